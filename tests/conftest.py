import hashlib
import random

import pytest
import torch


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs through libnt_mi355x.so)")


def _hash(text):
    return int(hashlib.sha256(text.encode("utf-8")).hexdigest(), 16) % 2**32


@pytest.fixture(autouse=True)
def _seed_per_test(request):
    # Same scheme as the reference suite (tests/conftest.py:8-37): seeds derived from
    # the SHA-256 of the test id.
    seed = _hash(f"{request.module.__name__}::{request.node.name}")
    random.seed(seed)
    torch.manual_seed(seed)
    yield


def gpu_available():
    return torch.cuda.is_available()


import os
import sys

# tests/programs.py and the repository root (for `oracle`) on the path.
_HERE = os.path.dirname(os.path.abspath(__file__))
for _p in (_HERE, os.path.dirname(_HERE)):
    if _p not in sys.path:
        sys.path.insert(0, _p)
