"""The reference's CompileRequest fields (reference src/ninetoothed/compiler/driver.py:37-54), test double."""

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True, kw_only=True)
class CompileRequest:
    arrangement: Any = None
    application: Any
    tensors: tuple = ()
    backend: Any = None
    caller: str = "torch"
    kernel_name: str = None
    num_warps: Any = None
    num_stages: Any = None
    max_num_configs: Any = None
    backend_options: Any = None
