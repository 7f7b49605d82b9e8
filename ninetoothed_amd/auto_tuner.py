"""Auto-tuning: pick the fastest of several candidate launchers per argument key.

The reference's contract (``src/ninetoothed/auto_tuner.py:14-202``): ``AutoTuner(funcs,
keys, *, benchmark=None, cache_namespace=None, validator=None)``; a call validates the
arguments, looks up the best candidate for their key (shapes, strides, dtypes, devices
and the other values), benchmarks every candidate the first time a key is seen — a
candidate that raises gets an infinite timing and the reason is kept — and runs the
winner.  Timings persist per candidate and per selection in JSON files under the cache
directory (``$NINETOOTHED_AMD_CACHE_DIR``, default ``~/.cache/ninetoothed_amd``), in a
folder named by a digest of the namespace and the candidate keys, so a new process
reuses them without benchmarking.

Handles use it when ``make``/``jit`` get ``max_num_configs`` > 1: the candidates are the
kernel plans of every family whose pattern and geometry fit the call (e.g. the
elementwise add kernel and the generic kernel), never for programs that update a tensor
they also read.
"""

import hashlib
import json
import math
import os
import threading
import time
from pathlib import Path


def cache_dir():
    root = os.environ.get("NINETOOTHED_AMD_CACHE_DIR")
    return Path(root) if root else Path.home() / ".cache" / "ninetoothed_amd"


def _digest(obj):
    return hashlib.sha256(json.dumps(obj, sort_keys=True, default=str).encode()).hexdigest()[:24]


def _read(path):
    try:
        return json.loads(Path(path).read_text())
    except (OSError, ValueError):
        return None


def _write(path, data):
    path = Path(path)
    tmp = path.with_suffix(f".{os.getpid()}.{threading.get_ident()}.tmp")
    tmp.write_text(json.dumps(data, indent=1, sort_keys=True))
    os.replace(tmp, path)


def _candidate_id(key):
    return key if isinstance(key, str) else json.dumps(key, sort_keys=True, default=str)


class AutoTuner:
    """Select a runtime candidate using an injectable benchmark strategy."""

    _process_lock = threading.Lock()

    def __init__(self, funcs, keys, *, benchmark=None, cache_namespace=None, validator=None):
        self._funcs = tuple(funcs)
        self._keys = tuple(keys)
        if not self._funcs or len(self._funcs) != len(self._keys):
            raise ValueError("AutoTuner requires one key for every candidate.")
        self._benchmark = benchmark or _default_benchmark
        self._validator = validator
        self._lock = threading.Lock()
        self._key_ids = tuple(_candidate_id(k) for k in self._keys)
        self._func_to_key = dict(zip(self._funcs, self._key_ids))
        namespace = cache_namespace or "default"
        self._cache_dir = cache_dir() / "auto_tuning" / _digest(
            {"schema": 1, "namespace": namespace, "candidate_ids": self._key_ids})
        self._cache_dir.mkdir(parents=True, exist_ok=True)
        self._cache_path = self._cache_dir / "selection.json"
        self._selection_timings = dict((_read(self._cache_path) or {}).get("timings", {}))
        self._candidate_timings = {k: {} for k in self._key_ids}
        self._best_func = {}

    def __call__(self, *args, **kwargs):
        if self._validator is not None:
            self._validator(args, kwargs)
        arg_key = self._make_arg_key(args, kwargs)
        with self._lock:
            best = self._best_func.get(arg_key)
            if best is None:
                timings = self._get_timings(args, kwargs)
                if all(math.isinf(t) for t in timings):
                    raise RuntimeError(self._all_candidates_failed_message(arg_key))
                best = self._funcs[timings.index(min(timings))]
                self._best_func[arg_key] = best
        return best(*args, **kwargs)

    def best(self, *args, **kwargs):
        """The candidate key chosen for these arguments (benchmarking them if needed)."""
        arg_key = self._make_arg_key(args, kwargs)
        with self._lock:
            timings = self._get_timings(args, kwargs)
        return self._keys[timings.index(min(timings))]

    def _get_timings(self, args, kwargs):
        arg_key = self._make_arg_key(args, kwargs)
        with self._process_lock:
            self._selection_timings.update((_read(self._cache_path) or {}).get("timings", {}))
            cached = self._selection_timings.get(arg_key)
            if cached is not None and not all(math.isinf(t) for t in cached):
                return list(cached)
            timings = [self._get_timing(f, args, kwargs) for f in self._funcs]
            self._selection_timings[arg_key] = timings
            _write(self._cache_path, {"schema": 1, "timings": self._selection_timings})
        return timings

    def _get_timing(self, func, args, kwargs):
        key_id = self._func_to_key[func]
        data = self._candidate_timings[key_id]
        arg_key = self._make_arg_key(args, kwargs)
        if arg_key in data and not math.isinf(data[arg_key]):
            return data[arg_key]
        path = self._get_func_cache_path(func)
        manifest = _read(path) or {}
        data.update(manifest.get("timings", {}))
        if arg_key in data and not math.isinf(data[arg_key]):
            return data[arg_key]
        failures = dict(manifest.get("failures", {}))
        try:
            timing = float(self._benchmark(func, args, kwargs))
            failures.pop(arg_key, None)
        except Exception as exc:  # noqa: BLE001  (a failing candidate is recorded, not raised)
            timing = float("inf")
            failures[arg_key] = f"{type(exc).__name__}: {exc}"
        data[arg_key] = timing
        _write(path, {"schema": 1, "timings": data, "failures": failures})
        return timing

    def _get_func_cache_path(self, func):
        return self._cache_dir / f"{_digest({'schema': 1, 'candidate_id': self._func_to_key[func]})}.json"

    def _all_candidates_failed_message(self, arg_key):
        reasons = []
        for func, key_id in zip(self._funcs, self._key_ids):
            manifest = _read(self._get_func_cache_path(func)) or {}
            reasons.append(f"{key_id}: " + manifest.get("failures", {}).get(arg_key,
                                                                              "benchmark returned an infinite timing"))
        return "All auto-tuning candidates failed: " + "; ".join(reasons)

    @staticmethod
    def _make_arg_key(args, kwargs):
        def one(a):
            if hasattr(a, "shape") and hasattr(a, "dtype"):
                stride = tuple(a.stride()) if hasattr(a, "stride") else None
                return (f"tensor(shape={tuple(a.shape)}, stride={stride}, dtype={str(a.dtype).split('.')[-1]}, "
                        f"device={getattr(a, 'device', None)})")
            return str(a)

        parts = [one(a) for a in args] + [f"{k}={one(v)}" for k, v in sorted(kwargs.items())]
        return ", ".join(parts)


def _default_benchmark(function, args, kwargs, *, warmup=2, repeat=10):
    """Median time in milliseconds of ``function(*args, **kwargs)`` on the current stream."""
    import torch

    if not torch.cuda.is_available():
        start = time.perf_counter()
        for _ in range(repeat):
            function(*args, **kwargs)
        return (time.perf_counter() - start) * 1e3 / repeat
    for _ in range(warmup):
        function(*args, **kwargs)
    times = []
    for _ in range(repeat):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        function(*args, **kwargs)
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    return times[len(times) // 2]
