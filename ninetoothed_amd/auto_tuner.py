"""Auto-tuning: time every candidate launcher of a call once, then always run the fastest.

Public contract (the reference's constructor and call, ``src/ninetoothed/auto_tuner.py:14-30``):
``AutoTuner(funcs, keys, *, benchmark=None, cache_namespace=None, validator=None)`` with one
key per candidate; ``tuner(*args, **kwargs)`` runs ``validator(args, kwargs)`` if given,
chooses a candidate for the call's signature and returns that candidate's result.  A
candidate whose benchmark raises is never chosen; when all of them raise, ``RuntimeError``
names every candidate with its reason.  ``benchmark(func, args, kwargs)`` returns a time
(any unit, smaller is better).

How it is organised here:

* **Signature** of a call (``signature``): a JSON string of each argument's description.
  Tensors are described by dtype, shape, strides, device and whether the data pointer is
  16-byte aligned (kernels with vector loads accept only aligned operands, so an aligned
  and a misaligned call of one shape are different tuning problems); other values by
  their ``repr``.
* **Timing book** (``TimingBook``): one JSON file per (namespace, candidate keys, kernel
  library build) under ``$NINETOOTHED_AMD_CACHE_DIR/tuning`` (default
  ``~/.cache/ninetoothed_amd``), holding ``{signature: {candidate label: milliseconds or
  "error: ..."}}``.  The build is a digest of ``libnt_mi355x.so``, so timings of one
  build never choose among another build's kernels.  Entries are merged into the file
  under a process-wide lock and written atomically, so several tuners and processes
  share what was measured and a new process re-times no candidate it finds timed there.
* **Election**: the first call with a new signature benchmarks every candidate of its row
  that has no finite time yet (a recorded failure counts as none, as the reference's
  infinite timing does, so a transient failure or a fixed bug is retried), takes the
  smallest time, runs the winner, and remembers it in memory only once that run returned
  (a winner that raises is not kept).

Handles use it when ``make``/``jit`` get ``max_num_configs`` > 1: the candidates are the
kernel plans (and kernel configurations) that fit the call; programs that update a tensor
they read are never tuned, since timing them would change their output.
"""

import hashlib
import json
import math
import os
import threading
import time
from pathlib import Path

_BOOK_LOCK = threading.Lock()


def cache_dir():
    root = os.environ.get("NINETOOTHED_AMD_CACHE_DIR")
    return Path(root) if root else Path.home() / ".cache" / "ninetoothed_amd"


def _describe(value):
    if hasattr(value, "shape") and hasattr(value, "dtype"):
        stride = list(value.stride()) if hasattr(value, "stride") else None
        pointer = value.data_ptr() if hasattr(value, "data_ptr") else 0
        return ["tensor", str(value.dtype).replace("torch.", ""), list(value.shape), stride,
                str(getattr(value, "device", "")), pointer % 16 == 0]
    return repr(value)


def signature(args, kwargs):
    """The tuning key of a call: what a kernel's speed and admissibility depend on."""
    return json.dumps([[_describe(a) for a in args], [[k, _describe(v)] for k, v in sorted(kwargs.items())]],
                      separators=(",", ":"))


def _label(key):
    return key if isinstance(key, str) else json.dumps(key, sort_keys=True, default=str)


_BUILD = None


def library_build():
    """Digest of the kernel library this process loads ("none" when it is not built)."""
    global _BUILD
    if _BUILD is None:
        from ninetoothed_amd import _lib

        try:
            _BUILD = hashlib.sha256(Path(_lib.LIBRARY_PATH).read_bytes()).hexdigest()[:16]
        except OSError:
            _BUILD = "none"
    return _BUILD


class TimingBook:
    """Measured times per call signature and candidate label, persisted as one JSON file."""

    def __init__(self, namespace, labels):
        ident = json.dumps({"namespace": namespace, "labels": list(labels), "build": library_build()},
                           sort_keys=True)
        digest = hashlib.sha256(ident.encode()).hexdigest()[:20]
        self.path = cache_dir() / "tuning" / f"{digest}.json"
        self.rows = {}

    def _load(self):
        try:
            data = json.loads(self.path.read_text())
        except (OSError, ValueError):
            return {}
        return data.get("rows", {}) if isinstance(data, dict) else {}

    def row(self, sig):
        """What is known for ``sig`` (re-reading the file when this process knows nothing yet)."""
        if sig not in self.rows:
            stored = self._load().get(sig)
            if stored:
                self.rows[sig] = dict(stored)
        return dict(self.rows.get(sig, {}))

    def record(self, sig, entries):
        with _BOOK_LOCK:
            rows = self._load()
            merged = dict(rows.get(sig, {}))
            merged.update(entries)
            rows[sig] = merged
            self.rows[sig] = merged
            self.path.parent.mkdir(parents=True, exist_ok=True)
            tmp = self.path.with_name(f"{self.path.name}.{os.getpid()}.{threading.get_ident()}")
            tmp.write_text(json.dumps({"rows": rows}, indent=1, sort_keys=True))
            os.replace(tmp, self.path)


def _time_of(entry):
    return float(entry) if isinstance(entry, (int, float)) else math.inf


class AutoTuner:
    """Run the fastest of several interchangeable launchers, timed once per call signature."""

    def __init__(self, funcs, keys, *, benchmark=None, cache_namespace=None, validator=None):
        funcs, keys = tuple(funcs), tuple(keys)
        if not funcs or len(funcs) != len(keys):
            raise ValueError("AutoTuner requires one key for every candidate.")
        self.candidates = funcs
        self.labels = tuple(_label(k) for k in keys)
        self.keys = keys
        self.book = TimingBook(cache_namespace or "default", self.labels)
        self._measure = benchmark or default_benchmark
        self._validator = validator
        self._winners = {}  # signature -> candidate index, kept once the winner has run
        self._lock = threading.Lock()

    def __call__(self, *args, **kwargs):
        if self._validator is not None:
            self._validator(args, kwargs)
        sig = signature(args, kwargs)
        index = self._winners.get(sig)
        if index is not None:
            return self.candidates[index](*args, **kwargs)
        with self._lock:
            index = self._elect(sig, args, kwargs)
            result = self.candidates[index](*args, **kwargs)
            self._winners[sig] = index
        return result

    def choose(self, *args, **kwargs):
        """Index of the candidate chosen for these arguments (timing them if needed), without running it."""
        sig = signature(args, kwargs)
        with self._lock:
            return self._elect(sig, args, kwargs)

    def timings(self, *args, **kwargs):
        """Candidate label -> recorded time or error for these arguments (empty before any election)."""
        return self.book.row(signature(args, kwargs))

    def _elect(self, sig, args, kwargs):
        row = self.book.row(sig)
        fresh = {}
        for func, label in zip(self.candidates, self.labels):
            if not math.isinf(_time_of(row.get(label))):
                continue  # timed before; a failure (or no entry) is timed again
            try:
                fresh[label] = float(self._measure(func, args, kwargs))
            except Exception as exc:  # noqa: BLE001  (a failing candidate is recorded, not raised)
                fresh[label] = f"error: {type(exc).__name__}: {exc}"
        if fresh:
            self.book.record(sig, fresh)
            row.update(fresh)
        times = [_time_of(row.get(label)) for label in self.labels]
        best = min(range(len(times)), key=times.__getitem__)
        if math.isinf(times[best]):
            reasons = "; ".join(f"{label}: {_reason(row.get(label))}" for label in self.labels)
            raise RuntimeError(f"All auto-tuning candidates failed: {reasons}")
        return best


def _reason(entry):
    if isinstance(entry, str) and entry.startswith("error: "):
        return entry[len("error: "):]
    return f"no finite timing ({entry})"


def default_benchmark(func, args, kwargs, *, target_ms=20.0, max_calls=200):
    """Milliseconds per call of ``func(*args, **kwargs)``.

    On a GPU: one untimed call, one timed call to size the batch, then a batch of calls
    lasting about ``target_ms`` timed with events on the current stream (the stream the
    launchers use).  Without a GPU: wall clock over a batch of the same size."""
    import torch

    if not torch.cuda.is_available():
        func(*args, **kwargs)
        start = time.perf_counter()
        func(*args, **kwargs)
        once = max(time.perf_counter() - start, 1e-6) * 1e3
        calls = max(1, min(max_calls, int(target_ms / once)))
        start = time.perf_counter()
        for _ in range(calls):
            func(*args, **kwargs)
        return (time.perf_counter() - start) * 1e3 / calls
    stream = torch.cuda.current_stream()
    func(*args, **kwargs)
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    func(*args, **kwargs)
    end.record(stream)
    end.synchronize()
    once = max(begin.elapsed_time(end), 1e-3)
    calls = max(3, min(max_calls, int(target_ms / once)))
    begin.record(stream)
    for _ in range(calls):
        func(*args, **kwargs)
    end.record(stream)
    end.synchronize()
    return begin.elapsed_time(end) / calls
