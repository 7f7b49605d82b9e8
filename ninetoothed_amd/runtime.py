"""Handle: the callable that ``make``/``jit`` return, and its call contract.

Mirrors the reference's runtime contract (``src/ninetoothed/compiler/runtime.py``):
  - ``handle(*public_args, **meta_or_public_kwargs)``, public args in application order;
  - ``TypeError`` for too many / duplicate / unknown / missing arguments
    (runtime.py:1147-1185), for rank or static-dim mismatches, for tensors that are not
    on the GPU (device type ``cuda`` under PyTorch-ROCm) or not all on one GPU
    (runtime.py:1218-1264), and for dtype mismatches with declared dtypes
    (runtime.py:1282-1294);
  - an empty output launches nothing and returns the first output (runtime.py:1411-1422);
  - otherwise launch on the caller's current stream and return the first output;
  - a non-zero library status raises ``KernelLaunchError`` (runtime.py:31-35).
Dtype-less tensors are specialised lazily per call-time key (dtypes, shapes,
strides, constexpr and meta values), as the reference does for non-Triton backends
(runtime.py:158-243); each key is matched once to a kernel family and cached.

A call with every public argument given positionally goes through a second cache
keyed on (dtype, shape, strides, device, data-pointer alignment) of each tensor, the value of each
constexpr, the type of each other scalar and the meta keywords; the tensors' part of that key is
built in C++ (`_fastkey`, from csrc/fastkey.cpp) where that module is built.  A key enters it
only after a call with that key passed every check above, so a hit goes straight
to the bound launcher (which reads data pointers, scalars and the current stream).
"""

import threading

from ninetoothed_amd import jagged
from ninetoothed_amd.dtype import normalize_dtype

try:  # the call key in C++ (csrc/fastkey.cpp, built by ninetoothed_amd._build); else built in Python
    from ninetoothed_amd import _fastkey
except ImportError:
    _fastkey = None
from ninetoothed_amd.errors import KernelLaunchError, LoweringError  # noqa: F401  (re-exported)


def _device_type_description(device_types):
    labels = ["CUDA" if d == "cuda" else d.upper() for d in device_types]
    return f"a {labels[0]} device" if len(labels) == 1 else f"one of these devices: {', '.join(labels)}"


class Handle:
    """A compiled NineToothed kernel bound to the MI355X backend."""

    def __init__(self, compilation, library_path=None):
        self._compilation = compilation
        self._artifact = compilation.artifact
        self._backend = compilation.target.backend.value
        self._platform = compilation.target.platform.name
        self._library = None if library_path is None else str(library_path)
        self._kernel = compilation.kernel
        self._abi = compilation.launch_abi
        self._plans = {}
        self._lock = threading.Lock()
        self._device_types = compilation.target.platform.device_types
        names = self._abi["public_args"]
        specs = {spec.name: spec for spec in self._kernel.param_specs}
        self._index = {n: i for i, n in enumerate(names)}
        # per position: 0 tensor, 1 constexpr scalar, 2 runtime scalar
        self._kinds = tuple(
            0 if specs[n].source_ndim != 0 else (1 if specs[n].constexpr else 2) for n in names
        )
        outputs = self._abi["outputs"]
        self._ret = self._index[outputs[0]] if outputs else None
        self._tensor_pos = tuple(i for i, k in enumerate(self._kinds) if k == 0)
        self._all_tensors = len(self._tensor_pos) == len(self._kinds)
        self._launchers = {}
        # max_num_configs > 1: pick among every fitting kernel by timing (auto_tuner.AutoTuner)
        request = compilation.request
        configs = getattr(request, "max_num_configs", None) if request is not None else None
        self._tune = isinstance(configs, int) and configs > 1

    # --------------------------------------------------------------- contract
    def __call__(self, *args, **kwargs):
        if len(args) == len(self._kinds):
            try:
                key = self._fast_key(args, kwargs)
                launch = self._launchers.get(key)
            except (AttributeError, TypeError):  # not a tensor, or unhashable: the checks below report it
                key = launch = None
            if launch is not None:
                launch(args)
                return None if self._ret is None else args[self._ret]
        else:
            key = None
        public, meta = self._public_values(args, kwargs)
        outputs = self._abi["outputs"]
        if any(hasattr(public.get(n), "numel") and public[n].numel() == 0 for n in outputs):
            return public[outputs[0]] if outputs else None
        plan_key = self._key(public, meta)
        plan = self._plans.get(plan_key)
        if plan is None:
            with self._lock:
                plan = self._plans.get(plan_key)
                if plan is None:
                    plan = self._kernel.specialize(public, meta, tune=self._tune)
                    self._plans[plan_key] = plan
        if key is not None:
            launch = plan.bind(public, self._index)
            launch(args)
            self._launchers[key] = launch
        else:
            plan.run(public)
        return public[outputs[0]] if outputs else None

    def _fast_key(self, args, kwargs):
        # A tensor's data-pointer alignment is part of the key: a launcher bound (or tuned)
        # for 16-byte aligned operands may have chosen a kernel that needs them.  The device
        # enters as its index (get_device: -1 off the GPU), which hashes far faster than a
        # torch.device object and tells the same tensors apart (all GPU tensors here report
        # one device type).
        if _fastkey is not None:
            tensors = args if self._all_tensors else tuple([args[i] for i in self._tensor_pos])
            key = _fastkey.key(tensors)
            if key is None:
                raise TypeError("not a tensor")  # the checks of the full path report it
            if not self._all_tensors:
                key = (key, tuple([v if kind == 1 else type(v) for v, kind in zip(args, self._kinds) if kind != 0]))
        else:
            if any(getattr(args[i], "is_nested", False) for i in self._tensor_pos):
                raise TypeError("a nested tensor")  # jagged calls take the full path every time
            key = tuple([
                (v.dtype, v.shape, v.stride(), v.get_device(), v.data_ptr() & 15) if kind == 0
                else (v if kind == 1 else type(v))
                for v, kind in zip(args, self._kinds)
            ])
        if kwargs:
            key = (key, tuple(sorted(kwargs.items())))
        return key

    def _public_values(self, args, kwargs):
        abi = self._abi
        names = abi["public_args"]
        if len(args) > len(names):
            raise TypeError(f"Expected at most {len(names)} arguments.")
        positional = names[: len(args)]
        duplicates = [n for n in positional if n in kwargs]
        if duplicates:
            raise TypeError(f"Kernel arguments passed twice: {', '.join(sorted(duplicates))}.")
        accepted = set(names) | set(abi["meta_args"])
        unknown = [n for n in kwargs if n not in accepted]
        if unknown:
            raise TypeError(f"Unknown kernel arguments: {', '.join(sorted(unknown))}.")
        values = dict(zip(names, args))
        meta = {}
        for k, v in kwargs.items():
            (values if k in names else meta)[k] = v
        missing = [n for n in names if n not in values]
        if missing:
            raise TypeError(f"Missing kernel arguments: {', '.join(missing)}.")
        self._validate(values)
        return values, meta

    def _validate(self, values):
        expected_device = None
        for spec in self._kernel.param_specs:
            value = values[spec.name]
            if spec.source_ndim == 0:
                continue
            shape = getattr(value, "shape", None)
            if shape is None:
                raise TypeError(f"Kernel argument `{spec.name}` must be a tensor.")
            if len(shape) != spec.source_ndim:
                raise TypeError(f"Kernel argument `{spec.name}` has rank {len(shape)}; expected {spec.source_ndim}.")
            if jagged.is_jagged(value) or getattr(value, "is_nested", False) or spec.jagged_dim is not None:
                if spec.jagged_dim is None or not jagged.is_jagged(value) or jagged.ragged_dim(value) != spec.jagged_dim:
                    raise TypeError(
                        f"Kernel argument `{spec.name}` must be "
                        + (f"a jagged nested tensor ragged in dimension {spec.jagged_dim}." if spec.jagged_dim is not None
                           else "a strided tensor (its Tensor has no `jagged_dim`).")
                    )
                shape = jagged.padded_shape(value)
            for axis, (actual, expected) in enumerate(zip(shape, spec.static_shape)):
                if expected is not None and actual != expected:
                    raise TypeError(
                        f"Kernel argument `{spec.name}` has shape {tuple(shape)}; expected dimension {axis} to be {expected}."
                    )
            device = getattr(value, "device", None)
            if device is not None:
                if device.type not in self._device_types:
                    raise TypeError(f"Kernel argument `{spec.name}` must be on {_device_type_description(self._device_types)}.")
                if expected_device is not None and device != expected_device:
                    raise TypeError("All tensor arguments must use the same CUDA device.")
                expected_device = expected_device or device
            if spec.dtype is not None and hasattr(value, "dtype"):
                actual = str(value.dtype).split(".")[-1]
                expected = normalize_dtype(spec.dtype)
                if actual != expected:
                    raise TypeError(f"Kernel argument `{spec.name}` has dtype {actual}; expected {expected}.")

    def _key(self, public, meta):
        parts = []
        for spec in self._kernel.param_specs:
            v = public[spec.name]
            if spec.source_ndim == 0:
                parts.append((spec.name, v if spec.constexpr else type(v).__name__))
            elif jagged.is_jagged(v):
                # the plan depends on the padded shape; index tables are built per call
                parts.append((spec.name, v.dtype, "jagged", jagged.padded_shape(v), v.values().stride()))
            else:
                parts.append((spec.name, v.dtype, tuple(v.shape), v.stride()))
        parts.append(tuple(sorted(meta.items())))
        return tuple(parts)

    # ---------------------------------------------------------- introspection
    def plans(self):
        """Matched kernel families so far, one per specialisation key."""
        return [p.describe() for p in self._plans.values()]

    @property
    def library(self):
        return self._library
