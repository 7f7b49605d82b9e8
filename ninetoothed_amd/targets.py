"""Platform profile of the MI355X backend.

The reference keeps per-vendor ``PlatformProfile`` records and resolves the target
from arguments and ``NINETOOTHED_BACKEND`` / ``NINETOOTHED_PLATFORM`` /
``NINETOOTHED_COMPUTE_ARCH`` (``src/ninetoothed/targets.py:16-204, 630-658``).  Here
there is one profile: AMD Instinct MI355X, gfx950, whose PyTorch-ROCm tensors report
device type ``cuda``.
"""

import os
from dataclasses import dataclass

from ninetoothed_amd.backends.core import Target, normalize_target


@dataclass(frozen=True)
class PlatformProfile:
    name: str
    vendor: str
    compute_arch: str
    device_types: tuple
    backend_modes: tuple
    wavefront_size: int
    compute_units: int
    lds_bytes_per_cu: int
    hbm_bytes: int
    peak_hbm_bytes_per_s: float
    peak_mfma_flops: dict


MI355X = PlatformProfile(
    name="amd-mi355x",
    vendor="amd",
    compute_arch="gfx950",
    device_types=("cuda",),
    backend_modes=(Target.HIP,),
    wavefront_size=64,
    compute_units=256,
    lds_bytes_per_cu=160 * 1024,
    hbm_bytes=288 * 1024**3,
    peak_hbm_bytes_per_s=8.0e12,
    peak_mfma_flops={"float16": 2.5166e15, "bfloat16": 2.5166e15, "float32": 157.3e12, "float64": 78.6e12},
)

PROFILES = {MI355X.name: MI355X, "mi355x": MI355X, "gfx950": MI355X}


@dataclass(frozen=True)
class TargetContext:
    backend: Target
    platform: PlatformProfile
    compute_arch: str


def resolve_target_context(backend=None, platform=None, compute_arch=None) -> TargetContext:
    backend = normalize_target(backend if backend is not None else os.environ.get("NINETOOTHED_BACKEND") or None)
    platform_name = platform or os.environ.get("NINETOOTHED_PLATFORM") or MI355X.name
    try:
        profile = PROFILES[str(platform_name).lower()]
    except KeyError:
        raise ValueError(f"Unsupported platform `{platform_name}`. Available: {', '.join(sorted(PROFILES))}.") from None
    arch = compute_arch or os.environ.get("NINETOOTHED_COMPUTE_ARCH") or profile.compute_arch
    if arch != profile.compute_arch:
        raise ValueError(f"The MI355X backend compiles for {profile.compute_arch}, not {arch}.")
    if backend not in profile.backend_modes:
        raise ValueError(f"Platform `{profile.name}` does not run backend `{backend.value}`.")
    return TargetContext(backend, profile, arch)
