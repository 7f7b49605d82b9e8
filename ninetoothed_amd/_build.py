"""Build libnt_mi355x.so from the hand-written gfx950 HIP sources in ``csrc/``.

Each ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` into an
object in ``_build/`` and the objects are linked into ``libnt_mi355x.so`` next to
this file.  The library is built in-tree so it travels with the source tree; the
runtime (``ninetoothed_amd._lib``) only loads what is already built.
"""

import concurrent.futures
import os
import shutil
import subprocess
import sysconfig
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY_NAME = "libnt_mi355x.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
OFFLOAD_ARCH = "gfx950"

# Packed-FP32 VALU forms are switched off: hipcc -O3 would otherwise emit them from
# ordinary float code.
COMMON_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
)


# Per-source flags.  attention.hip: builtin MFMAs keep their accumulators in VGPRs (its
# one-wave-per-SIMD kernel puts only the output accumulators in AGPRs, through inline
# assembly); without this the compiler would move every MFMA to AGPRs in that kernel and
# copy the scores back and forth.
FILE_FLAGS = {"attention.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form=1")}


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libnt_mi355x.so.")
    return found


def sources() -> list[Path]:
    return sorted(SOURCE_DIR.glob("*.hip"))


def _compile(source: Path, extra: tuple[str, ...]) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [
        hipcc(),
        *COMMON_FLAGS,
        *FILE_FLAGS.get(source.name, ()),
        *extra,
        f"-I{INCLUDE_DIR}",
        f"-I{SOURCE_DIR}",
        "-c",
        str(source),
        "-o",
        str(obj),
    ]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return obj


def build(verbose: bool = False, extra_flags: tuple[str, ...] = (), jobs: int | None = None) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {SOURCE_DIR}")
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, tuple(extra_flags)), srcs))
    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects), "-lhiprtc", "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    build_fastkey()
    if verbose:
        print(f"built {LIBRARY_PATH} from {len(srcs)} sources, and {fastkey_path().name}", file=sys.stderr)
    return LIBRARY_PATH


def fastkey_path() -> Path:
    return PACKAGE_DIR / ("_fastkey" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_fastkey() -> Path:
    """Compile csrc/fastkey.cpp (the Handle's call key in C++, a CPython module over torch's
    tensor metadata) with the host compiler against the installed torch."""
    import torch

    torch_dir = Path(torch.__path__[0])
    out = fastkey_path()
    tmp = out.with_name(out.name + ".tmp")
    cmd = [
        shutil.which("g++") or "g++", "-O2", "-shared", "-fPIC", "-std=c++17",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        f"-I{sysconfig.get_paths()['include']}", f"-I{torch_dir / 'include'}",
        f"-I{torch_dir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        str(SOURCE_DIR / "fastkey.cpp"), f"-L{torch_dir / 'lib'}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-Wl,-rpath,{torch_dir / 'lib'}", "-o", str(tmp),
    ]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"fastkey.cpp failed to build:\n{result.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build(verbose=True, extra_flags=tuple(sys.argv[1:]))
