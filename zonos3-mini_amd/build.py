"""Build ``libzonos3_gdn.so`` (all HIP sources under ``csrc/``) for gfx950 with hipcc, in-tree.

Usage: ``python zonos3-mini_amd/build.py`` (or ``build()`` from Python). Each ``.hip`` compiles to an object
in ``_build/`` in parallel, then one shared library ``lib/libzonos3_gdn.so`` is linked. Always rebuilds.
``python zonos3-mini_amd/build.py --asan`` (``build_asan()``) builds the AddressSanitizer check program of the
C ABI's validation paths instead.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = PKG / "lib"
LIB_NAME = "libzonos3_gdn.so"
ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the gated-DeltaNet kernels)")
    return path


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` and link ``lib/libzonos3_gdn.so``; returns the library path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    build_dir = PKG / "_build"
    build_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    objs = [build_dir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        list(pool.map(_compile, sources, objs))
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


# AddressSanitizer on the host code only (the device code is built as usual).
ASAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def build_asan(verbose: bool = False) -> Path:
    """The C-ABI validation checks (``tests/asan/abi_checks.cpp``) linked against every ``csrc/*.hip`` built
    with AddressSanitizer on its host code: ``_build/asan/abi_checks``, a CPU program (no GPU needed). Returns
    its path."""
    sources = sorted(CSRC.glob("*.hip"))
    asan_dir = PKG / "_build" / "asan"
    asan_dir.mkdir(parents=True, exist_ok=True)
    objs = [asan_dir / (s.stem + ".o") for s in sources]
    flags = [f if f != "-O3" else "-O1" for f in HIP_FLAGS] + ["-g", *ASAN_HOST]

    def one(src: Path, obj: Path) -> None:
        cmd = [hipcc(), *flags, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc (asan) failed on {src.name}:\n{' '.join(cmd)}\n{res.stderr}")

    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        list(pool.map(one, sources, objs))
    driver = ROOT / "tests" / "asan" / "abi_checks.cpp"
    exe = asan_dir / "abi_checks"
    rocm = Path(hipcc()).resolve().parent.parent
    gxx = shutil.which("g++") or "g++"
    cmd = [gxx, "-std=c++17", "-g", "-O1", "-fsanitize=address", f"-I{INCLUDE}", str(driver), *map(str, objs),
           f"-L{rocm / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{rocm / 'lib'}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"asan link failed:\n{' '.join(cmd)}\n{res.stderr}")
    if verbose:
        print(f"built {exe}")
    return exe


if __name__ == "__main__":
    if "--asan" in sys.argv:
        build_asan(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
