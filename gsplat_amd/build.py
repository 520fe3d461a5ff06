"""Build recipe for libgsplat_hip.so (gfx950) -- plain hipcc, no torch headers.

Every ``gsplat_amd/csrc/*.hip`` file is compiled to an object for gfx950 and
linked into ``gsplat_amd/lib/libgsplat_hip.so``, the C-ABI library declared in
``include/gsplat_hip.h``.  The library links only against the HIP runtime, so
it can be loaded from any host language; the Python package reaches it through
``ctypes`` (``gsplat_amd/_lib.py``).

Run ``python gsplat_amd/build.py`` (or ``__graft_entry__.build()``): by path, since
importing the package loads the library this rebuilds.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shlex
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent


def _header_abi_hash() -> str:
    """abi.header_abi_hash(), with abi.py loaded by path: importing the
    package would load the library that is about to be rebuilt (and refuse a
    stale one)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_gsplat_amd_abi", PKG_DIR / "abi.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.header_abi_hash()

CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
OBJ_DIR = LIB_DIR / "obj"
LIB_PATH = LIB_DIR / "libgsplat_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=fast-honor-pragmas: fuse multiply-adds except where a
#   `#pragma clang fp contract(off)` region asks for exact IEEE op order
#   (the parts whose results must be reproducible bit for bit on the host).
# -packed-fp32-ops: packed FP32 instructions stay disabled on this pool.
# -munsafe-fp-atomics: float atomicAdd lowers to the native global atomic
#   (all buffers are ordinary device allocations).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast-honor-pragmas",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def _compile(src: Path, defines=()) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {src.name}:\n{shlex.join(cmd)}\n{res.stdout}\n{res.stderr}"
        )
    noisy = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l]
    if any(l.strip() for l in noisy):
        sys.stderr.write("\n".join(noisy) + "\n")
    return obj


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every HIP source and link libgsplat_hip.so; returns its path."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(8, os.cpu_count() or 4)
    # the interface digest the library reports from gsplat_abi_version()
    defines = [f'-DGSPLAT_ABI_HASH="{_header_abi_hash()}"']
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, defines), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{shlex.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[gsplat_amd.build] built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build()
