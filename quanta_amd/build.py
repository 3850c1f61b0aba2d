"""Build the gfx950 HIP extension `quanta_amd/_qmoe.so` in-tree with hipcc.

    python -m quanta_amd.build          # compile (always recompiles)

The library is a plain C-ABI shared object (include/quanta_moe.h) loaded with ctypes; no torch
headers are involved, so the build needs only ROCm's hipcc. Objects are compiled in parallel
into quanta_amd/_build/ and linked into quanta_amd/_qmoe.so.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "_qmoe.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-but-set-variable",
    # Packed FP32 VALU forms are kept out of every kernel (hipcc otherwise forms them from
    # scalar float code); the host pass warns that it does not know the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the quanta_amd extension needs ROCm's hipcc")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(PKG.parent / "include"), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    warn = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if warn.strip():
        print(f"[quanta_amd.build] {src.name}:\n{warn}", file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link quanta_amd/_qmoe.so. Always recompiles."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError("no HIP sources found")
    workers = min(len(srcs), max(1, (os.cpu_count() or 4) // 2), 8)
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[quanta_amd.build] built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
