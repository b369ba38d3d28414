"""Build libmono_gfx950.so in-tree with hipcc for gfx950 (no JIT, no cache outside the tree).

``python -m sgl_amd_mono_amd.build`` compiles every ``csrc/*.hip`` and ``csrc/*.cpp``
to ``_build/*.o`` in parallel and links the shared library next to this file.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmono_gfx950.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed-FP32 VALU forms stay off: the compiler may still emit scalar FP32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


# Per-source flags. The multi-layer kernel runs every phase in a loop over the layers:
# without machine loop-invariant code motion the compiler keeps each phase's constants
# where they are used instead of holding them across the loop (they would spill).
EXTRA = {
    "layer_stack.hip": ["-mllvm", "-disable-machine-licm"],
}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + src.suffix.replace(".", "_") + ".o")
    cmd = [hipcc(), *COMMON, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile and link; returns the library path. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
