"""Build recipe for ``libyapd_t3.so`` (gfx950 only).

Compiles every ``csrc/*.hip`` and ``csrc/*.cpp`` with ``hipcc`` into
``yapd_amd/_lib/libyapd_t3.so`` in-tree, so the built library travels with
the source tree.  Usage: ``python -m yapd_amd.build`` (or ``build()``).
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
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libyapd_t3.so"
OBJDIR = PKG / "_build"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # Packed fp32 VALU ops (v_pk_*_f32) are kept off on purpose.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]
# Files whose fp32 op order must follow the reference exactly (no FMA contraction).
PER_FILE_FLAGS = {
    "score.hip": ["-ffp-contract=off"],
    "voc_stitch.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build yapd_amd")
    return path


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.name + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def sources():
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, os.cpu_count() or 1, len(srcs))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    # export only the C ABI (yapd_*); internal C++ helpers stay local to the library
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={CSRC / 'exports.map'}",
           "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
