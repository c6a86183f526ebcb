"""Build libppo_hip.so (all HIP sources under csrc/) for gfx950 with hipcc, in-tree.

Usage: ``python -m tt_rsl_rl_amd.build`` (or ``__graft_entry__.build()``).  Sources are compiled in parallel
to objects under ``csrc/_build/`` and linked into ``tt_rsl_rl_amd/libppo_hip.so``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
BUILD_DIR = CSRC / "_build"
LIB = PKG / "libppo_hip.so"
ARCH = os.environ.get("PPO_HIP_ARCH", "gfx950")

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 by itself on this target.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
# PPO_HIP_TUNING=1 at build time compiles the tile / split / wave variants and their environment overrides used for
# tuning sweeps; the default library holds only the configurations the tests cover.
if os.environ.get("PPO_HIP_TUNING") == "1":
    HIPCC_FLAGS.append("-DPPO_HIP_TUNING")


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libppo_hip.so")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip and link libppo_hip.so.  Always rebuilds."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources for {ARCH}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
