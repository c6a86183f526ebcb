"""Host-side sanitizer run of libppo_hip.so, on the CPU only (no GPU is touched).

``python -m tt_rsl_rl_amd.sanitize_host`` compiles every csrc/*.hip with AddressSanitizer and UndefinedBehaviorSanitizer
on the host code only (device code is compiled as usual, unsanitized), links ``tt_rsl_rl_amd/libppo_hip_asan.so``, and
runs the tests that call the library's host paths without a GPU -- the C ABI's argument validation and status codes
(tests/test_lib_abi.py: every entry point's checks, struct layouts, the MT19937 / randperm ranges of the native
permutation) and the CPU-generator skipping (tests/test_host_rng.py) -- in a child process with the sanitizer runtime
preloaded.  Any sanitizer report aborts the run (halt_on_error, no recovery from undefined behaviour).  Leak checks are
off: the Python interpreter itself keeps allocations until exit.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

from . import build as B

LIB_ASAN = B.PKG / "libppo_hip_asan.so"
BUILD_DIR = B.CSRC / "_build_asan"
# the sanitizers apply to the host compilation only: each host flag goes behind its own -Xarch_host
HOST_SANITIZE = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=undefined",
                 "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]
TESTS = ["tests/test_lib_abi.py", "tests/test_host_rng.py"]


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [B.hipcc(), *B.HIPCC_FLAGS, *HOST_SANITIZE, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build() -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as pool:
        objs = list(pool.map(_compile, B.sources()))
    cmd = [B.hipcc(), f"--offload-arch={B.ARCH}", "-shared", "-fPIC", *HOST_SANITIZE, "-o", str(LIB_ASAN),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    return LIB_ASAN


def runtime() -> str:
    """The compiler's AddressSanitizer runtime (it carries the UndefinedBehaviorSanitizer handlers too)."""
    out = subprocess.run([B.hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True).stdout.strip()
    if not out or not Path(out).exists():
        raise RuntimeError("libclang_rt.asan-x86_64.so not found next to hipcc's clang")
    return out


def run_tests(extra: list[str] | None = None) -> int:
    env = dict(os.environ)
    env.update({"PPO_HIP_LIB": str(LIB_ASAN), "LD_PRELOAD": runtime(),
                "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1",
                "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1", "HIP_VISIBLE_DEVICES": ""})
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *TESTS, *(extra or [])]
    return subprocess.run(cmd, cwd=B.PKG.parent, env=env).returncode


if __name__ == "__main__":
    print(f"built {build()}", flush=True)
    sys.exit(run_tests(sys.argv[1:]))
