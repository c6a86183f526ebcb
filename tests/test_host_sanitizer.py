"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU: a build with the host
compilation sanitized (device code as usual) runs the C-ABI and host-RNG tests in a child process with the sanitizer
runtime preloaded; any report fails the run (tt_rsl_rl_amd/sanitize_host.py)."""

from __future__ import annotations

import shutil

import pytest


@pytest.mark.timeout(900)
def test_host_paths_clean_under_asan_and_ubsan():
    if shutil.which("hipcc") is None and not shutil.os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    try:
        from tt_rsl_rl_amd import sanitize_host
    except ImportError:
        pytest.skip("the sanitizer recipe is not part of this copy of the tree")
    sanitize_host.build()
    assert sanitize_host.run_tests() == 0
