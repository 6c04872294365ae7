"""The C-ABI library's host code under AddressSanitizer (CPU only): the library rebuilt with ASan on the host side
(arcagi2_flashnext_dots3_amd/build_asan.py), loaded behind the clang ASan runtime, runs every argument check of
tests/test_abi.py; any ASan report fails the test. Skipped where hipcc or the ASan runtime is absent."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_abi_argument_checks_under_host_asan():
    from arcagi2_flashnext_dots3_amd import build, build_asan
    rt = build_asan.asan_runtime()
    if rt is None or not os.path.exists(build.HIPCC):
        pytest.skip("hipcc or the clang ASan runtime is not installed")
    lib = build_asan.build_asan()
    env = dict(os.environ, LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0", SPMLA_LIB=lib)
    probe = ("from arcagi2_flashnext_dots3_amd import _lib; _lib.lib(); "
             "print(open('/proc/self/maps').read().count('libspmla_gfx950_asan'))")
    r = subprocess.run([sys.executable, "-c", probe], cwd=REPO, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and int(r.stdout.strip().splitlines()[-1]) > 0, r.stderr[-2000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "tests/test_abi.py", "-q", "-m", "not gpu", "-p",
                        "no:cacheprovider"], cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
