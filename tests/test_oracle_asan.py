"""The oracle's C restatement under AddressSanitizer and UBSan (CPU).

`make -C oracle asan` builds the same sources with -fsanitize=address,undefined
(liboracle_asan.so); the oracle's own CPU tests then run on that build in a
child process (QVEX_ORACLE_LIB names it, libasan is preloaded because the
interpreter itself is not instrumented, leak checks are off for the same
reason). Any out-of-bounds access or undefined behaviour in the index
arithmetic of oracle/*.c fails the run."""

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
ORACLE_TESTS = ["tests/test_oracle_qmv.py", "tests/test_oracle_affine.py", "tests/test_oracle_gdn.py",
                "tests/test_oracle_rng.py", "tests/test_oracle_spec.py", "tests/test_oracle_spec_filter.py",
                "tests/test_golden.py"]


def _libasan():
    if shutil.which("gcc") is None:
        return None
    r = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    p = r.stdout.strip()
    return p if r.returncode == 0 and os.path.isabs(p) and os.path.exists(p) else None


def test_oracle_tests_clean_under_asan_ubsan():
    asan = _libasan()
    if asan is None:
        pytest.skip("gcc with libasan not available")
    r = subprocess.run(["make", "-B", "-C", str(REPO / "oracle"), "asan"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ)
    env.update({"LD_PRELOAD": asan, "QVEX_ORACLE_LIB": str(REPO / "oracle" / "liboracle_asan.so"),
                "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
                "OMP_NUM_THREADS": "4"})
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
                        *ORACLE_TESTS], cwd=REPO, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    print(out[-3000:])
    assert r.returncode == 0, out[-6000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out
    assert " passed" in out
