"""The oracle's C source under AddressSanitizer and UndefinedBehaviorSanitizer.

The CPU oracle checks every GPU result, so an out-of-bounds access or
undefined arithmetic in it would corrupt the parity tests silently.  This
test builds oracle/_asan/liboracle.so (`make -C oracle asan`: the checker's
source with -fsanitize=address,undefined and no OpenMP), then runs the
oracle's own CPU test files against that build in a child process with
libasan preloaded.  Any sanitizer report fails the child (UBSan halts on the
first error; ASan aborts on its first)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")
FILES = ["test_oracle_ring.py", "test_oracle_golden.py", "test_oracle_kernels.py",
         "test_oracle_model.py", "test_oracle_model_ref.py", "test_oracle_codec.py"]


def _libasan():
    try:
        path = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                              text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None
    return os.path.realpath(path) if os.path.isabs(path) and os.path.exists(path) else None


def test_oracle_tests_pass_under_asan_and_ubsan():
    asan = _libasan()
    if asan is None:
        pytest.skip("gcc's libasan is not available")
    subprocess.run(["make", "-s", "-C", ORACLE, "asan"], check=True)
    lib = os.path.join(ORACLE, "_asan", "liboracle.so")
    env = dict(os.environ, LD_PRELOAD=asan, MB_ORACLE_LIB=lib,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    # the child checks that it really loaded the sanitized build
    probe = ("from oracle import oracle; oracle.lib(); import os; "
             "m = open('/proc/self/maps').read(); "
             "assert os.environ['MB_ORACLE_LIB'] in m and 'libasan' in m")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    # (the mutant cases change only the numpy restatement, not the C code)
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "-m", "not gpu", "-k", "not mutant",
                        *[os.path.join("tests", f) for f in FILES]],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    print(out.strip().splitlines()[-1])
