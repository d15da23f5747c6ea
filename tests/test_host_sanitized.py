"""The host side of the boundary under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU.

The C ABI's host code (argument checks, context set-up and its error and
clean-up paths, in the csrc/*.hip files) and the N-API addon's marshalling
(mb_napi.cc) run here instrumented: mockbird_amd.build.build_sanitized()
builds them with -fsanitize=address,undefined on the host side only (the GPU
code is compiled as usual), and the boundary's own CPU tests -- the export
list and null-context sweep of test_abi.py, the JS engine's exports, weight
resolution and argument errors of test_engine_js.py -- run against that build
in a child process with clang's ASan runtime preloaded (Python and Node
themselves are not instrumented).  Any sanitizer report fails the child:
UBSan halts on its first error, ASan aborts on its first.  Leak checking is
off (the interpreters keep their allocations to the end)."""
import os
import subprocess
import sys

import pytest

from mockbird_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FILES = ["test_abi.py", "test_engine_js.py"]


def test_boundary_host_code_under_asan_and_ubsan():
    rt = build.asan_runtime()
    if rt is None:
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    if build.sanitized_stale():
        build.build_sanitized()
    env = dict(os.environ, LD_PRELOAD=rt, MB_HIP_LIB=build.ASAN_LIB,
               MB_HIP_ADDON=build.ASAN_ADDON,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    # the child checks that it really loaded the sanitized builds
    probe = ("import mockbird_amd as mb; mb.load(); import os; "
             "m = open('/proc/self/maps').read(); "
             "assert os.environ['MB_HIP_LIB'] in m and 'libclang_rt.asan' in m")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    r = subprocess.run(["node", "-e", "const fs = require('fs'); "
                        "process.dlopen({exports: {}}, process.env.MB_HIP_ADDON); "
                        "const m = fs.readFileSync('/proc/self/maps', 'utf8'); "
                        "if (!m.includes(process.env.MB_HIP_LIB) || !m.includes('libclang_rt.asan')) "
                        "process.exit(3);"], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "-m", "not gpu", *[os.path.join("tests", f) for f in FILES]],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    print(out.strip().splitlines()[-1])
