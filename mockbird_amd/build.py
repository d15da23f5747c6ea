"""Build libmockbird_hip.so (gfx950) and the Node N-API addon in-tree.

    python -m mockbird_amd.build            # library + addon
    python -m mockbird_amd.build --lib-only
    python -m mockbird_amd.build --sanitized  # also the host-sanitized build

hipcc compiles each csrc/*.hip file for gfx950 only; objects go to
mockbird_amd/_build/ and the shared library to mockbird_amd/libmockbird_hip.so.
Packed fp32 instructions are disabled on every HIP compile line.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libmockbird_hip.so")
PROBE_LIB = os.path.join(PKG, "libmb_probe.so")
TIMELINE_LIB = os.path.join(PKG, "libmockbird_hip_timeline.so")
ADDON = os.path.join(PKG, "engine", "mockbird_hip.node")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"),
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"compile failed: {cmd[-1] if cmd else ''}")
    if r.stderr.strip():
        # keep warnings visible, minus hipcc's host-pass note about the packed-fp32 feature
        lines = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if any(ln.strip() for ln in lines):
            sys.stderr.write("\n".join(lines) + "\n")


def build_lib(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = []
    cmds = []
    for src in sources:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, LIB)
    return LIB


def build_probe() -> str:
    """libmb_probe.so: bench.py's HBM read-ceiling kernel (measurement only)."""
    src = os.path.join(CSRC, "probe", "hbm_read.hip")
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", src, "-o", tmp, f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_timeline() -> str:
    """libmockbird_hip_timeline.so: the library with ring.hip built under
    -DMB_BLOCK_TIMELINE=1, so that every decode-attention block records its
    start and end times and the CU that ran it (mb_probe_block_stamps).  For
    bench.py's timeline leg only (measurement, loaded through MB_HIP_LIB);
    links the other objects of build_lib()."""
    obj = os.path.join(BUILD, "ring.timeline.o")
    _run([HIPCC, *HIP_FLAGS, "-DMB_BLOCK_TIMELINE=1", "-c", os.path.join(CSRC, "ring.hip"),
          "-o", obj])
    objs = [os.path.join(BUILD, os.path.basename(src) + ".o")
            for src in sorted(glob.glob(os.path.join(CSRC, "*.hip")))
            if os.path.basename(src) != "ring.hip"]
    tmp = TIMELINE_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, obj,
          f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, TIMELINE_LIB)
    return TIMELINE_LIB


def build_addon() -> str | None:
    """The N-API addon links libmockbird_hip.so by rpath $ORIGIN/.."""
    src = os.path.join(CSRC, "napi", "mb_napi.cc")
    if not os.path.exists(src):
        return None
    node_inc = "/usr/include/node"
    if not os.path.exists(os.path.join(node_inc, "node_api.h")):
        sys.stderr.write("node_api.h not found; skipping the N-API addon\n")
        return None
    os.makedirs(os.path.dirname(ADDON), exist_ok=True)
    tmp = ADDON + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-I", node_inc,
          "-I", os.path.join(ROOT, "include"), src, "-o", tmp, "-L", PKG, "-lmockbird_hip",
          "-Wl,-rpath,$ORIGIN/..", "-Wl,--allow-shlib-undefined"])
    os.replace(tmp, ADDON)
    return ADDON


ASAN_DIR = os.path.join(PKG, "_asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libmockbird_hip.so")
ASAN_ADDON = os.path.join(ASAN_DIR, "engine", "mockbird_hip.node")
# the runtime both sanitized builds link against (clang's, as hipcc's)
ASAN_RUNTIME = os.path.join(ROCM, "llvm", "lib", "clang")
SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-shared-libasan"]


def asan_runtime() -> str | None:
    """clang's AddressSanitizer runtime (to preload into python / node)."""
    for path in sorted(glob.glob(os.path.join(ASAN_RUNTIME, "*", "lib", "linux",
                                              "libclang_rt.asan-x86_64.so"))):
        return path
    return None


def sanitized_stale() -> bool:
    """Whether the host-sanitized build is missing or older than a source."""
    if not (os.path.exists(ASAN_LIB) and os.path.exists(ASAN_ADDON)):
        return True
    built = min(os.path.getmtime(ASAN_LIB), os.path.getmtime(ASAN_ADDON))
    sources = (glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.h")) +
               glob.glob(os.path.join(CSRC, "napi", "*.cc")) +
               glob.glob(os.path.join(ROOT, "include", "*.h")))
    return any(os.path.getmtime(f) > built for f in sources)


def build_sanitized(jobs: int = 8) -> tuple[str, str | None]:
    """The C ABI and the N-API addon with their host code under
    AddressSanitizer and UndefinedBehaviorSanitizer (the GPU code is built
    as usual): mockbird_amd/_asan/libmockbird_hip.so and
    mockbird_amd/_asan/engine/mockbird_hip.node, which links it.  For the
    CPU tests of the boundary (tests/test_host_sanitized.py); run with
    clang's ASan runtime preloaded (asan_runtime())."""
    obj_dir = os.path.join(ASAN_DIR, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    flags = [f for f in HIP_FLAGS if f != "-O3"] + ["-O1", "-g", "-fno-omit-frame-pointer"] + SAN_HOST
    cmds, objs = [], []
    for src in sorted(glob.glob(os.path.join(CSRC, "*.hip"))):
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *flags, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = ASAN_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *SAN_HOST, "-o", tmp, *objs,
          f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, ASAN_LIB)
    src = os.path.join(CSRC, "napi", "mb_napi.cc")
    node_inc = "/usr/include/node"
    if not os.path.exists(os.path.join(node_inc, "node_api.h")):
        return ASAN_LIB, None
    os.makedirs(os.path.dirname(ASAN_ADDON), exist_ok=True)
    tmp = ASAN_ADDON + ".tmp"
    _run([os.path.join(ROCM, "llvm", "bin", "clang++"), "-O1", "-g", "-fPIC", "-shared",
          "-std=c++17", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
          "-fno-sanitize-recover=undefined", "-shared-libasan",
          # globals uninstrumented: Node 12 registers the addon's module-name
          # literal with ASan twice and ASan then reports it as misaligned;
          # heap and stack accesses stay checked
          "-mllvm", "-asan-globals=0", "-I", node_inc, "-I",
          os.path.join(ROOT, "include"), src, "-o", tmp, "-L", ASAN_DIR, "-lmockbird_hip",
          "-Wl,-rpath,$ORIGIN/..", "-Wl,--allow-shlib-undefined"])
    os.replace(tmp, ASAN_ADDON)
    return ASAN_LIB, ASAN_ADDON


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("--sanitized", action="store_true",
                    help="also build the host-sanitized library and addon (mockbird_amd/_asan)")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args(argv)
    print(build_lib(a.j))
    if not a.lib_only:
        print(build_probe())
        print(build_timeline())
        addon = build_addon()
        if addon:
            print(addon)
    if a.sanitized:
        print(*build_sanitized(a.j))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
