"""The CPU test suite once more against host builds instrumented with AddressSanitizer and
UndefinedBehaviorSanitizer: the oracle (all of oracle/*.cpp) and the library's host code (the
C-ABI validation in capi.cpp, the ggml adapter, every launcher; device code is built as
usual), both with clang's shared sanitizer runtime, which the child process preloads.  Any
sanitizer report aborts the child (halt_on_error), so the run must pass as the plain one
does.  No kernel is launched: the CPU tests stop at argument validation."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "turing-sm75_amd")
ROCM = "/opt/rocm"
CLANG = os.path.join(ROCM, "llvm", "bin", "clang++")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
       "-fno-omit-frame-pointer"]
LIB_SOURCES = ["attn_fwd.hip", "attn_valu.hip", "gdn_recurrent.hip", "gdn_chunked.hip",
               "gdn_ops.hip", "layout.hip", "capi.cpp", "ggml_adapter.cpp"]


def _runtime():
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(out) or not os.path.exists(out):
        # older layouts keep it under lib/linux of the resource directory
        res = subprocess.run([CLANG, "-print-resource-dir"], capture_output=True, text=True).stdout.strip()
        out = os.path.join(res, "lib", "linux", "libclang_rt.asan-x86_64.so")
    return out


def _build(tmp):
    oracle_src = [os.path.join(ROOT, "oracle", f) for f in ("inputs.cpp", "attn_oracle.cpp", "gdn_oracle.cpp")]
    orc = os.path.join(tmp, "liboracle.so")
    jobs = [subprocess.Popen([CLANG, "-O1", "-g", "-std=c++17", "-fPIC", "-fopenmp", "-mavx2", "-mfma",
                              "-ffp-contract=off", *SAN, "-shared-libsan", "-shared", *oracle_src,
                              "-Wl,-rpath," + os.path.join(ROCM, "llvm", "lib"), "-o", orc])]
    objs = []
    host_san = [x for f in SAN for x in ("-Xarch_host", f)]  # instrument the host pass only
    for src in LIB_SOURCES:
        obj = os.path.join(tmp, src + ".o")
        objs.append(obj)
        jobs.append(subprocess.Popen(
            [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-Xclang",
             "-target-feature", "-Xclang", "-packed-fp32-ops", *host_san, "-x", "hip", "-c",
             os.path.join(PKG, "csrc", src), "-o", obj],
            stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL))
    assert all(j.wait() == 0 for j in jobs), "sanitizer build failed"
    lib = os.path.join(tmp, "libtsa.so")
    # link against clang's shared sanitizer runtime by name (the host objects need it)
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", *objs, _runtime(), "-o", lib],
                   check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    return orc, lib


@pytest.mark.skipif(not (os.path.exists(CLANG) and os.path.exists(HIPCC)), reason="no ROCm clang")
def test_cpu_suite_under_asan_and_ubsan(tmp_path):
    orc, lib = _build(str(tmp_path))
    rt = _runtime()
    assert os.path.exists(rt), rt
    env = dict(os.environ, LD_PRELOAD=rt, TSA_LIB_PATH=lib, TSA_ORACLE_LIB_PATH=orc,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",  # the interpreter itself leaks
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    # the instrumented builds are the ones loaded, with the runtime active
    probe = ("import sys; sys.path[:0] = sys.argv[1:3]; import tsa, oracle; "
             "print(tsa.load()._name, oracle.load()._name); "
             "print(any('libclang_rt.asan' in l for l in open('/proc/self/maps')))")
    r = subprocess.run([sys.executable, "-c", probe, ROOT, PKG], env=env, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.split() == [lib, orc, "True"], r.stdout
    tests = sorted(os.path.join(ROOT, "tests", f) for f in os.listdir(os.path.join(ROOT, "tests"))
                   if f.startswith("test_") and f.endswith(".py") and f != "test_sanitizers.py")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider", *tests], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=900)
    print(r.stdout[-3000:], r.stderr[-3000:])
    assert r.returncode == 0
    assert " passed" in r.stdout and "failed" not in r.stdout
