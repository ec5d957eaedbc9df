"""The two lab drivers on the GPU: bin/attn_sm75 (src/attn_sm75.cu:442-554) and bin/gdn
(src/gdn_sm75.cu:1246-1412) run as child processes at the reference's shapes and at the
workloads' own sizes.  Each run must exit 0 and every check line it prints must pass the
reference's 0.02 gate (and the 1e-3 relative state gate for GDN); the values are parsed and
re-checked here, so a driver that printed OK for a failing value would be caught too."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "turing-sm75_amd", "bin")

ATTN_LINE = re.compile(r"^max \|(\w+)-naive\| : ([0-9.eE+-]+|nan|inf)\s+(OK|FAIL)\s*$")
GDN_LINE = re.compile(r"^max \|(\w+)-naive\| : ([0-9.eE+-]+|nan|inf)\s+(OK|FAIL)\s+"
                      r"state rel ([0-9.eE+-]+|nan|inf)\s+(OK|FAIL)\s*$")
# the chunk decomposition against the token-serial kernel (src/gdn_sm75.cu:1283-1289)
CHUNK_SERIAL_LINE = re.compile(r"^max \|chunk-serial\| : ([0-9.eE+-]+|nan|inf)\s+(OK|FAIL)\s*$")


def _run(argv, timeout=300):
    exe = os.path.join(BIN, argv[0])
    assert os.path.exists(exe), "build the drivers first (make -C turing-sm75_amd)"
    print("driver:", " ".join(argv), flush=True)
    r = subprocess.run([exe] + argv[1:], capture_output=True, text=True, timeout=timeout)
    sys.stdout.write(r.stdout)
    sys.stderr.write(r.stderr)
    return r


@pytest.mark.gpu
@pytest.mark.parametrize("args", [
    ["1", "4", "256", "128", "--causal", "0"],   # the reference's `make run` shape, non-causal
    ["1", "4", "256", "128"],                    # the same, causal (the reference's default)
    ["2", "8", "512", "64"],                     # causal D=64
    [],                                          # the reference's default 2 8 512 128
    ["1", "32", "8192", "128", "--outlier", "0.01", "--iters", "5"],  # long context
    ["1", "24", "512", "256", "--hkv", "4", "--gate", "1"],           # gated GQA, D=256
])
def test_attn_driver(args):
    r = _run(["attn_sm75"] + args)
    assert r.returncode == 0, (r.returncode, r.stderr)
    checks = [ATTN_LINE.match(l) for l in r.stdout.splitlines() if l.startswith("max |")]
    assert checks and all(checks), r.stdout
    names = [m.group(1) for m in checks]
    assert "mfma" in names
    gqa = "--hkv" in args
    assert ("valu" in names) != gqa  # the VALU opponent runs beside plain attention only
    for m in checks:
        err = float(m.group(2))
        assert err < 0.02 and m.group(3) == "OK", m.group(0)
    assert re.search(r"^mfma  \(gfx950\)  :\s+[0-9.]+ ms", r.stdout, re.M), r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("args", [
    ["512"],                                     # the reference's `make gdn`: LCG, Hv=48, fp32 I/O
    ["512", "--io", "f16"],                      # the same inputs rounded to fp16 I/O
    ["100"],                                     # ragged T (one full and one partial chunk)
    ["4096", "--hv", "32", "--dist", "normal", "--iters", "5"],   # the prefill workload
    ["--mode", "decode", "--steps", "64"],       # 16 sequences, step-major decode layout
    ["--mode", "decode", "--steps", "8", "--batch", "3", "--hv", "32"],
])
def test_gdn_driver(args):
    r = _run(["gdn"] + args)
    assert r.returncode == 0, (r.returncode, r.stderr)
    lines = r.stdout.splitlines()
    cs = [CHUNK_SERIAL_LINE.match(l) for l in lines if l.startswith("max |chunk-serial|")]
    checks = [GDN_LINE.match(l) for l in lines if l.startswith("max |") and not l.startswith("max |chunk-serial|")]
    assert checks and all(checks), r.stdout
    if "decode" in args:
        assert not cs, r.stdout
    else:  # printed once, before the per-kernel checks, as the reference does
        assert len(cs) == 1 and cs[0] and lines.index(cs[0].group(0)) < lines.index(checks[0].group(0)), r.stdout
        assert float(cs[0].group(1)) < 0.02 and cs[0].group(2) == "OK", cs[0].group(0)
    names = {m.group(1) for m in checks}
    assert names == ({"decode"} if "decode" in args else {"chunked", "recurrent"}), names
    for m in checks:
        eo, es = float(m.group(2)), float(m.group(4))
        assert eo < 0.02 and m.group(3) == "OK", m.group(0)
        assert es < 1e-3 and m.group(5) == "OK", m.group(0)
    assert "x48 layers" in r.stdout or "ms/step" in r.stdout
