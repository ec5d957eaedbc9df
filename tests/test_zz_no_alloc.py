"""tsa_gdn_chunked_fwd_noalloc, the chunked prefill on the library's fixed device scratch
array instead of a caller workspace, called through the C-ABI and checked against
tsa_gdn_chunked_fwd (the same kernels, so bit for bit) on two calls in a row, the second
smaller than the first, on the largest shape the 64 MiB scratch holds, and on shapes where
the call splits the sequence."""
import ctypes
import math

import numpy as np
import pytest

import tsa

pytestmark = pytest.mark.gpu
D = 128


def _inputs(rng, B, T, Hq, Hv):
    l2n = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    q = l2n(rng.standard_normal((B, T, Hq, D))).astype(np.float16)
    k = l2n(rng.standard_normal((B, T, Hq, D))).astype(np.float16)
    v = rng.standard_normal((B, T, Hv, D)).astype(np.float16)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))).astype(np.float32)
    g = (-np.logaddexp(0.0, rng.standard_normal((B, T, Hv)))).astype(np.float32)
    st = (0.02 * rng.standard_normal((B, Hv, D, D))).astype(np.float32)
    return q, k, v, g, beta, st


def _case(dev, seed, B, T, Hq, Hv):
    import torch
    print(f"no-alloc case B={B} T={T} Hq={Hq} Hv={Hv}", flush=True)
    rng = np.random.default_rng(seed)
    q, k, v, g, beta, st = (torch.from_numpy(a).to(dev) for a in _inputs(rng, B, T, Hq, Hv))
    s_ref = st.clone()
    o_ref = tsa.gdn_chunked_fwd(q, k, v, g, beta, s_ref)
    s_new = st.clone()
    o_new = torch.empty_like(v)
    stream = torch.cuda.current_stream()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = tsa.load().tsa_gdn_chunked_fwd_noalloc(
        p(q), p(k), p(v), p(g), p(beta), p(s_new), p(o_new), B, T, Hq, Hv, D, D, 64,
        1.0 / math.sqrt(D), ctypes.c_void_p(stream.cuda_stream))
    assert rc == tsa.TSA_OK, tsa.strerror(rc)
    torch.cuda.synchronize()
    assert torch.equal(o_new, o_ref) and torch.equal(s_new, s_ref)
    assert bool(torch.isfinite(o_new.float()).all())


def test_noalloc_two_calls_second_smaller(dev):
    _case(dev, 11, 1, 1100, 16, 32)
    _case(dev, 12, 2, 300, 4, 8)


def test_noalloc_largest_shape(dev):
    assert tsa.gdn_chunked_workspace_bytes(1, 2240, 16, 32) <= 64 << 20
    _case(dev, 13, 1, 2240, 16, 32)
    _case(dev, 14, 1, 70, 2, 3)


def test_noalloc_sequence_split(dev):
    """Few heads and many chunks: the call splits the sequence (its Phi / Z / entry slots in
    the scratch too), on two calls in a row, the second smaller."""
    for B, T, Hq, Hv in ((1, 2048, 2, 4), (1, 1000, 1, 2)):
        split = tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv)
        assert split > tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv, nseg=1)
    _case(dev, 15, 1, 2048, 2, 4)
    _case(dev, 16, 1, 1000, 1, 2)


def test_noalloc_runs_whole_where_the_split_does_not_fit(dev):
    """4 V-heads, T = 9000: the split's workspace (71 MB) exceeds the 64 MiB scratch, so the
    no-allocation call runs the chunk carry whole (33 MB) instead of failing; it equals the
    workspace entry point with the split turned off, bit for bit."""
    import torch
    B, T, Hq, Hv = 1, 9000, 2, 4
    assert tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv) > 64 << 20
    assert tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv, nseg=1) <= 64 << 20
    print(f"no-alloc case B={B} T={T} Hq={Hq} Hv={Hv}, whole carry", flush=True)
    rng = np.random.default_rng(17)
    q, k, v, g, beta, st = (torch.from_numpy(a).to(dev) for a in _inputs(rng, B, T, Hq, Hv))
    s_ref = st.clone()
    o_ref = tsa.gdn_chunked_fwd(q, k, v, g, beta, s_ref, nseg=1)  # split off
    torch.cuda.synchronize()
    s_new, o_new = st.clone(), torch.empty_like(v)
    stream = torch.cuda.current_stream()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = tsa.load().tsa_gdn_chunked_fwd_noalloc(
        p(q), p(k), p(v), p(g), p(beta), p(s_new), p(o_new), B, T, Hq, Hv, D, D, 64,
        1.0 / math.sqrt(D), ctypes.c_void_p(stream.cuda_stream))
    assert rc == tsa.TSA_OK, tsa.strerror(rc)
    torch.cuda.synchronize()
    assert torch.equal(o_new, o_ref) and torch.equal(s_new, s_ref)


_FIRST_CALL_CAPTURED = r"""
import ctypes, math, sys
import numpy as np
import torch
sys.path[:0] = sys.argv[1:3]
import tsa
dev = torch.device("cuda:0")
B, T, Hq, Hv, D = 1, 700, 4, 8, 128
rng = np.random.default_rng(18)
l2n = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
arrays = (l2n(rng.standard_normal((B, T, Hq, D))).astype(np.float16),
          l2n(rng.standard_normal((B, T, Hq, D))).astype(np.float16),
          rng.standard_normal((B, T, Hv, D)).astype(np.float16),
          (-np.logaddexp(0.0, rng.standard_normal((B, T, Hv)))).astype(np.float32),
          (1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))).astype(np.float32),
          (0.02 * rng.standard_normal((B, Hv, D, D))).astype(np.float32))
q, k, v, g, beta, st0 = (torch.from_numpy(a).to(dev) for a in arrays)
lib = tsa.load()
p = lambda t: ctypes.c_void_p(t.data_ptr())
def noalloc(ts, out, stream):
    return lib.tsa_gdn_chunked_fwd_noalloc(p(q), p(k), p(v), p(g), p(beta), p(ts), p(out), B, T, Hq, Hv,
                                           D, D, 64, 1.0 / math.sqrt(D), ctypes.c_void_p(stream.cuda_stream))
ts, out = st0.clone(), torch.empty_like(v)
torch.cuda.synchronize()
side = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
print("first no-allocation call of the process, inside a graph capture", flush=True)
with torch.cuda.graph(graph, stream=side):
    rc = noalloc(ts, out, side)
assert rc == tsa.TSA_OK, tsa.strerror(rc)
s_ref = st0.clone()
o_ref = tsa.gdn_chunked_fwd(q, k, v, g, beta, s_ref)
torch.cuda.synchronize()
for i in range(2):
    ts.copy_(st0)
    out.fill_(3.0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, o_ref) and torch.equal(ts, s_ref), f"replay {i}"
ts2, out2 = st0.clone(), torch.empty_like(v)
assert noalloc(ts2, out2, torch.cuda.current_stream()) == tsa.TSA_OK
torch.cuda.synchronize()
assert torch.equal(out2, o_ref) and torch.equal(ts2, s_ref)
print("replays and an eager call equal the workspace entry point bit for bit", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(dev):
    """A fresh process whose first no-allocation call (the one that looks up the scratch
    array's device address) is made while a stream is being captured: the captured graph's
    replays, and an eager call after them, equal tsa_gdn_chunked_fwd bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root, os.path.join(root, "turing-sm75_amd")],
                       capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-3000:])
    assert r.returncode == 0
