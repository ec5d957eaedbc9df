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


def test_noalloc_sequence_split(dev, monkeypatch):
    """Few heads and many chunks: the call splits the sequence (its Phi / Z / entry slots in
    the scratch too), on two calls in a row, the second smaller."""
    monkeypatch.delenv("TSA_GDN_SEGMENTS", raising=False)
    for B, T, Hq, Hv in ((1, 2048, 2, 4), (1, 1000, 1, 2)):
        split = tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv)
        monkeypatch.setenv("TSA_GDN_SEGMENTS", "1")
        assert split > tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv)
        monkeypatch.delenv("TSA_GDN_SEGMENTS")
    _case(dev, 15, 1, 2048, 2, 4)
    _case(dev, 16, 1, 1000, 1, 2)


def test_noalloc_runs_whole_where_the_split_does_not_fit(dev, monkeypatch):
    """4 V-heads, T = 9000: the split's workspace (71 MB) exceeds the 64 MiB scratch, so the
    no-allocation call runs the chunk carry whole (33 MB) instead of failing; it equals the
    workspace entry point with the split turned off, bit for bit."""
    import torch
    monkeypatch.delenv("TSA_GDN_SEGMENTS", raising=False)
    B, T, Hq, Hv = 1, 9000, 2, 4
    assert tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv) > 64 << 20
    monkeypatch.setenv("TSA_GDN_SEGMENTS", "1")
    assert tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv) <= 64 << 20
    print(f"no-alloc case B={B} T={T} Hq={Hq} Hv={Hv}, whole carry", flush=True)
    rng = np.random.default_rng(17)
    q, k, v, g, beta, st = (torch.from_numpy(a).to(dev) for a in _inputs(rng, B, T, Hq, Hv))
    s_ref = st.clone()
    o_ref = tsa.gdn_chunked_fwd(q, k, v, g, beta, s_ref)  # split off
    torch.cuda.synchronize()
    monkeypatch.delenv("TSA_GDN_SEGMENTS")
    s_new, o_new = st.clone(), torch.empty_like(v)
    stream = torch.cuda.current_stream()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = tsa.load().tsa_gdn_chunked_fwd_noalloc(
        p(q), p(k), p(v), p(g), p(beta), p(s_new), p(o_new), B, T, Hq, Hv, D, D, 64,
        1.0 / math.sqrt(D), ctypes.c_void_p(stream.cuda_stream))
    assert rc == tsa.TSA_OK, tsa.strerror(rc)
    torch.cuda.synchronize()
    assert torch.equal(o_new, o_ref) and torch.equal(s_new, s_ref)
