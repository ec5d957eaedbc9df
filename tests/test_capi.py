"""C-ABI surface on CPU: the library loads, exports every function include/tsa.h declares,
and rejects invalid arguments with the documented codes before touching the GPU.
The lab drivers reject bad command lines with exit code 2 (src/attn_sm75.cu:449-460,
src/gdn_sm75.cu:1249-1252)."""
import ctypes
import os
import subprocess

import pytest

import tsa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "turing-sm75_amd", "bin")
NULL = None
DUMMY = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation


def test_exports_every_declared_symbol():
    lib = tsa.load()
    names = tsa.header_symbols()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", tsa.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported


def test_version_and_strerror():
    lib = tsa.load()
    assert lib.tsa_version().decode().startswith("tsa ")
    for code in range(8):
        assert tsa.strerror(code)
    assert "unknown" in tsa.strerror(99)


def _attn(*, q=DUMMY, B=1, H=1, S=16, D=128, scale=0.1, causal=1):
    return tsa.load().tsa_attn_fwd(q, DUMMY, DUMMY, DUMMY, B, H, S, D, scale, causal, NULL)


def test_attn_argument_errors():
    assert _attn(q=NULL) == tsa.TSA_ERR_NULL
    assert _attn(S=0) == tsa.TSA_ERR_SHAPE
    assert _attn(B=-1) == tsa.TSA_ERR_SHAPE
    assert _attn(D=96) == tsa.TSA_ERR_UNSUPPORTED
    assert _attn(D=512) == tsa.TSA_ERR_UNSUPPORTED
    assert _attn(causal=2) == tsa.TSA_ERR_ARG
    assert _attn(scale=0.0) == tsa.TSA_ERR_ARG
    assert _attn(scale=-0.1) == tsa.TSA_ERR_ARG
    assert _attn(scale=float("nan")) == tsa.TSA_ERR_ARG
    assert _attn(B=1 << 16, H=1 << 16, S=1) == tsa.TSA_ERR_SHAPE
    lib = tsa.load()
    assert lib.tsa_attn_naive(DUMMY, DUMMY, NULL, DUMMY, 1, 1, 4, 64, 0.1, 0, NULL) == tsa.TSA_ERR_NULL


def test_attn_valu_argument_errors():
    # the VALU opponent validates exactly as tsa_attn_fwd
    f = tsa.load().tsa_attn_fwd_valu
    assert f(DUMMY, NULL, DUMMY, DUMMY, 1, 1, 16, 128, 0.1, 1, NULL) == tsa.TSA_ERR_NULL
    assert f(DUMMY, DUMMY, DUMMY, DUMMY, 1, 1, 0, 128, 0.1, 1, NULL) == tsa.TSA_ERR_SHAPE
    assert f(DUMMY, DUMMY, DUMMY, DUMMY, 1, 1, 16, 96, 0.1, 1, NULL) == tsa.TSA_ERR_UNSUPPORTED
    assert f(DUMMY, DUMMY, DUMMY, DUMMY, 1, 1, 16, 64, 0.1, 3, NULL) == tsa.TSA_ERR_ARG
    assert f(DUMMY, DUMMY, DUMMY, DUMMY, 1, 1, 16, 64, float("inf"), 0, NULL) == tsa.TSA_ERR_ARG


def _gqa(*, q=DUMMY, gate=NULL, B=1, Hq=24, Hkv=4, S=16, D=256, scale=0.1, causal=1):
    return tsa.load().tsa_attn_gqa_fwd(q, DUMMY, DUMMY, gate, DUMMY, B, Hq, Hkv, S, D, scale,
                                       causal, NULL)


def test_attn_gqa_argument_errors():
    # gate may be NULL; every other pointer is required
    assert _gqa(q=NULL) == tsa.TSA_ERR_NULL
    assert _gqa(Hkv=5) == tsa.TSA_ERR_SHAPE    # 24 % 5 != 0
    assert _gqa(Hkv=0) == tsa.TSA_ERR_SHAPE
    assert _gqa(Hkv=48) == tsa.TSA_ERR_SHAPE   # more K/V heads than query heads
    assert _gqa(D=96) == tsa.TSA_ERR_UNSUPPORTED
    assert _gqa(causal=3) == tsa.TSA_ERR_ARG
    assert _gqa(scale=float("inf")) == tsa.TSA_ERR_ARG
    lib = tsa.load()
    assert lib.tsa_attn_gqa_naive(DUMMY, NULL, DUMMY, NULL, DUMMY, 1, 2, 1, 4, 64, 0.1, 0,
                                  NULL) == tsa.TSA_ERR_NULL


def _chunked(*, T=64, Hv=2, dk=128, dv=128, chunk=64, ws=DUMMY, ws_bytes=1 << 30, st=DUMMY):
    return tsa.load().tsa_gdn_chunked_fwd(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, st, DUMMY,
                                          1, T, 1, Hv, dk, dv, chunk, 0.1, ws, ws_bytes, NULL)


def test_gdn_chunked_argument_errors():
    need = tsa.gdn_chunked_workspace_bytes(1, 64, 1, 2)
    assert need > 0
    assert _chunked(st=NULL) == tsa.TSA_ERR_NULL
    assert _chunked(T=0) == tsa.TSA_ERR_SHAPE
    assert _chunked(dk=64, dv=64) == tsa.TSA_ERR_UNSUPPORTED
    assert _chunked(chunk=16) == tsa.TSA_ERR_UNSUPPORTED
    assert _chunked(chunk=0) == tsa.TSA_ERR_SHAPE
    assert _chunked(ws=NULL) == tsa.TSA_ERR_WORKSPACE
    assert _chunked(ws_bytes=need - 1) == tsa.TSA_ERR_WORKSPACE


def test_gdn_f32_entry_points_validate_like_fp16():
    lib = tsa.load()
    args = [DUMMY] * 7
    need32 = tsa.gdn_chunked_workspace_bytes(1, 100, 2, 4, f32=True)
    assert need32 == tsa.gdn_chunked_workspace_bytes(1, 100, 2, 4) + 2 * 49152 * 4  # + K, Q, K_lo rows
    ch = lambda ws=DUMMY, nb=need32, dk=128, T=100: lib.tsa_gdn_chunked_fwd_f32(
        *args, 1, T, 2, 4, dk, 128, 64, 0.1, ws, nb, NULL)
    assert ch(ws=NULL) == tsa.TSA_ERR_WORKSPACE
    assert ch(nb=need32 - 1) == tsa.TSA_ERR_WORKSPACE
    assert ch(dk=64) == tsa.TSA_ERR_UNSUPPORTED
    assert ch(T=0) == tsa.TSA_ERR_SHAPE
    assert lib.tsa_gdn_recurrent_fwd_f32(*args[:6], NULL, 1, 4, 1, 2, 128, 128, 0.1, NULL) == tsa.TSA_ERR_NULL
    assert lib.tsa_gdn_decode_step_f32(*args, 4, 1, 2, 128, 96, 0.1, NULL) == tsa.TSA_ERR_UNSUPPORTED
    assert lib.tsa_gdn_naive_f32(*args, 1, 1, 0, 2, 128, 128, 0.1, NULL) == tsa.TSA_ERR_SHAPE
    assert lib.tsa_gdn_chunked_workspace_bytes_f32(1, 64, 16, 32, 128, 128, 32) == 0


def test_gdn_workspace_bytes_scales_with_chunks():
    # per (sequence, V-head): a 58 368-byte chunk workspace and a 4-byte ready flag per chunk,
    # and a 4-byte abort word for each of the 4 carry workgroups (32 state columns each)
    per_head = lambda nch: nch * (58368 + 4) + 4 * 4
    assert tsa.gdn_chunked_workspace_bytes(1, 64, 16, 32) == 32 * per_head(1)
    assert tsa.gdn_chunked_workspace_bytes(1, 65, 16, 32) == 32 * per_head(2)
    assert tsa.gdn_chunked_workspace_bytes(2, 4096, 16, 32) == 2 * 32 * per_head(64)
    assert tsa.gdn_chunked_workspace_bytes(1, 64, 16, 32, dk=64) == 0
    assert tsa.gdn_chunked_workspace_bytes(1, 64, 16, 32, chunk=32) == 0


def test_gdn_workspace_bytes_with_sequence_split():
    # few heads and many chunks split the sequence: after the flags and abort words, at a
    # 256-byte boundary, three 64 KiB fp32 slots (entry state, Z, Phi) per head and segment,
    # then per head two fp32 rows of 128 (the maps' O_Z and M) per token after segment 0
    base = lambda BHv, nch: BHv * (nch * (58368 + 4) + 4 * 4)
    rows = lambda BHv, T, L: 2 * BHv * (T - 64 * L) * 512
    split = lambda BHv, nch, nseg, T, L: ((base(BHv, nch) + 255) // 256 * 256 + BHv * nseg * 3 * 65536 +
                                           rows(BHv, T, L))
    ws = tsa.gdn_chunked_workspace_bytes
    # 4 heads, 64 chunks: 8 segments of 8 chunks (the maps launch, 15 units x 4 workgroups x
    # 4 heads, fits 256 CUs; sqrt(64) = 8)
    assert ws(1, 4096, 2, 4) == split(4, 64, 8, 4096, 8)
    # 1 head: 8 segments at 64 chunks, 16 of 16 chunks at 256, 2 of 8 at 16 (8 chunks at least)
    assert ws(1, 4096, 1, 1) == split(1, 64, 8, 4096, 8)
    assert ws(1, 16384, 1, 1) == split(1, 256, 16, 16384, 16)
    assert ws(1, 1024, 1, 1) == split(1, 16, 2, 1024, 8)
    # 16 heads: 2 segments (3 units x 64 workgroups); 32 heads: the carry already takes half
    # the CUs, no split; 11 chunks: too short to split
    assert ws(1, 4096, 8, 16) == split(16, 64, 2, 4096, 32)
    assert ws(1, 4096, 16, 32) == base(32, 64)
    assert ws(1, 704, 2, 4) == base(4, 11)
    # the library's plan is a function of the shapes: nseg = 0 is the same query
    for shape in ((1, 4096, 2, 4), (1, 4096, 16, 32), (1, 1024, 1, 1)):
        assert ws(*shape, nseg=0) == ws(*shape)
        assert ws(*shape, f32=True, nseg=0) == ws(*shape, f32=True)
    # explicit plans
    assert ws(1, 4096, 2, 4, nseg=1) == base(4, 64)
    assert ws(1, 1000, 1, 2, nseg=3) == split(2, 16, 3, 1000, 6)  # 6 + 6 + 4
    assert ws(1, 128, 1, 2, nseg=3) == split(2, 2, 2, 128, 1)  # 2 chunks: 2 of 1
    assert ws(1, 64, 1, 2, nseg=3) == base(2, 1)  # 1 chunk: no split
    assert ws(2, 777, 3, 4, nseg=5) == split(8, 13, 5, 777, 3)  # 3 x 4 + 1
    assert ws(2, 777, 3, 4, nseg=1000) == split(8, 13, 13, 777, 1)  # one chunk each
    # fp32 I/O: the chunk workspace also holds the fp16 K / Q rows
    f32base = 4 * (18 * (58368 + 49152 + 4) + 4 * 4)
    assert ws(1, 1100, 2, 4, f32=True, nseg=4) == (f32base + 255) // 256 * 256 + 4 * 4 * 3 * 65536 + rows(4, 1100, 5)
    # invalid requests
    lib = tsa.load()
    assert lib.tsa_gdn_chunked_plan_workspace_bytes(1, 64, 1, 2, 128, 128, 64, 0, -1) == 0
    assert lib.tsa_gdn_chunked_plan_workspace_bytes(1, 64, 1, 2, 128, 128, 64, 2, 0) == 0
    assert lib.tsa_gdn_chunked_plan_workspace_bytes(1, 64, 1, 2, 128, 128, 32, 0, 0) == 0


def test_gdn_plan_fwd_argument_errors():
    # validated before any HIP call
    lib = tsa.load()
    f = lambda io=0, nseg=0, T=64, ws=DUMMY, wsb=1 << 30: lib.tsa_gdn_chunked_plan_fwd(
        DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, T, 1, 2, 128, 128, 64, 0.1, io, nseg, ws, wsb, NULL)
    assert f(io=2) == tsa.TSA_ERR_ARG
    assert f(nseg=-1) == tsa.TSA_ERR_ARG
    assert f(ws=NULL) == tsa.TSA_ERR_WORKSPACE
    need = tsa.gdn_chunked_workspace_bytes(1, 1000, 1, 2, nseg=3)
    assert f(T=1000, nseg=3, wsb=need - 1) == tsa.TSA_ERR_WORKSPACE
    assert lib.tsa_gdn_chunked_plan_fwd(NULL, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 1, 64, 1, 2, 128, 128, 64,
                                        0.1, 0, 0, DUMMY, 1 << 30, NULL) == tsa.TSA_ERR_NULL


def test_gdn_noalloc_argument_errors():
    # validated before any HIP call; shapes whose workspace exceeds the fixed 64 MiB scratch
    # are refused with their own code (32 V-heads: T = 2240 fits, T = 2241 does not)
    lib = tsa.load()
    f = lambda q=DUMMY, B=1, T=64, Hv=32, dk=128, chunk=64, scale=0.1: lib.tsa_gdn_chunked_fwd_noalloc(
        q, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, B, T, 16, Hv, dk, 128, chunk, scale, NULL)
    assert f(q=NULL) == tsa.TSA_ERR_NULL
    assert f(T=0) == tsa.TSA_ERR_SHAPE
    assert f(dk=64) == tsa.TSA_ERR_UNSUPPORTED
    assert f(chunk=16) == tsa.TSA_ERR_UNSUPPORTED
    assert f(scale=float("nan")) == tsa.TSA_ERR_ARG
    assert tsa.gdn_chunked_workspace_bytes(1, 2240, 16, 32) <= 64 << 20
    assert tsa.gdn_chunked_workspace_bytes(1, 2241, 16, 32) > 64 << 20
    assert f(T=2241) == tsa.TSA_ERR_SCRATCH
    assert f(B=2, T=1200) == tsa.TSA_ERR_SCRATCH
    assert "64 MiB" in tsa.strerror(tsa.TSA_ERR_SCRATCH)


def test_gdn_redo_count_argument_errors():
    lib = tsa.load()
    c = ctypes.c_int(-1)
    need = tsa.gdn_chunked_workspace_bytes(1, 100, 2, 4)
    f = lambda ws=DUMMY, nb=need, T=100, dk=128, io=0, cnt=ctypes.byref(c): lib.tsa_gdn_chunked_redo_count(
        ws, nb, 1, T, 2, 4, dk, 128, 64, io, cnt, NULL)
    assert f(ws=NULL) == tsa.TSA_ERR_NULL
    assert f(io=2) == tsa.TSA_ERR_ARG
    assert f(io=1) == tsa.TSA_ERR_WORKSPACE  # the fp32-I/O workspace is larger
    assert f(cnt=None) == tsa.TSA_ERR_NULL
    assert f(T=0) == tsa.TSA_ERR_SHAPE
    assert f(dk=64) == tsa.TSA_ERR_UNSUPPORTED
    assert f(nb=need - 4) == tsa.TSA_ERR_WORKSPACE
    assert c.value == -1  # nothing was written


def test_binding_rejects_wrong_out_shape(monkeypatch):
    # the binding's output check runs before any library call: a smaller out would be written
    # past its end (CPU tensors stand in here, so the device check is bypassed)
    import torch
    monkeypatch.setattr(tsa, "_need", lambda *a, **k: None)
    like = torch.empty(1, 70, 2, 128, dtype=torch.float16)
    with pytest.raises(ValueError):
        tsa._out(torch.empty(1, 69, 2, 128, dtype=torch.float16), like)
    ok = torch.empty_like(like)
    assert tsa._out(ok, like) is ok


def test_gdn_recurrent_and_decode_argument_errors():
    lib = tsa.load()
    args = [DUMMY] * 7
    assert lib.tsa_gdn_recurrent_fwd(*args, 1, 4, 1, 2, 128, 64, 0.1, NULL) == tsa.TSA_ERR_UNSUPPORTED
    assert lib.tsa_gdn_recurrent_fwd(*args, 1, 0, 1, 2, 128, 128, 0.1, NULL) == tsa.TSA_ERR_SHAPE
    assert lib.tsa_gdn_decode_step(*args[:6], NULL, 4, 1, 2, 128, 128, 0.1, NULL) == tsa.TSA_ERR_NULL
    assert lib.tsa_gdn_decode_step(*args, 4, 1, 2, 128, 128, float("inf"), NULL) == tsa.TSA_ERR_ARG
    assert lib.tsa_gdn_naive(*args, 1, 1, 0, 2, 128, 128, 0.1, NULL) == tsa.TSA_ERR_SHAPE


@pytest.mark.parametrize("argv", [
    ["attn_sm75", "1", "2", "3"],
    ["attn_sm75", "1", "2", "64", "96"],
    ["attn_sm75", "--causal"],
    ["gdn", "0"],
    ["gdn", "64", "--mode", "train"],
    ["gdn", "64", "--io", "f64"],
])
def test_drivers_usage_errors_exit_2(argv):
    exe = os.path.join(BIN, argv[0])
    assert os.path.exists(exe), "build the drivers first (make -C turing-sm75_amd)"
    r = subprocess.run([exe] + argv[1:], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)


def test_gdn_fused_and_op_argument_errors():
    lib = tsa.load()
    inf, nan = float("inf"), float("nan")
    # chunked fused: q k v a b dt A state out | B T Hq Hv dk dv chunk | scale eps | ws ws_bytes stream
    def fused(*, A=DUMMY, dk=128, chunk=64, eps=1e-6, ws=DUMMY, ws_bytes=1 << 30, T=64):
        return lib.tsa_gdn_chunked_fused_fwd(DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, A, DUMMY,
                                             DUMMY, 1, T, 1, 2, dk, 128, chunk, 0.1, eps, ws,
                                             ws_bytes, NULL)
    assert fused(A=NULL) == tsa.TSA_ERR_NULL
    assert fused(eps=0.0) == tsa.TSA_ERR_ARG
    assert fused(eps=nan) == tsa.TSA_ERR_ARG
    assert fused(dk=64) == tsa.TSA_ERR_UNSUPPORTED
    assert fused(chunk=32) == tsa.TSA_ERR_UNSUPPORTED
    assert fused(T=0) == tsa.TSA_ERR_SHAPE
    assert fused(ws=NULL) == tsa.TSA_ERR_WORKSPACE
    # decode fused: q k v a b dt A state out | B Hq Hv dk dv | scale eps | stream
    args = [DUMMY] * 9
    assert lib.tsa_gdn_decode_fused_step(*args, 4, 1, 2, 128, 128, 0.1, -1.0, NULL) == tsa.TSA_ERR_ARG
    assert lib.tsa_gdn_decode_fused_step(*args, 4, 1, 2, 128, 128, inf, 1e-6, NULL) == tsa.TSA_ERR_ARG
    assert lib.tsa_gdn_decode_fused_step(*args, 4, 1, 2, 96, 128, 0.1, 1e-6, NULL) == tsa.TSA_ERR_UNSUPPORTED
    assert lib.tsa_gdn_decode_fused_step(*args[:5], NULL, *args[6:], 4, 1, 2, 128, 128, 0.1, 1e-6,
                                         NULL) == tsa.TSA_ERR_NULL
    # preprocess: q k a b dt A q_out k_out g beta | B T Hq Hv dk | eps | stream
    pa = [DUMMY] * 10
    assert lib.tsa_gdn_preprocess(*pa[:9], NULL, 1, 8, 2, 4, 128, 1e-6, NULL) == tsa.TSA_ERR_NULL
    assert lib.tsa_gdn_preprocess(*pa, 1, 8, 2, 4, 64, 1e-6, NULL) == tsa.TSA_ERR_UNSUPPORTED
    assert lib.tsa_gdn_preprocess(*pa, 1, 0, 2, 4, 128, 1e-6, NULL) == tsa.TSA_ERR_SHAPE
    assert lib.tsa_gdn_preprocess(*pa, 1, 8, 2, 4, 128, 0.0, NULL) == tsa.TSA_ERR_ARG
    # gated rmsnorm: x z w y | B T Hv dv | eps | stream
    assert lib.tsa_gdn_gated_rmsnorm(DUMMY, NULL, DUMMY, DUMMY, 1, 2, 3, 128, 1e-6, NULL) == tsa.TSA_ERR_NULL
    assert lib.tsa_gdn_gated_rmsnorm(DUMMY, DUMMY, DUMMY, DUMMY, 1, 2, 3, 64, 1e-6, NULL) == tsa.TSA_ERR_UNSUPPORTED
    assert lib.tsa_gdn_gated_rmsnorm(DUMMY, DUMMY, DUMMY, DUMMY, 1, 0, 3, 128, 1e-6, NULL) == tsa.TSA_ERR_SHAPE
    assert lib.tsa_gdn_gated_rmsnorm(DUMMY, DUMMY, DUMMY, DUMMY, 1, 2, 3, 128, inf, NULL) == tsa.TSA_ERR_ARG


def _tt(ne, typ=0, data=0x1000, nb=None):
    t = tsa.TsaTensor()
    t.data = data
    t.type = typ
    es = 2 if typ == 1 else 4
    if nb is None:
        nb = [es]
        for i in range(3):
            nb.append(nb[-1] * ne[i])
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    return t


def test_ggml_adapter_argument_errors():
    lib = tsa.load()
    B, T, Hk, Hv, S = 1, 8, 2, 4, 128

    def call(**over):
        d = dict(q=_tt([S, Hk, T, B]), k=_tt([S, Hk, T, B]), v=_tt([S, Hv, T, B]),
                 g=_tt([Hv, T, B, 1]), beta=_tt([Hv, T, B, 1]), state=_tt([S, S, Hv, B]),
                 out=_tt([S, Hv, T, B]), state_out=_tt([S, S, Hv, B], data=0x2000))
        scale = over.pop("scale", 0.1)
        ws = over.pop("ws", DUMMY)
        d.update(over)
        args = [ctypes.byref(d[n]) if d[n] is not None else None
                for n in ("q", "k", "v", "g", "beta", "state", "out", "state_out")]
        return lib.tsa_ggml_gated_delta_net(*args, scale, ws, 1 << 40, NULL)

    assert call(k=None) == tsa.TSA_ERR_NULL
    assert call(v=_tt([S, Hv, T, B], data=0)) == tsa.TSA_ERR_NULL
    assert call(q=_tt([S, Hk, T, B], typ=7)) == tsa.TSA_ERR_ARG
    assert call(g=_tt([Hv, T, B, 1], typ=1)) == tsa.TSA_ERR_UNSUPPORTED   # gates are fp32
    assert call(state=_tt([S, S, Hv, B], typ=1)) == tsa.TSA_ERR_UNSUPPORTED
    assert call(k=_tt([S, Hk + 1, T, B])) == tsa.TSA_ERR_SHAPE
    assert call(out=_tt([S, Hv, T + 1, B])) == tsa.TSA_ERR_SHAPE
    assert call(beta=_tt([Hv, T, B, 2])) == tsa.TSA_ERR_SHAPE
    assert call(q=_tt([S, Hk, 0, B]), k=_tt([S, Hk, 0, B])) == tsa.TSA_ERR_SHAPE
    q64 = _tt([64, Hk, T, B])
    assert call(q=q64, k=_tt([64, Hk, T, B]), state=_tt([64, S, Hv, B]),
                state_out=_tt([64, S, Hv, B], data=0x2000)) == tsa.TSA_ERR_UNSUPPORTED
    assert call(scale=float("nan")) == tsa.TSA_ERR_ARG
    # in place must be the same view
    assert call(state_out=_tt([S, S, Hv, B], nb=[4, 1024, 65536, 4 * 65536])) == tsa.TSA_ERR_ARG
    assert call(ws=NULL) == tsa.TSA_ERR_WORKSPACE


def test_ggml_workspace_bytes():
    lib = tsa.load()
    ws = lambda T, Hk=2, Hv=4, S=128: lib.tsa_ggml_gdn_workspace_bytes(
        ctypes.byref(_tt([S, Hk, T, 1])), ctypes.byref(_tt([S, Hv, T, 1])))
    assert ws(8, S=64) == 0 and ws(0) == 0
    small, big = ws(31), ws(32)
    # from 32 tokens on (the chunked prefill's dispatch), its workspace is included
    assert big - small >= tsa.gdn_chunked_workspace_bytes(1, 32, 2, 4)
    assert ws(128) > ws(64) > 0
