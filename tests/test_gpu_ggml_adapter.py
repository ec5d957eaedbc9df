"""GPU: tsa_ggml_gated_delta_net (the ggml-layout adapter) against the direct entry points
and the oracle.

The adapter only moves data (gathers strided views into the kernels' dense layout, scatters
the output back) and dispatches on the tokens per sequence and the operands' types, so its
results must equal the direct entry point's bit for bit: tsa_gdn_decode_step (T = 1),
tsa_gdn_recurrent_fwd (T < 32), tsa_gdn_chunked_fwd (T >= 32), or their *_f32 forms when any
of q / k / v / out is fp32 (fp32 operands are never narrowed to fp16 in memory).  Cases:
dense fp16 operands (used in place), fp32 views into a fused projection buffer with an fp32
strided output, a separate and a padded (non-dense) state_out, the dispatch boundary T = 31
/ 32, and one case against the recurrence oracle with its gates.
"""
import numpy as np
import pytest

import tsa

pytestmark = pytest.mark.gpu
D = 128


def _data(rng, B, T, Hk, Hv):
    l2n = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    q = l2n(rng.standard_normal((B, T, Hk, D))).astype(np.float16)
    k = l2n(rng.standard_normal((B, T, Hk, D))).astype(np.float16)
    v = rng.standard_normal((B, T, Hv, D)).astype(np.float16)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))).astype(np.float32)
    g = (-np.logaddexp(0.0, rng.standard_normal((B, T, Hv)))).astype(np.float32)
    st = (0.05 * rng.standard_normal((B, Hv, D, D))).astype(np.float32)
    return q, k, v, g, beta, st


def _t(dev, x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _direct(dev, q, k, v, g, beta, st, f32=False):
    import torch
    tq, tk, tv, tg, tb, ts = (_t(dev, x) for x in (q, k, v, g, beta, st))
    if f32:  # the fp32-I/O entry points
        tq, tk, tv = tq.float(), tk.float(), tv.float()
    T = q.shape[1]
    if T == 1:
        o = tsa.gdn_decode_step(tq[:, 0], tk[:, 0], tv[:, 0], tg[:, 0], tb[:, 0], ts)[:, None]
    elif T < 32:
        o = tsa.gdn_recurrent_fwd(tq, tk, tv, tg, tb, ts)
    else:
        o = tsa.gdn_chunked_fwd(tq, tk, tv, tg, tb, ts)
    torch.cuda.synchronize()
    return o.cpu(), ts.cpu()


@pytest.mark.parametrize("T", [1, 20, 31, 32, 300, 1500])  # 1500: 2 x 6 heads, the sequence split
def test_dense_fp16_in_place(dev, T):
    import torch
    B, Hk, Hv = 2, 2, 6
    q, k, v, g, beta, st = _data(np.random.default_rng(T), B, T, Hk, Hv)
    o_ref, s_ref = _direct(dev, q, k, v, g, beta, st)
    tq, tk, tv, tg, tb, ts = (_t(dev, x) for x in (q, k, v, g, beta, st))
    out = torch.empty_like(tv)
    tsa.ggml_gated_delta_net(tq, tk, tv, tg, tb, ts, out)  # state in place
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), o_ref) and torch.equal(ts.cpu(), s_ref)


@pytest.mark.parametrize("T", [1, 33, 200])
def test_fp32_views_of_a_fused_projection(dev, T):
    """q, k, v as fp32 column blocks of one [B, T, (2 Hk + Hv) * D] projection output (the
    layout llama.cpp's graph slices), g / beta as views of a [B, T, 2 Hv] buffer, the output
    written as fp32 into every other row of a wider buffer, state_out a separate tensor."""
    import torch
    B, Hk, Hv = 2, 2, 4
    q, k, v, g, beta, st = _data(np.random.default_rng(50 + T), B, T, Hk, Hv)
    o_ref, s_ref = _direct(dev, q, k, v, g, beta, st, f32=True)
    o16, s16 = _direct(dev, q, k, v, g, beta, st)
    W = (2 * Hk + Hv) * D
    proj = torch.zeros(B, T, W, device=dev)
    proj[:, :, :Hk * D] = _t(dev, q).float().reshape(B, T, -1)
    proj[:, :, Hk * D:2 * Hk * D] = _t(dev, k).float().reshape(B, T, -1)
    proj[:, :, 2 * Hk * D:] = _t(dev, v).float().reshape(B, T, -1)
    qv = proj[:, :, :Hk * D].view(B, T, Hk, D)
    kv = proj[:, :, Hk * D:2 * Hk * D].view(B, T, Hk, D)
    vv = proj[:, :, 2 * Hk * D:].view(B, T, Hv, D)
    gb = torch.zeros(B, T, 2 * Hv, device=dev)
    gb[:, :, :Hv], gb[:, :, Hv:] = _t(dev, g), _t(dev, beta)
    outbuf = torch.full((B, T, 2, Hv, D), 7.0, device=dev)
    out = outbuf[:, :, 0]                      # non-dense fp32 output
    ts_in = _t(dev, st)
    ts_out = torch.empty_like(ts_in)
    assert not qv.is_contiguous() and not out.is_contiguous()
    tsa.ggml_gated_delta_net(qv, kv, vv, gb[:, :, :Hv], gb[:, :, Hv:], ts_in, out, ts_out)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and torch.equal(out.cpu(), o_ref)
    assert torch.equal(ts_out.cpu(), s_ref)
    # on fp16-exact inputs the decode and token-serial fp32 paths (T < 32) carry the fp16 path's
    # state bit for bit (their outputs may differ in the last rounding, tests/test_gpu_gdn.py
    # covers that); the chunked fp32 path takes its W S state operand and W's A operand as
    # fp16 hi + lo pairs, so its state agrees with the fp16 path's to the latter's rounding
    if T < 32:
        assert torch.equal(s_ref, s16)
    else:
        assert float((s_ref - s16).abs().max() / s16.abs().max()) < 3e-4
    assert torch.equal(ts_in.cpu(), torch.from_numpy(st))        # input state untouched
    assert bool((outbuf[:, :, 1] == 7.0).all())                    # the gaps untouched


def test_padded_state_out(dev):
    import torch
    B, T, Hk, Hv = 1, 96, 2, 4
    q, k, v, g, beta, st = _data(np.random.default_rng(9), B, T, Hk, Hv)
    o_ref, s_ref = _direct(dev, q, k, v, g, beta, st)
    tq, tk, tv, tg, tb, ts = (_t(dev, x) for x in (q, k, v, g, beta, st))
    pad = torch.full((B, Hv, D, D + 8), -1.0, device=dev)
    s_out = pad[:, :, :, :D]                   # rows 8 floats apart: not dense
    out = torch.empty_like(tv)
    tsa.ggml_gated_delta_net(tq, tk, tv, tg, tb, ts, out, s_out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), o_ref) and torch.equal(s_out.cpu(), s_ref)
    assert bool((pad[:, :, :, D:] == -1.0).all())


def test_against_oracle(dev, orc):
    import torch
    B, T, Hk, Hv = 1, 512, 16, 48   # the target model's GDN head counts
    q, k, v, g, beta, st = _data(np.random.default_rng(77), B, T, Hk, Hv)
    tq, tk, tv, tg, tb, ts = (_t(dev, x) for x in (q, k, v, g, beta, st))
    out = torch.empty(B, T, Hv, D, device=dev)   # fp32 output, as ggml's op writes
    tsa.ggml_gated_delta_net(tq.float(), tk.float(), tv.float(), tg, tb, ts, out)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.gdn_serial(q, k, v, g, beta, st)
    eo = float(np.abs(out.cpu().numpy() - o_ref).max())
    es = float(np.abs(ts.cpu().numpy() - s_ref).max() / np.abs(s_ref).max())
    print(f"ggml adapter T={T} Hv={Hv}: out max-abs {eo:.2e}  state rel {es:.2e}")
    assert eo < 2e-3 and es < 3e-4
