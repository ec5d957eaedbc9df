"""GPU parity of the GDN layer's pre/post ops: tsa_gdn_preprocess, tsa_gdn_gated_rmsnorm,
and the fused entry points tsa_gdn_chunked_fused_fwd / tsa_gdn_decode_fused_step, against
the oracle (oracle.gdn_preprocess / gated_rmsnorm in float64, then the pinned recurrence
oracle oracle.gdn_serial on the pre-processed inputs).

Inputs are the raw quantities of the layer: q, k ~ N(0,1) rows (not normalised), gate
projections a, b ~ N(0,1), dt_bias ~ N(0, 0.5), A = -exp(N(0, 0.5)).  Gates: the recurrence
gates (outputs max-abs < 0.02, state within 1e-3 relative); the pre-op outputs are fp16
rows of unit norm (abs 2e-3) and fp32 gates (rel 1e-5); the post-op output abs 2e-2 /
rel 1e-2 of an fp16 value.  Cases: shapes of the target model's layer and the T=4096, Hq=16, Hv=32
prefill, ragged T, Hv % Hq != 0, batches, in-place forms, decode continuity.
"""
import numpy as np
import pytest

import tsa

pytestmark = pytest.mark.gpu
D = 128
OUT_GATE, STATE_GATE = 2e-2, 1e-3


def _raw(rng, B, T, Hq, Hv, sstd=0.0, lead=None):
    lead = (B, T) if lead is None else lead
    q = rng.standard_normal(lead + (Hq, D)).astype(np.float16)
    k = rng.standard_normal(lead + (Hq, D)).astype(np.float16)
    v = rng.standard_normal(lead + (Hv, D)).astype(np.float16)
    a = rng.standard_normal(lead + (Hv,)).astype(np.float32)
    b = rng.standard_normal(lead + (Hv,)).astype(np.float32)
    dt = (0.5 * rng.standard_normal(Hv)).astype(np.float32)
    A = (-np.exp(0.5 * rng.standard_normal(Hv))).astype(np.float32)
    st = ((sstd * rng.standard_normal((B, Hv, D, D))).astype(np.float32) if sstd
          else np.zeros((B, Hv, D, D), np.float32))
    return q, k, v, a, b, dt, A, st


def _dev(dev, *arrays):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in arrays]


def _rel(x, ref):
    return float(np.abs(x - ref).max() / max(np.abs(ref).max(), 1e-30))


def _ref_recurrence(orc, q, k, v, a, b, dt, A, st, eps=1e-6):
    qn, kn, g, beta = orc.gdn_preprocess(q.astype(np.float64), k.astype(np.float64), a, b, dt, A, eps)
    return orc.gdn_serial(qn, kn, v, g, beta, st)


def test_preprocess(dev, orc):
    import torch
    rng = np.random.default_rng(11)
    q, k, v, a, b, dt, A, _ = _raw(rng, 2, 37, 3, 5)
    q[0, 0, 0] = 0.0  # a zero row stays zero
    tq, tk, ta, tb, tdt, tA = _dev(dev, q, k, a, b, dt, A)
    qn, kn, g, beta = tsa.gdn_preprocess(tq, tk, ta, tb, tdt, tA)
    torch.cuda.synchronize()
    rq, rk, rg, rb = orc.gdn_preprocess(q, k, a, b, dt, A)
    eq = float(np.abs(qn.float().cpu().numpy() - rq).max())
    ek = float(np.abs(kn.float().cpu().numpy() - rk).max())
    eg, eb = _rel(g.cpu().numpy(), rg), _rel(beta.cpu().numpy(), rb)
    print(f"preprocess q {eq:.2e} k {ek:.2e} g rel {eg:.2e} beta rel {eb:.2e}")
    assert eq < 2e-3 and ek < 2e-3 and eg < 1e-5 and eb < 1e-5
    assert np.all(qn[0, 0, 0].cpu().numpy() == 0)


def test_preprocess_in_place(dev):
    import torch
    rng = np.random.default_rng(12)
    q, k, _, a, b, dt, A, _ = _raw(rng, 1, 64, 4, 8)
    tq, tk, ta, tb, tdt, tA = _dev(dev, q, k, a, b, dt, A)
    qn, kn, _, _ = tsa.gdn_preprocess(tq, tk, ta, tb, tdt, tA)
    g, beta = torch.empty_like(ta), torch.empty_like(tb)
    tsa._check(tsa.load().tsa_gdn_preprocess(
        tsa._ptr(tq), tsa._ptr(tk), tsa._ptr(ta), tsa._ptr(tb), tsa._ptr(tdt), tsa._ptr(tA),
        tsa._ptr(tq), tsa._ptr(tk), tsa._ptr(g), tsa._ptr(beta), 1, 64, 4, 8, D, 1e-6, None))
    torch.cuda.synchronize()
    assert torch.equal(tq, qn) and torch.equal(tk, kn)


@pytest.mark.parametrize("shape", [(1, 5, 48), (2, 33, 32), (1, 1, 1)])
def test_gated_rmsnorm(dev, orc, shape):
    import torch
    B, T, Hv = shape
    rng = np.random.default_rng(13 + T)
    x = (3 * rng.standard_normal((B, T, Hv, D))).astype(np.float16)
    z = rng.standard_normal((B, T, Hv, D)).astype(np.float16)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    tx, tz, tw = _dev(dev, x, z, w)
    y = tsa.gdn_gated_rmsnorm(tx, tz, tw)
    torch.cuda.synchronize()
    ref = orc.gated_rmsnorm(x, z, w)
    err = np.abs(y.float().cpu().numpy() - ref)
    print(f"gated rmsnorm {shape}: max-abs {err.max():.2e}")
    assert np.all(err <= 2e-2 * np.maximum(1.0, np.abs(ref)) * 0.5 + 1e-3)
    # in place (y aliases x) gives the same bits
    y2 = tsa.gdn_gated_rmsnorm(tx, tz, tw, out=tx)
    torch.cuda.synchronize()
    assert torch.equal(y2, y)


CASES = [  # B, T, Hq, Hv
    (1, 64, 2, 4),
    (1, 100, 3, 5),      # ragged T, Hv % Hq != 0
    (2, 130, 2, 6),      # batch, ragged
    (1, 1, 1, 1),
    (1, 4096, 16, 32),   # the T=4096, Hq=16, Hv=32 prefill from raw inputs
    (1, 2048, 2, 4),     # few heads, 32 chunks: the call splits the sequence (4 segments)
    (1, 1500, 1, 3),     # split into 3 segments of 8 chunks, the last chunk ragged
]


@pytest.mark.parametrize("case", CASES)
def test_chunked_fused(dev, orc, case):
    import torch
    B, T, Hq, Hv = case
    rng = np.random.default_rng(100 + T + Hv)
    q, k, v, a, b, dt, A, st = _raw(rng, B, T, Hq, Hv, sstd=0.05)
    tq, tk, tv, ta, tb, tdt, tA, ts = _dev(dev, q, k, v, a, b, dt, A, st)
    o = tsa.gdn_chunked_fused_fwd(tq, tk, tv, ta, tb, tdt, tA, ts)
    torch.cuda.synchronize()
    o_ref, s_ref = _ref_recurrence(orc, q, k, v, a, b, dt, A, st)
    eo, es = float(np.abs(o.float().cpu().numpy() - o_ref).max()), _rel(ts.cpu().numpy(), s_ref)
    print(f"chunked fused {case}: out max-abs {eo:.2e}  state rel {es:.2e}")
    assert eo < min(2e-3, OUT_GATE) and es < min(3e-4, STATE_GATE)


def test_chunked_fused_matches_preprocess_then_chunked(dev):
    import torch
    rng = np.random.default_rng(7)
    q, k, v, a, b, dt, A, st = _raw(rng, 1, 640, 4, 8, sstd=0.05)
    tq, tk, tv, ta, tb, tdt, tA, ts1 = _dev(dev, q, k, v, a, b, dt, A, st)
    ts2 = ts1.clone()
    o1 = tsa.gdn_chunked_fused_fwd(tq, tk, tv, ta, tb, tdt, tA, ts1)
    qn, kn, g, beta = tsa.gdn_preprocess(tq, tk, ta, tb, tdt, tA)
    o2 = tsa.gdn_chunked_fwd(qn, kn, tv, g, beta, ts2)
    torch.cuda.synchronize()
    eo = float((o1.float() - o2.float()).abs().max())
    es = float((ts1 - ts2).abs().max() / ts2.abs().max())
    print(f"fused vs unfused: out {eo:.2e}  state rel {es:.2e}")
    assert eo < 2e-3 and es < 1e-3


@pytest.mark.parametrize("shape", [(16, 16, 32), (3, 16, 48), (1, 1, 1)])
def test_decode_fused(dev, orc, shape):
    import torch
    B, Hq, Hv = shape
    rng = np.random.default_rng(200 + B + Hv)
    steps = 32
    st = (0.02 * rng.standard_normal((B, Hv, D, D))).astype(np.float32)
    raws = [_raw(rng, B, 1, Hq, Hv, lead=(B,)) for _ in range(steps)]
    ts = _dev(dev, st)[0]
    s_ref = st
    outs = []
    for q, k, v, a, b, dt, A, _ in raws:
        tq, tk, tv, ta, tb, tdt, tA = _dev(dev, q, k, v, a, b, dt, A)
        outs.append(tsa.gdn_decode_fused_step(tq, tk, tv, ta, tb, tdt, tA, ts))
    torch.cuda.synchronize()
    eo = 0.0
    for (q, k, v, a, b, dt, A, _), o in zip(raws, outs):
        o_ref, s_ref = _ref_recurrence(orc, q[:, None], k[:, None], v[:, None], a[:, None],
                                       b[:, None], dt, A, s_ref)
        eo = max(eo, float(np.abs(o.float().cpu().numpy() - o_ref[:, 0]).max()))
    es = _rel(ts.cpu().numpy(), s_ref)
    print(f"decode fused {shape} x{steps}: out max-abs {eo:.2e}  state rel {es:.2e}")
    assert eo < min(2e-3, OUT_GATE) and es < min(1e-5, STATE_GATE)
