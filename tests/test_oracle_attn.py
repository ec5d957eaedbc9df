"""Oracle: naive attention (restating src/attn_sm75.cu:55-94).

Pins, each chosen so a plausible mistake (wrong scale, missing max subtraction, a mask
off by one, swapped operands, wrong head offset) fails at least one:
  * the float64 dense-softmax fixtures (tests/golden/attn_golden.npz), tolerance set by the
    final fp16 rounding of O;
  * closed forms: S = 1 gives O = V; Q = 0 gives the (prefix) mean of V; constant V rows
    give O = V; a causal row ignores every later key; row 0 of a causal head is V[0];
  * permutation equivariance of non-causal attention over (K, V) rows;
  * a planted mistake (scale x 1.1) is caught by the fixture check.
"""
import numpy as np
import pytest


def _case(g, i):
    B, H, S, D, causal = (int(x) for x in g[f"c{i}_meta"])
    return g[f"c{i}_q"], g[f"c{i}_k"], g[f"c{i}_v"], g[f"c{i}_o"], bool(causal)


def _err(a, b):
    return float(np.abs(a.astype(np.float64) - b.astype(np.float64)).max())


@pytest.mark.parametrize("i", range(4))
def test_oracle_matches_f64_golden(orc, golden, i):
    q, k, v, o, causal = _case(golden("attn_golden.npz"), i)
    ours = orc.attn_naive(q, k, v, causal)
    # fp16 output rounding (|O| <= ~3: half-ulp <= 2^-10) plus fp32 accumulation
    assert _err(ours, o) < 2.5e-3


def test_planted_scale_error_is_caught(orc, golden):
    q, k, v, o, causal = _case(golden("attn_golden.npz"), 0)
    D = q.shape[-1]
    wrong = orc.attn_naive(q, k, v, causal, scale=1.1 / np.sqrt(D))
    assert _err(wrong, o) > 1e-2


def test_rows_api_matches_full(orc):
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((2, 3, 50, 64)).astype(np.float16) for _ in range(3))
    full = orc.attn_naive(q, k, v, True)
    rows = np.array([0, 7, 49, 50, 99, 151, 299])
    r, o32, o16 = orc.attn_rows(q, k, v, rows, True)
    flat = full.reshape(-1, 64)
    assert np.array_equal(o16.view(np.uint16), flat[r].view(np.uint16))
    assert np.array_equal(o32.astype(np.float16).view(np.uint16), flat[r].view(np.uint16))


@pytest.mark.parametrize("causal", [False, True])
def test_single_key_returns_v(orc, causal):
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((2, 2, 1, 128)).astype(np.float16) for _ in range(3))
    assert np.array_equal(orc.attn_naive(q, k, v, causal).view(np.uint16), v.view(np.uint16))


def test_zero_query_gives_prefix_mean(orc):
    rng = np.random.default_rng(5)
    S = 40
    q = np.zeros((1, 1, S, 64), np.float16)
    k = rng.standard_normal((1, 1, S, 64)).astype(np.float16)
    v = rng.standard_normal((1, 1, S, 64)).astype(np.float16)
    v64 = v.astype(np.float64)[0, 0]
    causal = orc.attn_naive(q, k, v, True).astype(np.float64)[0, 0]
    prefix = np.cumsum(v64, axis=0) / np.arange(1, S + 1)[:, None]
    assert np.abs(causal - prefix).max() < 2e-3
    full = orc.attn_naive(q, k, v, False).astype(np.float64)[0, 0]
    assert np.abs(full - v64.mean(axis=0)).max() < 2e-3


def test_constant_v_rows(orc):
    rng = np.random.default_rng(6)
    q, k = (rng.standard_normal((1, 2, 30, 64)).astype(np.float16) for _ in range(2))
    v = np.broadcast_to(rng.standard_normal((1, 2, 1, 64)), (1, 2, 30, 64)).astype(np.float16).copy()
    for causal in (False, True):
        o = orc.attn_naive(q, k, v, causal)
        assert _err(o, v) < 2e-3


def test_causal_ignores_future_keys(orc):
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 1, 64, 64)).astype(np.float16) for _ in range(3))
    o = orc.attn_naive(q, k, v, True)
    k2, v2 = k.copy(), v.copy()
    k2[0, 0, 40:] = rng.standard_normal((24, 64)).astype(np.float16)
    v2[0, 0, 40:] = rng.standard_normal((24, 64)).astype(np.float16)
    o2 = orc.attn_naive(q, k2, v2, True)
    assert np.array_equal(o[0, 0, :40].view(np.uint16), o2[0, 0, :40].view(np.uint16))
    assert not np.array_equal(o[0, 0, 40:].view(np.uint16), o2[0, 0, 40:].view(np.uint16))
    assert np.array_equal(o[0, 0, 0].view(np.uint16), v[0, 0, 0].view(np.uint16))


def test_noncausal_key_permutation(orc):
    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((1, 2, 45, 128)).astype(np.float16) for _ in range(3))
    perm = rng.permutation(45)
    a = orc.attn_naive(q, k, v, False)
    b = orc.attn_naive(q, k[:, :, perm].copy(), v[:, :, perm].copy(), False)
    assert _err(a, b) < 2e-3  # only the fp32 summation order changes


def test_heads_are_independent(orc):
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((2, 3, 20, 64)).astype(np.float16) for _ in range(3))
    o = orc.attn_naive(q, k, v, True)
    o1 = orc.attn_naive(q[1:2, 2:3].copy(), k[1:2, 2:3].copy(), v[1:2, 2:3].copy(), True)
    assert np.array_equal(o[1, 2].view(np.uint16), o1[0, 0].view(np.uint16))


# ---- gated grouped-query attention (oracle.attn_gqa_rows) ----
def _dense_gqa_f64(q, k, v, gate, causal, scale):
    """Independent float64 dense softmax with an explicit K/V head map and gate."""
    B, Hq, S, D = q.shape
    grp = Hq // k.shape[1]
    out = np.empty((B, Hq, S, D))
    for b in range(B):
        for h in range(Hq):
            kk, vv = k[b, h // grp].astype(np.float64), v[b, h // grp].astype(np.float64)
            s = scale * (q[b, h].astype(np.float64) @ kk.T)
            if causal:
                s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            o = (p / p.sum(axis=1, keepdims=True)) @ vv
            if gate is not None:
                o = o / (1.0 + np.exp(-gate[b, h].astype(np.float64)))
            out[b, h] = o
    return out


@pytest.mark.parametrize("Hq,Hkv,D,causal,gated", [(6, 1, 64, True, True), (4, 2, 128, False, True),
                                                   (24, 4, 256, True, True), (3, 3, 64, True, False)])
def test_gqa_matches_dense_f64(orc, Hq, Hkv, D, causal, gated):
    rng = np.random.default_rng(700 + Hq + D)
    B, S = 1, 37
    q = rng.standard_normal((B, Hq, S, D)).astype(np.float16)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    gate = rng.standard_normal((B, Hq, S, D)).astype(np.float16) if gated else None
    rows = np.arange(B * Hq * S)
    _, o = orc.attn_gqa_rows(q, k, v, gate, rows, causal)
    ref = _dense_gqa_f64(q, k, v, gate, causal, 1.0 / np.sqrt(D)).reshape(-1, D)
    assert np.abs(o - ref).max() < 1e-5


def test_gqa_equal_heads_is_plain_attention(orc):
    rng = np.random.default_rng(710)
    q, k, v = (rng.standard_normal((1, 3, 50, 64)).astype(np.float16) for _ in range(3))
    rows = np.arange(3 * 50)
    _, o = orc.attn_gqa_rows(q, k, v, None, rows, True)
    _, o32, _ = orc.attn_rows(q, k, v, rows, True)
    assert np.array_equal(o, o32.astype(np.float64))


def test_gqa_gate_closed_forms(orc):
    rng = np.random.default_rng(711)
    q = rng.standard_normal((1, 4, 20, 64)).astype(np.float16)
    k, v = (rng.standard_normal((1, 2, 20, 64)).astype(np.float16) for _ in range(2))
    rows = np.arange(4 * 20)
    _, plain = orc.attn_gqa_rows(q, k, v, None, rows, False)
    _, half = orc.attn_gqa_rows(q, k, v, np.zeros_like(q), rows, False)
    _, closed = orc.attn_gqa_rows(q, k, v, np.full_like(q, -60000.0), rows, False)
    assert np.allclose(half, plain / 2, rtol=0, atol=1e-12)   # sigmoid(0) = 1/2
    assert np.abs(closed).max() < 1e-20                     # sigmoid(-60000) ~ 0


def test_gqa_planted_head_map_error_is_caught(orc):
    # a head map h % Hkv instead of h // (Hq // Hkv) must not pass the dense comparison
    rng = np.random.default_rng(712)
    q = rng.standard_normal((1, 4, 16, 64)).astype(np.float16)
    k, v = (rng.standard_normal((1, 2, 16, 64)).astype(np.float16) for _ in range(2))
    rows = np.arange(4 * 16)
    _, o = orc.attn_gqa_rows(q, k, v, None, rows, True)
    wrong = np.stack([k[0, h % 2] for h in range(4)])[None], np.stack([v[0, h % 2] for h in range(4)])[None]
    _, o_wrong = orc.attn_gqa_rows(q, wrong[0], wrong[1], None, rows, True)
    assert np.abs(o - o_wrong).max() > 0.1
