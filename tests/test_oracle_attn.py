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
