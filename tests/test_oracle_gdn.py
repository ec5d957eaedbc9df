"""Oracle: Gated DeltaNet serial recurrence and chunk decomposition.

The serial oracle restates gdn_cpu (src/gdn_sm75.cu:1078-1106); the chunked oracle restates
the chunk structure of gdn_chunked_cpu (:1109-1244).

Why the chunk form is exact with Tm = (I + A)^-1 (rows = tokens t of one chunk, G = in-chunk
inclusive cumsum of g_log, S0 the state entering the chunk, S as dk x dv):
  unrolling S_t = e^{g_t} S_{t-1} + k_t (x) d_t gives
    S_t = e^{G_t} S0 + sum_{s<=t} e^{G_t - G_s} k_s (x) d_s,
  and d_t = beta_t (v_t - e^{g_t} S_{t-1}^T k_t) becomes
    d_t + sum_{s<t} A[t][s] d_s = beta_t v_t - beta_t e^{G_t} S0^T k_t,
    A[t][s] = beta_t (k_t . k_s) e^{G_t - G_s},
  so D = (I + A)^-1 (diag(beta) V - diag(beta e^G) K S0) = U - W S0,
    out_t = scale (e^{G_t} S0^T q_t + sum_{s<=t} e^{G_t - G_s} (k_s . q_t) d_s),
    S_C = e^{G_C} S0 + sum_s e^{G_C - G_s} k_s (x) d_s.
The reference's loop (:1161-1180) stores attn[i + t*C] and reads it as Tm[t][i]; its
forward substitution produces I - (I + A)^-1 A^T in that storage instead of (I + A^T)^-1,
which agrees with the exact inverse only to first order in A (C = 2: entry (1,1) is 1 + a^2
instead of 1).  The build pins chunked GDN to the serial recurrence, never to that loop.

Pins: float64 matrix-form fixtures (tests/golden/gdn_golden.npz); closed forms (beta = 0,
one token from a zero state, the delta rule's exact write of v under key k, orthonormal
keys); chunked(f64, exact) == serial for C = 16/32/64 and ragged T; the C = 2 closed form of
the reference's solve; prefill/decode state continuity; the affine segment map the
sequence split composes; a planted head-map mistake.
"""
import numpy as np
import pytest

D = 128


def _inputs(rng, B, T, Hq, Hv, sstd=0.0, d=D):
    l2n = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    q = l2n(rng.standard_normal((B, T, Hq, d))).astype(np.float16).astype(np.float32)
    k = l2n(rng.standard_normal((B, T, Hq, d))).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((B, T, Hv, d)).astype(np.float16).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))).astype(np.float32)
    g = (-np.logaddexp(0.0, rng.standard_normal((B, T, Hv)))).astype(np.float32)
    st = (sstd * rng.standard_normal((B, Hv, d, d))).astype(np.float32)
    return q, k, v, g, beta, st


def _rel(a, ref):
    return float(np.abs(a - ref).max() / max(np.abs(ref).max(), 1e-30))


def _golden_case(g, i):
    keys = ("q", "k", "v", "g", "beta", "state0", "out", "state1")
    q, k, v, gl, beta, s0, out, s1 = (g[f"c{i}_{n}"] for n in keys)
    f = lambda a: a.astype(np.float32)
    return f(q), f(k), f(v), f(gl), f(beta), f(s0), out, s1


@pytest.mark.parametrize("i", range(3))
def test_serial_matches_f64_golden(orc, golden, i):
    q, k, v, g, beta, s0, out, s1 = _golden_case(golden("gdn_golden.npz"), i)
    o, s = orc.gdn_serial(q, k, v, g, beta, s0)
    assert np.abs(o - out).max() < 1e-5
    assert _rel(s, s1) < 1e-5


@pytest.mark.parametrize("i", range(3))
@pytest.mark.parametrize("C", [16, 64])
def test_chunked_exact_matches_f64_golden(orc, golden, i, C):
    q, k, v, g, beta, s0, out, s1 = _golden_case(golden("gdn_golden.npz"), i)
    o, s = orc.gdn_chunked(q, k, v, g, beta, s0, chunk=C, exact=True, f64=True)
    assert np.abs(o - out).max() < 1e-6
    assert _rel(s, s1) < 1e-6


def test_planted_head_map_error_is_caught(orc, golden):
    q, k, v, g, beta, s0, out, s1 = _golden_case(golden("gdn_golden.npz"), 0)
    # V-head h must read QK head h % Hq; give every V-head QK head 0 instead
    q2, k2 = q.copy(), k.copy()
    q2[:, :, 1], k2[:, :, 1] = q[:, :, 0], k[:, :, 0]
    o, s = orc.gdn_serial(q2, k2, v, g, beta, s0)
    assert np.abs(o - out).max() > 1e-3 and _rel(s, s1) > 1e-2


def test_beta_zero_is_pure_decay(orc):
    rng = np.random.default_rng(11)
    q, k, v, g, beta, st = _inputs(rng, 1, 7, 1, 2, sstd=0.1)
    beta[:] = 0
    o, s = orc.gdn_serial(q, k, v, g, beta, st)
    G = np.cumsum(g.astype(np.float64), axis=1)  # [B,T,Hv]
    for h in range(2):
        S0 = st[0, h].astype(np.float64)  # [dv][dk]
        assert _rel(s[0, h], np.exp(G[0, -1, h]) * S0) < 1e-5
        for t in range(7):
            ref = np.exp(G[0, t, h]) * (S0 @ q[0, t, 0].astype(np.float64)) / np.sqrt(D)
            assert np.abs(o[0, t, h] - ref).max() < 1e-6


def test_one_token_from_zero_state(orc):
    rng = np.random.default_rng(12)
    q, k, v, g, beta, st = _inputs(rng, 2, 1, 1, 3)
    o, s = orc.gdn_serial(q, k, v, g, beta, st)
    for b in range(2):
        for h in range(3):
            kk, vv, bb = k[b, 0, 0].astype(np.float64), v[b, 0, h].astype(np.float64), beta[b, 0, h]
            assert _rel(s[b, h], bb * np.outer(vv, kk)) < 1e-6  # S[c][i] = beta v_c k_i
            ref = bb * (kk @ q[b, 0, 0]) * vv / np.sqrt(D)
            assert np.abs(o[b, 0, h] - ref).max() < 1e-6


def test_delta_rule_writes_v_under_unit_key(orc):
    # g = 0 (no decay) and beta = 1: after the update S^T k = v exactly, whatever S was.
    rng = np.random.default_rng(13)
    q, k, v, g, beta, st = _inputs(rng, 1, 5, 1, 2, sstd=0.3)
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32)
    g[:] = 0
    beta[:] = 1
    for t in range(1, 6):
        _, s = orc.gdn_serial(q[:, :t], k[:, :t], v[:, :t], g[:, :t], beta[:, :t], st)
        for h in range(2):
            read = s[0, h].astype(np.float64) @ k[0, t - 1, 0].astype(np.float64)
            assert np.abs(read - v[0, t - 1, h]).max() < 1e-4


def test_orthonormal_keys_retrieve_values(orc):
    rng = np.random.default_rng(14)
    T = 6
    basis = np.linalg.qr(rng.standard_normal((D, D)))[0][:, :T].T.astype(np.float32)
    k = basis[None, :, None, :].copy()
    q = np.zeros_like(k)
    v = rng.standard_normal((1, T, 1, D)).astype(np.float32)
    g = np.zeros((1, T, 1), np.float32)
    beta = np.ones((1, T, 1), np.float32)
    _, s = orc.gdn_serial(q, k, v, g, beta, np.zeros((1, 1, D, D), np.float32))
    for t in range(T):
        assert np.abs(s[0, 0] @ basis[t] - v[0, t, 0]).max() < 1e-4


@pytest.mark.parametrize("T,C", [(64, 64), (100, 64), (130, 32), (77, 16), (5, 64)])
def test_chunked_exact_equals_serial(orc, T, C):
    rng = np.random.default_rng(T * 131 + C)
    q, k, v, g, beta, st = _inputs(rng, 2, T, 2, 4, sstd=0.05)
    o_s, s_s = orc.gdn_serial(q, k, v, g, beta, st)
    o_c, s_c = orc.gdn_chunked(q, k, v, g, beta, st, chunk=C, exact=True, f64=True)
    assert np.abs(o_c - o_s).max() < 1e-5
    assert _rel(s_c, s_s) < 1e-5
    o_f, s_f = orc.gdn_chunked(q, k, v, g, beta, st, chunk=C, exact=True, f64=False)
    assert np.abs(o_f - o_s).max() < 1e-4 and _rel(s_f, s_s) < 1e-4


def test_chunk_size_invariance(orc):
    rng = np.random.default_rng(15)
    q, k, v, g, beta, st = _inputs(rng, 1, 128, 1, 2)
    res = [orc.gdn_chunked(q, k, v, g, beta, st, chunk=C) for C in (16, 32, 64)]
    for o, s in res[1:]:
        assert np.abs(o - res[0][0]).max() < 1e-6 and _rel(s, res[0][1]) < 1e-6


def test_reference_solve_closed_form_c2(orc):
    # kb in ggml [i + j*C] order; only the strictly-upper entry (i=0, j=1) = a is used.
    a = 0.37
    kb = np.array([0.0, 0.0, a, 0.0], np.float32)  # kb[0 + 1*2] = a
    attn = orc.ref_solve(kb)
    # reference loop: I - (I + A)^-1 A^T  ->  [[1, -a], [0, 1 + a^2]] read column-major
    assert np.allclose(attn, [1.0, 0.0, -a, 1.0 + a * a], atol=1e-7)
    # the exact (I + A^T)^-1 has 1 in that diagonal slot
    exact = np.linalg.inv(np.eye(2) + np.array([[0, a], [0, 0]])).T.reshape(-1)
    assert np.allclose(exact, [1.0, 0.0, -a, 1.0])


def test_reference_solve_is_only_first_order(orc):
    rng = np.random.default_rng(16)
    q, k, v, g, beta, st = _inputs(rng, 1, 256, 1, 2)
    o_s, s_s = orc.gdn_serial(q, k, v, g, beta, st)
    _, s_ref = orc.gdn_chunked(q, k, v, g, beta, st, chunk=64, exact=False, f64=False)
    _, s_ex = orc.gdn_chunked(q, k, v, g, beta, st, chunk=64, exact=True, f64=False)
    assert _rel(s_ex, s_s) < 1e-5
    assert _rel(s_ref, s_s) > 10 * _rel(s_ex, s_s)


def test_prefill_then_decode_equals_serial(orc):
    rng = np.random.default_rng(17)
    q, k, v, g, beta, st = _inputs(rng, 2, 70, 2, 2, sstd=0.02)
    o_all, s_all = orc.gdn_serial(q, k, v, g, beta, st)
    _, s1 = orc.gdn_chunked(q[:, :69], k[:, :69], v[:, :69], g[:, :69], beta[:, :69], st, chunk=64)
    o2, s2 = orc.gdn_serial(q[:, 69:], k[:, 69:], v[:, 69:], g[:, 69:], beta[:, 69:], s1)
    assert _rel(s2, s_all) < 1e-5
    assert np.abs(o2[:, 0] - o_all[:, 69]).max() < 1e-5


def test_segment_state_map_is_affine(orc):
    """The premise of the chunked prefill's sequence split: over a segment the state update is
    affine in the entering state, S_out = Phi S_in + Z, where Z is the segment run from a zero
    state and Phi the segment run with v = 0 from the identity.  With the state stored
    [dv][dk] that reads st_out = st_in @ st_Phi + st_Z (the combine's E' = E P + Z).  A slow
    gate keeps Phi far from both zero and the identity; the transposed composition fails."""
    rng = np.random.default_rng(23)
    B, T, Hq, Hv = 1, 150, 1, 2
    q, k, v, g, beta, _ = _inputs(rng, B, T, Hq, Hv)
    g = (-0.01 * (1 + 0.5 * rng.standard_normal(g.shape))).astype(np.float32)
    s_in = (0.5 * rng.standard_normal((B, Hv, D, D))).astype(np.float32)
    eye = np.broadcast_to(np.eye(D, dtype=np.float32), (B, Hv, D, D)).copy()
    _, s_out = orc.gdn_serial(q, k, v, g, beta, s_in)
    _, z = orc.gdn_serial(q, k, v, g, beta, np.zeros_like(s_in))
    _, phi = orc.gdn_serial(q, k, np.zeros_like(v), g, beta, eye)
    s64, p64 = s_in.astype(np.float64), phi.astype(np.float64)
    assert _rel(np.einsum("bhjd,bhde->bhje", s64, p64) + z, s_out) < 1e-5
    assert np.abs(phi - eye).max() > 0.05 and np.abs(phi).max() > 0.1
    assert _rel(np.einsum("bhjd,bhed->bhje", s64, p64) + z, s_out) > 1e-2


def test_serial_thread_count_does_not_change_results(orc):
    rng = np.random.default_rng(18)
    q, k, v, g, beta, st = _inputs(rng, 2, 9, 2, 4, sstd=0.02)
    a = orc.gdn_serial(q, k, v, g, beta, st, nthreads=1)
    b = orc.gdn_serial(q, k, v, g, beta, st, nthreads=4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
