"""The GDN pre/post-op oracle (oracle.l2norm_rows, softplus, sigmoid, gdn_gates,
gated_rmsnorm) pinned by closed forms and invariants.

The reference tree holds no implementation of these ops (its inputs assume them applied;
their definitions follow llama.cpp's graph around gated_delta_net, src/gdn_sm75.cu:3), so
parity against ggml itself is unpinned.  Each check below is chosen so that a plausible
mistake (sum instead of mean, a missing eps guard, a sign error in the gate, a dropped
silu factor) fails one of them; test_planted_mistakes_are_caught shows that for some.
"""
import math

import numpy as np

import oracle


def test_l2norm_unit_rows_and_scale_invariance():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 7, 128))
    y = oracle.l2norm_rows(x)
    assert np.allclose(np.linalg.norm(y, axis=-1), 1.0, atol=1e-12)
    assert np.allclose(oracle.l2norm_rows(3.5 * x), y, atol=1e-12)
    # direction kept: y is a positive multiple of x
    assert np.all(np.sum(y * x, axis=-1) > 0)


def test_l2norm_eps_guard():
    # ||x|| below eps divides by eps (ggml's max(norm, eps)), zero rows stay zero
    x = np.zeros((2, 128))
    x[1, 3] = 1e-8
    y = oracle.l2norm_rows(x, eps=1e-6)
    assert np.all(y[0] == 0)
    assert math.isclose(y[1, 3], 1e-8 / 1e-6, rel_tol=1e-12)


def test_softplus_sigmoid_closed_forms():
    x = np.linspace(-15, 15, 301)
    sp = oracle.softplus(x)
    assert math.isclose(float(oracle.softplus(0.0)), math.log(2.0), rel_tol=1e-15)
    assert np.allclose(sp - oracle.softplus(-x), x, atol=1e-12)      # softplus(x) - softplus(-x) = x
    assert np.allclose(np.exp(sp), 1 + np.exp(x), rtol=1e-12)
    assert float(oracle.softplus(25.0)) == 25.0                        # pass-through above 20
    assert float(oracle.sigmoid(0.0)) == 0.5
    assert np.allclose(oracle.sigmoid(x) + oracle.sigmoid(-x), 1.0, atol=1e-15)
    # sigmoid is the derivative of softplus
    h = 1e-6
    assert np.allclose((oracle.softplus(x + h) - oracle.softplus(x - h)) / (2 * h), oracle.sigmoid(x), atol=1e-8)


def test_gdn_gates():
    Hv = 6
    dt = np.linspace(-1, 1, Hv)
    A = -np.exp(np.linspace(-0.5, 0.5, Hv))
    a = -dt[None, :] + np.zeros((3, Hv))      # softplus(0) = ln 2
    b = np.zeros((3, Hv))
    g, beta = oracle.gdn_gates(a, b, dt, A)
    assert np.allclose(g, math.log(2.0) * A[None, :], atol=1e-15)
    assert np.all(beta == 0.5)
    # A < 0 and softplus > 0: every log-decay is negative, every decay in (0, 1)
    g2, _ = oracle.gdn_gates(np.random.default_rng(1).standard_normal((4, Hv)), b[:1], dt, A)
    assert np.all(g2 < 0) and np.all(np.exp(g2) < 1)


def test_gated_rmsnorm_closed_forms():
    rng = np.random.default_rng(2)
    w = rng.uniform(0.5, 1.5, 128)
    z = rng.standard_normal((3, 128))
    silu = z / (1 + np.exp(-z))
    # constant rows: x / rms(x) = sign(c) (up to eps)
    for c in (2.0, -0.5):
        x = np.full((3, 128), c)
        y = oracle.gated_rmsnorm(x, z, w, eps=0.0)
        assert np.allclose(y, np.sign(c) * w * silu, atol=1e-12)
    # eps enters as rms = sqrt(mean(x^2) + eps)
    x = np.full((1, 128), 1e-3)
    y = oracle.gated_rmsnorm(x, np.full((1, 128), 50.0), np.ones(128), eps=1e-6)
    assert np.allclose(y, 1e-3 / math.sqrt(1e-6 + 1e-6) * 50.0, rtol=1e-12)
    # z = 0 gates everything off; the normalised part has unit rms
    x = rng.standard_normal((4, 128)) * 7
    assert np.all(oracle.gated_rmsnorm(x, np.zeros_like(x), w) == 0)
    ones = np.full_like(x, 40.0)   # silu(40) = 40 to double precision
    y = oracle.gated_rmsnorm(x, ones, np.ones(128), eps=0.0) / 40.0
    assert np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, atol=1e-12)


def test_preprocess_composes_with_the_recurrence():
    # the pre-ops feed the pinned recurrence oracle: with already-normalised rows and
    # g / beta given directly, l2norm is the identity (to rounding) and the result is the same
    rng = np.random.default_rng(3)
    B, T, Hq, Hv = 1, 20, 2, 4
    q = oracle.l2norm_rows(rng.standard_normal((B, T, Hq, 128)))
    k = oracle.l2norm_rows(rng.standard_normal((B, T, Hq, 128)))
    assert np.allclose(oracle.l2norm_rows(q), q, atol=1e-15)
    v = rng.standard_normal((B, T, Hv, 128)).astype(np.float32)
    g, beta = oracle.gdn_gates(rng.standard_normal((B, T, Hv)), rng.standard_normal((B, T, Hv)),
                               np.zeros(Hv), -np.ones(Hv))
    st = np.zeros((B, Hv, 128, 128), np.float32)
    o1, s1 = oracle.gdn_serial(q, k, v, g, beta, st)
    qn, kn, g2, b2 = oracle.gdn_preprocess(3 * q, 0.5 * k, rng.standard_normal((B, T, Hv)) * 0,
                                           np.zeros((B, T, Hv)), np.zeros(Hv), -np.ones(Hv))
    o2, s2 = oracle.gdn_serial(qn, kn, v, g, beta, st)
    assert np.allclose(o1, o2, atol=1e-6) and np.allclose(s1, s2, atol=1e-6)
    assert np.allclose(g2, -math.log(2.0)) and np.all(b2 == 0.5)


def test_planted_mistakes_are_caught():
    """Plausible wrong versions of the post-op fail the closed-form checks above."""
    rng = np.random.default_rng(4)
    w, z = np.ones(128), np.full((2, 128), 40.0)
    x = rng.standard_normal((2, 128))

    def sum_not_mean(x, z, w, eps=0.0):
        return x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + eps) * w * (z * oracle.sigmoid(z))

    def no_silu(x, z, w, eps=0.0):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w * z

    def unit_rms(f):
        y = f(x, z, w, 0.0) / 40.0
        return np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, atol=1e-9)

    assert unit_rms(oracle.gated_rmsnorm)
    assert not unit_rms(sum_not_mean)
    zz = np.full((2, 128), -1.0)   # silu(-1) = -0.2689..., not -1
    assert not np.allclose(no_silu(x, zz, w), oracle.gated_rmsnorm(x, zz, w, eps=0.0))
