"""Generate the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference (cookys/turing-sm75) commits no golden vectors and its code is CUDA, which
cannot run here, so these fixtures are computed from the mathematics the reference states,
in float64 numpy, in a formulation independent of the oracle's C++ loops:

  attention  O = softmax(scale Q K^T + mask) V as a dense matrix per head, float64
             (src/attn_sm75.cu:55-94 states the same two-pass softmax).
  GDN        per V-head h (QK head h % Hq, src/gdn_sm75.cu:11,68), with S as a dk x dv
             matrix:  S <- e^g S;  S <- S + outer(k, beta (v - S^T k));  o = scale S^T q
             (src/gdn_sm75.cu:6-11,1078-1106), float64, stored back in the reference's
             [Hv][dv][dk] state layout.
  LCG        the first values of the GDN driver's generator (src/gdn_sm75.cu:1270-1279)
             computed with Python integers.

Inputs are drawn with numpy's seeded generator and stored (fp16 inputs as float16), so
the fixtures are data only.
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def attn_f64(q, k, v, causal, scale):
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    B, H, S, D = q.shape
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    if causal:
        s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, v)


def gdn_f64(q, k, v, g, beta, state, scale):
    q, k, v, g, beta = (x.astype(np.float64) for x in (q, k, v, g, beta))
    B, T, Hq, dk = q.shape
    Hv, dv = v.shape[2], v.shape[3]
    out = np.zeros((B, T, Hv, dv))
    st = np.zeros((B, Hv, dv, dk))
    for b in range(B):
        for h in range(Hv):
            S = state[b, h].astype(np.float64).T.copy()  # dk x dv
            hq = h % Hq
            for t in range(T):
                kt, qt = k[b, t, hq], q[b, t, hq]
                S *= np.exp(g[b, t, h])
                S += np.outer(kt, beta[b, t, h] * (v[b, t, h] - S.T @ kt))
                out[b, t, h] = scale * (S.T @ qt)
            st[b, h] = S.T
    return out, st


def lcg_first(count):
    s, vals = 1, []
    for _ in range(count):
        s = (s * 1664525 + 1013904223) % 2**32
        vals.append((s >> 8) / 16777216.0 - 0.5)
    return np.array(vals)


def l2n(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def main():
    rng = np.random.default_rng(20261201)
    # ---- attention ----
    cases = [(1, 2, 33, 64, 1), (1, 3, 70, 128, 0), (2, 1, 129, 128, 1), (1, 1, 1, 64, 1)]
    arrays = {}
    for i, (B, H, S, D, causal) in enumerate(cases):
        q = rng.standard_normal((B, H, S, D)).astype(np.float16)
        k = rng.standard_normal((B, H, S, D)).astype(np.float16)
        v = rng.standard_normal((B, H, S, D)).astype(np.float16)
        scale = np.float32(1.0 / np.sqrt(np.float32(D)))
        arrays[f"c{i}_q"], arrays[f"c{i}_k"], arrays[f"c{i}_v"] = q, k, v
        arrays[f"c{i}_o"] = attn_f64(q, k, v, causal, float(scale)).astype(np.float32)
        arrays[f"c{i}_meta"] = np.array([B, H, S, D, causal], np.int64)
    np.savez_compressed(os.path.join(HERE, "attn_golden.npz"), **arrays)

    # ---- GDN (d = 128: the shape the kernels support) ----
    arrays = {}
    gcases = [  # B, T, Hq, Hv, state std
        (2, 37, 2, 2, 0.0),
        (1, 150, 1, 1, 0.0),
        (2, 5, 1, 2, 0.02),
    ]
    for i, (B, T, Hq, Hv, sstd) in enumerate(gcases):
        d = 128
        q = l2n(rng.standard_normal((B, T, Hq, d))).astype(np.float16)
        k = l2n(rng.standard_normal((B, T, Hq, d))).astype(np.float16)
        v = rng.standard_normal((B, T, Hv, d)).astype(np.float16)
        beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))).astype(np.float32)
        g = (-np.logaddexp(0.0, rng.standard_normal((B, T, Hv)))).astype(np.float32)
        # stored as fp16 values (exact in fp32) to keep the fixture small
        state = (sstd * rng.standard_normal((B, Hv, d, d))).astype(np.float16)
        scale = float(np.float32(1.0 / np.sqrt(np.float32(d))))
        out, st = gdn_f64(q, k, v, g, beta, state, scale)
        for name, a in (("q", q), ("k", k), ("v", v), ("beta", beta), ("g", g),
                        ("state0", state), ("out", out.astype(np.float32)),
                        ("state1", st.astype(np.float32))):
            arrays[f"c{i}_{name}"] = a
        arrays[f"c{i}_meta"] = np.array([B, T, Hq, Hv, d], np.int64)
    np.savez_compressed(os.path.join(HERE, "gdn_golden.npz"), **arrays)

    # ---- the GDN driver's LCG for T = 1, Hq = 16, Hv = 48, d = 128: q takes the first
    # 2048 draws, k the next 2048 (x0.2 each) ----
    nq = 1 * 16 * 128
    r = lcg_first(nq + 8)
    # rnd() is exact in float32; the reference then multiplies by 0.2f in float32
    r32 = r.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "lcg_golden.npz"),
                        q_first=r32[:8] * np.float32(0.2),
                        k_first=r32[nq:nq + 8] * np.float32(0.2))


if __name__ == "__main__":
    main()
