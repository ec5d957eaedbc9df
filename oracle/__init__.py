"""numpy wrapper of oracle/liboracle.so -- the CPU restatement of the reference's naive paths.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the reference results are compared with or the timed CPU
baseline, never as the product.
The C++ sources cite the reference file:line each function restates (oracle.h).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_p = ctypes.c_void_p
_i, _f, _i64, _u32, _sz = ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_uint32, ctypes.c_size_t
_SIG = {
    "orc_f2h": [_p, _p, _sz],
    "orc_h2f": [_p, _p, _sz],
    "orc_mt_normal_half": [_u32, _f, _f, _sz, _i, _p],
    "orc_gdn_lcg_inputs": [_i, _i, _i, _i, _p, _p, _p, _p, _p],
    "orc_attn_rows": [_p, _p, _p, _i, _i, _i, _i, _f, _i, _p, _i64, _p, _p, _i],
    "orc_attn_naive": [_p, _p, _p, _p, _i, _i, _i, _i, _f, _i, _i],
    "orc_gdn_serial": [_p] * 7 + [_i] * 6 + [_f, _i],
    "orc_gdn_chunked_f64": [_p] * 7 + [_i] * 7 + [_f, _i, _i],
    "orc_gdn_chunked_f32": [_p] * 7 + [_i] * 7 + [_f, _i, _i],
    "orc_ref_solve": [_p, _p, _i],
}


def load():
    """Load liboracle.so once; TSA_ORACLE_LIB_PATH names another build (the sanitizer run)."""
    global _lib
    if _lib is None:
        path = os.environ.get("TSA_ORACLE_LIB_PATH") or LIB_PATH
        if not os.path.exists(path):
            raise OSError(f"{path} not found: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        for name, args in _SIG.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _threads(n):
    """Thread count for the parallel (b, h) loops: n, else $OMP_NUM_THREADS, else all cores."""
    if n:
        return int(n)
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def f2h(x) -> np.ndarray:
    """float32 -> fp16 bits (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().orc_f2h(_ptr(x), _ptr(out), x.size)
    return out


def h2f(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    load().orc_h2f(_ptr(h), _ptr(out), h.size)
    return out


def mt_normal_half(seed: int, mean: float, std: float, n: int, ntensors: int) -> np.ndarray:
    """The reference's make_tensor sequence: uint16 fp16 bits, shape [ntensors, n]."""
    out = np.empty((ntensors, n), dtype=np.uint16)
    load().orc_mt_normal_half(seed, mean, std, n, ntensors, _ptr(out))
    return out


def gdn_lcg_inputs(T: int, Hq: int, Hv: int, d: int = 128):
    """The GDN driver's LCG inputs (q, k [T,Hq,d], v [T,Hv,d], g_log, beta [T,Hv]) fp32."""
    q = np.empty((T, Hq, d), np.float32)
    k = np.empty((T, Hq, d), np.float32)
    v = np.empty((T, Hv, d), np.float32)
    g = np.empty((T, Hv), np.float32)
    b = np.empty((T, Hv), np.float32)
    load().orc_gdn_lcg_inputs(T, Hq, Hv, d, _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(b))
    return q, k, v, g, b


def _as_h16(a):
    a = np.asarray(a)
    if a.dtype == np.float16:
        return np.ascontiguousarray(a).view(np.uint16)
    assert a.dtype == np.uint16
    return np.ascontiguousarray(a)


def attn_naive(q, k, v, causal: bool, scale: float | None = None, nthreads=None) -> np.ndarray:
    """Naive attention on fp16 [B,H,S,D] arrays; returns fp16 [B,H,S,D]."""
    q, k, v = _as_h16(q), _as_h16(k), _as_h16(v)
    B, H, S, D = q.shape
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(D))
    out = np.empty_like(q)
    load().orc_attn_naive(_ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, S, D, float(scale),
                          int(causal), _threads(nthreads))
    return out.view(np.float16)


def attn_rows(q, k, v, rows, causal: bool, scale: float | None = None, nthreads=None):
    """Naive attention for the listed flat rows (bh*S + q).  Returns (fp32 acc/l, fp16)."""
    q, k, v = _as_h16(q), _as_h16(k), _as_h16(v)
    B, H, S, D = q.shape
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(D))
    rows = np.ascontiguousarray(np.sort(np.asarray(rows, dtype=np.int64)))
    o32 = np.empty((rows.size, D), np.float32)
    o16 = np.empty((rows.size, D), np.uint16)
    load().orc_attn_rows(_ptr(q), _ptr(k), _ptr(v), B, H, S, D, float(scale), int(causal),
                         _ptr(rows), rows.size, _ptr(o32), _ptr(o16), _threads(nthreads))
    return rows, o32, o16.view(np.float16)


def attn_gqa_rows(q, k, v, gate, rows, causal: bool, scale: float | None = None, nthreads=None):
    """Gated grouped-query attention for the listed flat rows (bh*S + q of q's [B,Hq,S,D]).

    Not a reference routine: the attention layer of the reference's target model (query
    head h reads K/V head h // (Hq // Hkv), output times sigmoid(gate), docs/qwen38-27b.md:13)
    defined on top of the pinned attention oracle: K/V repeated per query-head group, then
    the gate applied in float64.  Returns (rows, float64 [n, D])."""
    q, k, v = _as_h16(q), _as_h16(k), _as_h16(v)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0 and k.shape == (B, Hkv, S, D) and v.shape == k.shape
    grp = Hq // Hkv
    kr = np.ascontiguousarray(np.repeat(k, grp, axis=1))
    vr = np.ascontiguousarray(np.repeat(v, grp, axis=1))
    rows, o32, _ = attn_rows(q, kr, vr, rows, causal, scale, nthreads)
    o = o32.astype(np.float64)
    if gate is not None:
        gf = np.asarray(gate, dtype=np.float64).reshape(-1, D)[rows]
        with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: sigmoid 0
            o = o / (1.0 + np.exp(-gf))
    return rows, o


def _gdn_prep(q, k, v, g, b, state):
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32)
    q, k, v, g, b = f(q), f(k), f(v), f(g), f(b)
    B, T, Hq, dk = q.shape
    Hv, dv = v.shape[2], v.shape[3]
    st = np.array(state, dtype=np.float32, copy=True, order="C")
    assert st.shape == (B, Hv, dv, dk), st.shape
    out = np.empty((B, T, Hv, dv), np.float32)
    return q, k, v, g, b, st, out, (B, T, Hq, Hv, dk, dv)


def gdn_serial(q, k, v, g_log, beta, state, scale=None, nthreads=None):
    """gdn_cpu on [B,T,...] arrays (any float dtype, converted exactly to fp32).
    Returns (out fp32 [B,T,Hv,dv], new state fp32 [B,Hv,dv,dk])."""
    q, k, v, g, b, st, out, (B, T, Hq, Hv, dk, dv) = _gdn_prep(q, k, v, g_log, beta, state)
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(dk))
    load().orc_gdn_serial(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(b), _ptr(st), _ptr(out),
                          B, T, Hq, Hv, dk, dv, float(scale), _threads(nthreads))
    return out, st


def gdn_chunked(q, k, v, g_log, beta, state, chunk, exact=True, f64=True, scale=None,
                nthreads=None):
    """Chunk decomposition (exact inverse, or the reference's solve loop when exact=False)."""
    q, k, v, g, b, st, out, (B, T, Hq, Hv, dk, dv) = _gdn_prep(q, k, v, g_log, beta, state)
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(dk))
    fn = load().orc_gdn_chunked_f64 if f64 else load().orc_gdn_chunked_f32
    fn(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(b), _ptr(st), _ptr(out), B, T, Hq, Hv, dk, dv,
       int(chunk), float(scale), int(exact), _threads(nthreads))
    return out, st


def ref_solve(kb: np.ndarray) -> np.ndarray:
    """The C x C matrix the reference's solve loop returns for kb (ggml [i + j*C] order)."""
    kb = np.ascontiguousarray(kb, dtype=np.float32)
    C = int(round(np.sqrt(kb.size)))
    out = np.empty(C * C, np.float32)
    load().orc_ref_solve(_ptr(kb.reshape(-1)), _ptr(out), C)
    return out


# ---------------------------------------------------------------------------------------
# GDN pre/post ops of the target model's Gated DeltaNet layer (docs/qwen38-27b.md:15; the
# kernel's semantic source is llama.cpp's gated_delta_net, gdn_sm75.cu:3).  The reference
# tree holds no implementation of them: these restate the published definitions in float64
# (ggml's l2_norm, sigmoid, softplus and rms_norm, and the layer's gate g = softplus(a +
# dt_bias) * A with A = -exp(A_log)).  Parity against ggml itself is unpinned; the tests
# pin them by closed forms and invariants.
# ---------------------------------------------------------------------------------------
def l2norm_rows(x, eps: float = 1e-6) -> np.ndarray:
    """x / max(||x||_2, eps) over the last axis, float64 (ggml_l2_norm's definition)."""
    x = np.asarray(x, dtype=np.float64)
    n = np.sqrt(np.sum(x * x, axis=-1, keepdims=True))
    return x / np.maximum(n, eps)


def softplus(x) -> np.ndarray:
    """log(1 + e^x), float64; x above 20 passes through (the threshold ggml and torch use)."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def sigmoid(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-x))


def gdn_gates(a, b, dt_bias, A):
    """(g_log, beta) from the layer's projections: a, b [..., Hv]; dt_bias, A [Hv]."""
    g = softplus(np.asarray(a, np.float64) + np.asarray(dt_bias, np.float64)) * np.asarray(A, np.float64)
    return g, sigmoid(b)


def gdn_preprocess(q, k, a, b, dt_bias, A, eps: float = 1e-6):
    """The pre-ops: l2-normalised q, k (float64) and g_log, beta (float64)."""
    g, beta = gdn_gates(a, b, dt_bias, A)
    return l2norm_rows(q, eps), l2norm_rows(k, eps), g, beta


def gated_rmsnorm(x, z, w, eps: float = 1e-6) -> np.ndarray:
    """The post-op: x / sqrt(mean(x^2) + eps) * w * silu(z) over the last axis, float64."""
    x = np.asarray(x, dtype=np.float64)
    z = np.asarray(z, dtype=np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * np.asarray(w, np.float64) * (z * sigmoid(z))
