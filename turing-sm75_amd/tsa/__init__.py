"""ctypes binding of libtsa.so, the C-ABI declared in include/tsa.h, for torch tensors.

torch is only plumbing here (device memory and the current HIP stream); every call goes
straight to the hand-written gfx950 kernels.  There is no fallback: if the library is
missing or a call fails, an exception is raised.

Shapes and dtypes mirror the reference labs (cookys/turing-sm75):
  attention  q, k, v, o      [B, H, S, D] fp16                (src/attn_sm75.cu:64,254)
  GDN        q, k            [B, T, Hq, dk] fp16              (src/gdn_sm75.cu:75-77)
             v, out          [B, T, Hv, dv] fp16
             g_log, beta     [B, T, Hv] fp32
             state           [B, Hv, dv, dk] fp32, updated in place (:71-72,1094)
  decode     q, k [B, Hq, dk], v/out [B, Hv, dv], g_log/beta [B, Hv]
"""
from __future__ import annotations

import ctypes
import math
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libtsa.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_ROOT), "include", "tsa.h")

TSA_OK = 0
TSA_ERR_NULL = 1
TSA_ERR_SHAPE = 2
TSA_ERR_UNSUPPORTED = 3
TSA_ERR_WORKSPACE = 4
TSA_ERR_LAUNCH = 5
TSA_ERR_ARG = 6
TSA_ERR_SCRATCH = 7

TSA_TYPE_F32, TSA_TYPE_F16 = 0, 1


class TsaTensor(ctypes.Structure):
    """The tsa_tensor view of include/tsa.h (the fields of a ggml_tensor view)."""
    _fields_ = [("data", ctypes.c_void_p), ("type", ctypes.c_int),
                ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4)]


_tp = ctypes.POINTER(TsaTensor)


_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_SIGNATURES = {
    "tsa_strerror": (ctypes.c_char_p, [_i]),
    "tsa_version": (ctypes.c_char_p, []),
    "tsa_attn_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp]),
    "tsa_attn_naive": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp]),
    "tsa_attn_fwd_valu": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp]),
    "tsa_attn_gqa_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp]),
    "tsa_attn_gqa_naive": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp]),
    "tsa_gdn_chunked_workspace_bytes": (_sz, [_i] * 7),
    "tsa_gdn_chunked_fwd": (_i, [_vp] * 7 + [_i] * 7 + [_f, _vp, _sz, _vp]),
    "tsa_gdn_chunked_fwd_noalloc": (_i, [_vp] * 7 + [_i] * 7 + [_f, _vp]),
    "tsa_gdn_chunked_redo_count": (_i, [_vp, _sz] + [_i] * 8 + [ctypes.POINTER(ctypes.c_int), _vp]),
    "tsa_gdn_chunked_workspace_bytes_f32": (_sz, [_i] * 7),
    "tsa_gdn_chunked_plan_workspace_bytes": (_sz, [_i] * 9),
    "tsa_gdn_chunked_plan_fwd": (_i, [_vp] * 7 + [_i] * 7 + [_f, _i, _i, _vp, _sz, _vp]),
    "tsa_gdn_chunked_fwd_f32": (_i, [_vp] * 7 + [_i] * 7 + [_f, _vp, _sz, _vp]),
    "tsa_gdn_recurrent_fwd_f32": (_i, [_vp] * 7 + [_i] * 6 + [_f, _vp]),
    "tsa_gdn_decode_step_f32": (_i, [_vp] * 7 + [_i] * 5 + [_f, _vp]),
    "tsa_gdn_naive_f32": (_i, [_vp] * 7 + [_i] * 6 + [_f, _vp]),
    "tsa_gdn_recurrent_fwd": (_i, [_vp] * 7 + [_i] * 6 + [_f, _vp]),
    "tsa_gdn_decode_step": (_i, [_vp] * 7 + [_i] * 5 + [_f, _vp]),
    "tsa_gdn_naive": (_i, [_vp] * 7 + [_i] * 6 + [_f, _vp]),
    "tsa_gdn_chunked_fused_fwd": (_i, [_vp] * 9 + [_i] * 7 + [_f, _f, _vp, _sz, _vp]),
    "tsa_gdn_decode_fused_step": (_i, [_vp] * 9 + [_i] * 5 + [_f, _f, _vp]),
    "tsa_gdn_preprocess": (_i, [_vp] * 10 + [_i] * 5 + [_f, _vp]),
    "tsa_gdn_gated_rmsnorm": (_i, [_vp] * 4 + [_i] * 4 + [_f, _vp]),
    "tsa_ggml_gdn_workspace_bytes": (_sz, [_tp, _tp]),
    "tsa_ggml_gated_delta_net": (_i, [_tp] * 8 + [_f, _vp, _sz, _vp]),
}


class TsaError(RuntimeError):
    """A tsa_* entry point returned a non-zero code."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"tsa error {code}: {msg}")
        self.code = code


_lib = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Load libtsa.so once (raises OSError with a build hint when it is missing).  The
    environment variable TSA_LIB_PATH names another build of the same library (the tests'
    sanitizer run uses it)."""
    global _lib
    if _lib is None:
        path = path or os.environ.get("TSA_LIB_PATH") or LIB_PATH
        if not os.path.exists(path):
            raise OSError(f"{path} not found: build it with `make -C turing-sm75_amd` "
                          "(or __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions include/tsa.h declares."""
    text = open(path).read()
    return sorted(set(re.findall(r"\b(tsa_[a-z0-9_]+)\s*\(", text)))


def strerror(code: int) -> str:
    return load().tsa_strerror(code).decode()


def _check(code: int) -> None:
    if code != TSA_OK:
        raise TsaError(code, strerror(code))


def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _need(t, dtype, ndim, name):
    import torch
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype or t.dim() != ndim or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous {ndim}-d {dtype} CUDA tensor, got "
                         f"{tuple(t.shape)} {t.dtype} on {t.device}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _out(out, like, name="out"):
    """The output tensor: a new one shaped like `like`, or the caller's, which must have
    exactly that shape (a smaller one would be written past its end)."""
    import torch
    if out is None:
        return torch.empty_like(like)
    _need(out, like.dtype, like.dim(), name)
    if out.shape != like.shape:
        raise ValueError(f"{name}: expected shape {tuple(like.shape)}, got {tuple(out.shape)}")
    return out


def _scratch(nbytes, device, stream):
    """A workspace for one call.  It is allocated on the stream the kernels run on, so the
    caching allocator does not hand it out again before they have finished with it."""
    import torch
    s = torch.cuda.current_stream(device) if stream is None else stream
    with torch.cuda.stream(s):
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------
def attn_fwd(q, k, v, out=None, scale=None, causal=True, stream=None, naive=False, valu=False):
    """O = softmax(scale Q K^T [+ causal mask]) V on the MFMA kernel (or the naive one, or the
    VALU opponent with valu=True)."""
    import torch
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(t, torch.float16, 4, name)
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    B, H, S, D = q.shape
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.float16, 4, "out")
    if out.shape != q.shape:
        raise ValueError("out shape differs from q")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if naive and valu:
        raise ValueError("naive and valu select different kernels")
    fn = load().tsa_attn_naive if naive else (load().tsa_attn_fwd_valu if valu else load().tsa_attn_fwd)
    _check(fn(_ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, S, D, float(scale), int(bool(causal)),
              _stream(stream)))
    return out


def attn_gqa_fwd(q, k, v, gate=None, out=None, scale=None, causal=True, stream=None, naive=False):
    """Gated grouped-query attention: q, gate [B, Hq, S, D]; k, v [B, Hkv, S, D] with
    Hq % Hkv == 0; O = softmax(scale Q K^T [+ causal mask]) V, times sigmoid(gate) if given."""
    import torch
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(t, torch.float16, 4, name)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, S, D) or v.shape != k.shape:
        raise ValueError(f"k, v must be [B, Hkv, S, D] with q's B, S, D: {tuple(q.shape)} "
                         f"{tuple(k.shape)} {tuple(v.shape)}")
    if gate is not None:
        _need(gate, torch.float16, 4, "gate")
        if gate.shape != q.shape:
            raise ValueError("gate shape differs from q")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.float16, 4, "out")
    if out.shape != q.shape:
        raise ValueError("out shape differs from q")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    fn = load().tsa_attn_gqa_naive if naive else load().tsa_attn_gqa_fwd
    gp = _ptr(gate) if gate is not None else ctypes.c_void_p(0)
    _check(fn(_ptr(q), _ptr(k), _ptr(v), gp, _ptr(out), B, Hq, Hkv, S, D, float(scale),
              int(bool(causal)), _stream(stream)))
    return out


# ---------------------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------------------
def _gdn_shapes(q, k, v, g_log, beta, state, batched_t: bool):
    """Shapes of a GDN call; q, k, v are all fp16 (the library's I/O type) or all fp32 (the
    *_f32 entry points, the reference's own I/O)."""
    import torch
    nd = 4 if batched_t else 3
    io = q.dtype if isinstance(q, torch.Tensor) and q.dtype in (torch.float16, torch.float32) else torch.float16
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(t, io, nd, name)
    _need(g_log, torch.float32, nd - 1, "g_log")
    _need(beta, torch.float32, nd - 1, "beta")
    _need(state, torch.float32, 4, "state")
    if batched_t:
        B, T, Hq, dk = q.shape
        Hv, dv = v.shape[2], v.shape[3]
        ok = (k.shape == q.shape and v.shape[:2] == (B, T) and g_log.shape == (B, T, Hv)
              and beta.shape == (B, T, Hv) and state.shape == (B, Hv, dv, dk))
    else:
        B, Hq, dk = q.shape
        Hv, dv = v.shape[1], v.shape[2]
        T = 1
        ok = (k.shape == q.shape and v.shape[0] == B and g_log.shape == (B, Hv)
              and beta.shape == (B, Hv) and state.shape == (B, Hv, dv, dk))
    if not ok:
        raise ValueError("inconsistent GDN shapes: q %s k %s v %s g %s beta %s state %s" % (
            tuple(q.shape), tuple(k.shape), tuple(v.shape), tuple(g_log.shape),
            tuple(beta.shape), tuple(state.shape)))
    return B, T, Hq, Hv, dk, dv


def gdn_chunked_workspace_bytes(B, T, Hq, Hv, dk=128, dv=128, chunk=64, f32=False, nseg=None) -> int:
    """Workspace bytes of one chunked call.  With few heads and many chunks the library's plan
    splits the sequence and needs more; the plan is a function of the shapes.  nseg asks for
    an explicit plan (0 = the library's, 1 = no split, n >= 2 = n segments)."""
    if nseg is not None:
        return int(load().tsa_gdn_chunked_plan_workspace_bytes(B, T, Hq, Hv, dk, dv, chunk, int(bool(f32)),
                                                               int(nseg)))
    fn = load().tsa_gdn_chunked_workspace_bytes_f32 if f32 else load().tsa_gdn_chunked_workspace_bytes
    return int(fn(B, T, Hq, Hv, dk, dv, chunk))


def gdn_chunked_fwd(q, k, v, g_log, beta, state, out=None, scale=None, chunk=64, ws=None,
                    stream=None, nseg=None):
    """Chunked prefill; state [B, Hv, dv, dk] is updated in place; returns out.  fp32 q/k/v
    select tsa_gdn_chunked_fwd_f32 (fp32 out).  With few heads (B*Hv <= 21) and at least 16
    chunks the library splits the sequence into segments run side by side (same results to
    fp32 rounding).  nseg (through tsa_gdn_chunked_plan_fwd) asks for an explicit plan: 0 =
    the library's, 1 = no split, n >= 2 = n segments."""
    import torch
    B, T, Hq, Hv, dk, dv = _gdn_shapes(q, k, v, g_log, beta, state, True)
    out = _out(out, v)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    f32 = q.dtype == torch.float32
    need = gdn_chunked_workspace_bytes(B, T, Hq, Hv, dk, dv, chunk, f32=f32, nseg=nseg)
    if ws is None:
        ws = _scratch(need, q.device, stream)
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(g_log), _ptr(beta), _ptr(state), _ptr(out),
            B, T, Hq, Hv, dk, dv, chunk, float(scale))
    tail = (_ptr(ws), ws.numel() * ws.element_size(), _stream(stream))
    if nseg is not None:
        _check(load().tsa_gdn_chunked_plan_fwd(*args, int(f32), int(nseg), *tail))
    else:
        fn = load().tsa_gdn_chunked_fwd_f32 if f32 else load().tsa_gdn_chunked_fwd
        _check(fn(*args, *tail))
    return out


def gdn_chunked_redo_count(ws, B, T, Hq, Hv, dk=128, dv=128, chunk=64, f32=False, stream=None) -> int:
    """Carry workgroups of the last chunked call on ws that were redone after a timed-out wait
    (0 when prep and carry ran side by side); synchronises the stream."""
    c = ctypes.c_int(-1)
    _check(load().tsa_gdn_chunked_redo_count(_ptr(ws), ws.numel() * ws.element_size(), B, T, Hq,
                                             Hv, dk, dv, chunk, int(bool(f32)), ctypes.byref(c),
                                             _stream(stream)))
    return c.value


def gdn_recurrent_fwd(q, k, v, g_log, beta, state, out=None, scale=None, stream=None,
                      naive=False):
    """Token-serial recurrence over T tokens (or the naive check kernel); state in place.
    fp32 q/k/v select the *_f32 entry points."""
    import torch
    B, T, Hq, Hv, dk, dv = _gdn_shapes(q, k, v, g_log, beta, state, True)
    out = _out(out, v)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    sfx = "_f32" if q.dtype == torch.float32 else ""
    fn = getattr(load(), ("tsa_gdn_naive" if naive else "tsa_gdn_recurrent_fwd") + sfx)
    _check(fn(_ptr(q), _ptr(k), _ptr(v), _ptr(g_log), _ptr(beta), _ptr(state), _ptr(out),
              B, T, Hq, Hv, dk, dv, float(scale), _stream(stream)))
    return out


def gdn_decode_step(q, k, v, g_log, beta, state, out=None, scale=None, stream=None):
    """One token per sequence: q/k [B, Hq, dk], v [B, Hv, dv]; state in place (fp16 or fp32
    q/k/v/out)."""
    import torch
    B, _, Hq, Hv, dk, dv = _gdn_shapes(q, k, v, g_log, beta, state, False)
    out = _out(out, v)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    fn = load().tsa_gdn_decode_step_f32 if q.dtype == torch.float32 else load().tsa_gdn_decode_step
    _check(fn(
        _ptr(q), _ptr(k), _ptr(v), _ptr(g_log), _ptr(beta), _ptr(state), _ptr(out),
        B, Hq, Hv, dk, dv, float(scale), _stream(stream)))
    return out


def gdn_naive(q, k, v, g_log, beta, state, out=None, scale=None, stream=None):
    """The naive on-device check kernel (one thread per state column)."""
    return gdn_recurrent_fwd(q, k, v, g_log, beta, state, out, scale, stream, naive=True)


# ---- the layer's pre / post ops (q, k l2 norm; beta = sigmoid(b); g_log = softplus(a +
# dt_bias) * A; gated RMSNorm of the output), fused or as passes of their own ----
def _gates(a, b, dt_bias, A, lead, Hv):
    import torch
    for name, t in (("a", a), ("b", b)):
        _need(t, torch.float32, len(lead) + 1, name)
        if tuple(t.shape) != tuple(lead) + (Hv,):
            raise ValueError(f"{name}: expected shape {tuple(lead) + (Hv,)}, got {tuple(t.shape)}")
    for name, t in (("dt_bias", dt_bias), ("A", A)):
        _need(t, torch.float32, 1, name)
        if t.numel() != Hv:
            raise ValueError(f"{name}: expected {Hv} values, got {t.numel()}")


def gdn_chunked_fused_fwd(q, k, v, a, b, dt_bias, A, state, out=None, scale=None, eps=1e-6,
                          chunk=64, ws=None, stream=None):
    """Chunked prefill from raw q, k [B,T,Hq,dk] and raw gate projections a, b [B,T,Hv]
    (fp16 q / k / v / out)."""
    import torch
    _need(q, torch.float16, 4, "q")
    B, T, Hq, Hv, dk, dv = _gdn_shapes(q, k, v, a, b, state, True)
    _gates(a, b, dt_bias, A, (B, T), Hv)
    out = _out(out, v)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    need = gdn_chunked_workspace_bytes(B, T, Hq, Hv, dk, dv, chunk)
    if ws is None:
        ws = _scratch(need, q.device, stream)
    _check(load().tsa_gdn_chunked_fused_fwd(
        _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(dt_bias), _ptr(A), _ptr(state),
        _ptr(out), B, T, Hq, Hv, dk, dv, chunk, float(scale), float(eps), _ptr(ws),
        ws.numel() * ws.element_size(), _stream(stream)))
    return out


def gdn_decode_fused_step(q, k, v, a, b, dt_bias, A, state, out=None, scale=None, eps=1e-6,
                          stream=None):
    """One decode step from raw q, k [B,Hq,dk] and raw gate projections a, b [B,Hv] (fp16
    q / k / v / out)."""
    import torch
    _need(q, torch.float16, 3, "q")
    B, _, Hq, Hv, dk, dv = _gdn_shapes(q, k, v, a, b, state, False)
    _gates(a, b, dt_bias, A, (B,), Hv)
    out = _out(out, v)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    _check(load().tsa_gdn_decode_fused_step(
        _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(dt_bias), _ptr(A), _ptr(state),
        _ptr(out), B, Hq, Hv, dk, dv, float(scale), float(eps), _stream(stream)))
    return out


def gdn_preprocess(q, k, a, b, dt_bias, A, eps=1e-6, stream=None):
    """The pre-ops as a pass: returns (q_n, k_n, g_log, beta) for raw q, k [B,T,Hq,dk]."""
    import torch
    _need(q, torch.float16, 4, "q")
    _need(k, torch.float16, 4, "k")
    if k.shape != q.shape:
        raise ValueError("q and k must have the same shape")
    B, T, Hq, dk = q.shape
    Hv = a.shape[-1]
    _gates(a, b, dt_bias, A, (B, T), Hv)
    qn, kn = torch.empty_like(q), torch.empty_like(k)
    g_log, beta = torch.empty_like(a), torch.empty_like(b)
    _check(load().tsa_gdn_preprocess(
        _ptr(q), _ptr(k), _ptr(a), _ptr(b), _ptr(dt_bias), _ptr(A), _ptr(qn), _ptr(kn),
        _ptr(g_log), _ptr(beta), B, T, Hq, Hv, dk, float(eps), _stream(stream)))
    return qn, kn, g_log, beta


def gdn_gated_rmsnorm(x, z, w, out=None, eps=1e-6, stream=None):
    """y = x / sqrt(mean(x^2) + eps) * w * silu(z) over dv; x, z [B,T,Hv,dv] fp16, w [dv]."""
    import torch
    _need(x, torch.float16, 4, "x")
    _need(z, torch.float16, 4, "z")
    _need(w, torch.float32, 1, "w")
    if z.shape != x.shape or w.numel() != x.shape[3]:
        raise ValueError("inconsistent shapes: x %s z %s w %s" % (tuple(x.shape), tuple(z.shape),
                                                                 tuple(w.shape)))
    out = _out(out, x)
    B, T, Hv, dv = x.shape
    _check(load().tsa_gdn_gated_rmsnorm(_ptr(x), _ptr(z), _ptr(w), _ptr(out), B, T, Hv, dv,
                                        float(eps), _stream(stream)))
    return out


# ---- ggml-layout adapter ----
def ggml_view(t) -> TsaTensor:
    """The ggml view of a torch tensor of up to 4 dims: ne / nb are its shape / strides in
    reverse order (ne[0] = the innermost dimension), padded with 1s."""
    import torch
    if t.dtype not in (torch.float32, torch.float16):
        raise ValueError(f"ggml views are fp32 or fp16, got {t.dtype}")
    if t.dim() > 4 or not t.is_cuda:
        raise ValueError("a ggml view is a CUDA tensor of at most 4 dims")
    ne = list(reversed(t.shape)) + [1] * (4 - t.dim())
    es = t.element_size()
    nb = [st * es for st in reversed(t.stride())]
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1] if nb else es)
    v = TsaTensor()
    v.data = t.data_ptr()
    v.type = TSA_TYPE_F16 if t.dtype == torch.float16 else TSA_TYPE_F32
    for i in range(4):
        v.ne[i] = int(ne[i])
        v.nb[i] = int(nb[i])
    return v


def ggml_gdn_workspace_bytes(q, v) -> int:
    return int(load().tsa_ggml_gdn_workspace_bytes(ctypes.byref(ggml_view(q)), ctypes.byref(ggml_view(v))))


def ggml_gated_delta_net(q, k, v, g_log, beta, state, out, state_out=None, scale=None, ws=None,
                         stream=None):
    """Torch tensors in the kernels' index order ([B, T, H, S] for q / k / v / out,
    [B, T, Hv] for g_log / beta, [B, Hv, S, S] for the states), any strides / fp32 or fp16:
    passed as ggml views.  state_out defaults to state (in place)."""
    import torch
    if state_out is None:
        state_out = state
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    views = [ggml_view(x) for x in (q, k, v, g_log, beta, state, out, state_out)]
    need = int(load().tsa_ggml_gdn_workspace_bytes(ctypes.byref(views[0]), ctypes.byref(views[2])))
    if ws is None:
        ws = _scratch(need, q.device, stream)
    _check(load().tsa_ggml_gated_delta_net(*[ctypes.byref(x) for x in views], float(scale),
                                           _ptr(ws), ws.numel() * ws.element_size(), _stream(stream)))
    return out
