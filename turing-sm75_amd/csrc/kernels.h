// kernels.h -- internal launch functions behind the C-ABI (capi.cpp).  Arguments are
// validated by the caller; every function only enqueues work on `stream`.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace tsa {

// q, gate, o: [B][Hq][S][D]; k, v: [B][Hkv][S][D]; gate may be null; Hq % Hkv == 0.
hipError_t attn_fwd(const void* q, const void* k, const void* v, const void* gate, void* o, int B,
                    int Hq, int Hkv, int S, int D, float scale, int causal, hipStream_t stream);
hipError_t attn_naive(const void* q, const void* k, const void* v, const void* gate, void* o,
                      int B, int Hq, int Hkv, int S, int D, float scale, int causal,
                      hipStream_t stream);
// The VALU opponent (no MFMA): q, k, v, o [B][H][S][D].
hipError_t attn_valu(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                     int D, float scale, int causal, hipStream_t stream);

// Raw inputs of the fused pre-ops (the target model's layer): a, b [B][T][Hv]; dt_bias, A
// [Hv] (A = -exp(A_log)); eps of the q / k l2 norms.  g_log = softplus(a + dt_bias) * A,
// beta = sigmoid(b), q and k normalised per head row.
struct GdnRawGates {
    const float* a;
    const float* b;
    const float* dt_bias;
    const float* A;
    float eps;
};

// f32: q / k / v / out are fp32 (the reference's own I/O; a larger workspace), else fp16.
// nseg: the sequence-split plan, 0 = the library's (a function of the shapes), 1 = no split,
// n >= 2 = n segments (fewer when the sequence has fewer chunks).
size_t gdn_chunked_ws_bytes(int B, int T, int Hv, bool f32 = false, int nseg = 0);
hipError_t gdn_chunked(const void* q, const void* k, const void* v, const float* g_log,
                       const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                       float scale, void* ws, bool f32, hipStream_t stream, int nseg = 0);
// The chunked prefill without a caller workspace: the library's fixed device scratch array
// (gdn_chunked_noalloc_max_bytes() bytes per GPU) stands in for it; no allocation, no side
// stream.  The caller checks gdn_chunked_ws_bytes(...) against the maximum.
size_t gdn_chunked_noalloc_max_bytes();
// Workspace bytes of a no-allocation call: it splits the sequence only where that fits.
size_t gdn_chunked_noalloc_ws_bytes(int B, int T, int Hv);
hipError_t gdn_chunked_noalloc(const void* q, const void* k, const void* v, const float* g_log,
                               const float* beta, float* state, void* out, int B, int T, int Hq,
                               int Hv, float scale, hipStream_t stream);
// Carry workgroups of the last call on ws that gave up waiting and were redone by the second
// launch (synchronises `stream`).
hipError_t gdn_chunked_redo_count(const void* ws, int B, int T, int Hv, bool f32, int* count,
                                  hipStream_t stream);
// f32: q / k / v / out are fp32 (the reference's own I/O), else fp16.
hipError_t gdn_recurrent(const void* q, const void* k, const void* v, const float* g_log,
                         const float* beta, float* state, void* out, int B, int T, int Hq,
                         int Hv, float scale, bool f32, hipStream_t stream);
hipError_t gdn_chunked_fused(const void* q, const void* k, const void* v, const GdnRawGates& gates,
                             float* state, void* out, int B, int T, int Hq, int Hv, float scale,
                             void* ws, hipStream_t stream);
hipError_t gdn_decode_fused(const void* q, const void* k, const void* v, const GdnRawGates& gates,
                            float* state, void* out, int B, int Hq, int Hv, float scale,
                            hipStream_t stream);
hipError_t gdn_preprocess(const void* q, const void* k, const float* a, const float* b,
                          const float* dt_bias, const float* A, void* q_out, void* k_out,
                          float* g_log, float* beta, int B, int T, int Hq, int Hv, float eps,
                          hipStream_t stream);
hipError_t gdn_gated_rmsnorm(const void* x, const void* z, const float* w, void* y, int B, int T,
                             int Hv, float eps, hipStream_t stream);
// A strided 4-D view: ne[0] innermost, nb[i] byte strides (ggml's convention).
struct View4 {
    long long ne[4];
    long long nb[4];
};
// dst(view d, type dst_f16 ? fp16 : fp32) <- src(view s, likewise); d.ne must equal s.ne.
hipError_t copy4d(const void* src, int src_f16, const View4& s, void* dst, int dst_f16,
                  const View4& d, hipStream_t stream);

hipError_t gdn_naive(const void* q, const void* k, const void* v, const float* g_log,
                     const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                     int dk, int dv, float scale, bool f32, hipStream_t stream);

}  // namespace tsa
