// capi.cpp -- the extern "C" boundary declared in include/tsa.h.
//
// Validation happens here, before any HIP call, so argument errors are reported the same
// way on machines without a GPU.  The launch functions in kernels.h assume valid input.
#include <climits>
#include <cmath>

#include "../../include/tsa.h"
#include "kernels.h"

namespace {

inline int from_hip(hipError_t e) { return e == hipSuccess ? TSA_OK : TSA_ERR_LAUNCH; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// a * b * c fits in an int (workgroup counts and per-dimension products).
inline bool fits_int(long long a, long long b, long long c = 1) {
    return a >= 0 && b >= 0 && c >= 0 && a * b <= INT_MAX && a * b * c <= INT_MAX;
}

int check_attn(const void* q, const void* k, const void* v, const void* o, int B, int H, int S,
               int D, float scale, int causal, int Hkv = -1) {
    if (!q || !k || !v || !o) return TSA_ERR_NULL;
    if (Hkv == -1) Hkv = H;
    if (B < 1 || H < 1 || Hkv < 1 || S < 1 || D < 1) return TSA_ERR_SHAPE;
    if (H % Hkv != 0) return TSA_ERR_SHAPE;
    if (D != 64 && D != 128 && D != 256) return TSA_ERR_UNSUPPORTED;
    if (causal != 0 && causal != 1) return TSA_ERR_ARG;
    // The running max is taken over raw q.k, which is the max of the scaled scores only
    // for scale > 0 (the reference's scale is 1/sqrt(D), src/attn_sm75.cu:462).
    if (!(scale > 0.f) || !std::isfinite(scale)) return TSA_ERR_ARG;
    // workgroups: B*H*ceil(S/128) for the MFMA kernel, B*H*ceil(S/64) for the VALU one,
    // B*H*S/128 for the naive one
    if (!fits_int(B, H, S)) return TSA_ERR_SHAPE;
    return TSA_OK;
}

int check_gdn(const void* q, const void* k, const void* v, const float* g, const float* beta,
              const float* state, const void* out, int B, int T, int Hq, int Hv, int dk, int dv,
              float scale) {
    if (!q || !k || !v || !g || !beta || !state || !out) return TSA_ERR_NULL;
    if (B < 1 || T < 1 || Hq < 1 || Hv < 1 || dk < 1 || dv < 1) return TSA_ERR_SHAPE;
    if (!std::isfinite(scale)) return TSA_ERR_ARG;
    // element offsets are 64-bit in every kernel; only workgroup counts must fit an int
    if (!fits_int(B, Hv, dv)) return TSA_ERR_SHAPE;
    return TSA_OK;
}

// The raw gate inputs of the fused pre-ops and the l2-norm eps.
int check_gates(const float* a, const float* b, const float* dt_bias, const float* A, float eps) {
    if (!a || !b || !dt_bias || !A) return TSA_ERR_NULL;
    if (!(eps > 0.f) || !std::isfinite(eps)) return TSA_ERR_ARG;
    return TSA_OK;
}

}  // namespace

extern "C" const char* tsa_strerror(int code) {
    switch (code) {
        case TSA_OK: return "ok";
        case TSA_ERR_NULL: return "a required pointer is NULL";
        case TSA_ERR_SHAPE: return "invalid shape (size < 1, too large, or inconsistent)";
        case TSA_ERR_UNSUPPORTED: return "shape not supported by this library (attention: D in {64,128,256}; GDN: dk = dv = 128, chunk = 64)";
        case TSA_ERR_WORKSPACE: return "workspace is NULL or smaller than the required size";
        case TSA_ERR_LAUNCH: return "the HIP runtime rejected a kernel launch";
        case TSA_ERR_ARG: return "invalid argument (causal not 0/1, scale not finite / not > 0, or eps not finite / not > 0)";
        case TSA_ERR_SCRATCH: return "the shapes need more than the 64 MiB device scratch of tsa_gdn_chunked_fwd_noalloc (use tsa_gdn_chunked_fwd with a workspace)";
        default: return "unknown tsa error code";
    }
}

extern "C" const char* tsa_version(void) { return "tsa 0.1 gfx950"; }

extern "C" int tsa_attn_fwd(const void* q, const void* k, const void* v, void* o, int B, int H,
                            int S, int D, float scale, int causal, void* stream) {
    const int rc = check_attn(q, k, v, o, B, H, S, D, scale, causal);
    if (rc) return rc;
    return from_hip(tsa::attn_fwd(q, k, v, nullptr, o, B, H, H, S, D, scale, causal,
                                  as_stream(stream)));
}

extern "C" int tsa_attn_naive(const void* q, const void* k, const void* v, void* o, int B,
                              int H, int S, int D, float scale, int causal, void* stream) {
    const int rc = check_attn(q, k, v, o, B, H, S, D, scale, causal);
    if (rc) return rc;
    return from_hip(tsa::attn_naive(q, k, v, nullptr, o, B, H, H, S, D, scale, causal,
                                    as_stream(stream)));
}

extern "C" int tsa_attn_fwd_valu(const void* q, const void* k, const void* v, void* o, int B,
                                 int H, int S, int D, float scale, int causal, void* stream) {
    const int rc = check_attn(q, k, v, o, B, H, S, D, scale, causal);
    if (rc) return rc;
    return from_hip(tsa::attn_valu(q, k, v, o, B, H, S, D, scale, causal, as_stream(stream)));
}

extern "C" int tsa_attn_gqa_fwd(const void* q, const void* k, const void* v, const void* gate,
                                void* o, int B, int Hq, int Hkv, int S, int D, float scale,
                                int causal, void* stream) {
    const int rc = check_attn(q, k, v, o, B, Hq, S, D, scale, causal, Hkv);
    if (rc) return rc;
    return from_hip(tsa::attn_fwd(q, k, v, gate, o, B, Hq, Hkv, S, D, scale, causal,
                                  as_stream(stream)));
}

extern "C" int tsa_attn_gqa_naive(const void* q, const void* k, const void* v, const void* gate,
                                  void* o, int B, int Hq, int Hkv, int S, int D, float scale,
                                  int causal, void* stream) {
    const int rc = check_attn(q, k, v, o, B, Hq, S, D, scale, causal, Hkv);
    if (rc) return rc;
    return from_hip(tsa::attn_naive(q, k, v, gate, o, B, Hq, Hkv, S, D, scale, causal,
                                    as_stream(stream)));
}

extern "C" size_t tsa_gdn_chunked_workspace_bytes(int B, int T, int Hq, int Hv, int dk, int dv,
                                                  int chunk) {
    if (B < 1 || T < 1 || Hq < 1 || Hv < 1 || dk != 128 || dv != 128 || chunk != 64) return 0;
    return tsa::gdn_chunked_ws_bytes(B, T, Hv, false);
}

extern "C" size_t tsa_gdn_chunked_workspace_bytes_f32(int B, int T, int Hq, int Hv, int dk, int dv,
                                                      int chunk) {
    if (B < 1 || T < 1 || Hq < 1 || Hv < 1 || dk != 128 || dv != 128 || chunk != 64) return 0;
    return tsa::gdn_chunked_ws_bytes(B, T, Hv, true);
}

extern "C" size_t tsa_gdn_chunked_plan_workspace_bytes(int B, int T, int Hq, int Hv, int dk, int dv,
                                                       int chunk, int io_f32, int nseg) {
    if (B < 1 || T < 1 || Hq < 1 || Hv < 1 || dk != 128 || dv != 128 || chunk != 64) return 0;
    if ((io_f32 != 0 && io_f32 != 1) || nseg < 0) return 0;
    return tsa::gdn_chunked_ws_bytes(B, T, Hv, io_f32 != 0, nseg);
}

namespace {
int chunked(const void* q, const void* k, const void* v, const float* g_log, const float* beta,
            float* state, void* out, int B, int T, int Hq, int Hv, int dk, int dv, int chunk,
            float scale, void* ws, size_t ws_bytes, bool f32, void* stream, int nseg = 0) {
    int rc = check_gdn(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale);
    if (rc) return rc;
    if (chunk < 1) return TSA_ERR_SHAPE;
    if (dk != 128 || dv != 128 || chunk != 64) return TSA_ERR_UNSUPPORTED;
    if (nseg < 0) return TSA_ERR_ARG;
    const long long nch = (T + 63LL) / 64;
    if (!fits_int(B, Hv, nch) || !fits_int(B, Hv, 8)) return TSA_ERR_SHAPE;
    const size_t need = tsa::gdn_chunked_ws_bytes(B, T, Hv, f32, nseg);
    if (!ws || ws_bytes < need) return TSA_ERR_WORKSPACE;
    return from_hip(tsa::gdn_chunked(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, scale, ws, f32,
                                     as_stream(stream), nseg));
}
}  // namespace

extern "C" int tsa_gdn_chunked_plan_fwd(const void* q, const void* k, const void* v,
                                        const float* g_log, const float* beta, float* state, void* out,
                                        int B, int T, int Hq, int Hv, int dk, int dv, int chunk,
                                        float scale, int io_f32, int nseg, void* ws, size_t ws_bytes,
                                        void* stream) {
    if (io_f32 != 0 && io_f32 != 1) return TSA_ERR_ARG;
    return chunked(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, chunk, scale, ws, ws_bytes,
                   io_f32 != 0, stream, nseg);
}

extern "C" int tsa_gdn_chunked_fwd(const void* q, const void* k, const void* v,
                                   const float* g_log, const float* beta, float* state, void* out,
                                   int B, int T, int Hq, int Hv, int dk, int dv, int chunk,
                                   float scale, void* ws, size_t ws_bytes, void* stream) {
    return chunked(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, chunk, scale, ws, ws_bytes,
                   false, stream);
}

extern "C" int tsa_gdn_chunked_fwd_f32(const float* q, const float* k, const float* v,
                                       const float* g_log, const float* beta, float* state, float* out,
                                       int B, int T, int Hq, int Hv, int dk, int dv, int chunk,
                                       float scale, void* ws, size_t ws_bytes, void* stream) {
    return chunked(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, chunk, scale, ws, ws_bytes,
                   true, stream);
}

extern "C" int tsa_gdn_chunked_fwd_noalloc(const void* q, const void* k, const void* v,
                                           const float* g_log, const float* beta, float* state,
                                           void* out, int B, int T, int Hq, int Hv, int dk, int dv,
                                           int chunk, float scale, void* stream) {
    int rc = check_gdn(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale);
    if (rc) return rc;
    if (chunk < 1) return TSA_ERR_SHAPE;
    if (dk != 128 || dv != 128 || chunk != 64) return TSA_ERR_UNSUPPORTED;
    const long long nch = (T + 63LL) / 64;
    if (!fits_int(B, Hv, nch) || !fits_int(B, Hv, 8)) return TSA_ERR_SHAPE;
    if (tsa::gdn_chunked_noalloc_ws_bytes(B, T, Hv) > tsa::gdn_chunked_noalloc_max_bytes()) return TSA_ERR_SCRATCH;
    return from_hip(tsa::gdn_chunked_noalloc(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, scale,
                                             as_stream(stream)));
}

extern "C" int tsa_gdn_chunked_redo_count(const void* ws, size_t ws_bytes, int B, int T, int Hq,
                                          int Hv, int dk, int dv, int chunk, int io_f32, int* count,
                                          void* stream) {
    if (!ws || !count) return TSA_ERR_NULL;
    if (B < 1 || T < 1 || Hq < 1 || Hv < 1 || chunk < 1) return TSA_ERR_SHAPE;
    if (dk != 128 || dv != 128 || chunk != 64) return TSA_ERR_UNSUPPORTED;
    if (io_f32 != 0 && io_f32 != 1) return TSA_ERR_ARG;
    const long long nch = (T + 63LL) / 64;
    if (!fits_int(B, Hv, nch) || !fits_int(B, Hv, 8)) return TSA_ERR_SHAPE;
    if (ws_bytes < tsa::gdn_chunked_ws_bytes(B, T, Hv, io_f32 != 0)) return TSA_ERR_WORKSPACE;
    return from_hip(tsa::gdn_chunked_redo_count(ws, B, T, Hv, io_f32 != 0, count, as_stream(stream)));
}

namespace {
int recurrent(const void* q, const void* k, const void* v, const float* g_log, const float* beta,
              float* state, void* out, int B, int T, int Hq, int Hv, int dk, int dv, float scale,
              bool f32, void* stream) {
    int rc = check_gdn(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale);
    if (rc) return rc;
    if (dk != 128 || dv != 128) return TSA_ERR_UNSUPPORTED;
    if (!fits_int(B, Hv, 4)) return TSA_ERR_SHAPE;
    return from_hip(tsa::gdn_recurrent(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, scale, f32,
                                       as_stream(stream)));
}

int naive(const void* q, const void* k, const void* v, const float* g_log, const float* beta,
          float* state, void* out, int B, int T, int Hq, int Hv, int dk, int dv, float scale,
          bool f32, void* stream) {
    int rc = check_gdn(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale);
    if (rc) return rc;
    return from_hip(tsa::gdn_naive(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, f32,
                                   as_stream(stream)));
}
}  // namespace

extern "C" int tsa_gdn_recurrent_fwd(const void* q, const void* k, const void* v,
                                     const float* g_log, const float* beta, float* state,
                                     void* out, int B, int T, int Hq, int Hv, int dk, int dv,
                                     float scale, void* stream) {
    return recurrent(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, false, stream);
}

extern "C" int tsa_gdn_recurrent_fwd_f32(const float* q, const float* k, const float* v,
                                         const float* g_log, const float* beta, float* state,
                                         float* out, int B, int T, int Hq, int Hv, int dk, int dv,
                                         float scale, void* stream) {
    return recurrent(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, true, stream);
}

extern "C" int tsa_gdn_decode_step(const void* q, const void* k, const void* v,
                                   const float* g_log, const float* beta, float* state, void* out,
                                   int B, int Hq, int Hv, int dk, int dv, float scale,
                                   void* stream) {
    return recurrent(q, k, v, g_log, beta, state, out, B, 1, Hq, Hv, dk, dv, scale, false, stream);
}

extern "C" int tsa_gdn_decode_step_f32(const float* q, const float* k, const float* v,
                                       const float* g_log, const float* beta, float* state,
                                       float* out, int B, int Hq, int Hv, int dk, int dv, float scale,
                                       void* stream) {
    return recurrent(q, k, v, g_log, beta, state, out, B, 1, Hq, Hv, dk, dv, scale, true, stream);
}

extern "C" int tsa_gdn_naive(const void* q, const void* k, const void* v, const float* g_log,
                             const float* beta, float* state, void* out, int B, int T, int Hq,
                             int Hv, int dk, int dv, float scale, void* stream) {
    return naive(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, false, stream);
}

extern "C" int tsa_gdn_naive_f32(const float* q, const float* k, const float* v, const float* g_log,
                                 const float* beta, float* state, float* out, int B, int T, int Hq,
                                 int Hv, int dk, int dv, float scale, void* stream) {
    return naive(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, true, stream);
}

extern "C" int tsa_gdn_chunked_fused_fwd(const void* q, const void* k, const void* v, const float* a,
                                         const float* b, const float* dt_bias, const float* A,
                                         float* state, void* out, int B, int T, int Hq, int Hv,
                                         int dk, int dv, int chunk, float scale, float eps, void* ws,
                                         size_t ws_bytes, void* stream) {
    int rc = check_gdn(q, k, v, a, b, state, out, B, T, Hq, Hv, dk, dv, scale);
    if (rc) return rc;
    rc = check_gates(a, b, dt_bias, A, eps);
    if (rc) return rc;
    if (chunk < 1) return TSA_ERR_SHAPE;
    if (dk != 128 || dv != 128 || chunk != 64) return TSA_ERR_UNSUPPORTED;
    const long long nch = (T + 63LL) / 64;
    if (!fits_int(B, Hv, nch) || !fits_int(B, Hv, 8)) return TSA_ERR_SHAPE;
    const size_t need = tsa::gdn_chunked_ws_bytes(B, T, Hv, false);
    if (!ws || ws_bytes < need) return TSA_ERR_WORKSPACE;
    return from_hip(tsa::gdn_chunked_fused(q, k, v, tsa::GdnRawGates{a, b, dt_bias, A, eps}, state,
                                           out, B, T, Hq, Hv, scale, ws, as_stream(stream)));
}

extern "C" int tsa_gdn_decode_fused_step(const void* q, const void* k, const void* v, const float* a,
                                         const float* b, const float* dt_bias, const float* A,
                                         float* state, void* out, int B, int Hq, int Hv, int dk,
                                         int dv, float scale, float eps, void* stream) {
    int rc = check_gdn(q, k, v, a, b, state, out, B, 1, Hq, Hv, dk, dv, scale);
    if (rc) return rc;
    rc = check_gates(a, b, dt_bias, A, eps);
    if (rc) return rc;
    if (dk != 128 || dv != 128) return TSA_ERR_UNSUPPORTED;
    if (!fits_int(B, Hv, 8)) return TSA_ERR_SHAPE;
    return from_hip(tsa::gdn_decode_fused(q, k, v, tsa::GdnRawGates{a, b, dt_bias, A, eps}, state,
                                          out, B, Hq, Hv, scale, as_stream(stream)));
}

extern "C" int tsa_gdn_preprocess(const void* q, const void* k, const float* a, const float* b,
                                  const float* dt_bias, const float* A, void* q_out, void* k_out,
                                  float* g_log, float* beta, int B, int T, int Hq, int Hv, int dk,
                                  float eps, void* stream) {
    if (!q || !k || !q_out || !k_out || !g_log || !beta) return TSA_ERR_NULL;
    int rc = check_gates(a, b, dt_bias, A, eps);
    if (rc) return rc;
    if (B < 1 || T < 1 || Hq < 1 || Hv < 1 || dk < 1) return TSA_ERR_SHAPE;
    if (dk != 128) return TSA_ERR_UNSUPPORTED;
    // workgroups: 2 * B*T*Hq / 16 rows and B*T*Hv / 256 gates
    if (!fits_int(B, T, Hq) || !fits_int(B, T, Hv)) return TSA_ERR_SHAPE;
    return from_hip(tsa::gdn_preprocess(q, k, a, b, dt_bias, A, q_out, k_out, g_log, beta, B, T, Hq,
                                        Hv, eps, as_stream(stream)));
}

extern "C" int tsa_gdn_gated_rmsnorm(const void* x, const void* z, const float* w, void* y, int B,
                                     int T, int Hv, int dv, float eps, void* stream) {
    if (!x || !z || !w || !y) return TSA_ERR_NULL;
    if (B < 1 || T < 1 || Hv < 1 || dv < 1) return TSA_ERR_SHAPE;
    if (dv != 128) return TSA_ERR_UNSUPPORTED;
    if (!(eps > 0.f) || !std::isfinite(eps)) return TSA_ERR_ARG;
    if (!fits_int(B, T, Hv)) return TSA_ERR_SHAPE;
    return from_hip(tsa::gdn_gated_rmsnorm(x, z, w, y, B, T, Hv, eps, as_stream(stream)));
}
