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

size_t gdn_chunked_ws_bytes(int B, int T, int Hv);
hipError_t gdn_chunked(const void* q, const void* k, const void* v, const float* g_log,
                       const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                       float scale, void* ws, hipStream_t stream);
hipError_t gdn_recurrent(const void* q, const void* k, const void* v, const float* g_log,
                         const float* beta, float* state, void* out, int B, int T, int Hq,
                         int Hv, float scale, hipStream_t stream);
hipError_t gdn_naive(const void* q, const void* k, const void* v, const float* g_log,
                     const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                     int dk, int dv, float scale, hipStream_t stream);

}  // namespace tsa
