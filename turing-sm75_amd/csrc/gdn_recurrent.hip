// gdn_recurrent.hip -- token-serial Gated DeltaNet (decode step = T of 1) for gfx950.
//
// Per token and V-head (src/gdn_sm75.cu:6-11):
//   g = exp(g_log);  kv = S^T k;  d = (v - g*kv)*beta;  S = g*S + k (x) d;
//   out = scale * S^T q.
// With S' = g*S + k (x) d the output is scale*(g*(S^T q) + d*(k.q)), so both dot products
// come from the state as it is loaded and the state makes exactly one trip through the
// registers per launch: read once, written once.  That round trip is the whole HBM cost
// of a decode step, so the layout is chosen for it:
//   * state column c (128 fp32 = 512 B, contiguous) is owned by an aligned group of 8
//     lanes; lane j holds float4 chunks j, j+8, j+16, j+24 -- every load/store
//     instruction of a wave covers 8 whole 128-B lines;
//   * the two per-column reductions are 3 DPP steps inside the 8-lane group (no LDS);
//   * the state is read and written with nontemporal loads/stores: it is touched once
//     per launch, and keeping it out of the caches measured 4.6 -> 5.6 TB/s for the
//     in-place read-modify-write stream of a 16 x 32 head decode step;
//   * T > 1: a 256-thread workgroup owns 32 columns of one (b, h) for all T tokens;
//     decode (T = 1): a one-wave workgroup owns 8 columns, so a decode step of 16 x 32
//     heads is 8192 independent workgroups.
// The reference's token-serial family (serial/smem/occ/occ2/occ4/occ4p/occ8,
// src/gdn_sm75.cu:57-188,577-893) differs only in how many columns a warp owns; here the
// state stays fp32 (gdn_smem_kernel's fp16 state is not reproduced).
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kD = 128;          // dk = dv
constexpr int kThreads = 256;
constexpr int kColsPerBlock = kThreads / 8;  // 32
constexpr int kBlocksPerHead = kD / kColsPerBlock;
constexpr int kDecodeCols = 8;  // decode: columns per workgroup
constexpr int kDecodeLpc = 8;   // decode: lanes per column

// q / k / v / out are fp16 (TIO = half_t, the library's I/O type) or fp32 (TIO = float, the
// reference's own, src/gdn_sm75.cu:57-64): 4 consecutive elements as fp32 either way.
__device__ __forceinline__ float4_t load4(const half_t* p) {
    const half4_t h = *reinterpret_cast<const half4_t*>(p);
    return float4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}
__device__ __forceinline__ float4_t load4(const float* p) { return *reinterpret_cast<const float4_t*>(p); }

template <typename TIO>
__device__ __forceinline__ void load_row16(const TIO* __restrict__ p, int j, float (&x)[16]) {
    // rows 4*(it*8 + j) .. +3 for it = 0..3
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const float4_t h = load4(p + 4 * (it * 8 + j));
        x[4 * it + 0] = h[0];
        x[4 * it + 1] = h[1];
        x[4 * it + 2] = h[2];
        x[4 * it + 3] = h[3];
    }
}

template <typename TIO>
__global__ void __launch_bounds__(kThreads)
gdn_recurrent_kernel(const TIO* __restrict__ q, const TIO* __restrict__ k,
                     const TIO* __restrict__ v, const float* __restrict__ g_log,
                     const float* __restrict__ beta, float* __restrict__ state,
                     TIO* __restrict__ out, int T, int Hq, int Hv, float scale) {
    const int bh = blockIdx.x / kBlocksPerHead;
    const int cb = blockIdx.x % kBlocksPerHead;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const int tid = threadIdx.x;
    const int col = cb * kColsPerBlock + (tid >> 3);
    const int j = tid & 7;

    float4_t* Sc = reinterpret_cast<float4_t*>(state + ((size_t)bh * kD + col) * kD);
    float4_t s[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) s[it] = __builtin_nontemporal_load(Sc + it * 8 + j);

    for (int t = 0; t < T; ++t) {
        const size_t bt = (size_t)b * T + t;
        float kr[16], qr[16];
        load_row16(k + (bt * Hq + hq) * kD, j, kr);
        load_row16(q + (bt * Hq + hq) * kD, j, qr);
        const float gl = g_log[bt * Hv + h];
        const float be = beta[bt * Hv + h];
        const float vc = (float)v[(bt * Hv + h) * kD + col];
        float kv = 0.f, sq = 0.f, kq = 0.f;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            kv = fmaf(s[it][0], kr[4 * it + 0], kv);
            kv = fmaf(s[it][1], kr[4 * it + 1], kv);
            kv = fmaf(s[it][2], kr[4 * it + 2], kv);
            kv = fmaf(s[it][3], kr[4 * it + 3], kv);
            sq = fmaf(s[it][0], qr[4 * it + 0], sq);
            sq = fmaf(s[it][1], qr[4 * it + 1], sq);
            sq = fmaf(s[it][2], qr[4 * it + 2], sq);
            sq = fmaf(s[it][3], qr[4 * it + 3], sq);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) kq = fmaf(kr[i], qr[i], kq);
        kv = sum8(kv);
        sq = sum8(sq);
        kq = sum8(kq);
        const float g = __expf(gl);
        const float d = (vc - g * kv) * be;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            s[it][0] = fmaf(g, s[it][0], kr[4 * it + 0] * d);
            s[it][1] = fmaf(g, s[it][1], kr[4 * it + 1] * d);
            s[it][2] = fmaf(g, s[it][2], kr[4 * it + 2] * d);
            s[it][3] = fmaf(g, s[it][3], kr[4 * it + 3] * d);
        }
        if (j == 0) out[(bt * Hv + h) * kD + col] = (TIO)(scale * fmaf(g, sq, d * kq));
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) __builtin_nontemporal_store(s[it], Sc + it * 8 + j);
}

// Sum over each aligned group of kLpc lanes (4, 8 or 16); every lane of the group receives it.
template <int kLpc>
__device__ __forceinline__ float sum_lanes(float x) {
    x += dpp_mov<kDppXor1>(x);
    x += dpp_mov<kDppXor2>(x);
    if (kLpc >= 8) x += dpp_mov<kDppHalfMirror>(x);
    if (kLpc >= 16) x += dpp_mov<kDppRowMirror>(x);
    return x;
}

// Decode step (T = 1): one workgroup of kLpc * kCols threads per kCols columns of a head;
// each column is owned by an aligned group of kLpc lanes, lane j holding float4 chunks
// j, j + kLpc, ... of it.  The q and k rows (512 bytes shared by every column) come in
// through LDS: wave 0 loads them with one 8-byte load per lane instead of every thread
// issuing its own.  Measured over 16 x 32 heads with 16 state replicas cycled (µs per step):
// 8 columns x 8 lanes (one wave, 8192 workgroups) 12.2, 16 x 8 12.6, 32 x 8 12.5, 8 x 16
// 12.7, 4 x 16 12.9, 16 x 4 13.6; plain instead of nontemporal state loads / stores 15.0;
// walking several column blocks per workgroup with the next block prefetched gained
// nothing.  kFused: q / k are raw rows, normalised here (their norms come from the same
// lane-group sums as the dot products), and g_log / beta come from the raw projections
// a / b (gate arguments).
template <int kCols, int kLpc, bool kFused, typename TIO>
__global__ void __launch_bounds__(kLpc * kCols)
gdn_decode_kernel(const TIO* __restrict__ q, const TIO* __restrict__ k,
                  const TIO* __restrict__ v, const float* __restrict__ g_log,
                  const float* __restrict__ beta, GdnRawGates gates, float* __restrict__ state,
                  TIO* __restrict__ out, int Hq, int Hv, float scale) {
    static_assert(kLpc * kCols >= 64, "wave 0 loads the q / k rows");
    constexpr int kWgPerHead = kD / kCols;
    constexpr int kR = 32 / kLpc;  // float4 chunks of the column per lane
    const int bh = blockIdx.x / kWgPerHead;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const int tid = threadIdx.x, j = tid % kLpc;
    const int col = (blockIdx.x % kWgPerHead) * kCols + tid / kLpc;
    const size_t bt = (size_t)b;  // token index of sequence b (T = 1)
    const size_t vrow = (bt * Hv + h) * kD;

    typedef typename std::conditional<std::is_same<TIO, float>::value, float4_t, half4_t>::type row4_t;
    __shared__ row4_t kq_rows[2][kD / 4];
    float4_t* Sc = reinterpret_cast<float4_t*>(state + ((size_t)bh * kD + col) * kD);
    float4_t s[kR];
#pragma unroll
    for (int it = 0; it < kR; ++it)
        s[it] = __builtin_nontemporal_load(Sc + it * kLpc + j);
    // Wait for the state before issuing the q / k / v loads.  Measured over 16 x 32 heads with
    // 16 replicas cycled: 11.3 vs 12.2 us per step with the small loads issued under the
    // state loads (and 9.4 vs 10.4 us on a cache-resident state).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt left at their maxima
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 64) {  // wave 0 -- lanes 0-31: k row, 32-63: q row, 4 elements each
        const TIO* row = (tid < 32 ? k : q) + (bt * Hq + hq) * kD;
        kq_rows[tid >> 5][tid & 31] = *reinterpret_cast<const row4_t*>(row + 4 * (tid & 31));
    }
    const float vc = (float)v[vrow + col];
    float g, be;
    if (kFused) {
        g = __expf(gdn_softplus(gates.a[bt * Hv + h] + gates.dt_bias[h]) * gates.A[h]);
        be = gdn_sigmoid(gates.b[bt * Hv + h]);
    } else {
        g = __expf(g_log[bt * Hv + h]);
        be = beta[bt * Hv + h];
    }
    __syncthreads();
    float kr[4 * kR], qr[4 * kR];
#pragma unroll
    for (int it = 0; it < kR; ++it) {
        const row4_t hk = kq_rows[0][it * kLpc + j], hq4 = kq_rows[1][it * kLpc + j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kr[4 * it + e] = (float)hk[e];
            qr[4 * it + e] = (float)hq4[e];
        }
    }
    float kv = 0.f, sq = 0.f, kq = 0.f;
#pragma unroll
    for (int it = 0; it < kR; ++it)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kv = fmaf(s[it][e], kr[4 * it + e], kv);
            sq = fmaf(s[it][e], qr[4 * it + e], sq);
        }
#pragma unroll
    for (int i = 0; i < 4 * kR; ++i) kq = fmaf(kr[i], qr[i], kq);
    kv = sum_lanes<kLpc>(kv);
    sq = sum_lanes<kLpc>(sq);
    kq = sum_lanes<kLpc>(kq);
    if (kFused) {  // k -> k / max(||k||, eps), q likewise: scale the sums and k itself
        float kk = 0.f, qq = 0.f;
#pragma unroll
        for (int i = 0; i < 4 * kR; ++i) {
            kk = fmaf(kr[i], kr[i], kk);
            qq = fmaf(qr[i], qr[i], qq);
        }
        const float kn = 1.f / fmaxf(sqrtf(sum_lanes<kLpc>(kk)), gates.eps);
        const float qn = 1.f / fmaxf(sqrtf(sum_lanes<kLpc>(qq)), gates.eps);
        kv *= kn;
        sq *= qn;
        kq *= kn * qn;
#pragma unroll
        for (int i = 0; i < 4 * kR; ++i) kr[i] *= kn;
    }
    const float d = (vc - g * kv) * be;
#pragma unroll
    for (int it = 0; it < kR; ++it) {
        float4_t x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = fmaf(g, s[it][e], kr[4 * it + e] * d);
        __builtin_nontemporal_store(x, Sc + it * kLpc + j);
    }
    if (j == 0) out[vrow + col] = (TIO)(scale * fmaf(g, sq, d * kq));
}

// Naive check kernel: one thread per state column, gdn_cpu order (src/gdn_sm75.cu:1090-1102).
template <typename TIO>
__global__ void __launch_bounds__(128)
gdn_naive_kernel(const TIO* __restrict__ q, const TIO* __restrict__ k,
                 const TIO* __restrict__ v, const float* __restrict__ g_log,
                 const float* __restrict__ beta, float* __restrict__ state,
                 TIO* __restrict__ out, int B, int T, int Hq, int Hv, int dk, int dv,
                 float scale) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)B * Hv * dv) return;
    const int c = (int)(idx % dv);
    const long long bh = idx / dv;
    const int b = (int)(bh / Hv), h = (int)(bh % Hv), hq = h % Hq;
    float* Sc = state + ((size_t)bh * dv + c) * dk;
    for (int t = 0; t < T; ++t) {
        const size_t bt = (size_t)b * T + t;
        const TIO* qt = q + (bt * Hq + hq) * dk;
        const TIO* kt = k + (bt * Hq + hq) * dk;
        const float g = expf(g_log[bt * Hv + h]);
        const float be = beta[bt * Hv + h];
        float kv = 0.f;
        for (int i = 0; i < dk; ++i) kv += Sc[i] * (float)kt[i];
        const float d = ((float)v[(bt * Hv + h) * dv + c] - g * kv) * be;
        float attn = 0.f;
        for (int i = 0; i < dk; ++i) {
            const float sn = g * Sc[i] + (float)kt[i] * d;
            Sc[i] = sn;
            attn += sn * (float)qt[i];
        }
        out[(bt * Hv + h) * dv + c] = (TIO)(attn * scale);
    }
}

template <typename TIO>
hipError_t launch_recurrent(const void* q, const void* k, const void* v, const float* g_log,
                            const float* beta, float* state, void* out, int B, int T, int Hq,
                            int Hv, float scale, hipStream_t stream) {
    auto Q = static_cast<const TIO*>(q);
    auto K = static_cast<const TIO*>(k);
    auto V = static_cast<const TIO*>(v);
    auto O = static_cast<TIO*>(out);
    if (T == 1) {
        const unsigned blocks = (unsigned)(B * Hv * (kD / kDecodeCols));
        hipLaunchKernelGGL((gdn_decode_kernel<kDecodeCols, kDecodeLpc, false, TIO>), dim3(blocks),
                           dim3(kDecodeLpc * kDecodeCols), 0, stream, Q, K, V, g_log, beta,
                           GdnRawGates{}, state, O, Hq, Hv, scale);
        return hipGetLastError();
    }
    const unsigned blocks = (unsigned)(B * Hv * kBlocksPerHead);
    hipLaunchKernelGGL(gdn_recurrent_kernel<TIO>, dim3(blocks), dim3(kThreads), 0, stream, Q, K, V,
                       g_log, beta, state, O, T, Hq, Hv, scale);
    return hipGetLastError();
}

template <typename TIO>
hipError_t launch_naive(const void* q, const void* k, const void* v, const float* g_log,
                        const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                        int dk, int dv, float scale, hipStream_t stream) {
    const long long cols = (long long)B * Hv * dv;
    const unsigned blocks = (unsigned)((cols + 127) / 128);
    hipLaunchKernelGGL(gdn_naive_kernel<TIO>, dim3(blocks), dim3(128), 0, stream,
                       static_cast<const TIO*>(q), static_cast<const TIO*>(k),
                       static_cast<const TIO*>(v), g_log, beta, state, static_cast<TIO*>(out), B, T,
                       Hq, Hv, dk, dv, scale);
    return hipGetLastError();
}

}  // namespace

hipError_t gdn_recurrent(const void* q, const void* k, const void* v, const float* g_log,
                         const float* beta, float* state, void* out, int B, int T, int Hq,
                         int Hv, float scale, bool f32, hipStream_t stream) {
    return f32 ? launch_recurrent<float>(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, scale, stream)
               : launch_recurrent<half_t>(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, scale, stream);
}

hipError_t gdn_decode_fused(const void* q, const void* k, const void* v, const GdnRawGates& gates,
                            float* state, void* out, int B, int Hq, int Hv, float scale,
                            hipStream_t stream) {
    const unsigned blocks = (unsigned)(B * Hv * (kD / kDecodeCols));
    hipLaunchKernelGGL((gdn_decode_kernel<kDecodeCols, kDecodeLpc, true, half_t>), dim3(blocks),
                       dim3(kDecodeLpc * kDecodeCols), 0, stream, static_cast<const half_t*>(q),
                       static_cast<const half_t*>(k), static_cast<const half_t*>(v), nullptr, nullptr,
                       gates, state, static_cast<half_t*>(out), Hq, Hv, scale);
    return hipGetLastError();
}

hipError_t gdn_naive(const void* q, const void* k, const void* v, const float* g_log,
                     const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                     int dk, int dv, float scale, bool f32, hipStream_t stream) {
    return f32 ? launch_naive<float>(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, stream)
               : launch_naive<half_t>(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, scale, stream);
}

}  // namespace tsa
