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
//   * a 256-thread workgroup owns 32 columns of one (b, h); the 4 workgroups of a head
//     and the B*Hv heads are independent, so a decode step of 16 x 32 heads is 2048
//     workgroups.
// The reference's token-serial family (serial/smem/occ/occ2/occ4/occ4p/occ8,
// src/gdn_sm75.cu:57-188,577-893) differs only in how many columns a warp owns; here the
// state stays fp32 (gdn_smem_kernel's fp16 state is not reproduced).
#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kD = 128;          // dk = dv
constexpr int kThreads = 256;
constexpr int kColsPerBlock = kThreads / 8;  // 32
constexpr int kBlocksPerHead = kD / kColsPerBlock;

__device__ __forceinline__ void load_row16(const half_t* __restrict__ p, int j, float (&x)[16]) {
    // rows 4*(it*8 + j) .. +3 for it = 0..3
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const half4_t h = *reinterpret_cast<const half4_t*>(p + 4 * (it * 8 + j));
        x[4 * it + 0] = (float)h[0];
        x[4 * it + 1] = (float)h[1];
        x[4 * it + 2] = (float)h[2];
        x[4 * it + 3] = (float)h[3];
    }
}

__global__ void __launch_bounds__(kThreads)
gdn_recurrent_kernel(const half_t* __restrict__ q, const half_t* __restrict__ k,
                     const half_t* __restrict__ v, const float* __restrict__ g_log,
                     const float* __restrict__ beta, float* __restrict__ state,
                     half_t* __restrict__ out, int T, int Hq, int Hv, float scale) {
    const int bh = blockIdx.x / kBlocksPerHead;
    const int cb = blockIdx.x % kBlocksPerHead;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const int tid = threadIdx.x;
    const int col = cb * kColsPerBlock + (tid >> 3);
    const int j = tid & 7;

    float4* Sc = reinterpret_cast<float4*>(state + ((size_t)bh * kD + col) * kD);
    float4 s[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) s[it] = Sc[it * 8 + j];

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
            kv = fmaf(s[it].x, kr[4 * it + 0], kv);
            kv = fmaf(s[it].y, kr[4 * it + 1], kv);
            kv = fmaf(s[it].z, kr[4 * it + 2], kv);
            kv = fmaf(s[it].w, kr[4 * it + 3], kv);
            sq = fmaf(s[it].x, qr[4 * it + 0], sq);
            sq = fmaf(s[it].y, qr[4 * it + 1], sq);
            sq = fmaf(s[it].z, qr[4 * it + 2], sq);
            sq = fmaf(s[it].w, qr[4 * it + 3], sq);
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
            s[it].x = fmaf(g, s[it].x, kr[4 * it + 0] * d);
            s[it].y = fmaf(g, s[it].y, kr[4 * it + 1] * d);
            s[it].z = fmaf(g, s[it].z, kr[4 * it + 2] * d);
            s[it].w = fmaf(g, s[it].w, kr[4 * it + 3] * d);
        }
        if (j == 0) out[(bt * Hv + h) * kD + col] = (half_t)(scale * fmaf(g, sq, d * kq));
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) Sc[it * 8 + j] = s[it];
}

// Naive check kernel: one thread per state column, gdn_cpu order (src/gdn_sm75.cu:1090-1102).
__global__ void __launch_bounds__(128)
gdn_naive_kernel(const half_t* __restrict__ q, const half_t* __restrict__ k,
                 const half_t* __restrict__ v, const float* __restrict__ g_log,
                 const float* __restrict__ beta, float* __restrict__ state,
                 half_t* __restrict__ out, int B, int T, int Hq, int Hv, int dk, int dv,
                 float scale) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)B * Hv * dv) return;
    const int c = (int)(idx % dv);
    const long long bh = idx / dv;
    const int b = (int)(bh / Hv), h = (int)(bh % Hv), hq = h % Hq;
    float* Sc = state + ((size_t)bh * dv + c) * dk;
    for (int t = 0; t < T; ++t) {
        const size_t bt = (size_t)b * T + t;
        const half_t* qt = q + (bt * Hq + hq) * dk;
        const half_t* kt = k + (bt * Hq + hq) * dk;
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
        out[(bt * Hv + h) * dv + c] = (half_t)(attn * scale);
    }
}

}  // namespace

hipError_t gdn_recurrent(const void* q, const void* k, const void* v, const float* g_log,
                         const float* beta, float* state, void* out, int B, int T, int Hq,
                         int Hv, float scale, hipStream_t stream) {
    const unsigned blocks = (unsigned)(B * Hv * kBlocksPerHead);
    hipLaunchKernelGGL(gdn_recurrent_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                       static_cast<const half_t*>(q), static_cast<const half_t*>(k),
                       static_cast<const half_t*>(v), g_log, beta, state,
                       static_cast<half_t*>(out), T, Hq, Hv, scale);
    return hipGetLastError();
}

hipError_t gdn_naive(const void* q, const void* k, const void* v, const float* g_log,
                     const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                     int dk, int dv, float scale, hipStream_t stream) {
    const long long cols = (long long)B * Hv * dv;
    const unsigned blocks = (unsigned)((cols + 127) / 128);
    hipLaunchKernelGGL(gdn_naive_kernel, dim3(blocks), dim3(128), 0, stream,
                       static_cast<const half_t*>(q), static_cast<const half_t*>(k),
                       static_cast<const half_t*>(v), g_log, beta, state,
                       static_cast<half_t*>(out), B, T, Hq, Hv, dk, dv, scale);
    return hipGetLastError();
}

}  // namespace tsa
