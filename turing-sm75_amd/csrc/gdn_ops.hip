// gdn_ops.hip -- the element-wise operations on either side of the Gated DeltaNet recurrence
// in the target model's layer (docs/qwen38-27b.md:15; the recurrence's semantic source is
// llama.cpp's gated_delta_net, src/gdn_sm75.cu:3):
//   pre:  q, k <- x / max(||x||_2, eps) per head row;  beta = sigmoid(b);
//         g_log = softplus(a + dt_bias[h]) * A[h]   (A = -exp(A_log), per V-head)
//   post: y = x / sqrt(mean(x^2) + eps) * w * silu(z)   per (token, V-head) row
// All are HBM-bound streams of 256-byte rows: a row belongs to 16 lanes that each move 16
// bytes, so every instruction covers whole 128-byte lines, and the row sums are 4 DPP
// steps inside the 16-lane group.  The fused prefill / decode entry points apply the
// pre-ops inside the recurrence kernels instead (gdn_chunked.hip, gdn_recurrent.hip).
#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kD = 128;
constexpr int kRowsPerBlock = 16;  // 256 threads, 16 per row
// Rows per 16-lane group: every row's loads are issued before any is used (rows past the end
// clamped to the last row, their results not stored), so a thread keeps kGroupRows 16-byte
// loads per input in flight instead of one.
constexpr int kGroupRows = 4;

// Sum over each aligned group of 16 lanes by DPP (no LDS round trip): the 8-lane sums, then
// each lane adds the mirror lane of the other half of its row.
__device__ __forceinline__ float sum16_dpp(float x) {
    x = sum8(x);
    return x + dpp_mov<kDppRowMirror>(x);
}

// Rows [0, rows) of x0 and then rows [0, rows) of x1, normalised into y0 / y1.
__global__ void __launch_bounds__(256)
l2norm_rows_kernel(const half_t* x0, half_t* y0, const half_t* x1,  // y may alias x
                   half_t* y1, long long rows, float eps) {
    const long long r0 = (long long)blockIdx.x * (kRowsPerBlock * kGroupRows) + (threadIdx.x >> 4);
    const int c = threadIdx.x & 15;
    half8_t v[kGroupRows];
#pragma unroll
    for (int i = 0; i < kGroupRows; ++i) {
        const long long r = min(r0 + (long long)kRowsPerBlock * i, 2 * rows - 1);
        const bool second = r >= rows;
        v[i] = *reinterpret_cast<const half8_t*>((second ? x1 : x0) + (second ? r - rows : r) * kD + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < kGroupRows; ++i) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf((float)v[i][e], (float)v[i][e], ss);
        const float inv = 1.f / fmaxf(sqrtf(sum16_dpp(ss)), eps);
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (half_t)((float)v[i][e] * inv);
        const long long r = r0 + (long long)kRowsPerBlock * i;
        const bool second = r >= rows;
        if (r < 2 * rows)
            *reinterpret_cast<half8_t*>((second ? y1 : y0) + (second ? r - rows : r) * kD + 8 * c) = o;
    }
}

__global__ void __launch_bounds__(256)
gdn_gates_kernel(const float* __restrict__ a, const float* __restrict__ b,
                 const float* __restrict__ dt_bias, const float* __restrict__ A,
                 float* __restrict__ g_log, float* __restrict__ beta, long long n, int Hv) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int h = (int)(i % Hv);
    g_log[i] = gdn_softplus(a[i] + dt_bias[h]) * A[h];
    beta[i] = gdn_sigmoid(b[i]);
}

// silu(z) = z sigmoid(z) on the hardware exp2 and reciprocal (both ~1 ulp): for z below
// about -88 the exponential is +inf and the result the limit -0.
__device__ __forceinline__ float silu_fast(float z) {
    return z * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-z * kLog2e));
}


__global__ void __launch_bounds__(256)
gated_rmsnorm_kernel(const half_t* x, const half_t* __restrict__ z,
                     const float* __restrict__ w, half_t* y, long long rows, float eps) {  // y may alias x
    const long long r0 = (long long)blockIdx.x * (kRowsPerBlock * kGroupRows) + (threadIdx.x >> 4);
    const int c = threadIdx.x & 15;
    half8_t xv[kGroupRows], zv[kGroupRows];
#pragma unroll
    for (int i = 0; i < kGroupRows; ++i) {
        const long long r = min(r0 + (long long)kRowsPerBlock * i, rows - 1);
        xv[i] = *reinterpret_cast<const half8_t*>(x + r * kD + 8 * c);
        zv[i] = *reinterpret_cast<const half8_t*>(z + r * kD + 8 * c);
    }
    const float4 w0 = *reinterpret_cast<const float4*>(w + 8 * c);
    const float4 w1 = *reinterpret_cast<const float4*>(w + 8 * c + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < kGroupRows; ++i) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf((float)xv[i][e], (float)xv[i][e], ss);
        const float rs = 1.f / sqrtf(sum16_dpp(ss) * (1.f / kD) + eps);
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (half_t)((float)xv[i][e] * rs * wv[e] * silu_fast((float)zv[i][e]));
        const long long r = r0 + (long long)kRowsPerBlock * i;
        if (r < rows) *reinterpret_cast<half8_t*>(y + r * kD + 8 * c) = o;
    }
}

}  // namespace

hipError_t gdn_preprocess(const void* q, const void* k, const float* a, const float* b,
                          const float* dt_bias, const float* A, void* q_out, void* k_out,
                          float* g_log, float* beta, int B, int T, int Hq, int Hv, float eps,
                          hipStream_t stream) {
    const long long rows = (long long)B * T * Hq;
    const long long nb = (2 * rows + kRowsPerBlock * kGroupRows - 1) / (kRowsPerBlock * kGroupRows);
    hipLaunchKernelGGL(l2norm_rows_kernel, dim3((unsigned)nb), dim3(256), 0, stream,
                       static_cast<const half_t*>(q), static_cast<half_t*>(q_out),
                       static_cast<const half_t*>(k), static_cast<half_t*>(k_out), rows, eps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const long long n = (long long)B * T * Hv;
    hipLaunchKernelGGL(gdn_gates_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a,
                       b, dt_bias, A, g_log, beta, n, Hv);
    return hipGetLastError();
}

hipError_t gdn_gated_rmsnorm(const void* x, const void* z, const float* w, void* y, int B, int T,
                             int Hv, float eps, hipStream_t stream) {
    const long long rows = (long long)B * T * Hv;
    const long long nb = (rows + kRowsPerBlock * kGroupRows - 1) / (kRowsPerBlock * kGroupRows);
    hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3((unsigned)nb), dim3(256), 0, stream,
                       static_cast<const half_t*>(x), static_cast<const half_t*>(z), w,
                       static_cast<half_t*>(y), rows, eps);
    return hipGetLastError();
}

}  // namespace tsa
