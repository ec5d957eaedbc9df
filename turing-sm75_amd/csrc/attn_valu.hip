// attn_valu.hip -- the VALU flash-attention forward for gfx950: the same recurrence as
// attn_fwd_kernel with no matrix cores, kept as its same-binary opponent, as
// flash_attn_sm75_ffma (src/attn_sm75.cu:107-233) is the CUDA-core opponent of the WMMA
// kernel in the reference's lab.
//
// Layout for wave64 VALU work rather than a 16x16 thread tile:
//   * a workgroup is 4 waves and owns 64 query rows; row r belongs to 4 consecutive lanes,
//     each holding a D/4 slice of q and of the O accumulator in fp32 registers;
//   * K and V tiles of 64 keys are staged in LDS (fp16); every lane of a wave that reads a
//     key reads one of only 4 slice addresses, so the reads are broadcasts;
//   * a score is an fp32 FMA dot over the lane's slice plus a 4-lane DPP sum; the tile's 64
//     scores stay in registers, the online softmax runs in the exp2 domain, and O += P V
//     reads the V rows back from LDS slice by slice;
//   * causal: tiles past the workgroup's last row are skipped, the longest query tiles are
//     issued first.
#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kVThreads = 256;
constexpr int kVRows = 64;  // query rows per workgroup (4 lanes per row)
constexpr int kVKeys = 64;  // keys per LDS tile

// Sum over each aligned group of 4 lanes; every lane of the group receives the total.
__device__ __forceinline__ float sum4(float x) {
    x += dpp_mov<kDppXor1>(x);
    x += dpp_mov<kDppXor2>(x);
    return x;
}

template <int D, bool kCausal>
__global__ void __launch_bounds__(kVThreads)
attn_valu_kernel(const half_t* __restrict__ Q, const half_t* __restrict__ K,
                 const half_t* __restrict__ V, half_t* __restrict__ O, int S, int n_qt,
                 float c2 /* scale * log2(e) */) {
    constexpr int kSl = D / 4;  // dims per lane
    __shared__ __align__(16) half_t Ks[kVKeys * D];
    __shared__ __align__(16) half_t Vs[kVKeys * D];

    const int tid = threadIdx.x, sl = tid & 3;
    const int bh = blockIdx.x / n_qt;
    const int rank = blockIdx.x % n_qt;
    const int qt = kCausal ? n_qt - 1 - rank : rank;
    const int q0 = qt * kVRows;
    const int my_q = q0 + (tid >> 2);
    const size_t head = (size_t)bh * S * D;

    float qv[kSl], o[kSl];
#pragma unroll
    for (int i = 0; i < kSl; i += 8) {
        half8_t h8 = {};
        if (my_q < S) h8 = *reinterpret_cast<const half8_t*>(Q + head + (size_t)my_q * D + sl * kSl + i);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qv[i + e] = (float)h8[e];
            o[i + e] = 0.f;
        }
    }
    float m = -INFINITY;  // running max of the raw scores q . k
    float l = 0.f;        // running sum of exp2((s - m) c2)

    const int kv_end = kCausal ? min(S, q0 + kVRows) : S;
    for (int k0 = 0; k0 < kv_end; k0 += kVKeys) {
        __syncthreads();  // every wave is done with the previous tile
        constexpr int kChunks = kVKeys * D / 8;  // 16-byte pieces per tile
#pragma unroll
        for (int e = tid; e < kChunks; e += kVThreads) {
            const int row = e / (D / 8), c = e % (D / 8);
            const int key = k0 + row;
            uint4 kx = make_uint4(0, 0, 0, 0), vx = kx;
            if (key < S) {
                kx = *reinterpret_cast<const uint4*>(K + head + (size_t)key * D + c * 8);
                vx = *reinterpret_cast<const uint4*>(V + head + (size_t)key * D + c * 8);
            }
            *reinterpret_cast<uint4*>(Ks + row * D + c * 8) = kx;
            *reinterpret_cast<uint4*>(Vs + row * D + c * 8) = vx;
        }
        __syncthreads();

        // scores of this row against the tile's keys
        float s[kVKeys];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < kVKeys; ++j) {
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < kSl; i += 8) {
                const half8_t k8 = *reinterpret_cast<const half8_t*>(Ks + j * D + sl * kSl + i);
#pragma unroll
                for (int e = 0; e < 8; ++e) dot = fmaf(qv[i + e], (float)k8[e], dot);
            }
            dot = sum4(dot);
            const int key = k0 + j;
            s[j] = (key >= S || (kCausal && key > my_q)) ? -INFINITY : dot;
            mx = fmaxf(mx, s[j]);
        }
        // online softmax: rescale O and l to the new max (rows with nothing unmasked yet keep
        // m = -inf and contribute nothing)
        const float m_new = fmaxf(m, mx);
        if (m_new != -INFINITY) {
            const float alpha = fast_exp2((m - m_new) * c2);  // 0 on the first unmasked tile
            m = m_new;
            l *= alpha;
#pragma unroll
            for (int i = 0; i < kSl; ++i) o[i] *= alpha;
            const float mc = m * c2;
#pragma unroll
            for (int j = 0; j < kVKeys; ++j) {
                const float p = fast_exp2(fmaf(s[j], c2, -mc));
                l += p;
#pragma unroll
                for (int i = 0; i < kSl; i += 8) {
                    const half8_t v8 = *reinterpret_cast<const half8_t*>(Vs + j * D + sl * kSl + i);
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[i + e] = fmaf(p, (float)v8[e], o[i + e]);
                }
            }
        }
    }

    if (my_q < S) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        half_t* orow = O + head + (size_t)my_q * D + sl * kSl;
#pragma unroll
        for (int i = 0; i < kSl; i += 8) {
            half8_t h8;
#pragma unroll
            for (int e = 0; e < 8; ++e) h8[e] = (half_t)(o[i + e] * inv);
            *reinterpret_cast<half8_t*>(orow + i) = h8;
        }
    }
}

template <int D, bool kCausal>
hipError_t launch_valu(const half_t* q, const half_t* k, const half_t* v, half_t* o, int BH, int S,
                       float scale, hipStream_t stream) {
    const int n_qt = (S + kVRows - 1) / kVRows;
    hipLaunchKernelGGL((attn_valu_kernel<D, kCausal>), dim3(BH * n_qt), dim3(kVThreads), 0, stream, q, k,
                       v, o, S, n_qt, scale * kLog2e);
    return hipGetLastError();
}

}  // namespace

hipError_t attn_valu(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                     int D, float scale, int causal, hipStream_t stream) {
    auto Q = static_cast<const half_t*>(q);
    auto Kp = static_cast<const half_t*>(k);
    auto Vp = static_cast<const half_t*>(v);
    auto Op = static_cast<half_t*>(o);
    const int BH = B * H;
    if (D == 256)
        return causal ? launch_valu<256, true>(Q, Kp, Vp, Op, BH, S, scale, stream)
                      : launch_valu<256, false>(Q, Kp, Vp, Op, BH, S, scale, stream);
    if (D == 128)
        return causal ? launch_valu<128, true>(Q, Kp, Vp, Op, BH, S, scale, stream)
                      : launch_valu<128, false>(Q, Kp, Vp, Op, BH, S, scale, stream);
    return causal ? launch_valu<64, true>(Q, Kp, Vp, Op, BH, S, scale, stream)
                  : launch_valu<64, false>(Q, Kp, Vp, Op, BH, S, scale, stream);
}

}  // namespace tsa
