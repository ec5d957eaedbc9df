// attn_fwd.hip -- softmax flash-attention forward for gfx950 (fp16 MFMA, fp32 softmax).
//
// Same recurrence as flash_attn_sm75_wmma (src/attn_sm75.cu:239-375): stream K/V tiles,
// keep running (m, l, O) per query row, O = O*alpha + P V, finally O / l.  The tiling is
// CDNA4-shaped instead of a 16x16 warp tile:
//   * a workgroup is 4 waves and owns 128 query rows (32 per wave); K/V tiles of 64 keys
//     are double-buffered in LDS (64 KiB at D = 128) so two workgroups share a CU;
//   * each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_f16 (A = K rows from LDS,
//     B = its 32 Q rows held in registers for the whole loop), so a lane owns one query
//     and 16 keys per 32-key block: the row max / row sum are register reductions plus
//     one exchange with lane l^32;
//   * P^T stays in registers (the S^T accumulator converted to fp16 is exactly the B
//     operand layout of the next MFMA) and O^T += V^T P^T reads V^T straight out of the
//     row-major V tile with ds_read_b64_tr_b16 -- no transpose pass;
//   * softmax in the exp2 domain with scale*log2(e) folded into one FMA per score;
//   * causal: tiles above a wave's diagonal are skipped, only diagonal / ragged tiles
//     are masked; heavy (late) query tiles are scheduled first, and all query tiles of
//     one (b, h) land on one XCD so its K/V stay in that XCD's L2.
#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kThreads = 256;
constexpr int kQRows = 128;  // query rows per workgroup
constexpr int kKRows = 64;   // keys per LDS tile

// 16-byte chunk swizzle of an LDS tile row: chunk c of row r lives at c ^ swz(r).
// swz is a permutation of r % 16, so 16 consecutive rows read at one chunk (the K
// operand reads) hit 16 different bank groups, and for every aligned group of 4 rows
// the values swz >> 1 differ, so the transposing V reads (4 rows x 2 chunks) do too.
__device__ __forceinline__ int swz(int r) {
    return 2 * (r & 3) + ((r >> 2) & 1) + 8 * ((r >> 3) & 1);
}

template <int D>
struct Cfg {
    static constexpr int kChunks = D / 8;                        // 16-B chunks per row
    static constexpr int kTile = kKRows * D;                     // halfs per K or V tile
    static constexpr int kLoads = kKRows * kChunks / kThreads;   // 16-B loads per thread
    static constexpr int kKSteps = D / 16;                       // k-steps of S^T = K Q^T
    static constexpr int kDBlocks = D / 32;                      // 32-row blocks of O^T
    static constexpr int kLdsBytes = 2 * 2 * kTile * 2;          // 2 buffers x (K, V)
    static_assert(kLoads * kThreads == kKRows * kChunks, "tile not covered");
};

template <int D>
__device__ __forceinline__ int chunk_pos(int r, int c) {
    return c ^ (swz(r) & (D / 8 - 1));
}

// Map the linear workgroup id to (bh, query tile).  Workgroups are dispatched round
// robin over the 8 XCDs; when BH is a multiple of 8, head bh runs on XCD bh % 8.  Causal
// runs issue the longest (highest) query tiles first.
__device__ __forceinline__ void map_block(int bid, int BH, int n_qt, bool causal, int& bh,
                                          int& qt) {
    int rank;
    if ((BH & 7) == 0) {
        const int xcd = bid & 7, slot = bid >> 3, hpx = BH >> 3;
        bh = (slot % hpx) * 8 + xcd;
        rank = slot / hpx;
    } else {
        bh = bid % BH;
        rank = bid / BH;
    }
    qt = causal ? (n_qt - 1 - rank) : rank;
}

template <int D>
__device__ __forceinline__ void load_tile(const half_t* __restrict__ src, int k0, int S,
                                          uint4 (&reg)[Cfg<D>::kLoads]) {
    const int tid = threadIdx.x;
    const bool full = k0 + kKRows <= S;
#pragma unroll
    for (int it = 0; it < Cfg<D>::kLoads; ++it) {
        const int id = it * kThreads + tid;
        const int row = id / Cfg<D>::kChunks, c = id % Cfg<D>::kChunks;
        if (full || k0 + row < S)
            reg[it] = *reinterpret_cast<const uint4*>(src + (size_t)(k0 + row) * D + c * 8);
        else
            reg[it] = make_uint4(0, 0, 0, 0);
    }
}

template <int D>
__device__ __forceinline__ void store_tile(half_t* dst, const uint4 (&reg)[Cfg<D>::kLoads]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < Cfg<D>::kLoads; ++it) {
        const int id = it * kThreads + tid;
        const int row = id / Cfg<D>::kChunks, c = id % Cfg<D>::kChunks;
        *reinterpret_cast<uint4*>(dst + row * D + chunk_pos<D>(row, c) * 8) = reg[it];
    }
}

template <int D, bool kCausal>
__global__ void __launch_bounds__(kThreads, 2)
attn_fwd_kernel(const half_t* __restrict__ Q, const half_t* __restrict__ K,
                const half_t* __restrict__ V, half_t* __restrict__ O, int S, int BH, int n_qt,
                float c2 /* scale * log2(e) */) {
    using C = Cfg<D>;
    extern __shared__ __align__(16) half_t lds[];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hi = lane >> 5;  // which half of the wave
    int bh, qt;
    map_block(blockIdx.x, BH, n_qt, kCausal, bh, qt);
    const size_t head = (size_t)bh * S * D;
    const int q0 = qt * kQRows;
    const int qw0 = q0 + 32 * wave;
    const int my_q = qw0 + (lane & 31);

    // This wave's 32 query rows as the B operand of S^T = K Q^T: slot s of k-step kk is
    // Q[my_q][16*kk + 8*hi + s].
    half8_t qf[C::kKSteps];
#pragma unroll
    for (int kk = 0; kk < C::kKSteps; ++kk) {
        if (my_q < S)
            qf[kk] = *reinterpret_cast<const half8_t*>(Q + head + (size_t)my_q * D + 16 * kk + 8 * hi);
        else
            qf[kk] = half8_t{};
    }

    const int kv_end = kCausal ? min(S, q0 + kQRows) : S;
    const int n_tiles = (kv_end + kKRows - 1) / kKRows;
    const int wave_kv_end = kCausal ? min(S, qw0 + 32) : S;

    float16_t o[C::kDBlocks];
#pragma unroll
    for (int i = 0; i < C::kDBlocks; ++i) o[i] = float16_t{};
    float m = -INFINITY;  // running max of raw scores (q . k), per query
    float l = 0.f;        // running sum of this lane's half of the keys

    // Lane-constant parts of the LDS addresses.
    const int krow = lane & 31;            // K operand row within a 32-key block
    const int ksw = swz(krow) & (D / 8 - 1);
    const int g16 = lane >> 4, i16 = lane & 15;
    const int vj = i16 >> 2, vm = i16 & 3;  // transposed-read source row / column group
    // V^T operand: source row 16*ks + 8*e + 4*hi + vj, columns 32*db + 16*(g16&1) + 4*vm.
    const int vchunk = 2 * (g16 & 1) + (vm >> 1);
    const int vsub = 4 * (vm & 1);

    uint4 kreg[C::kLoads], vreg[C::kLoads];
    load_tile<D>(K + head, 0, S, kreg);
    load_tile<D>(V + head, 0, S, vreg);
    store_tile<D>(lds, kreg);
    store_tile<D>(lds + C::kTile, vreg);
    __syncthreads();

    for (int t = 0; t < n_tiles; ++t) {
        const int k0 = t * kKRows;
        const bool more = t + 1 < n_tiles;
        if (more) {
            load_tile<D>(K + head, k0 + kKRows, S, kreg);
            load_tile<D>(V + head, k0 + kKRows, S, vreg);
        }
        if (k0 < wave_kv_end) {
            const half_t* Kt = lds + (t & 1) * 2 * C::kTile;
            const half_t* Vt = Kt + C::kTile;
            // ---- S^T = K Q^T for two 32-key blocks ----
            float16_t s[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                s[kb] = float16_t{};
                const half_t* kr = Kt + (kb * 32 + krow) * D;
#pragma unroll
                for (int kk = 0; kk < C::kKSteps; ++kk) {
                    const half8_t a = *reinterpret_cast<const half8_t*>(kr + (((2 * kk + hi) ^ ksw) * 8));
                    s[kb] = mfma32(a, qf[kk], s[kb]);
                }
            }
            // ---- masks: causal diagonal and keys past S ----
            if ((kCausal && k0 + kKRows - 1 > qw0) || k0 + kKRows > S) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + 32 * kb + 8 * (r >> 2) + 4 * hi + (r & 3);
                        if ((kCausal && key > my_q) || key >= S) s[kb][r] = -INFINITY;
                    }
            }
            // ---- online softmax (exp2 domain) ----
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m, mx);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = fast_exp2((m - m_use) * c2);
            m = m_new;
            const float mc = m_use * c2;
            half8_t p[4];
            float rs = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = fast_exp2(fmaf(s[kb][r], c2, -mc));
                    rs += pv;
                    p[2 * kb + (r >> 3)][r & 7] = (half_t)pv;
                }
            l = fmaf(l, alpha, rs);
#pragma unroll
            for (int db = 0; db < C::kDBlocks; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
            // ---- O^T += V^T P^T ----
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int db = 0; db < C::kDBlocks; ++db) {
                    const int r0 = 16 * ks + 4 * hi + vj;      // e = 0 row
                    const int r1 = r0 + 8;                       // e = 1 row
                    const int ch = 4 * db + vchunk;
                    const half4_t lo = lds_read_tr16(Vt + r0 * D + chunk_pos<D>(r0, ch) * 8 + vsub);
                    const half4_t up = lds_read_tr16(Vt + r1 * D + chunk_pos<D>(r1, ch) * 8 + vsub);
                    const half8_t a = {lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
                    o[db] = mfma32(a, p[ks], o[db]);
                }
            }
        }
        if (more) {
            half_t* nxt = lds + ((t + 1) & 1) * 2 * C::kTile;
            store_tile<D>(nxt, kreg);
            store_tile<D>(nxt + C::kTile, vreg);
        }
        __syncthreads();
    }

    // ---- epilogue: O = O^T / l, 4 consecutive d per store ----
    l += __shfl_xor(l, 32);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (my_q < S) {
        half_t* orow = O + head + (size_t)my_q * D;
#pragma unroll
        for (int db = 0; db < C::kDBlocks; ++db)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const half4_t v4 = {(half_t)(o[db][4 * rg] * inv), (half_t)(o[db][4 * rg + 1] * inv),
                                    (half_t)(o[db][4 * rg + 2] * inv), (half_t)(o[db][4 * rg + 3] * inv)};
                *reinterpret_cast<half4_t*>(orow + 32 * db + 8 * rg + 4 * hi) = v4;
            }
    }
}

template <int D, bool kCausal>
hipError_t launch(const half_t* q, const half_t* k, const half_t* v, half_t* o, int B, int H,
                  int S, float scale, hipStream_t stream) {
    const int BH = B * H;
    const int n_qt = (S + kQRows - 1) / kQRows;
    const int lds = Cfg<D>::kLdsBytes;
    hipLaunchKernelGGL((attn_fwd_kernel<D, kCausal>), dim3(BH * n_qt), dim3(kThreads), lds,
                       stream, q, k, v, o, S, BH, n_qt, scale * kLog2e);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Naive check kernel: one thread per query row (src/attn_sm75.cu:55-94 math).
// ---------------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(128)
attn_naive_kernel(const half_t* __restrict__ Q, const half_t* __restrict__ K,
                  const half_t* __restrict__ V, half_t* __restrict__ O, int S, long long rows,
                  float scale, int causal) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows) return;
    const long long bh = idx / S;
    const int qi = (int)(idx % S);
    const size_t off = (size_t)bh * S * D;
    float qf[D];
#pragma unroll
    for (int d = 0; d < D; ++d) qf[d] = (float)Q[off + (size_t)qi * D + d];
    const int kend = causal ? qi + 1 : S;
    float m = -INFINITY;
    for (int kk = 0; kk < kend; ++kk) {
        const half_t* kr = K + off + (size_t)kk * D;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < D; ++d) dot = fmaf(qf[d], (float)kr[d], dot);
        m = fmaxf(m, dot * scale);
    }
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = 0.f;
    float l = 0.f;
    for (int kk = 0; kk < kend; ++kk) {
        const half_t* kr = K + off + (size_t)kk * D;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < D; ++d) dot = fmaf(qf[d], (float)kr[d], dot);
        const float p = expf(fmaf(dot, scale, -m));
        l += p;
        const half_t* vr = V + off + (size_t)kk * D;
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = fmaf(p, (float)vr[d], acc[d]);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) O[off + (size_t)qi * D + d] = (half_t)(acc[d] / l);
}

}  // namespace

hipError_t attn_fwd(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                    int D, float scale, int causal, hipStream_t stream) {
    auto Q = static_cast<const half_t*>(q);
    auto K = static_cast<const half_t*>(k);
    auto Vp = static_cast<const half_t*>(v);
    auto Op = static_cast<half_t*>(o);
    if (D == 128)
        return causal ? launch<128, true>(Q, K, Vp, Op, B, H, S, scale, stream)
                      : launch<128, false>(Q, K, Vp, Op, B, H, S, scale, stream);
    return causal ? launch<64, true>(Q, K, Vp, Op, B, H, S, scale, stream)
                  : launch<64, false>(Q, K, Vp, Op, B, H, S, scale, stream);
}

hipError_t attn_naive(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                      int D, float scale, int causal, hipStream_t stream) {
    const long long rows = (long long)B * H * S;
    const unsigned blocks = (unsigned)((rows + 127) / 128);
    auto Q = static_cast<const half_t*>(q);
    auto K = static_cast<const half_t*>(k);
    auto Vp = static_cast<const half_t*>(v);
    auto Op = static_cast<half_t*>(o);
    if (D == 128)
        hipLaunchKernelGGL(attn_naive_kernel<128>, dim3(blocks), dim3(128), 0, stream, Q, K, Vp,
                           Op, S, rows, scale, causal);
    else
        hipLaunchKernelGGL(attn_naive_kernel<64>, dim3(blocks), dim3(128), 0, stream, Q, K, Vp,
                           Op, S, rows, scale, causal);
    return hipGetLastError();
}

}  // namespace tsa
