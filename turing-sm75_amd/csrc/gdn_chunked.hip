// gdn_chunked.hip -- chunked Gated DeltaNet prefill for gfx950 (fp16 MFMA, fp32 state).
//
// Chunk algebra (the chunk structure of gdn_chunked_cpu, src/gdn_sm75.cu:1109-1244, with
// the exact inverse).  Per V-head and chunk of C = 64 tokens, rows = tokens t, with
// G_t = in-chunk inclusive cumsum of g_log:
//   A[t][s]   = beta_t (k_t . k_s) e^{G_t - G_s}      s < t        (strictly lower)
//   Tm        = (I + A)^-1
//   W         = Tm diag(beta e^G) K          (C x dk)
//   U         = Tm diag(beta) V              (C x dv)
//   Aqk[t][s] = (q_t . k_s) e^{G_t - G_s}      s <= t
//   Vnew      = U - W S                      (S is dk x dv, the state entering the chunk)
//   O         = scale (diag(e^G) Q S + Aqk Vnew)
//   S'        = e^{G_{C-1}} S + K^T diag(e^{G_{C-1} - G}) Vnew
// Only differences G_t - G_s with s <= t are exponentiated, so nothing overflows.
//
// Two kernels:
//   gdn_chunk_prep  -- one workgroup per (b, h, chunk), all chunks in parallel:
//                      G, K K^T and Q K^T on MFMA, the exact blocked (I + A)^-1 in fp32,
//                      W and U on MFMA; writes W, U, Aqk (fp16) and G (fp32) to ws.
//   gdn_chunk_carry -- one workgroup per (b, h, 16-column strip of S), sequential over the
//                      chunks: Vnew = U - W S and Q S, O, and the state update, all on
//                      v_mfma_f32_16x16x32_f16 with the state kept in fp32 accumulators;
//                      the next chunk's W/Q/K/Aqk/U/G are prefetched while the current
//                      one is computed (double-buffered LDS).
#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kC = 64;     // chunk
constexpr int kD = 128;    // dk = dv
constexpr int kThreads = 256;
constexpr int kStrip = 16;  // state columns per carry workgroup

// Workspace per (b, h, chunk).
constexpr int kWsW = 0;                          // fp16 [64][128]
constexpr int kWsU = kWsW + kC * kD * 2;         // fp16 [64][128]
constexpr int kWsAqk = kWsU + kC * kD * 2;       // fp16 [64][64]
constexpr int kWsG = kWsAqk + kC * kC * 2;       // fp32 [64]
constexpr int kWsChunk = kWsG + kC * 4;          // 41216 B, multiple of 256

// 16-B chunk swizzle for [rows][128] fp16 LDS tiles (see attn_fwd.hip for the argument):
// 16 consecutive rows at one chunk and 4 aligned rows x 2 chunks are conflict free.
__device__ __forceinline__ int swz(int r) {
    return 2 * (r & 3) + ((r >> 2) & 1) + 8 * ((r >> 3) & 1);
}
__device__ __forceinline__ int tile_off(int r, int c /*16-B chunk*/) {
    return r * kD + ((c ^ swz(r)) << 3);
}
// Transposed read of a [rows][128] tile: result lane holds column col0 + lane%16 (of its
// 16-lane group) for rows row0 + j, j = 0..3, where this lane supplies row0 + (l%16)/4.
__device__ __forceinline__ half4_t tile_read_tr(const half_t* tile, int row0, int col0) {
    const int i16 = threadIdx.x & 15;
    const int r = row0 + (i16 >> 2);
    const int col = col0 + 4 * (i16 & 3);
    return lds_read_tr16(tile + tile_off(r, col >> 3) + (col & 7));
}

// ----------------------------------------------------------------------------------
// Prep
// ----------------------------------------------------------------------------------
struct PrepLds {
    half_t K[kC * kD];
    half_t Q[kC * kD];
    half_t V[kC * kD];
    float A[kC][kC + 1];
    float Tm[kC][kC + 4];
    float X[3][16][17];
    float G[kC];
    float bt[kC];
    float bg[kC];
};

__global__ void __launch_bounds__(kThreads)
gdn_chunk_prep(const half_t* __restrict__ q, const half_t* __restrict__ k,
               const half_t* __restrict__ v, const float* __restrict__ g_log,
               const float* __restrict__ beta, unsigned char* __restrict__ ws, int T, int Hq,
               int Hv, int nch) {
    __shared__ PrepLds sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hi = lane >> 5;
    const int ch = blockIdx.x % nch;
    const int bh = blockIdx.x / nch;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const int t0 = ch * kC;
    unsigned char* wsc = ws + ((size_t)bh * nch + ch) * kWsChunk;

    // ---- load K, Q, V rows of the chunk (zero past T), g and beta ----
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        const int r = id >> 4, c = id & 15;
        const int tt = t0 + r;
        uint4 kv = make_uint4(0, 0, 0, 0), qv = kv, vv = kv;
        if (tt < T) {
            const size_t bt = (size_t)b * T + tt;
            kv = *reinterpret_cast<const uint4*>(k + (bt * Hq + hq) * kD + c * 8);
            qv = *reinterpret_cast<const uint4*>(q + (bt * Hq + hq) * kD + c * 8);
            vv = *reinterpret_cast<const uint4*>(v + (bt * Hv + h) * kD + c * 8);
        }
        *reinterpret_cast<uint4*>(sm.K + tile_off(r, c)) = kv;
        *reinterpret_cast<uint4*>(sm.Q + tile_off(r, c)) = qv;
        *reinterpret_cast<uint4*>(sm.V + tile_off(r, c)) = vv;
    }
    for (int e = tid; e < kC * (kC + 4); e += kThreads) (&sm.Tm[0][0])[e] = 0.f;
    if (wave == 0) {
        const int tt = t0 + lane;
        const size_t bt = (size_t)b * T + tt;
        float x = tt < T ? g_log[bt * Hv + h] : 0.f;
        const float be = tt < T ? beta[bt * Hv + h] : 0.f;
        // inclusive prefix sum over the 64 tokens
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        sm.G[lane] = x;
        sm.bt[lane] = be;
        sm.bg[lane] = be * __expf(x);
        reinterpret_cast<float*>(wsc + kWsG)[lane] = x;
    }
    __syncthreads();

    // ---- K K^T and Q K^T: wave w owns the 32x32 tile (mt, nt) of both ----
    {
        const int mt = wave >> 1, nt = wave & 1;
        const int ra = 32 * mt + (lane & 31), rb = 32 * nt + (lane & 31);
        float16_t kk = {}, qk = {};
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) {
            const int c = 2 * s + hi;
            const half8_t ak = *reinterpret_cast<const half8_t*>(sm.K + tile_off(ra, c));
            const half8_t aq = *reinterpret_cast<const half8_t*>(sm.Q + tile_off(ra, c));
            const half8_t bk = *reinterpret_cast<const half8_t*>(sm.K + tile_off(rb, c));
            kk = mfma32(ak, bk, kk);
            qk = mfma32(aq, bk, qk);
        }
        half_t* aqk = reinterpret_cast<half_t*>(wsc + kWsAqk);
        const int s_ = rb;  // column = key token
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
            const float dec = (s_ <= t) ? __expf(sm.G[t] - sm.G[s_]) : 0.f;
            sm.A[t][s_] = (s_ < t) ? sm.bt[t] * kk[r] * dec : 0.f;
            aqk[t * kC + s_] = (half_t)(qk[r] * dec);
        }
    }
    __syncthreads();

    // ---- Tm = (I + A)^-1, 16x16 blocks: diagonal blocks by forward substitution ----
    if (wave == 0) {
        const int bi = lane >> 4, cj = lane & 15;
        float x[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float acc = (t == cj) ? 1.f : 0.f;
#pragma unroll
            for (int s = 0; s < t; ++s) acc = fmaf(-sm.A[16 * bi + t][16 * bi + s], x[s], acc);
            x[t] = acc;
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) sm.Tm[16 * bi + t][16 * bi + cj] = x[t];
    }
    __syncthreads();
    // off-diagonal blocks, block row by block row: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj
    {
        const int r = tid >> 4, c = tid & 15;
        for (int i = 1; i < 4; ++i) {
            for (int j = 0; j < i; ++j) {
                float x = 0.f;
                for (int kb = j; kb < i; ++kb)
#pragma unroll
                    for (int m = 0; m < 16; ++m)
                        x = fmaf(sm.A[16 * i + r][16 * kb + m], sm.Tm[16 * kb + m][16 * j + c], x);
                sm.X[j][r][c] = x;
            }
            __syncthreads();
            for (int j = 0; j < i; ++j) {
                float x = 0.f;
#pragma unroll
                for (int m = 0; m < 16; ++m)
                    if (m <= r) x = fmaf(sm.Tm[16 * i + r][16 * i + m], sm.X[j][m][c], x);
                sm.Tm[16 * i + r][16 * j + c] = -x;
            }
            __syncthreads();
        }
    }

    // ---- W = Tm diag(beta e^G) K and U = Tm diag(beta) V ----
    // wave w: row tile mt = w >> 1, column tiles nt = 2*(w & 1) + {0, 1}, for W and U.
    {
        const int mt = wave >> 1;
        const int trow = 32 * mt + (lane & 31);
        half8_t aw[4], au[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
            for (int qd = 0; qd < 8; ++qd) {
                const int s = 16 * ks + 8 * hi + qd;
                const float tv = sm.Tm[trow][s];
                aw[ks][qd] = (half_t)(tv * sm.bg[s]);
                au[ks][qd] = (half_t)(tv * sm.bt[s]);
            }
        }
        half_t* Wg = reinterpret_cast<half_t*>(wsc + kWsW);
        half_t* Ug = reinterpret_cast<half_t*>(wsc + kWsU);
        const int g16 = lane >> 4;
#pragma unroll
        for (int n2 = 0; n2 < 2; ++n2) {
            const int nt = 2 * (wave & 1) + n2;
            float16_t w_acc = {}, u_acc = {};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int row0 = 16 * ks + 8 * hi;
                const int col0 = 32 * nt + 16 * (g16 & 1);
                const half4_t k0 = tile_read_tr(sm.K, row0, col0);
                const half4_t k1 = tile_read_tr(sm.K, row0 + 4, col0);
                const half4_t v0 = tile_read_tr(sm.V, row0, col0);
                const half4_t v1 = tile_read_tr(sm.V, row0 + 4, col0);
                const half8_t bk = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
                const half8_t bv = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                w_acc = mfma32(aw[ks], bk, w_acc);
                u_acc = mfma32(au[ks], bv, u_acc);
            }
            const int col = 32 * nt + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
                Wg[t * kD + col] = (half_t)w_acc[r];
                Ug[t * kD + col] = (half_t)u_acc[r];
            }
        }
    }
}

// ----------------------------------------------------------------------------------
// Carry
// ----------------------------------------------------------------------------------
constexpr int kPadS = kD + 8;    // S16T row pitch (halfs): 272 B, conflict-free 16-B reads
constexpr int kPadV = kC + 8;    // VnT / VsT / Aqk row pitch: 144 B
struct CarryBuf {
    half_t W[kC * kD];
    half_t Q[kC * kD];
    half_t K[kC * kD];
    half_t Aqk[kC * kPadV];
    half_t U[kC * kStrip];
    float G[kC];
};
struct CarryLds {
    CarryBuf buf[2];
    half_t S16T[kStrip * kPadS];
    half_t VnT[kStrip * kPadV];
    half_t VsT[kStrip * kPadV];
};

// Per-thread share of one chunk's inputs: 4 x 16 B of each of W, Q, K; 2 of Aqk; one of
// U (threads 0..127) or G (threads 128..143).
struct ChunkRegs {
    uint4 w[4], q[4], k[4], a[2], x;
};

__device__ __forceinline__ void carry_load(ChunkRegs& R, const unsigned char* __restrict__ wsc,
                                           const half_t* __restrict__ q,
                                           const half_t* __restrict__ k, int b, int T, int Hq,
                                           int hq, int t0, int c0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        const int r = id >> 4, c = id & 15;
        const int tt = t0 + r;
        R.w[it] = *reinterpret_cast<const uint4*>(wsc + kWsW + (size_t)(r * kD + c * 8) * 2);
        if (tt < T) {
            const size_t bt = (size_t)b * T + tt;
            R.q[it] = *reinterpret_cast<const uint4*>(q + (bt * Hq + hq) * kD + c * 8);
            R.k[it] = *reinterpret_cast<const uint4*>(k + (bt * Hq + hq) * kD + c * 8);
        } else {
            R.q[it] = make_uint4(0, 0, 0, 0);
            R.k[it] = make_uint4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = it * kThreads + tid;  // 512 chunks of Aqk: row id/8, chunk id%8
        R.a[it] = *reinterpret_cast<const uint4*>(wsc + kWsAqk + (size_t)id * 16);
    }
    if (tid < 128) {  // U strip: row tid/2, half (tid&1) of the 16 columns
        const int r = tid >> 1, hv = tid & 1;
        R.x = *reinterpret_cast<const uint4*>(wsc + kWsU + (size_t)(r * kD + c0 + 8 * hv) * 2);
    } else if (tid < 144) {
        R.x = *reinterpret_cast<const uint4*>(wsc + kWsG + (size_t)(tid - 128) * 16);
    }
}

__device__ __forceinline__ void carry_store(const ChunkRegs& R, CarryBuf& B) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        const int r = id >> 4, c = id & 15;
        *reinterpret_cast<uint4*>(B.W + tile_off(r, c)) = R.w[it];
        *reinterpret_cast<uint4*>(B.Q + tile_off(r, c)) = R.q[it];
        *reinterpret_cast<uint4*>(B.K + tile_off(r, c)) = R.k[it];
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = it * kThreads + tid;
        const int r = id >> 3, c = id & 7;
        *reinterpret_cast<uint4*>(B.Aqk + r * kPadV + c * 8) = R.a[it];
    }
    if (tid < 128) {
        const int r = tid >> 1, hv = tid & 1;
        *reinterpret_cast<uint4*>(B.U + r * kStrip + 8 * hv) = R.x;
    } else if (tid < 144) {
        *reinterpret_cast<uint4*>(B.G + 4 * (tid - 128)) = R.x;
    }
}

__global__ void __launch_bounds__(kThreads, 1)
gdn_chunk_carry(const half_t* __restrict__ q, const half_t* __restrict__ k,
                const unsigned char* __restrict__ ws, float* __restrict__ state,
                half_t* __restrict__ out, int T, int Hq, int Hv, int nch, int BHv,
                float scale) {
    __shared__ CarryLds sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    // block id = strip * BHv + bh: all strips of one head share an XCD when BHv % 8 == 0.
    const int strip = blockIdx.x / BHv;
    const int bh = blockIdx.x % BHv;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const int c0 = strip * kStrip;
    const unsigned char* wsh = ws + (size_t)bh * nch * kWsChunk;

    // State strip: wave w owns rows i in [32w, 32w + 32) as two 16x16 accumulator tiles;
    // lane holds column c0 + c, rows 32w + 16m + 4g + r.
    float* Sg = state + ((size_t)bh * kD + c0 + c) * kD;
    float4_t s_acc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const float4 v4 = *reinterpret_cast<const float4*>(Sg + 32 * wave + 16 * m + 4 * g);
        s_acc[m] = float4_t{v4.x, v4.y, v4.z, v4.w};
        const half4_t hv = {(half_t)v4.x, (half_t)v4.y, (half_t)v4.z, (half_t)v4.w};
        *reinterpret_cast<half4_t*>(sm.S16T + c * kPadS + 32 * wave + 16 * m + 4 * g) = hv;
    }
    {
        ChunkRegs R;
        carry_load(R, wsh, q, k, b, T, Hq, hq, 0, c0);
        carry_store(R, sm.buf[0]);
    }
    __syncthreads();

    for (int ch = 0; ch < nch; ++ch) {
        const int t0 = ch * kC;
        const bool more = ch + 1 < nch;
        CarryBuf& B = sm.buf[ch & 1];
        ChunkRegs R;
        if (more) carry_load(R, wsh + (size_t)(ch + 1) * kWsChunk, q, k, b, T, Hq, hq, t0 + kC, c0);

        // ---- W S and Q S for token tile w (tokens 16w .. 16w+15) ----
        float4_t wsv = {}, qsv = {};
        const int trow = 16 * wave + c;  // A-operand row (token) of this lane
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const half8_t bS = *reinterpret_cast<const half8_t*>(sm.S16T + c * kPadS + 32 * ks + 8 * g);
            const half8_t aW = *reinterpret_cast<const half8_t*>(B.W + tile_off(trow, 4 * ks + g));
            const half8_t aQ = *reinterpret_cast<const half8_t*>(B.Q + tile_off(trow, 4 * ks + g));
            wsv = mfma16(aW, bS, wsv);
            qsv = mfma16(aQ, bS, qsv);
        }
        // ---- Vnew = U - W S (lane: column c, tokens 16w + 4g + r) ----
        const float GC = B.G[kC - 1];
        half4_t vn4, vs4;
        float eG[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * wave + 4 * g + r;
            const float Gt = B.G[t];
            const float vn = (float)B.U[t * kStrip + c] - wsv[r];
            vn4[r] = (half_t)vn;
            vs4[r] = (half_t)(vn * __expf(GC - Gt));
            eG[r] = __expf(Gt);
        }
        *reinterpret_cast<half4_t*>(sm.VnT + c * kPadV + 16 * wave + 4 * g) = vn4;
        *reinterpret_cast<half4_t*>(sm.VsT + c * kPadV + 16 * wave + 4 * g) = vs4;
        __syncthreads();

        // ---- O = scale (e^G Q S + Aqk Vnew) ----
        {
            float4_t av = {};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8_t aA = *reinterpret_cast<const half8_t*>(B.Aqk + trow * kPadV + 32 * ks + 8 * g);
                const half8_t bV = *reinterpret_cast<const half8_t*>(sm.VnT + c * kPadV + 32 * ks + 8 * g);
                av = mfma16(aA, bV, av);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tt = t0 + 16 * wave + 4 * g + r;
                if (tt < T)
                    out[(((size_t)b * T + tt) * Hv + h) * kD + c0 + c] = (half_t)(scale * fmaf(eG[r], qsv[r], av[r]));
            }
        }
        // ---- S = e^{G_C} S + K^T diag(e^{G_C - G}) Vnew ----
        {
            const float eGC = __expf(GC);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s_acc[m][r] *= eGC;
                const int i0 = 32 * wave + 16 * m;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const half4_t k0 = tile_read_tr(B.K, 32 * ks + 8 * g, i0);
                    const half4_t k1 = tile_read_tr(B.K, 32 * ks + 8 * g + 4, i0);
                    const half8_t aK = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
                    const half8_t bV = *reinterpret_cast<const half8_t*>(sm.VsT + c * kPadV + 32 * ks + 8 * g);
                    s_acc[m] = mfma16(aK, bV, s_acc[m]);
                }
                const half4_t hv = {(half_t)s_acc[m][0], (half_t)s_acc[m][1], (half_t)s_acc[m][2],
                                    (half_t)s_acc[m][3]};
                *reinterpret_cast<half4_t*>(sm.S16T + c * kPadS + i0 + 4 * g) = hv;
            }
        }
        if (more) carry_store(R, sm.buf[(ch + 1) & 1]);
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < 2; ++m)
        *reinterpret_cast<float4*>(Sg + 32 * wave + 16 * m + 4 * g) =
            make_float4(s_acc[m][0], s_acc[m][1], s_acc[m][2], s_acc[m][3]);
}

}  // namespace

size_t gdn_chunked_ws_bytes(int B, int T, int Hv) {
    const size_t nch = (size_t)(T + kC - 1) / kC;
    return (size_t)B * Hv * nch * kWsChunk;
}

hipError_t gdn_chunked(const void* q, const void* k, const void* v, const float* g_log,
                       const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                       float scale, void* ws, hipStream_t stream) {
    const int nch = (T + kC - 1) / kC;
    const int BHv = B * Hv;
    auto Q = static_cast<const half_t*>(q);
    auto K = static_cast<const half_t*>(k);
    auto W = static_cast<unsigned char*>(ws);
    hipLaunchKernelGGL(gdn_chunk_prep, dim3(BHv * nch), dim3(kThreads), 0, stream, Q, K,
                       static_cast<const half_t*>(v), g_log, beta, W, T, Hq, Hv, nch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gdn_chunk_carry, dim3(BHv * (kD / kStrip)), dim3(kThreads), 0, stream,
                       Q, K, W, state, static_cast<half_t*>(out), T, Hq, Hv, nch, BHv, scale);
    return hipGetLastError();
}

}  // namespace tsa
