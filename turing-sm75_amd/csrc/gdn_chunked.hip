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
// gdn_chunk_prep  -- one workgroup per (b, h, chunk), all chunks in parallel: G by a wave
//   scan, K K^T and Q K^T on v_mfma_f32_32x32x16_f16 (the all-zero upper tile skipped),
//   the exact (I + A)^-1 by 16x16 blocks in fp32 (diagonal blocks by forward substitution,
//   then each wave owns one block column, so no cross-wave dependency), W and U on MFMA
//   with K and V read transposed by ds_read_b64_tr_b16.  W, U, Aqk leave through LDS
//   staging as 16-byte stores, already in the operand layouts the carry kernel loads.
// gdn_chunk_carry -- one workgroup per (b, h, 32 state columns), sequential over chunks.
//   Two "chain" waves each own a 16-column strip of S in fp32 MFMA accumulators and run
//   only the loop-carried part: W S and the state update (32 v_mfma_f32_16x16x32_f16 per
//   chunk).  Two "output" waves trail by one chunk and compute Q S + Aqk Vnew from the
//   S / Vnew operands the chain waves leave in LDS.  Every operand tile is staged one chunk
//   ahead with gfx950 LDS-DMA (global_load_lds_dwordx4) into double-buffered slots, so no
//   register holds prefetched data and each wave reads its MFMA operands from LDS in
//   batches ahead of the MFMAs.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kC = 64;     // chunk
constexpr int kD = 128;    // dk = dv
constexpr int kThreads = 256;
constexpr int kA = 68;     // fp32 row pitch (floats) of the A / Tm tiles: 16-B aligned rows
constexpr int kStrips = 2; // 16-column strips per carry workgroup
constexpr int kCarryThreads = 512;  // waves 0-1 chain, 2-3 output, 4-7 DMA

// Workspace per (b, h, chunk).
constexpr int kWsW = 0;                     // fp16 [64 t][128]: column i stored at perm32(i)
constexpr int kWsU = kWsW + kC * kD * 2;    // fp16 [8 strip][4 mtile][64 lane][4]
constexpr int kWsAqk = kWsU + kC * kD * 2;  // fp16 [64 t][64]: column s stored at perm32(s)
constexpr int kWsG = kWsAqk + kC * kC * 2;  // fp32 [64] e^{G_t}, then fp32 [64] e^{G_63 - G_t}
constexpr int kWsChunk = kWsG + kC * 8;     // 41472 B, multiple of 256

// Within each aligned 32-block, index 16a + 4g + b is stored at 8g + 4a + b.  A 16x16x32
// MFMA lane of group g then finds its 8 k-values {16a + 4g + b} in one 16-byte run; that
// k order is the one in which a 16x16 accumulator (rows 4g + r) is reused as a B operand.
__device__ __forceinline__ int perm32(int i) {
    return (i & ~31) | (((i >> 2) & 3) << 3) | (((i >> 4) & 1) << 2) | (i & 3);
}

// 16-B chunk swizzle for [rows][128] fp16 LDS tiles (same argument as attn_fwd.hip): 16
// consecutive rows at one chunk, and 4 aligned rows x 2 chunks, are bank-conflict free.
__device__ __forceinline__ int swz(int r) {
    return 2 * (r & 3) + ((r >> 2) & 1) + 8 * ((r >> 3) & 1);
}
__device__ __forceinline__ int tile_off(int r, int c /*16-B chunk*/) {
    return r * kD + ((c ^ swz(r)) << 3);
}
// Transposed read of a [rows][128] tile: within each 16-lane group the result lane holds
// column col0 + lane%16 for rows row0 .. row0+3 (this lane supplies row0 + (l%16)/4).
__device__ __forceinline__ half4_t tile_read_tr(const half_t* tile, int row0, int col0) {
    const int i16 = threadIdx.x & 15;
    const int r = row0 + (i16 >> 2);
    const int col = col0 + 4 * (i16 & 3);
    return lds_read_tr16(tile + tile_off(r, col >> 3) + (col & 7));
}

// Orders this wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ half8_t cat8(const half4_t& a, const half4_t& b) {
    return half8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// ----------------------------------------------------------------------------------
// Prep
// ----------------------------------------------------------------------------------
struct PrepLds {
    half_t K[kC * kD];  // K rows, swizzled
    union {             // A during the solve; V afterwards; W staging at the end
        float A[kC][kA];
        half_t V[kC * kD];
        half_t Wst[kC * kD];
    };
    union {             // Tm; U staging at the end
        float Tm[kC][kA];
        half_t Ust[kC * kD];
    };
    half_t Aqk[kC * kC];  // Aqk staging
    float X[3][16][17];   // per-wave scratch of the off-diagonal solve
    float G[kC];
    float bt[kC];
    float bg[kC];
};

__global__ void __launch_bounds__(kThreads, 2)
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
    const int mt = wave >> 1, nt = wave & 1;  // this wave's 32x32 tile of K K^T / Q K^T

    // ---- 1. K rows to LDS, V rows and this wave's Q operand rows to registers ----
    uint4 vreg[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        const int r = id >> 4, c = id & 15;
        const int tt = t0 + r;
        uint4 kv = make_uint4(0, 0, 0, 0);
        vreg[it] = kv;
        if (tt < T) {
            const size_t bt = (size_t)b * T + tt;
            kv = *reinterpret_cast<const uint4*>(k + (bt * Hq + hq) * kD + c * 8);
            vreg[it] = *reinterpret_cast<const uint4*>(v + (bt * Hv + h) * kD + c * 8);
        }
        *reinterpret_cast<uint4*>(sm.K + tile_off(r, c)) = kv;
    }
    half8_t qa[kD / 16];
    {
        const int tt = t0 + 32 * mt + (lane & 31);
        const half_t* qrow = q + (((size_t)b * T + tt) * Hq + hq) * kD + 8 * hi;
#pragma unroll
        for (int s = 0; s < kD / 16; ++s)
            qa[s] = tt < T ? *reinterpret_cast<const half8_t*>(qrow + 16 * s) : half8_t{};
    }
    if (wave == 0) {
        const int tt = t0 + lane;
        const size_t bt = (size_t)b * T + tt;
        float x = tt < T ? g_log[bt * Hv + h] : 0.f;
        const float be = tt < T ? beta[bt * Hv + h] : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {  // inclusive prefix sum over the chunk
            const float y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        const float ex = __expf(x);
        sm.G[lane] = x;
        sm.bt[lane] = be;
        sm.bg[lane] = be * ex;
        reinterpret_cast<float*>(wsc + kWsG)[lane] = ex;
        reinterpret_cast<float*>(wsc + kWsG)[kC + lane] = __expf(__shfl(x, kC - 1) - x);
    }
    lds_barrier();

    // ---- 2. K K^T and Q K^T; A (fp32, strictly lower) and Aqk (fp16 staging) ----
    if (mt == 0 && nt == 1) {
        // every (t < 32, s >= 32) entry is above the diagonal: Aqk is zero there
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 8 * (r >> 2) + 4 * hi + (r & 3);
            sm.Aqk[t * kC + perm32(32 + (lane & 31))] = (half_t)0.f;
        }
    } else {
        const int ra = 32 * mt + (lane & 31), rb = 32 * nt + (lane & 31);
        float16_t kk = {}, qk = {};
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) {
            const int c = 2 * s + hi;
            const half8_t ak = *reinterpret_cast<const half8_t*>(sm.K + tile_off(ra, c));
            const half8_t bk = *reinterpret_cast<const half8_t*>(sm.K + tile_off(rb, c));
            kk = mfma32(ak, bk, kk);
            qk = mfma32(qa[s], bk, qk);
        }
        const float Gs = sm.G[rb];
        const int sp = perm32(rb);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
            const float dec = (rb <= t) ? __expf(sm.G[t] - Gs) : 0.f;
            if (rb < t) sm.A[t][rb] = sm.bt[t] * kk[r] * dec;
            sm.Aqk[t * kC + sp] = (half_t)(qk[r] * dec);
        }
    }
    lds_barrier();

    // ---- 3. Aqk out; Tm = (I + A)^-1 ----
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = it * kThreads + tid;
        *reinterpret_cast<uint4*>(wsc + kWsAqk + (size_t)id * 16) =
            *reinterpret_cast<const uint4*>(sm.Aqk + id * 8);
    }
    if (wave == 0) {  // the four 16x16 diagonal blocks, one column per lane
        const int bi = lane >> 4, cj = lane & 15;
        float x[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float acc = (t == cj) ? 1.f : 0.f;
            const float* arow = &sm.A[16 * bi + t][16 * bi];
#pragma unroll
            for (int s = 0; s < t; ++s) acc = fmaf(-arow[s], x[s], acc);
            x[t] = acc;
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) sm.Tm[16 * bi + t][16 * bi + cj] = x[t];
    }
    lds_barrier();
    if (wave < 3) {  // block column j = wave: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, i > j
        const int j = wave, rr = lane >> 4, cc = lane & 15;
        for (int i = j + 1; i < 4; ++i) {
            float x[4] = {0.f, 0.f, 0.f, 0.f};
            for (int kb = j; kb < i; ++kb) {
#pragma unroll
                for (int m4 = 0; m4 < 4; ++m4) {
                    float tv[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) tv[u] = sm.Tm[16 * kb + 4 * m4 + u][16 * j + cc];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float4 a4 = *reinterpret_cast<const float4*>(&sm.A[16 * i + 4 * rr + e][16 * kb + 4 * m4]);
                        x[e] = fmaf(a4.x, tv[0], x[e]);
                        x[e] = fmaf(a4.y, tv[1], x[e]);
                        x[e] = fmaf(a4.z, tv[2], x[e]);
                        x[e] = fmaf(a4.w, tv[3], x[e]);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) sm.X[j][4 * rr + e][cc] = x[e];
            wave_lds_sync();
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * rr + e;
                float acc = 0.f;
#pragma unroll
                for (int m = 0; m < 16; ++m)
                    if (m <= r) acc = fmaf(sm.Tm[16 * i + r][16 * i + m], sm.X[j][m][cc], acc);
                sm.Tm[16 * i + r][16 * j + cc] = -acc;
            }
            wave_lds_sync();
        }
    }
    lds_barrier();

    // ---- 4. V to LDS (over A), then W = Tm diag(beta e^G) K and U = Tm diag(beta) V ----
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        *reinterpret_cast<uint4*>(sm.V + tile_off(id >> 4, id & 15)) = vreg[it];
    }
    lds_barrier();
    float16_t w_acc[2], u_acc[2];
    {
        const int trow = 32 * mt + (lane & 31);
        const int g16 = lane >> 4;
        const int nks = mt == 0 ? 2 : 4;  // Tm[t < 32][s >= 32] = 0
        half8_t aw[4], au[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks >= nks) break;
            const float4 t0v = *reinterpret_cast<const float4*>(&sm.Tm[trow][16 * ks + 8 * hi]);
            const float4 t1v = *reinterpret_cast<const float4*>(&sm.Tm[trow][16 * ks + 8 * hi + 4]);
            const float tv[8] = {t0v.x, t0v.y, t0v.z, t0v.w, t1v.x, t1v.y, t1v.z, t1v.w};
#pragma unroll
            for (int qd = 0; qd < 8; ++qd) {
                const int s = 16 * ks + 8 * hi + qd;
                const float x = (s <= trow) ? tv[qd] : 0.f;  // Tm is lower triangular
                aw[ks][qd] = (half_t)(x * sm.bg[s]);
                au[ks][qd] = (half_t)(x * sm.bt[s]);
            }
        }
#pragma unroll
        for (int n2 = 0; n2 < 2; ++n2) {
            const int ntw = 2 * (wave & 1) + n2;
            w_acc[n2] = float16_t{};
            u_acc[n2] = float16_t{};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if (ks >= nks) break;
                const int row0 = 16 * ks + 8 * hi;
                const int col0 = 32 * ntw + 16 * (g16 & 1);
                const half8_t bk = cat8(tile_read_tr(sm.K, row0, col0), tile_read_tr(sm.K, row0 + 4, col0));
                const half8_t bv = cat8(tile_read_tr(sm.V, row0, col0), tile_read_tr(sm.V, row0 + 4, col0));
                w_acc[n2] = mfma32(aw[ks], bk, w_acc[n2]);
                u_acc[n2] = mfma32(au[ks], bv, u_acc[n2]);
            }
        }
    }
    lds_barrier();

    // ---- 5. stage W and U in their workspace layouts, then 16-byte stores ----
#pragma unroll
    for (int n2 = 0; n2 < 2; ++n2) {
        const int col = 32 * (2 * (wave & 1) + n2) + (lane & 31);
        const int cp = perm32(col);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
            sm.Wst[t * kD + cp] = (half_t)w_acc[n2][r];
            sm.Ust[((((col >> 4) * 4 + (t >> 4)) * 64 + ((t >> 2) & 3) * 16 + (col & 15)) << 2) + (t & 3)] =
                (half_t)u_acc[n2][r];
        }
    }
    lds_barrier();
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        *reinterpret_cast<uint4*>(wsc + kWsW + (size_t)id * 16) = *reinterpret_cast<const uint4*>(sm.Wst + id * 8);
        *reinterpret_cast<uint4*>(wsc + kWsU + (size_t)id * 16) = *reinterpret_cast<const uint4*>(sm.Ust + id * 8);
    }
}

// ----------------------------------------------------------------------------------
// Carry
// ----------------------------------------------------------------------------------
struct ChainSlot {                   // operands of the loop-carried part of one chunk
    half_t K[kC * kD];               // K rows, swizzled (read transposed by the update)
    half_t W[kC * kD];               // W rows (perm32 columns), swizzled
    half_t U[kStrips * 4 * 64 * 4];  // this workgroup's two U strips, accumulator order
    float E[kC];                     // e^{G_t}
    float Dg[kC];                    // e^{G_63 - G_t}
};
struct OutSlot {                     // operands of the output of one chunk
    half_t Q[kC * kD];               // Q rows, swizzled
    half_t A[kC * kC];               // Aqk rows (perm32 columns), 8-chunk swizzle
    float E[kC];                     // e^{G_t} (followed in the workspace by e^{G_63 - G_t})
    float Dg[kC];
};
struct CarryLds {
    ChainSlot cs[2];
    OutSlot os[2];
    uint4 XS[2][kStrips][6][64];     // chain -> output: S operands (4) and Vnew operands (2)
    half_t OS[2][32 * 32];           // per output wave: its 32 tokens x 32 columns of O
    unsigned PF[64];                 // landing words of the L2 prefetch (never read)
};

// 16-B chunk swizzle of the [64][64] Aqk tile: 16 consecutive rows at one chunk are
// conflict free (two rows share a 256-B bank period).
__device__ __forceinline__ int aqk_off(int r, int c) {
    return r * kC + ((c ^ ((r >> 1) & 7)) << 3);
}

typedef __attribute__((address_space(3))) void* lds_void_t;

// One LDS-DMA instruction: lane l copies 16 bytes from src into LDS dst_base + 16*l
// (M0 holds the wave's LDS base).  Written as inline asm on purpose: the compiler does not
// track LDS written by DMA slot by slot and would wait for every DMA in flight before the
// first LDS read of the other slot; the kernel orders DMA and reads itself with
// dma_barrier(), the only consumer-side wait these writes need.
__device__ __forceinline__ void dma16(const void* src, const void* dst_base) {
    const unsigned m0v = __builtin_amdgcn_readfirstlane(
        (unsigned)(uintptr_t)(lds_void_t)const_cast<void*>(dst_base));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(src), "{m0}"(m0v) : "memory");
}

// DMA of the chain operands of one chunk into a chain slot (37 one-KiB instructions) and
// of the output operands of one chunk into an out slot (25 instructions), spread over the
// four DMA waves (4-7).  A wave stalls at issue once its requests to far memory pile up,
// so the copies are issued by waves that do nothing else.  Rows past T are clamped to the
// last valid row: they only meet zero coefficients (U, W and beta are zero there).
__device__ __forceinline__ void dma_chain(ChainSlot& cs, const half_t* k, const unsigned char* wsc,
                                          int b, int T, int Hq, int hq, int t0, int pair) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = wave - 4; i < 37; i += 4) {
        if (i < 16) {                       // K tile, 1 KiB block i
            const int P = i * 64 + lane, row = P >> 4, cch = (P & 15) ^ swz(row);
            const int tt = min(t0 + row, T - 1);
            dma16(k + (((size_t)b * T + tt) * Hq + hq) * kD + cch * 8, cs.K + i * 512);
        } else if (i < 32) {                // W tile
            const int bi = i - 16, P = bi * 64 + lane, row = P >> 4, cch = (P & 15) ^ swz(row);
            dma16(wsc + kWsW + (size_t)(row * kD + cch * 8) * 2, cs.W + bi * 512);
        } else if (i < 36) {                // U strips 2*pair, 2*pair+1: 4 KiB linear
            const int bi = i - 32;
            dma16(wsc + kWsU + (size_t)pair * 4096 + (size_t)bi * 1024 + lane * 16, cs.U + bi * 512);
        } else if (lane < 32) {             // E, Dg: 512 B
            dma16(wsc + kWsG + lane * 16, cs.E);
        }
    }
}
__device__ __forceinline__ void dma_out(OutSlot& os, const half_t* q, const unsigned char* wsc,
                                        int b, int T, int Hq, int hq, int t0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = (wave - 3) & 3; i < 25; i += 4) {  // 62 instructions in all: 15 or 16 per wave
        if (i < 16) {                       // Q tile
            const int P = i * 64 + lane, row = P >> 4, cch = (P & 15) ^ swz(row);
            const int tt = min(t0 + row, T - 1);
            dma16(q + (((size_t)b * T + tt) * Hq + hq) * kD + cch * 8, os.Q + i * 512);
        } else if (i < 24) {                // Aqk tile
            const int bi = i - 16, P = bi * 64 + lane, row = P >> 3, cch = (P & 7) ^ ((row >> 1) & 7);
            dma16(wsc + kWsAqk + (size_t)(row * kC + cch * 8) * 2, os.A + bi * 512);
        } else if (lane < 32) {
            dma16(wsc + kWsG + lane * 16, os.E);
        }
    }
}

// L2 prefetch of one chunk: one 4-byte LDS-DMA per 128-byte line, landing in PF.  Lines
// shared by the four column workgroups of a head (K, Q, W, Aqk, E/Dg: 452 lines) are split
// four ways, each workgroup adds its own U strips (32 lines): 3 instructions, every lane
// active (spare lanes repeat the first E line).  Then the DMA of the chunk's tiles hits L2.
constexpr int kPfShared = 452 / 4;
constexpr int kPfInstr = 3;
__device__ __forceinline__ void prefetch_l2(const half_t* q, const half_t* k, const unsigned char* wsc,
                                            int b, int T, int Hq, int hq, int t0, int pair,
                                            const unsigned* pf) {
    const int lane = threadIdx.x & 63;
    const unsigned m0v = (unsigned)(uintptr_t)(lds_void_t)const_cast<unsigned*>(pf);
#pragma unroll
    for (int j = 0; j < kPfInstr; ++j) {
        const int slot = 64 * j + lane;
        const unsigned char* p = wsc + kWsG;
        if (slot < kPfShared) {
            const int L = pair + 4 * slot;  // < 452
            if (L < 256) {
                const int tt = min(t0 + ((L & 127) >> 1), T - 1);
                const half_t* base = L < 128 ? k : q;
                p = reinterpret_cast<const unsigned char*>(base + (((size_t)b * T + tt) * Hq + hq) * kD) + 128 * (L & 1);
            } else if (L < 384) {
                p = wsc + kWsW + (L - 256) * 128;
            } else if (L < 448) {
                p = wsc + kWsAqk + (L - 384) * 128;
            } else {
                p = wsc + kWsG + (L - 448) * 128;
            }
        } else if (slot < kPfShared + 32) {
            p = wsc + kWsU + pair * 4096 + (slot - kPfShared) * 128;
        }
        asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" :: "v"(p), "{m0}"(m0v) : "memory");
    }
}

// Wait for this wave's DMA, then a barrier over LDS: after it every wave sees every wave's
// DMA data.  The prefetching wave issued its kPfInstr prefetches last and vector loads
// complete in issue order, so vmcnt(kPfInstr) covers its DMA and leaves the prefetches in
// flight (vmcnt also counts stores; their completion is not needed here).
template <bool kPrefetcher>
__device__ __forceinline__ void dma_barrier() {
    if (kPrefetcher)
        __builtin_amdgcn_s_waitcnt(0x0F70 | kPfInstr);  // vmcnt(3)
    else
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt left at their maxima
    lds_barrier();
}

// Chain step for one chunk: strip S (fp32 accumulators) <- next state, and the S / Vnew
// operands handed to the output waves in XS.
__device__ __forceinline__ void chain_step(float4_t (&S)[8], const ChainSlot& cs, uint4* xs, int sl) {
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    half8_t Sb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        Sb[kk] = half8_t{(half_t)S[2 * kk][0], (half_t)S[2 * kk][1], (half_t)S[2 * kk][2], (half_t)S[2 * kk][3],
                         (half_t)S[2 * kk + 1][0], (half_t)S[2 * kk + 1][1], (half_t)S[2 * kk + 1][2], (half_t)S[2 * kk + 1][3]};
    half4_t u[4];
    float dg[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        u[mt] = *reinterpret_cast<const half4_t*>(cs.U + ((sl * 4 + mt) * 64 + lane) * 4);
        const float4 d4 = *reinterpret_cast<const float4*>(cs.Dg + 16 * mt + 4 * g);
        dg[mt][0] = d4.x; dg[mt][1] = d4.y; dg[mt][2] = d4.z; dg[mt][3] = d4.w;
    }
    const float eGC = cs.E[kC - 1];
    // W S in two batches of two row tiles; each batch's 8 W operands are read before its MFMAs
    float4_t wsv[4];
#pragma unroll
    for (int m0 = 0; m0 < 4; m0 += 2) {
        half8_t aW[2][4];
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                aW[mm][kk] = *reinterpret_cast<const half8_t*>(cs.W + tile_off(16 * (m0 + mm) + c, 4 * kk + g));
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
            wsv[m0 + mm] = float4_t{};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) wsv[m0 + mm] = mfma16(aW[mm][kk], Sb[kk], wsv[m0 + mm]);
        }
    }
    // Vnew = U - W S (lane: column c, tokens 16mt + 4g + r); Vs = Vnew e^{G_C - G_t}
    half8_t Vn[2], Vs[2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float vn = (float)u[mt][r] - wsv[mt][r];
            Vn[mt >> 1][4 * (mt & 1) + r] = (half_t)vn;
            Vs[mt >> 1][4 * (mt & 1) + r] = (half_t)(vn * dg[mt][r]);
        }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xs[kk * 64 + lane] = __builtin_bit_cast(uint4, Sb[kk]);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) xs[(4 + ks) * 64 + lane] = __builtin_bit_cast(uint4, Vn[ks]);
    // S = e^{G_C} S + K^T Vs: K^T operands read transposed, 8 row tiles in two batches
#pragma unroll
    for (int m0 = 0; m0 < 8; m0 += 4) {
        half8_t aK[4][2];
#pragma unroll
        for (int mm = 0; mm < 4; ++mm)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                aK[mm][ks] = cat8(tile_read_tr(cs.K, 32 * ks + 4 * g, 16 * (m0 + mm)),
                                  tile_read_tr(cs.K, 32 * ks + 16 + 4 * g, 16 * (m0 + mm)));
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            S[m0 + mm] *= eGC;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) S[m0 + mm] = mfma16(aK[mm][ks], Vs[ks], S[m0 + mm]);
        }
    }
}

// Output for one chunk, token tiles {2w, 2w+1} of both strips: O = scale (e^G Q S + Aqk Vnew).
__device__ __forceinline__ void out_step(const OutSlot& os, const uint4 (*xs)[6][64], half_t* ostage,
                                         int w, float scale) {
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    half8_t aQ[2][4], aA[2][2];
    float eg[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = 16 * (2 * w + j) + c;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const half4_t lo = *reinterpret_cast<const half4_t*>(
                os.Q + t * kD + (((4 * kk + (g >> 1)) ^ swz(t)) << 3) + 4 * (g & 1));
            const half4_t up = *reinterpret_cast<const half4_t*>(
                os.Q + t * kD + (((4 * kk + 2 + (g >> 1)) ^ swz(t)) << 3) + 4 * (g & 1));
            aQ[j][kk] = cat8(lo, up);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            aA[j][ks] = *reinterpret_cast<const half8_t*>(os.A + aqk_off(t, 4 * ks + g));
        const float4 e4 = *reinterpret_cast<const float4*>(os.E + 16 * (2 * w + j) + 4 * g);
        eg[j][0] = e4.x; eg[j][1] = e4.y; eg[j][2] = e4.z; eg[j][3] = e4.w;
    }
    float4_t qs[2][kStrips], av[2][kStrips];
#pragma unroll
    for (int s = 0; s < kStrips; ++s) {
        half8_t Sb[4], Vn[2];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) Sb[kk] = __builtin_bit_cast(half8_t, xs[s][kk][lane]);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) Vn[ks] = __builtin_bit_cast(half8_t, xs[s][4 + ks][lane]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            qs[j][s] = float4_t{};
            av[j][s] = float4_t{};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) qs[j][s] = mfma16(aQ[j][kk], Sb[kk], qs[j][s]);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) av[j][s] = mfma16(aA[j][ks], Vn[ks], av[j][s]);
        }
    }
    // O tile (32 tokens x 32 columns) staged in LDS; out_flush stores it
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int s = 0; s < kStrips; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                ostage[(16 * j + 4 * g + r) * 32 + 16 * s + c] =
                    (half_t)(scale * fmaf(eg[j][r], qs[j][s][r], av[j][s][r]));
}

// 16-byte stores of a staged O tile (tokens t0 + 32w .. +31, columns pair*32 .. +31).
// Called one iteration after out_step, so the stores drain behind a whole iteration of
// work instead of in front of the next barrier.
__device__ __forceinline__ void out_flush(const half_t* ostage, half_t* out, int b, int T, int Hv,
                                          int h, int t0, int pair, int w) {
    const int lane = threadIdx.x & 63;
    wave_lds_sync();
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int tl = 16 * hf + (lane >> 2);  // token within this wave's 32
        const int tt = t0 + 32 * w + tl;
        const uint4 v4 = *reinterpret_cast<const uint4*>(ostage + tl * 32 + 8 * (lane & 3));
        if (tt < T)
            *reinterpret_cast<uint4*>(out + (((size_t)b * T + tt) * Hv + h) * kD + pair * 32 + 8 * (lane & 3)) = v4;
    }
    wave_lds_sync();
}

__global__ void __launch_bounds__(kCarryThreads, 1)
gdn_chunk_carry(const half_t* __restrict__ q, const half_t* __restrict__ k,
                const unsigned char* __restrict__ ws, float* __restrict__ state,
                half_t* __restrict__ out, int T, int Hq, int Hv, int nch, int BHv, float scale) {
    __shared__ CarryLds sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    // block id = pair * BHv + bh: all column pairs of one head share an XCD when BHv % 8 == 0
    const int pair = blockIdx.x / BHv;
    const int bh = blockIdx.x % BHv;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const unsigned char* wsh = ws + (size_t)bh * nch * kWsChunk;
    const bool chain = wave < 2, outw = wave == 2 || wave == 3, dmaw = wave >= 4;
    const int sl = wave & 1;  // chain wave: its strip; output wave: w = wave - 2

    // Pipeline, iteration it.  Chain waves: process chunk it from cs[it&1].  Output waves:
    // store the O tile of chunk it-2 staged in LDS, then compute the output of chunk it-1
    // from os[(it-1)&1] and XS[(it-1)&1].  DMA waves: copy the chain operands of chunk it+1
    // into cs[(it+1)&1] and the output operands of chunk it into os[it&1]; wave 7 then
    // prefetches chunk it+3 into L2; wait for the copies.  Then the workgroup meets at a
    // barrier.
    float4_t S[8];
    float* Sg = state + ((size_t)bh * kD + (pair * kStrips + sl) * 16 + c) * kD;
    if (chain) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const float4 v4 = *reinterpret_cast<const float4*>(Sg + 16 * m + 4 * g);
            S[m] = float4_t{v4.x, v4.y, v4.z, v4.w};
        }
    }
    if (dmaw) {
        dma_chain(sm.cs[0], k, wsh, b, T, Hq, hq, 0, pair);
        if (wave == 7)
            for (int cp = 1; cp <= 2; ++cp) {
                const int cc = min(cp, nch - 1);
                prefetch_l2(q, k, wsh + (size_t)cc * kWsChunk, b, T, Hq, hq, cc * kC, pair, sm.PF);
            }
    }
    dma_barrier<false>();

    // Each role runs its own loop (one barrier per iteration in each), so no role's loop
    // state occupies registers in another role's code.  `it` runs 0..nch; the loop is
    // unrolled by two so slot indices are constants.
    if (chain) {
        for (int it = 0; it <= nch; it += 2) {
            if (it < nch) chain_step(S, sm.cs[0], &sm.XS[0][sl][0][0], sl);
            lds_barrier();  // chain waves issue no vector memory operations in the loop
            if (it + 1 > nch) break;
            if (it + 1 < nch) chain_step(S, sm.cs[1], &sm.XS[1][sl][0][0], sl);
            lds_barrier();
        }
    } else if (outw) {
        const int w = wave - 2;
        for (int it = 0; it <= nch; it += 2) {
            if (it >= 2) out_flush(sm.OS[w], out, b, T, Hv, h, (it - 2) * kC, pair, w);
            if (it >= 1) out_step(sm.os[1], sm.XS[1], sm.OS[w], w, scale);
            lds_barrier();  // the O stores need not complete before the barrier
            if (it + 1 > nch) break;
            if (it >= 1) out_flush(sm.OS[w], out, b, T, Hv, h, (it - 1) * kC, pair, w);
            out_step(sm.os[0], sm.XS[0], sm.OS[w], w, scale);
            lds_barrier();
        }
    } else {
        auto dma_step = [&](auto P, int it) {
            constexpr int p = decltype(P)::value;
            if (it + 1 < nch)
                dma_chain(sm.cs[p ^ 1], k, wsh + (size_t)(it + 1) * kWsChunk, b, T, Hq, hq, (it + 1) * kC, pair);
            if (it < nch) dma_out(sm.os[p], q, wsh + (size_t)it * kWsChunk, b, T, Hq, hq, it * kC);
            if (wave == 7) {
                const int cc = min(it + 3, nch - 1);
                prefetch_l2(q, k, wsh + (size_t)cc * kWsChunk, b, T, Hq, hq, cc * kC, pair, sm.PF);
                dma_barrier<true>();
            } else {
                dma_barrier<false>();
            }
        };
        for (int it = 0; it <= nch; it += 2) {
            dma_step(std::integral_constant<int, 0>{}, it);
            if (it + 1 > nch) break;
            dma_step(std::integral_constant<int, 1>{}, it + 1);
        }
    }
    if (chain) {
#pragma unroll
        for (int m = 0; m < 8; ++m)
            *reinterpret_cast<float4*>(Sg + 16 * m + 4 * g) = make_float4(S[m][0], S[m][1], S[m][2], S[m][3]);
    } else if (outw) {
        out_flush(sm.OS[wave - 2], out, b, T, Hv, h, (nch - 1) * kC, pair, wave - 2);
    }
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
    hipLaunchKernelGGL(gdn_chunk_carry, dim3(BHv * (kD / (16 * kStrips))), dim3(kCarryThreads), 0,
                       stream, Q, K, W, state, static_cast<half_t*>(out), T, Hq, Hv, nch, BHv,
                       scale);
    return hipGetLastError();
}

}  // namespace tsa
