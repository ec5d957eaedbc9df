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
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kC = 64;     // chunk
constexpr int kD = 128;    // dk = dv
constexpr int kThreads = 256;
constexpr int kStrips = 2; // 16-column strips per carry workgroup
constexpr int kCarryThreads = 512;  // waves 0-1 chain, 2-3 output, 4-7 DMA

// Workspace per (b, h, chunk).
constexpr int kWsW = 0;                     // fp16 [64 t][128]: column i stored at perm32(i)
constexpr int kWsU = kWsW + kC * kD * 2;    // fp32 [8 strip][4 mtile][64 lane][4]
constexpr int kWsAqk = kWsU + kC * kD * 4;  // fp16 [64 t][64]: column s stored at perm32(s)
// fp32 [64] e^{G_t} qn_t, [64] e^{G_63 - G_t} kn_t, [64] {e^{G_63}, 0, ...}, [64] zeros, where
// qn_t, kn_t are the l2-norm factors of the fused entry point's raw q / k rows (1 otherwise)
constexpr int kWsG = kWsAqk + kC * kC * 2;
constexpr int kWsChunk = kWsG + kC * 16;    // 58368 B, multiple of 256
// fp32 q / k / v / out (the reference's own I/O): the prep also leaves the chunk's K and Q
// rows in fp16, unswizzled [64 t][128], for the carry's copies (LDS-DMA cannot convert)
constexpr int kWsK = kWsChunk;
constexpr int kWsQ = kWsK + kC * kD * 2;
// and the low halves of the K rows (K - fp16(K), fp16): the state update takes K as an exact
// hi + lo pair, since rounding the fp32 K to one fp16 operand there is most of the fp32 path's
// state error (~2.3e-4 of 3.4e-4 on the reference's own inputs, numpy model)
constexpr int kWsKlo = kWsQ + kC * kD * 2;
constexpr int kWsChunkF32 = kWsKlo + kC * kD * 2;  // 107520 B
template <bool kF32> constexpr int ws_chunk() { return kF32 ? kWsChunkF32 : kWsChunk; }

// Ready flags, after all chunk workspaces: one word per (b, h, chunk), then an abort word per
// carry workgroup.  A call that runs the prep beside the carry first clears them with a small
// kernel on the caller's stream (gdn_flags_clear, a kernel rather than a memset so that a
// captured graph replays it correctly), so whatever the workspace held before, no flag reads
// as set before the prep sets it in this call.  A call that runs them in order writes and
// reads no flags (both kernels get a null flag pointer: the kernel boundary orders the prep's
// stores before the carry), and the carry zeroes the abort words itself.  Beside the carry
// the prep writes 1 there once the chunk's workspace is in memory; the carry's DMA waves wait
// for it before copying the chunk.
// A wait gives up after a limit on the 100 MHz real-time counter (2 ms; the environment
// variable TSA_GDN_CARRY_WAIT_US sets it in microseconds, 0 = give up whenever a chunk is
// not ready at the first look, which is how the tests exercise the path).  When the prep
// runs beside the carry, a workgroup that gave up leaves its state columns untouched and
// writes 1 to its abort word; a second launch of the carry, ordered after the prep on the
// caller's stream, runs exactly the workgroups whose abort word is 1 and exits at once in the
// others.  Waits time out when the two kernels do not run at the same time: a profiler or a
// runtime setting that serialises dispatches, or a device busy with other work.  The abort
// words stay in the workspace after the call (tsa_gdn_chunked_redo_count reads them).  A
// wait that times out where no second launch follows poisons the state with NaN.

// Wait limit of the second carry launch (1 s); it runs after the prep, so its flags are
// normally all set.
constexpr unsigned kRetryWaitTicks = 100000000u;

// Carry launch modes.
constexpr int kCarryInOrder = 0;  // after the prep on one stream: waits never block
constexpr int kCarryBeside = 1;   // beside the prep: a timed-out workgroup aborts
constexpr int kCarryRetry = 2;    // after the prep: only the first launch's aborted workgroups run

// Sequence split (few heads, many chunks): T is cut into nseg segments of seg_len chunks (the
// last takes the rest).  The state update is linear in the state and in U, so the state
// after a segment is an affine map of the state E entering it, S_out = Phi E + Z, where Z is
// the segment's chain run from S = 0 and Phi its chain run from S = I with U = 0; and a
// chunk's output, O = A S + B, is then O = O_Z + M E, where O_Z is the output of the Z chain
// and M = A Phi_<c the output of the Phi chain (U = 0 makes B vanish).  Three launches after
// the prep:
//   maps    -- segment 0's chain from the caller's state (its outputs, and its end state as
//              segment 1's entry), and, side by side, the Z and Phi chains of segments
//              1 .. nseg-1 with their outputs O_Z and M (fp32, to the workspace);
//   combine (gdn_seg_combine) -- E[s+1] = Phi_s E[s] + Z_s for s = 1 .. nseg-1, the last
//              one the call's final state;
//   fixup   (gdn_seg_fixup) -- O = O_Z + M E for every chunk of segments 1 .. nseg-1, all
//              chunks in parallel.
// The serial depth drops from nch chunk steps to seg_len chunk steps + nseg - 1 combine
// steps.  Per (b, h, segment) the workspace holds three [128 columns][128] fp32 slots
// (entry E, Z, Phi), and per (b, h) the O_Z and M rows of the tokens after segment 0.
constexpr int kJobPlain = 0, kJobMaps = 1;
constexpr int kSegSlots = 3, kSegEntry = 0, kSegZ = 1, kSegPhi = 2;
constexpr size_t kSegSlotFloats = (size_t)kD * kD;
struct CarryJob {
    int phase = kJobPlain;
    int nseg = 1, seg_len = 0;
    int Tr = 0;            // tokens after segment 0: rows of oz / om per (b, h)
    float* seg = nullptr;  // [B*Hv][nseg][kSegSlots][kD][kD]
    float* oz = nullptr;   // [B*Hv][Tr][kD]: O_Z, the Z chains' outputs
    float* om = nullptr;   // [B*Hv][Tr][kD]: M, the Phi chains' outputs
};

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

// Device-scope stores of the workspace (sc1): written through to the device's coherence
// point, so the carry, whose copies of them are device-scope loads too, sees them from any
// XCD as soon as this wave's vmcnt has drained -- no L2 write-back or invalidate needed
// (both measured far too slow to issue once per workgroup or chunk).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_dev(unsigned char* p, const uint4& v) {
    const u32x4_t x = {v.x, v.y, v.z, v.w};
    // s_nop 1: a store of more than 8 bytes may still read its data registers in the next
    // cycle, and the compiler does not see into this asm to keep them unchanged that long
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(x) : "memory");
}
__device__ __forceinline__ void store_dev(float* p, float v) {
    asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}

// 8 consecutive q / k / v elements as 8 fp16 values (one uint4), from fp16 or fp32 memory:
// fp32 inputs are converted in registers.
__device__ __forceinline__ uint4 load8h(const half_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint4 load8h(const float* p) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    const half8_t h = {(half_t)a.x, (half_t)a.y, (half_t)a.z, (half_t)a.w,
                       (half_t)b.x, (half_t)b.y, (half_t)b.z, (half_t)b.w};
    return __builtin_bit_cast(uint4, h);
}
// The same 8 fp32 elements as an exact pair of fp16 halves: hi = fp16(x), lo = fp16(x - hi).
__device__ __forceinline__ void load8hl(const float* p, uint4& hi, uint4& lo) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    half8_t h, l;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        h[e] = (half_t)x[e];
        l[e] = (half_t)(x[e] - (float)h[e]);
    }
    hi = __builtin_bit_cast(uint4, h);
    lo = __builtin_bit_cast(uint4, l);
}
__device__ __forceinline__ void load8hl(const half_t* p, uint4& hi, uint4& lo) {
    hi = *reinterpret_cast<const uint4*>(p);
    lo = make_uint4(0, 0, 0, 0);
}

// ----------------------------------------------------------------------------------
// Prep
// ----------------------------------------------------------------------------------
// Packed storage of the ten lower-triangular 16x16 fp32 blocks of a 64 x 64 matrix (A, Tm):
// block (i, j), j <= i, at (i(i+1)/2 + j) * 256 floats, element (r, c) of a block at
// 16 r + 4 ((c/4) ^ (r/4 % 4)) + c % 4.  The XOR of 16-byte chunks makes the MFMA operand
// reads of the block solve (16 rows x 4 columns, 4 rows x 16 columns) hit 64 distinct
// banks, and keeps 4 consecutive columns in one 16-byte chunk.
__device__ __forceinline__ int tri_off(int row, int col) {
    const int i = row >> 4, j = col >> 4, r = row & 15, c = col & 15;
    return (((i * (i + 1)) >> 1) + j) * 256 + r * 16 + ((((c >> 2) ^ (r >> 2)) & 3) << 2) + (c & 3);
}

// 37 KB, so four workgroups share a CU.  Region x holds A and Aqk / Tm during the solve,
// then V for the U product; K's region takes the W staging.
struct PrepLds {
    half_t K[kC * kD];          // K rows, swizzled; W staging at the end
    union {
        struct {
            float A[10 * 256];  // strictly lower A, packed blocks
            union {
                half_t Aqk[kC * kC];  // Aqk staging
                float Tm[10 * 256];   // (I + A)^-1, packed blocks
            };
        } s;
        half_t V[kC * kD];      // V rows, swizzled
    } x;
    float G[kC];
    float bt[kC];
    float bg[kC];
    float kn[kC];  // l2-norm factors 1 / max(||k_t||, eps), 1 / max(||q_t||, eps) (fused only)
    float qn[kC];
};

// kFused: q / k are the raw rows (normalised here: the factors scale A, Aqk, W and the
// workspace's e^G / e^{G_63 - G}, so the carry multiplies raw K / Q rows by them for free),
// and g_log / beta are computed from the raw projections a / b (gate arguments).
// TIO: the q / k / v element type (fp16, or fp32 with the K / Q rows left in fp16 in the
// workspace for the carry).
// Four workgroups per CU (128 VGPRs); the fp32-I/O form holds its fp32 loads before converting
// them and needs more registers, so it runs three per CU rather than spill.
template <typename TIO> constexpr int prep_wgs_per_cu() { return std::is_same<TIO, float>::value ? 3 : 4; }
template <bool kFused, typename TIO>
__global__ void __launch_bounds__(kThreads, prep_wgs_per_cu<TIO>())
gdn_chunk_prep(const TIO* __restrict__ q, const TIO* __restrict__ k,
               const TIO* __restrict__ v, const float* __restrict__ g_log,
               const float* __restrict__ beta, GdnRawGates gates, unsigned char* __restrict__ ws,
               unsigned* __restrict__ flags, int T, int Hq, int Hv, int nch, int BHv) {
    __shared__ __align__(16) PrepLds sm;
    // fp32 I/O: the low fp16 halves of the chunk's V rows (swizzled like V), 16 KiB more LDS
    __shared__ __align__(16) half_t vlo_lds[std::is_same<TIO, float>::value ? kC * kD : 8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hi = lane >> 5;
    // chunk-major: workgroups are dispatched in the order the carry consumes chunks, and
    // (b, h, chunk) lands on the XCD of the head's carry workgroups when BHv % 8 == 0
    const int ch = blockIdx.x / BHv;
    const int bh = blockIdx.x % BHv;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const int t0 = ch * kC;
    constexpr bool kF32 = std::is_same<TIO, float>::value;
    unsigned char* wsc = ws + ((size_t)bh * nch + ch) * ws_chunk<kF32>();
    const int mt = wave >> 1, nt = wave & 1;  // this wave's 32x32 tile of K K^T / Q K^T

    // ---- 1. K rows to LDS, V rows and this wave's Q operand rows to registers.  Every global
    // load of the phase is issued first (wave 0's gate inputs, K, V, Q), from row-clamped
    // addresses, and rows past T are zeroed where the values are consumed: a branch around a
    // load makes the compiler wait for every load in flight where the paths join, which had
    // serialised the phase into one memory latency per K row group ----
    const int lastt = T - 1;
    float gx = 0.f, gy = 0.f;  // wave 0: the gate inputs of token t0 + lane
    if (wave == 0) {
        const size_t bt = (size_t)b * T + min(t0 + lane, lastt);
        gx = kFused ? gates.a[bt * Hv + h] : g_log[bt * Hv + h];
        gy = kFused ? gates.b[bt * Hv + h] : beta[bt * Hv + h];
    }
    // with fp32 I/O K and V also keep their low fp16 halves: K_lo goes to the workspace for the
    // carry's state update, V_lo feeds the U product as a second B operand
    uint4 kreg[4], vreg[4], klo[4], vlo[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        const size_t bt = (size_t)b * T + min(t0 + (id >> 4), lastt);
        load8hl(k + (bt * Hq + hq) * kD + (id & 15) * 8, kreg[it], klo[it]);
        load8hl(v + (bt * Hv + h) * kD + (id & 15) * 8, vreg[it], vlo[it]);
    }
    half8_t qa[kD / 16];
    const int qt_row = t0 + 32 * mt + (lane & 31);
    {
        const TIO* qrow = q + (((size_t)b * T + min(qt_row, lastt)) * Hq + hq) * kD + 8 * hi;
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) qa[s] = __builtin_bit_cast(half8_t, load8h(qrow + 16 * s));
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        const int r = id >> 4, c = id & 15;
        const uint4 kv = t0 + r > lastt ? make_uint4(0, 0, 0, 0) : kreg[it];
        *reinterpret_cast<uint4*>(sm.K + tile_off(r, c)) = kv;
        if (kF32) {
            store_dev(wsc + kWsK + (size_t)(r * kD + c * 8) * 2, kv);
            store_dev(wsc + kWsKlo + (size_t)(r * kD + c * 8) * 2, t0 + r > lastt ? make_uint4(0, 0, 0, 0) : klo[it]);
        }
        if (kFused) {  // the row's 16 threads are 16 consecutive lanes of one wave
            const half8_t k8 = __builtin_bit_cast(half8_t, kv);
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf((float)k8[e], (float)k8[e], ss);
            ss += __shfl_xor(ss, 8);
            ss += __shfl_xor(ss, 4);
            ss += __shfl_xor(ss, 2);
            ss += __shfl_xor(ss, 1);
            if (c == 0) sm.kn[r] = 1.f / fmaxf(sqrtf(ss), gates.eps);
        }
    }
    {
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) qa[s] = qt_row > lastt ? half8_t{} : qa[s];
        if (kF32 && nt == 0) {  // waves 0 and 2 hold the chunk's 64 Q rows
            const int row = 32 * mt + (lane & 31);
#pragma unroll
            for (int s = 0; s < kD / 16; ++s)
                store_dev(wsc + kWsQ + (size_t)(row * kD + 16 * s + 8 * hi) * 2, __builtin_bit_cast(uint4, qa[s]));
        }
        if (kFused) {  // the two halves of the row are lanes l and l ^ 32
            float ss = 0.f;
#pragma unroll
            for (int s = 0; s < kD / 16; ++s)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = fmaf((float)qa[s][e], (float)qa[s][e], ss);
            ss += __shfl_xor(ss, 32);
            if (nt == 0 && hi == 0) sm.qn[32 * mt + (lane & 31)] = 1.f / fmaxf(sqrtf(ss), gates.eps);
        }
    }
    if (wave == 0) {
        float x = 0.f, be = 0.f;
        if (t0 + lane <= lastt) {
            if (kFused) {
                x = gdn_softplus(gx + gates.dt_bias[h]) * gates.A[h];
                be = gdn_sigmoid(gy);
            } else {
                x = gx;
                be = gy;
            }
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {  // inclusive prefix sum over the chunk
            const float y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        sm.G[lane] = x;
        sm.bt[lane] = be;
    }
    lds_barrier();

    // ---- 2. K K^T and Q K^T; A (fp32, strictly lower) and Aqk (fp16 staging) ----
    if (mt == 0 && nt == 1) {
        // every (t < 32, s >= 32) entry is above the diagonal: Aqk is zero there
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 8 * (r >> 2) + 4 * hi + (r & 3);
            sm.x.s.Aqk[t * kC + perm32(32 + (lane & 31))] = (half_t)0.f;
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
        const float kns = kFused ? sm.kn[rb] : 1.f;
        const int sp = perm32(rb);
        // this lane's rows t = 32mt + 8q + 4hi + 0..3: four 16-byte reads per factor (one
        // 4-byte read per row had made this phase a chain of ~65 small LDS round trips)
        float4 g4[4], b4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int t0q = 32 * mt + 8 * q + 4 * hi;
            if (!kFused) {
                g4[q] = *reinterpret_cast<const float4*>(sm.G + t0q);
                b4[q] = *reinterpret_cast<const float4*>(sm.bt + t0q);
            }
        }
        // A is stored only for blocks (t/16, rb/16) on or below the diagonal; in the one block
        // above it (mt == nt, rb in the upper half, t in the lower) the lane writes a slot of
        // sm.bg instead (rewritten in phase 3), so no store needs a branch.  Entries with
        // rb >= t inside stored diagonal blocks get zeros, which nothing reads.
        const bool upper = mt == nt && ((lane >> 4) & 1);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = r >> 2, e = r & 3;
            const int t = 32 * mt + 8 * q + 4 * hi + e;
            // the fused variant reads per row (holding the 32 values spills it)
            const float Gt = kFused ? sm.G[t] : e == 0 ? g4[q].x : e == 1 ? g4[q].y : e == 2 ? g4[q].z : g4[q].w;
            const float bt = kFused ? sm.bt[t] : e == 0 ? b4[q].x : e == 1 ? b4[q].y : e == 2 ? b4[q].z : b4[q].w;
            const float dec = (rb <= t) ? __expf(Gt - Gs) : 0.f;
            float aval = bt * kk[r] * dec, qval = qk[r] * dec;
            if (kFused) {  // per-row reads here: 16-byte ones would hold 32 more registers
                aval = bt * kk[r] * (dec * sm.kn[t] * kns);
                qval = qk[r] * (dec * sm.qn[t] * kns);
            }
            float* ap = (upper && r < 8) ? sm.bg + (lane & 63) : sm.x.s.A + tri_off(t, rb);
            *ap = rb < t ? aval : 0.f;
            sm.x.s.Aqk[t * kC + sp] = (half_t)qval;
        }
    }
    lds_barrier();

    // ---- 3. Aqk out (its staging shares LDS with Tm); wave 1: the decay block and the W
    // column scale beta e^G (kn); Tm = (I + A)^-1 ----
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = it * kThreads + tid;
        store_dev(wsc + kWsAqk + (size_t)id * 16, *reinterpret_cast<const uint4*>(sm.x.s.Aqk + id * 8));
    }
    if (wave == 1) {
        const float x = sm.G[lane], xc = sm.G[kC - 1];
        const float ex = __expf(x);
        const float kn = kFused ? sm.kn[lane] : 1.f, qn = kFused ? sm.qn[lane] : 1.f;
        sm.bg[lane] = sm.bt[lane] * ex * kn;
        float* wg = reinterpret_cast<float*>(wsc + kWsG);
        store_dev(wg + lane, ex * qn);
        store_dev(wg + kC + lane, __expf(xc - x) * kn);
        store_dev(wg + 2 * kC + lane, lane == 0 ? __expf(xc) : 0.f);
        store_dev(wg + 3 * kC + lane, 0.f);
    }
    lds_barrier();
    if (wave == 0) {  // the four 16x16 diagonal blocks, one column per lane
        const int bi = lane >> 4, cj = lane & 15;
        float x[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float acc = (t == cj) ? 1.f : 0.f;
#pragma unroll
            for (int s = 0; s < t; ++s) acc = fmaf(-sm.x.s.A[tri_off(16 * bi + t, 16 * bi + s)], x[s], acc);
            x[t] = acc;
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) sm.x.s.Tm[tri_off(16 * bi + t, 16 * bi + cj)] = x[t];
    }
    lds_barrier();
    if (wave < 3) {  // block column j = wave: T_ij = -T_ii X, X = sum_{k=j}^{i-1} A_ik T_kj, i > j
        // 16x16x16 fp32 block products on v_mfma_f32_16x16x4_f32 (lane l: A[l%16][l/16],
        // B[l/16][l%16], D[4*(l/16) + r][l%16]); the diagonal blocks hold zeros above the
        // diagonal, so no masking is needed.  X stays in registers: register s of lane l
        // holds X[4*(l/16) + s][l%16], which is the B operand of k-step s when the A operand
        // supplies column 4*(l/16) + s of T_ii.
        const int j = wave, r16 = lane & 15, k4 = lane >> 4;
        for (int i = j + 1; i < 4; ++i) {
            float4_t x = {};
            for (int kb = j; kb < i; ++kb)
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4)
                    x = mfma16f32(sm.x.s.A[tri_off(16 * i + r16, 16 * kb + 4 * s4 + k4)],
                                  sm.x.s.Tm[tri_off(16 * kb + 4 * s4 + k4, 16 * j + r16)], x);
            float4_t t = {};
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
                t = mfma16f32(sm.x.s.Tm[tri_off(16 * i + r16, 16 * i + 4 * k4 + s4)], x[s4], t);
#pragma unroll
            for (int r = 0; r < 4; ++r) sm.x.s.Tm[tri_off(16 * i + 4 * k4 + r, 16 * j + r16)] = -t[r];
            wave_lds_sync();
        }
    }
    lds_barrier();

    // ---- 4. W = Tm diag(beta e^G) K and U = Tm diag(beta) V.  The Tm rows become fp16 A
    // operands in registers; W's products run first, while Tm is still in LDS, then U's
    // operand is taken as an exact pair of fp16 halves (hi + lo, two MFMAs per step) and V
    // goes to LDS over A / Tm.  U is kept in fp32 (stored so): rounding its operand or its
    // value to fp16 were each ~3e-4 of relative state error at T = 4096 ----
    float16_t u_acc[2];
    {
        const int trow = 32 * mt + (lane & 31);
        const int g16 = lane >> 4;
        const int nks = mt == 0 ? 2 : 4;  // Tm[t < 32][s >= 32] = 0
        // the 8 Tm values of this lane's operand slots at k-step ks, zero above the diagonal
        auto tm_row = [&](int ks, float (&x)[8]) {
            // block (trow/16, ks) lies above the diagonal for ks > trow/16: Tm is zero there
            // and the masked read below goes to a stored block instead
            const int base = tri_off(trow, 16 * min(ks, trow >> 4) + 8 * hi);
            const float4 t0v = *reinterpret_cast<const float4*>(&sm.x.s.Tm[base]);
            const float4 t1v = *reinterpret_cast<const float4*>(&sm.x.s.Tm[base ^ 4]);
            const float tv[8] = {t0v.x, t0v.y, t0v.z, t0v.w, t1v.x, t1v.y, t1v.z, t1v.w};
#pragma unroll
            for (int qd = 0; qd < 8; ++qd) x[qd] = (16 * ks + 8 * hi + qd <= trow) ? tv[qd] : 0.f;
        };
        {
            // With fp32 I/O, W's A operand Tm diag(beta e^G) is taken as an exact pair of fp16
            // halves (two MFMAs per step): with the carry's W S state operand also split, the
            // state error of a slowly decaying gate halves (numpy model: 4.6e-5 -> 2.2e-5 at
            // T = 2048).  The fp16-I/O path keeps one operand: the pair cost 3 % of a call at
            // 32 heads, T = 4096 (A/B on one box).  One output tile at a time, its Tm operands
            // re-read per tile: two accumulators and a second operand would not fit the 128
            // registers of four workgroups per CU.
            float16_t w_acc[2];
#pragma unroll
            for (int n2 = 0; n2 < 2; ++n2) {
                const int ntw = 2 * (wave & 1) + n2;
                w_acc[n2] = float16_t{};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    if (ks >= nks) break;
                    float x[8];
                    tm_row(ks, x);
                    half8_t awh, awl;
#pragma unroll
                    for (int qd = 0; qd < 8; ++qd) {
                        const float y = x[qd] * sm.bg[16 * ks + 8 * hi + qd];
                        awh[qd] = (half_t)y;
                        awl[qd] = (half_t)(y - (float)awh[qd]);
                    }
                    const int row0 = 16 * ks + 8 * hi;
                    const int col0 = 32 * ntw + 16 * (g16 & 1);
                    const half8_t bk = cat8(tile_read_tr(sm.K, row0, col0), tile_read_tr(sm.K, row0 + 4, col0));
                    w_acc[n2] = mfma32(awh, bk, w_acc[n2]);
                    if (kF32) w_acc[n2] = mfma32(awl, bk, w_acc[n2]);
                }
            }
            lds_barrier();  // every wave's K reads done: W is staged over K
#pragma unroll
            for (int n2 = 0; n2 < 2; ++n2) {
                const int cp = perm32(32 * (2 * (wave & 1) + n2) + (lane & 31));
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int t = 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
                    sm.K[t * kD + cp] = (half_t)w_acc[n2][r];
                }
            }
        }
        half8_t au[4], al[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks >= nks) break;
            float x[8];
            tm_row(ks, x);
#pragma unroll
            for (int qd = 0; qd < 8; ++qd) {
                const float y = x[qd] * sm.bt[16 * ks + 8 * hi + qd];
                au[ks][qd] = (half_t)y;
                al[ks][qd] = (half_t)(y - (float)au[ks][qd]);
            }
        }
        lds_barrier();
#pragma unroll
        for (int it = 0; it < 4; ++it) {  // V rows past T (loaded from the last row) are zero
            const int id = it * kThreads + tid;
            const bool past = t0 + (id >> 4) > lastt;
            *reinterpret_cast<uint4*>(sm.x.V + tile_off(id >> 4, id & 15)) = past ? make_uint4(0, 0, 0, 0) : vreg[it];
            if (kF32)
                *reinterpret_cast<uint4*>(vlo_lds + tile_off(id >> 4, id & 15)) = past ? make_uint4(0, 0, 0, 0) : vlo[it];
        }
        lds_barrier();
#pragma unroll
        for (int n2 = 0; n2 < 2; ++n2) {
            const int ntw = 2 * (wave & 1) + n2;
            u_acc[n2] = float16_t{};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if (ks >= nks) break;
                const int row0 = 16 * ks + 8 * hi;
                const int col0 = 32 * ntw + 16 * (g16 & 1);
                const half8_t bv = cat8(tile_read_tr(sm.x.V, row0, col0), tile_read_tr(sm.x.V, row0 + 4, col0));
                u_acc[n2] = mfma32(au[ks], bv, u_acc[n2]);
                u_acc[n2] = mfma32(al[ks], bv, u_acc[n2]);
                if (kF32) {  // the low half of the fp32 V (lo x lo is below fp32 rounding)
                    const half8_t bvl = cat8(tile_read_tr(vlo_lds, row0, col0), tile_read_tr(vlo_lds, row0 + 4, col0));
                    u_acc[n2] = mfma32(au[ks], bvl, u_acc[n2]);
                }
            }
        }
    }

    // ---- 5. U stored from registers in fp32 (registers 4a..4a+3 are tokens t0..t0+3 of one
    // column: one 16-byte slot of the carry's layout); W from its staging, 16-byte stores ----
#pragma unroll
    for (int n2 = 0; n2 < 2; ++n2) {
        const int col = 32 * (2 * (wave & 1) + n2) + (lane & 31);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const int t0 = 32 * mt + 8 * a + 4 * hi;
            const int slot = ((col >> 4) * 4 + (t0 >> 4)) * 64 + ((t0 >> 2) & 3) * 16 + (col & 15);
            store_dev(wsc + kWsU + (size_t)slot * 16,
                      make_uint4(__float_as_uint(u_acc[n2][4 * a]), __float_as_uint(u_acc[n2][4 * a + 1]),
                                 __float_as_uint(u_acc[n2][4 * a + 2]), __float_as_uint(u_acc[n2][4 * a + 3])));
        }
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int id = it * kThreads + tid;
        store_dev(wsc + kWsW + (size_t)id * 16, *reinterpret_cast<const uint4*>(sm.K + id * 8));
    }

    // ---- 6. publish (beside the carry only): every wave's device-scope stores complete, then
    // the chunk's flag.  In order the kernel boundary orders the stores before the carry, so
    // the workgroup ends without waiting for them ----
    if (flags) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (tid == 0)
            __hip_atomic_store(flags + (size_t)bh * nch + ch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ----------------------------------------------------------------------------------
// Carry
// ----------------------------------------------------------------------------------
struct ChainSlot {                   // operands of the loop-carried part of one chunk
    half_t K[kC * kD];               // K rows, swizzled (read transposed by the update)
    half_t W[kC * kD];               // W rows (perm32 columns), swizzled
    float U[kStrips * 4 * 64 * 4];   // this workgroup's two U strips (fp32), accumulator order
    float E[kC];                     // e^{G_t} qn_t (the output's factor; unused here)
    float Dg[kC];                    // e^{G_63 - G_t} kn_t
    float Ec[2 * kC];                // e^{G_63} (the chunk's decay), then zeros
};
struct OutSlot {                     // operands of the output of one chunk
    half_t Q[kC * kD];               // Q rows, swizzled
    half_t A[kC * kC];               // Aqk rows (perm32 columns), 8-chunk swizzle
    float E[kC];                     // e^{G_t} qn_t (followed in the workspace by e^{G_63 - G_t} kn_t)
    float Dg[kC];
};
struct CarryLds {
    ChainSlot cs[2];
    OutSlot os[2];
    uint4 XS[2][kStrips][6][64];     // chain -> output: S operands (4) and Vnew operands (2)
    half_t OS[2][32 * 32];           // per output wave: its 32 tokens x 32 columns of O
    int err[4];                      // per DMA wave: a ready wait timed out
};

// 16-B chunk swizzle of the [64][64] Aqk tile: 16 consecutive rows at one chunk are
// conflict free (two rows share a 256-B bank period).
__device__ __forceinline__ int aqk_off(int r, int c) {
    return r * kC + ((c ^ ((r >> 1) & 7)) << 3);
}

typedef __attribute__((address_space(3))) void* lds_void_t;

// Per-chunk copies into LDS: 66 one-KiB LDS-DMA instructions (global_load_lds_dwordx4,
// lane l copies 16 bytes to M0 + 16*l).  Instruction n < 41 fills the chain slot at byte
// 1024*n (K tile n < 16, W tile, fp32 U strips 32..39, decay block 40); n >= 41 fills the out
// slot at byte 1024*(n-41) (Q tile, Aqk tile, E/Dg 65).  The structs' members are laid out in that
// order so that the LDS offset is just 1024 * tile index.  The four DMA waves (4-7) take
// n = w + 4j; each lane's source offset for its instructions is fixed for the whole loop
// and computed once, so an instruction costs a scalar M0 write and the DMA itself.
constexpr int kDmaN = 66, kDmaChain = 41;
constexpr int kDmaEOut = 65;  // a 512-byte copy: lanes 0-31 only
// With fp32 I/O the output waves load their operands from memory into registers and the out
// slots hold instead the low halves of the chain chunk's K rows (K_lo, 16 KiB): instructions
// 41 .. 56 copy them, swizzled like K, from the chunk's workspace.
constexpr int kDmaNF32 = kDmaChain + 16;
template <bool kF32> constexpr int dma_n() { return kF32 ? kDmaNF32 : kDmaN; }
__device__ __forceinline__ unsigned dma_src_off_klo(int i, int lane) {
    const int P = i * 64 + lane, row = P >> 4, cch = (P & 15) ^ swz(row);
    return kWsKlo + row * kD * 2 + cch * 16;
}

// Source byte offset of instruction n for this lane, from the instruction's base pointer:
// the row base of the chunk's first token (K / Q tiles, rows at rowbytes apart, rows
// past `lastrow` clamped to it: they only meet zero coefficients) or the chunk's workspace.
__device__ __forceinline__ unsigned dma_src_off(int n, int lane, unsigned rowbytes, int pair, int lastrow) {
    const int i = n < kDmaChain ? n : n - kDmaChain;
    const bool chainslot = n < kDmaChain;
    if (i < 16) {                                    // K or Q rows, swizzled 16-B chunks
        const int P = i * 64 + lane, row = P >> 4, cch = (P & 15) ^ swz(row);
        return (unsigned)min(row, lastrow) * rowbytes + cch * 16;
    }
    if (chainslot) {
        if (i < 32) {                                // W rows, swizzled
            const int P = (i - 16) * 64 + lane, row = P >> 4, cch = (P & 15) ^ swz(row);
            return kWsW + (row * kD + cch * 8) * 2;
        }
        if (i < 40) return kWsU + pair * 8192 + (i - 32) * 1024 + lane * 16;  // own U strips
        return kWsG + lane * 16;                     // the whole 1-KiB decay block
    }
    if (i < 24) {                                    // Aqk rows, 8-chunk swizzle
        const int P = (i - 16) * 64 + lane, row = P >> 3, cch = (P & 7) ^ ((row >> 1) & 7);
        return kWsAqk + (row * kC + cch * 8) * 2;
    }
    return kWsG + (lane & 31) * 16;
}

// Issue instruction n: src = base + off (saddr form: 64-bit base in SGPRs, 32-bit VGPR
// offset).  Written as inline asm on purpose: the compiler does not track LDS written by
// DMA slot by slot and would wait for every DMA in flight before the first LDS read of the
// other slot; the kernel orders the copies and the reads itself (dma_wait_barrier).
// Workspace tiles (dev) are device-scope loads (sc1), the counterpart of the prep's stores.
__device__ __forceinline__ void dma_issue(const void* base, unsigned off, unsigned lds_addr, bool half,
                                          bool dev) {
    if (!half || (threadIdx.x & 63) < 32) {
        if (dev)
            asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 sc1" :: "v"(off), "s"(base),
                         "{m0}"(lds_addr) : "memory");
        else
            asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(off), "s"(base),
                         "{m0}"(lds_addr) : "memory");
    }
}

// Wait for this wave's copies (vmcnt counts them), then a barrier over LDS: after it every
// wave sees every wave's copies.
__device__ __forceinline__ void dma_wait_barrier() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt left at their maxima
    lds_barrier();
}

// The loop of DMA wave W (0..3): instruction n = W + 4j is a constant in each unrolled
// step, so its kind, base pointer and LDS address fold.  Iteration it copies the chain
// operands of chunk it+1 into cs[(it+1)&1] and the output operands of chunk it into
// os[it&1] (the prologue: chunk 0 into cs[0]), then waits for them and meets the barrier.
// A chunk that ends past T recomputes its K / Q offsets with clamped rows.
// kh / qh: the K / Q rows of chunk 0 (the inputs' rows, or with kF32 the fp16 copies in the
// workspace, which the prep writes in this call and are therefore read device-scope), with
// rowbytes between rows and chunk_bytes between chunks.
template <int W, bool kF32>
__device__ __forceinline__ void dma_role(const unsigned (&slot_lds)[4], const unsigned char* kh,
                                         const unsigned char* qh, const unsigned char* wsh,
                                         const unsigned* fl, unsigned wait_ticks,
                                         int* err, unsigned rowbytes, size_t chunk_bytes, int pair,
                                         int T, int nch) {
    constexpr int kJ = (dma_n<kF32>() - W + 3) / 4;
    const int lane = threadIdx.x & 63;
    unsigned off[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const int n = W + 4 * j;
        off[j] = kF32 && n >= kDmaChain ? dma_src_off_klo(n - kDmaChain, lane)
                                        : dma_src_off(n, lane, rowbytes, pair, kC - 1);
    }
    // slot_lds: cs[0], cs[1], os[0], os[1]
    auto copies = [&](int pc, int po, int cn, int co) {
        const bool do_c = cn < nch, do_o = co >= 0 && co < nch;
        const int last_c = min(kC - 1, T - 1 - cn * kC), last_o = min(kC - 1, T - 1 - co * kC);
        const unsigned char* kb = kh + (size_t)cn * chunk_bytes;
        const unsigned char* wc = wsh + (size_t)cn * ws_chunk<kF32>();
        const unsigned char* qb = qh + (size_t)co * chunk_bytes;
        const unsigned char* wo = wsh + (size_t)co * ws_chunk<kF32>();
        auto issue_all = [&](auto Ragged) {
#pragma unroll
            for (int j = 0; j < kJ; ++j) {
                const int n = W + 4 * j;
                const bool chainslot = n < kDmaChain;
                const int i = chainslot ? n : n - kDmaChain;
                if (kF32 && !chainslot) {  // K_lo rows of the chain chunk, into its parity's out slot
                    if (do_c) dma_issue(wc, off[j], slot_lds[2 + pc] + 1024u * i, false, true);
                    continue;
                }
                const bool rows = i < 16;
                if (chainslot ? !do_c : !do_o) continue;
                unsigned o = off[j];
                if (decltype(Ragged)::value && rows)
                    o = dma_src_off(n, lane, rowbytes, pair, chainslot ? last_c : last_o);
                const unsigned char* base = chainslot ? (rows ? kb : wc) : (rows ? qb : wo);
                const unsigned lds = (chainslot ? slot_lds[pc] : slot_lds[2 + po]) + 1024u * i;
                dma_issue(base, o, lds, n == kDmaEOut, kF32 || !rows);
            }
        };
        if ((do_c && last_c < kC - 1) || (do_o && last_o < kC - 1))
            issue_all(std::true_type{});
        else
            issue_all(std::false_type{});
    };
    // fl[n] is chunk n's flag (device-scope loads, like the workspace copies that follow
    // it).  The flag of the next chunk is loaded right after a chunk's copies are issued, so
    // its round trip overlaps them and a chunk that is ready costs no wait.  After one
    // timed-out wait, no more waits (the workgroup's results are then discarded).
    auto peek = [&](int n) -> unsigned {
        if (!fl) return 1u;  // in order after the prep: every chunk is ready
        return n < nch ? __hip_atomic_load(fl + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    };
    // real-time counter (100 MHz), low 32 bits; readfirstlane keeps the wait loop uniform
    auto now = []() { return __builtin_amdgcn_readfirstlane((unsigned)__builtin_amdgcn_s_memrealtime()); };
    auto ready = [&](int n, unsigned v) {
        v = __builtin_amdgcn_readfirstlane(v);
        if (v != 0u || *err) return;
        const unsigned t0 = now();
        while (v == 0u) {
            if (now() - t0 >= wait_ticks) {
                *err = 1;
                return;
            }
            __builtin_amdgcn_s_sleep(8);
            v = __builtin_amdgcn_readfirstlane(
                __hip_atomic_load(fl + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
    };
    *err = 0;
    ready(0, peek(0));
    copies(0, 0, 0, -1);
    unsigned nxt = peek(1);
    dma_wait_barrier();
    for (int it = 0; it <= nch; it += 2) {
        if (it + 1 < nch) ready(it + 1, nxt);
        copies(1, 0, it + 1, it);
        nxt = peek(it + 2);
        dma_wait_barrier();
        if (it + 1 > nch) break;
        if (it + 2 < nch) ready(it + 2, nxt);
        copies(0, 1, it + 2, it + 1);
        nxt = peek(it + 3);
        dma_wait_barrier();
    }
}


// Per-lane LDS offsets (in halfs, within a tile) of the chain step's operand reads.  The
// swizzle makes them lane-dependent, but row-tile and slot steps are constant, so with
// these bases every read in the loop is a base register plus an immediate.
struct ChainOffs {
    int w[4];   // W operand, k-step kk, row tile 0 (row tile mt adds 16 * mt * kD)
    int k[8];   // K^T operand, row tile m of S, token rows 4g.. (token block ks adds 32*ks*kD)
};
__device__ __forceinline__ ChainOffs chain_offs() {
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15, i16 = lane & 15;
    ChainOffs o;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) o.w[kk] = tile_off(c, 4 * kk + g);
    const int r = 4 * g + (i16 >> 2);  // token row this lane supplies to the transposed read
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int col = 16 * m + 4 * (i16 & 3);
        o.k[m] = tile_off(r, col >> 3) + (col & 7);
    }
    return o;
}

// Chain step for one chunk: strip S (fp32 accumulators) <- next state, and the S / Vnew
// operands handed to the output waves in XS.  Every LDS read of the step (W and K^T
// operands, U, decay factors) depends only on the chunk's slot, so all of them are issued
// before the first MFMA and a scheduling barrier keeps them there: the MFMAs then find
// their operands arriving in order instead of waiting on each small batch.
// us: 1, or 0 for a transition map's chain (U = 0).
// kLo (fp32 I/O): klo is the chunk's K_lo tile, and the update takes K as an exact hi + lo
// pair (rounding the fp32 K to one fp16 operand there was ~2.3e-4 of relative state error on
// the reference's own inputs, numpy model); W S takes the state as hi + lo too (see below).
template <bool kLo>
__device__ __forceinline__ void chain_step(float4_t (&S)[8], const ChainSlot& cs, uint4* xs, int sl,
                                           const ChainOffs& off, float us, const half_t* klo) {
    const int lane = threadIdx.x & 63, g = lane >> 4;
    half8_t aW[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            aW[mt][kk] = *reinterpret_cast<const half8_t*>(cs.W + off.w[kk] + 16 * mt * kD);
    float4 u[4], d4[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        u[mt] = *reinterpret_cast<const float4*>(cs.U + ((sl * 4 + mt) * 64 + lane) * 4);
        d4[mt] = *reinterpret_cast<const float4*>(cs.Dg + 16 * mt + 4 * g);
    }
    const float eGC = cs.Ec[0];
    // K^T operands of the state update, read transposed
    half8_t aK[8][2];
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            aK[m][ks] = cat8(lds_read_tr16(cs.K + off.k[m] + 32 * ks * kD),
                             lds_read_tr16(cs.K + off.k[m] + (32 * ks + 16) * kD));
    __builtin_amdgcn_sched_barrier(0);

    half8_t Sb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        Sb[kk] = half8_t{(half_t)S[2 * kk][0], (half_t)S[2 * kk][1], (half_t)S[2 * kk][2], (half_t)S[2 * kk][3],
                         (half_t)S[2 * kk + 1][0], (half_t)S[2 * kk + 1][1], (half_t)S[2 * kk + 1][2], (half_t)S[2 * kk + 1][3]};
    // W S, the four row-tile chains interleaved.  With fp32 I/O (kLo) the state operand is an
    // exact pair of fp16 halves (hi + lo, a second MFMA per step reusing the W operand; with W's
    // own A operand split in the prep, the state error of a slowly decaying gate halves, numpy
    // model); the low halves are formed one k-step at a time, next to their MFMAs.  The fp16-I/O
    // path keeps one operand: the pair put 16 MFMAs on the chunk step's dependency chain
    // (+16 % per call at 32 heads, T = 4096, A/B on one box).
    float4_t wsv[4] = {float4_t{}, float4_t{}, float4_t{}, float4_t{}};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        half8_t Sl;
        if (kLo) {
#pragma unroll
            for (int e = 0; e < 8; ++e) Sl[e] = (half_t)(S[2 * kk + (e >> 2)][e & 3] - (float)Sb[kk][e]);
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            wsv[mt] = mfma16(aW[mt][kk], Sb[kk], wsv[mt]);
            if (kLo) wsv[mt] = mfma16(aW[mt][kk], Sl, wsv[mt]);
        }
    }
    // Vnew = U - W S (lane: column c, tokens 16mt + 4g + r); Vs = Vnew e^{G_C - G_t} as an
    // exact pair of fp16 halves (hi + lo): its rounding to one fp16 operand was ~3e-4 of
    // relative state error at T = 4096; the second MFMA per step reuses the K^T operand
    half8_t Vn[2], Vs[2], Vl[2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const float uu[4] = {u[mt].x, u[mt].y, u[mt].z, u[mt].w};
        const float dg[4] = {d4[mt].x, d4[mt].y, d4[mt].z, d4[mt].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float vn = fmaf(uu[r], us, -wsv[mt][r]);
            Vn[mt >> 1][4 * (mt & 1) + r] = (half_t)vn;
            const float vs = vn * dg[r];
            const half_t vh = (half_t)vs;
            Vs[mt >> 1][4 * (mt & 1) + r] = vh;
            Vl[mt >> 1][4 * (mt & 1) + r] = (half_t)(vs - (float)vh);
        }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xs[kk * 64 + lane] = __builtin_bit_cast(uint4, Sb[kk]);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) xs[(4 + ks) * 64 + lane] = __builtin_bit_cast(uint4, Vn[ks]);
    // S = e^{G_C} S + K^T (Vs hi + Vs lo)
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        S[m] *= eGC;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            S[m] = mfma16(aK[m][ks], Vs[ks], S[m]);
            S[m] = mfma16(aK[m][ks], Vl[ks], S[m]);
        }
    }
    // + K_lo^T Vs hi, one row tile's operands read at a time (the registers of the hoisted K^T
    // reads above are all in use)
    if (kLo) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8_t aKl = cat8(lds_read_tr16(klo + off.k[m] + 32 * ks * kD),
                                         lds_read_tr16(klo + off.k[m] + (32 * ks + 16) * kD));
                S[m] = mfma16(aKl, Vs[ks], S[m]);
            }
        }
    }
}

// A operands of one output wave's chunk: Q (token tiles 2w, 2w+1, in the state operand's
// k order), Aqk (perm32 columns) and the factors e^{G_t} qn_t of its D rows.
struct OutOps {
    half8_t aQ[2][4], aA[2][2];
    float4 eg[2];
};
// from the chunk's out slot in LDS (fp16 I/O)
__device__ __forceinline__ OutOps out_ops_lds(const OutSlot& os, int w) {
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    OutOps op;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = 16 * (2 * w + j) + c;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const half4_t lo = *reinterpret_cast<const half4_t*>(
                os.Q + t * kD + (((4 * kk + (g >> 1)) ^ swz(t)) << 3) + 4 * (g & 1));
            const half4_t up = *reinterpret_cast<const half4_t*>(
                os.Q + t * kD + (((4 * kk + 2 + (g >> 1)) ^ swz(t)) << 3) + 4 * (g & 1));
            op.aQ[j][kk] = cat8(lo, up);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            op.aA[j][ks] = *reinterpret_cast<const half8_t*>(os.A + aqk_off(t, 4 * ks + g));
        op.eg[j] = *reinterpret_cast<const float4*>(os.E + 16 * (2 * w + j) + 4 * g);
    }
    return op;
}
// from the chunk's workspace (fp32 I/O: the prep's fp16 Q rows, unswizzled)
__device__ __forceinline__ OutOps out_ops_mem(const unsigned char* wsc, int w) {
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const half_t* Q = reinterpret_cast<const half_t*>(wsc + kWsQ);
    const half_t* A = reinterpret_cast<const half_t*>(wsc + kWsAqk);
    const float* E = reinterpret_cast<const float*>(wsc + kWsG);
    OutOps op;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = 16 * (2 * w + j) + c;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            op.aQ[j][kk] = cat8(*reinterpret_cast<const half4_t*>(Q + t * kD + 32 * kk + 4 * g),
                                *reinterpret_cast<const half4_t*>(Q + t * kD + 32 * kk + 16 + 4 * g));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            op.aA[j][ks] = *reinterpret_cast<const half8_t*>(A + t * kC + 8 * (4 * ks + g));
        op.eg[j] = *reinterpret_cast<const float4*>(E + 16 * (2 * w + j) + 4 * g);
    }
    return op;
}

// Output for one chunk, token tiles {2w, 2w+1} of both strips: O = scale (e^G Q S + Aqk Vnew).
// With TIO = float the values go straight to the fp32 output (o32: this wave's first token
// row of the chunk and the workgroup's first column; rows past T are skipped) instead of
// through the fp16 staging tile.
template <typename TIO>
__device__ __forceinline__ void out_step(const OutOps& op, const uint4 (*xs)[6][64], half_t* ostage,
                                         int w, float scale, float* o32, size_t o32_row, int rows_left) {
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    float eg[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        eg[j][0] = op.eg[j].x; eg[j][1] = op.eg[j].y; eg[j][2] = op.eg[j].z; eg[j][3] = op.eg[j].w;
    }
    half8_t Sb[kStrips][4], Vn[kStrips][2];
#pragma unroll
    for (int s = 0; s < kStrips; ++s) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) Sb[s][kk] = __builtin_bit_cast(half8_t, xs[s][kk][lane]);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) Vn[s][ks] = __builtin_bit_cast(half8_t, xs[s][4 + ks][lane]);
    }
    __builtin_amdgcn_sched_barrier(0);  // every LDS read of the step ahead of the MFMAs
    float4_t qs[2][kStrips], av[2][kStrips];
#pragma unroll
    for (int s = 0; s < kStrips; ++s) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            qs[j][s] = float4_t{};
            av[j][s] = float4_t{};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) qs[j][s] = mfma16(op.aQ[j][kk], Sb[s][kk], qs[j][s]);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) av[j][s] = mfma16(op.aA[j][ks], Vn[s][ks], av[j][s]);
        }
    }
    if (std::is_same<TIO, float>::value) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tl = 16 * j + 4 * g + r;  // token within this wave's 32
                if (tl < rows_left)
#pragma unroll
                    for (int s = 0; s < kStrips; ++s)
                        o32[tl * o32_row + 16 * s + c] = scale * fmaf(eg[j][r], qs[j][s][r], av[j][s][r]);
            }
        return;
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
                                          int h, int t0, int pair, int w, int Tloc) {
    const int lane = threadIdx.x & 63;
    wave_lds_sync();
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int tl = 16 * hf + (lane >> 2);  // token within this wave's 32
        const int tt = t0 + 32 * w + tl;
        const uint4 v4 = *reinterpret_cast<const uint4*>(ostage + tl * 32 + 8 * (lane & 3));
        if (tt < Tloc)
            *reinterpret_cast<uint4*>(out + (((size_t)b * T + tt) * Hv + h) * kD + pair * 32 + 8 * (lane & 3)) = v4;
    }
    wave_lds_sync();
}

// TIO: the q / k / out element type.  With fp32 I/O the K / Q rows come from the prep's fp16
// copies in the workspace and the output is stored in fp32 straight from registers.
// job: the whole sequence (kJobPlain), or one launch of the sequence split (segments of the
// workgroup's unit, its start state and where its end state goes are derived below).
template <typename TIO>
__global__ void __launch_bounds__(kCarryThreads, 1)
gdn_chunk_carry(const TIO* __restrict__ q, const TIO* __restrict__ k,
                const unsigned char* __restrict__ ws, const unsigned* __restrict__ flags,
                unsigned* __restrict__ aborts, int mode, unsigned wait_ticks,
                float* __restrict__ state,
                TIO* __restrict__ out, int T, int Hq, int Hv, int nch_all, int BHv, float scale,
                CarryJob job) {
    constexpr bool kF32 = std::is_same<TIO, float>::value;
    __shared__ CarryLds sm;
    if (mode == kCarryRetry &&
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(aborts + blockIdx.x, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT)) == 0u)
        return;  // this workgroup finished in the launch beside the prep
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: role branches are scalar
    const int g = lane >> 4, c = lane & 15;
    // block id = (unit * 4 + pair) * BHv + bh: all column pairs of one head share an XCD when
    // BHv % 8 == 0
    const int unit = blockIdx.x / (4 * BHv);
    const int pair = (blockIdx.x / BHv) & 3;
    const int bh = blockIdx.x % BHv;
    const int b = bh / Hv, h = bh % Hv, hq = h % Hq;
    const bool chain = wave < 2, outw = wave == 2 || wave == 3, dmaw = wave >= 4;
    const int sl = wave & 1;  // chain wave: its strip; output wave: w = wave - 2

    // This workgroup's chunks [c0, c0 + nch), where its state starts (src: loaded; else zero,
    // or the identity for a transition map), where it ends (dst), where its outputs go (out,
    // or a map's fp32 rows in the workspace), and the U scale (0 for a transition map).
    int seg = 0, c0 = 0, nch = nch_all;
    bool ident = false;
    float us = 1.f;
    const float* src = state;
    float* dst = state;
    float* obuf = nullptr;  // a map's fp32 output rows (from segment 1's first token), or out
    // this head's slots (no slots in the plain job)
    float* segh = job.seg ? job.seg + (size_t)bh * job.nseg * kSegSlots * kSegSlotFloats : nullptr;
    auto slot = [&](int sg, int which) { return segh + ((size_t)sg * kSegSlots + which) * kSegSlotFloats; };
    if (job.phase == kJobMaps) {
        if (unit == 0) {            // segment 0 from the caller's state; its end enters segment 1
            dst = slot(1, kSegEntry);
        } else {                    // Z or Phi of segment 1 + (unit - 1) / 2
            seg = 1 + (unit - 1) / 2;
            const bool phi = ((unit - 1) & 1) != 0;
            src = nullptr;
            ident = phi;
            us = phi ? 0.f : 1.f;
            dst = slot(seg, phi ? kSegPhi : kSegZ);
            obuf = (phi ? job.om : job.oz) + ((size_t)bh * job.Tr + (size_t)(seg - 1) * job.seg_len * kC) * kD;
        }
    }
    if (job.phase != kJobPlain) {
        c0 = seg * job.seg_len;
        nch = seg == job.nseg - 1 ? nch_all - c0 : job.seg_len;
    }
    const int Tloc = T - c0 * kC;  // tokens from this workgroup's first chunk to the end of the sequence
    const unsigned char* wsh = ws + ((size_t)bh * nch_all + c0) * ws_chunk<kF32>();

    // Pipeline, iteration it.  Chain waves: process chunk it from cs[it&1].  Output waves:
    // store the O tile of chunk it-2 staged in LDS, then compute the output of chunk it-1
    // from os[(it-1)&1] and XS[(it-1)&1].  DMA waves: copy the chain operands of chunk it+1
    // into cs[(it+1)&1] and the output operands of chunk it into os[it&1], then wait for
    // the copies.  Then the workgroup meets at a barrier.
    float4_t S[8];
    // state layout [b*Hv + h][column][dk]: this lane's column, dk rows 16m + 4g + 0..3
    const int col = (pair * kStrips + sl) * 16 + c;
    const size_t soff = ((size_t)bh * kD + col) * kD, soff_seg = (size_t)col * kD;
    const float* Sg = src == state ? state + soff : src + soff_seg;
    if (chain) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            if (src) {
                const float4 v4 = *reinterpret_cast<const float4*>(Sg + 16 * m + 4 * g);
                S[m] = float4_t{v4.x, v4.y, v4.z, v4.w};
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) S[m][r] = ident && 16 * m + 4 * g + r == col ? 1.f : 0.f;
            }
        }
    }
    if (!dmaw) dma_wait_barrier();  // matches the DMA waves' prologue barrier
    // Each role runs its own loop (one barrier per iteration in each), so no role's loop
    // state occupies registers in another role's code.  `it` runs 0..nch; the loop is
    // unrolled by two so slot indices are constants.
    if (chain) {
        const ChainOffs off = chain_offs();
        for (int it = 0; it <= nch; it += 2) {
            if (it < nch)
                chain_step<kF32>(S, sm.cs[0], &sm.XS[0][sl][0][0], sl, off, us,
                                 reinterpret_cast<const half_t*>(&sm.os[0]));
            lds_barrier();  // chain waves issue no vector memory operations in the loop
            if (it + 1 > nch) break;
            if (it + 1 < nch)
                chain_step<kF32>(S, sm.cs[1], &sm.XS[1][sl][0][0], sl, off, us,
                                 reinterpret_cast<const half_t*>(&sm.os[1]));
            lds_barrier();
        }
    } else if (outw) {
        const int w = wave - 2;
        const size_t orow = (size_t)Hv * kD;
        // rows from this workgroup's first chunk on
        half_t* out16 = reinterpret_cast<half_t*>(out) + (size_t)c0 * kC * orow;
        // fp32 output (fp32 I/O, or a map's rows in the workspace): row of token t0 + 32 w of
        // chunk ch, column pair * 32
        const bool f32out = kF32 || obuf != nullptr;  // uniform
        const size_t o32_row = obuf ? (size_t)kD : orow;
        float* o32 = obuf ? obuf + (size_t)(32 * w) * kD + pair * 32
                          : reinterpret_cast<float*>(out) + ((size_t)b * T + c0 * kC + 32 * w) * orow +
                                (size_t)h * kD + pair * 32;
        // fp32 I/O: the operands come from memory into registers, Q one chunk ahead (ops[ch & 1]
        // holds chunk ch's), Aqk and e^G at the step (two full operand sets do not fit beside
        // the chain's registers); otherwise from the chunk's out slot
        OutOps ops[2];
        if (kF32) ops[0] = out_ops_mem(wsh, w);
        auto step = [&](int slot, int ch) {
            if (kF32) {
                const OutOps nx = out_ops_mem(wsh + (size_t)min(ch + 1, nch - 1) * ws_chunk<kF32>(), w);
                if (ch + 1 < nch) {
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) ops[slot ^ 1].aQ[j][kk] = nx.aQ[j][kk];
                }
                const OutOps cu = out_ops_mem(wsh + (size_t)ch * ws_chunk<kF32>(), w);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) ops[slot].aA[j][ks] = cu.aA[j][ks];
                    ops[slot].eg[j] = cu.eg[j];
                }
            } else {
                ops[slot] = out_ops_lds(sm.os[slot], w);
            }
            if (f32out)
                out_step<float>(ops[slot], sm.XS[slot], sm.OS[w], w, scale, o32 + (size_t)ch * kC * o32_row,
                                o32_row, Tloc - ch * kC - 32 * w);
            else
                out_step<TIO>(ops[slot], sm.XS[slot], sm.OS[w], w, scale, o32, o32_row, 0);
        };
        for (int it = 0; it <= nch; it += 2) {
            if (!f32out && it >= 2) out_flush(sm.OS[w], out16, b, T, Hv, h, (it - 2) * kC, pair, w, Tloc);
            if (it >= 1) step(1, it - 1);
            lds_barrier();  // the O stores need not complete before the barrier
            if (it + 1 > nch) break;
            if (!f32out && it >= 1) out_flush(sm.OS[w], out16, b, T, Hv, h, (it - 1) * kC, pair, w, Tloc);
            step(0, it);
            lds_barrier();
        }
    } else {
        // the inputs' K / Q rows, or with fp32 I/O the prep's fp16 copies in the workspace
        const unsigned rowbytes = kF32 ? (unsigned)kD * 2 : (unsigned)Hq * kD * 2;
        const size_t chunk_bytes = kF32 ? (size_t)kWsChunkF32 : (size_t)kC * rowbytes;
        const unsigned char* kh = kF32 ? wsh + kWsK
                                       : reinterpret_cast<const unsigned char*>(k + ((size_t)b * T * Hq + hq) * kD) +
                                             (size_t)c0 * chunk_bytes;
        const unsigned char* qh = kF32 ? wsh + kWsQ
                                       : reinterpret_cast<const unsigned char*>(q + ((size_t)b * T * Hq + hq) * kD) +
                                             (size_t)c0 * chunk_bytes;
        const unsigned slot_lds[4] = {(unsigned)(uintptr_t)(lds_void_t)(void*)&sm.cs[0],
                                      (unsigned)(uintptr_t)(lds_void_t)(void*)&sm.cs[1],
                                      (unsigned)(uintptr_t)(lds_void_t)(void*)&sm.os[0],
                                      (unsigned)(uintptr_t)(lds_void_t)(void*)&sm.os[1]};
        const unsigned* fl = flags ? flags + (size_t)bh * nch_all + c0 : nullptr;
        int* err = &sm.err[wave - 4];
        switch (wave) {
            case 4: dma_role<0, kF32>(slot_lds, kh, qh, wsh, fl, wait_ticks, err, rowbytes, chunk_bytes, pair, Tloc, nch); break;
            case 5: dma_role<1, kF32>(slot_lds, kh, qh, wsh, fl, wait_ticks, err, rowbytes, chunk_bytes, pair, Tloc, nch); break;
            case 6: dma_role<2, kF32>(slot_lds, kh, qh, wsh, fl, wait_ticks, err, rowbytes, chunk_bytes, pair, Tloc, nch); break;
            default: dma_role<3, kF32>(slot_lds, kh, qh, wsh, fl, wait_ticks, err, rowbytes, chunk_bytes, pair, Tloc, nch); break;
        }
    }
    if (chain) {
        // a timed-out wait means some chunk operands were read before they were published:
        // beside the prep, leave the state for the second launch; otherwise poison it
        const bool lost = (sm.err[0] | sm.err[1] | sm.err[2] | sm.err[3]) != 0;
        // the abort word (cleared at the start of the call) sends this workgroup into the
        // second launch
        if (mode == kCarryBeside && tid == 0 && lost)
            __hip_atomic_store(aborts + blockIdx.x, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        // in order after the prep the abort words were not cleared: the first unit's
        // workgroups zero theirs (a workgroup that runs in order never gives up)
        if (mode == kCarryInOrder && tid == 0 && blockIdx.x < 4 * BHv)
            __hip_atomic_store(aborts + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (dst && !(lost && mode == kCarryBeside)) {
            const float nan = __builtin_nanf("");
            float* Dg = dst == state ? state + soff : dst + soff_seg;
#pragma unroll
            for (int m = 0; m < 8; ++m)
                *reinterpret_cast<float4*>(Dg + 16 * m + 4 * g) =
                    lost ? make_float4(nan, nan, nan, nan) : make_float4(S[m][0], S[m][1], S[m][2], S[m][3]);
        }
    } else if (outw && !kF32 && !obuf) {
        out_flush(sm.OS[wave - 2], reinterpret_cast<half_t*>(out) + (size_t)c0 * kC * Hv * kD, b, T, Hv, h,
                  (nch - 1) * kC, pair, wave - 2, Tloc);
    }
}

// The combine of the sequence split: entry[s + 1] = Phi_s entry[s] + Z_s for s = 1 .. nseg - 1,
// in fp32; entry[nseg] is the call's final state (state, same layout).  Slots are stored [column][dk]; row j of the Phi slot is Phi's column j, so with
// E = entry[s] stored the same way, entry[s + 1][c][d] = sum_j E[c][j] Phi[j][d] + Z[c][d].
// State columns never mix: a workgroup takes R columns of one head through every step and
// waits for no other workgroup.  Only the E chain is serial: wave w sums over j in
// [32 w, 32 w + 32) with its lane's dk pair (2 lane, 2 lane + 1), holding that quarter of
// Phi_s in registers while the next step's quarter loads; the four partial sums meet in LDS.
// Every workgroup reads all of Phi_s per step whatever R is, while its FMA time grows with R:
// the host picks the smallest R that keeps about one workgroup per CU.
constexpr int kCombThreads = 256;
template <int R>
__global__ void __launch_bounds__(kCombThreads) gdn_seg_combine(float* __restrict__ seg, float* __restrict__ state,
                                                                int nseg) {
    const int bh = blockIdx.x / (kD / R), c0 = (blockIdx.x % (kD / R)) * R;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float* segh = seg + (size_t)bh * nseg * kSegSlots * kSegSlotFloats;
    auto slot = [&](int sg, int which) { return segh + ((size_t)sg * kSegSlots + which) * kSegSlotFloats; };
    constexpr int kOut = (R * kD + kCombThreads - 1) / kCombThreads;  // outputs per thread
    __shared__ __align__(16) float E[R][kD];
    __shared__ __align__(16) float part[4][R][kD];
    if (tid < R * kD / 4)
        reinterpret_cast<float4*>(&E[0][0])[tid] =
            reinterpret_cast<const float4*>(slot(1, kSegEntry) + (size_t)c0 * kD)[tid];
    auto quarter = [&](int sg, float2 (&p)[32]) {
        const float2* P = reinterpret_cast<const float2*>(slot(sg, kSegPhi) + (size_t)(32 * w) * kD) + lane;
#pragma unroll
        for (int jj = 0; jj < 32; ++jj) p[jj] = P[jj * (kD / 2)];
    };
    // this thread's outputs in the reduction: o = tid + 256 i < R * 128 is (row o / 128, dk o % 128)
    auto zload = [&](int sg, float (&z)[kOut]) {
        const float* Z = slot(sg, kSegZ) + (size_t)c0 * kD;
#pragma unroll
        for (int i = 0; i < kOut; ++i) z[i] = Z[min(tid + kCombThreads * i, R * kD - 1)];
    };
    // step sg computes with (pc, zc) while step sg + 1's quarter loads into (pn, zn); the loop
    // is unrolled by two so the two register sets swap roles without copies
    auto step = [&](int sg, const float2 (&pc)[32], const float (&zc)[kOut], float2 (&pn)[32], float (&zn)[kOut]) {
        // unconditional (the last step reloads its own slot): a branch around the loads would
        // make the compiler wait for them where the paths join
        const int nx = min(sg + 1, nseg - 1);
        quarter(nx, pn);
        zload(nx, zn);
        float2 acc[R] = {};
#pragma unroll
        for (int jj = 0; jj < 32; jj += 4) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float4 e = *reinterpret_cast<const float4*>(&E[r][32 * w + jj]);
                acc[r].x = fmaf(e.x, pc[jj].x, acc[r].x);
                acc[r].y = fmaf(e.x, pc[jj].y, acc[r].y);
                acc[r].x = fmaf(e.y, pc[jj + 1].x, acc[r].x);
                acc[r].y = fmaf(e.y, pc[jj + 1].y, acc[r].y);
                acc[r].x = fmaf(e.z, pc[jj + 2].x, acc[r].x);
                acc[r].y = fmaf(e.z, pc[jj + 2].y, acc[r].y);
                acc[r].x = fmaf(e.w, pc[jj + 3].x, acc[r].x);
                acc[r].y = fmaf(e.w, pc[jj + 3].y, acc[r].y);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) *reinterpret_cast<float2*>(&part[w][r][2 * lane]) = acc[r];
        __syncthreads();  // partial sums written, E read by every wave
        float* en = (sg + 1 < nseg ? slot(sg + 1, kSegEntry) : state + (size_t)bh * kSegSlotFloats) + (size_t)c0 * kD;
#pragma unroll
        for (int i = 0; i < kOut; ++i) {
            const int o = tid + kCombThreads * i, r = o / kD, d = o % kD;
            if (o < R * kD) {
                const float v = zc[i] + part[0][r][d] + part[1][r][d] + part[2][r][d] + part[3][r][d];
                E[r][d] = v;
                en[o] = v;
            }
        }
        __syncthreads();
    };
    float2 pa[32], pb[32];
    float za[kOut], zb[kOut];
    quarter(1, pa);
    zload(1, za);
    __syncthreads();
    for (int sg = 1; sg < nseg; sg += 2) {
        step(sg, pa, za, pb, zb);
        if (sg + 1 >= nseg) break;
        step(sg + 1, pb, zb, pa, za);
    }
}

// The fixup of the sequence split: O = O_Z + M E^T for the tokens of segments 1 .. nseg-1,
// every chunk in parallel (a workgroup per (b, h, chunk)).  M [token][dk] and O_Z
// [token][column] are the map chains' fp32 outputs (scale included), E [column][dk] the
// entry state of the chunk's segment.  The product runs on fp16 MFMAs with each fp32 operand
// as an exact hi + lo pair (hi hi + hi lo + lo hi).  E goes to LDS as the B operands' hi and lo
// halves, rows padded to kFixRow halfs so that the 16 rows one read touches fall in different
// banks; wave w takes tokens 16 (w % 4) .. + 15 of the chunk and columns 64 (w / 4) .. + 63.
constexpr int kFixRow = kD + 8;
constexpr int kFixThreads = 512;
template <typename TIO>
__global__ void __launch_bounds__(kFixThreads)
gdn_seg_fixup(const float* __restrict__ seg, const float* __restrict__ oz, const float* __restrict__ om,
              TIO* __restrict__ out, int T, int Hv, int nseg, int seg_len, int Tr, int nfix) {
    const int bh = blockIdx.x / nfix, cl = blockIdx.x % nfix;  // cl: chunk counted from segment 1's start
    const int b = bh / Hv, h = bh % Hv;
    const int sg = min(seg_len + cl, nseg * seg_len - 1) / seg_len;  // the chunk's segment (1 .. nseg-1)
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int w = (tid >> 6) & 3, n0 = 4 * (tid >> 8);  // token block; first 16-column tile
    __shared__ __align__(16) half_t Eh[kD * kFixRow];
    __shared__ __align__(16) half_t El[kD * kFixRow];
    // Every global load is issued before any is used (E's 16 float4s per thread, this lane's
    // M row, its 16 O_Z values), from clamped addresses, and only the stores are guarded: a
    // load behind a branch, or one per loop trip between LDS stores, waits out its own memory
    // latency.
    const float* E = seg + ((size_t)bh * nseg * kSegSlots + (size_t)sg * kSegSlots + kSegEntry) * kSegSlotFloats;
    constexpr int kEPer = kD * kD / 4 / kFixThreads;  // float4s of E per thread
    float4 ev[kEPer];
#pragma unroll
    for (int i = 0; i < kEPer; ++i) ev[i] = reinterpret_cast<const float4*>(E)[tid + kFixThreads * i];
    // A operands: this lane's token row of M (rows past T, which the buffers do not hold, read
    // the last row and are not stored), dk 32 ks + 8 g .. + 7
    const size_t base = (size_t)bh * Tr;
    const size_t ra = base + min((size_t)cl * kC + 16 * w + c, (size_t)Tr - 1);
    float4 mv[4][2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const float4* mp = reinterpret_cast<const float4*>(om + ra * kD + 32 * ks + 8 * g);
        mv[ks][0] = mp[0];
        mv[ks][1] = mp[1];
    }
    // O_Z of this lane's outputs: tokens 16 w + 4 g + r, columns 16 (n0 + nt) + c
    float zv[4][4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            zv[nt][r] = oz[(base + min((size_t)cl * kC + 16 * w + 4 * g + r, (size_t)Tr - 1)) * kD + 16 * (n0 + nt) + c];
#pragma unroll
    for (int i = 0; i < kEPer; ++i) {
        const float e4[4] = {ev[i].x, ev[i].y, ev[i].z, ev[i].w};
        half4_t hv, lv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            hv[q] = (half_t)e4[q];
            lv[q] = (half_t)(e4[q] - (float)hv[q]);
        }
        const int f = 4 * (tid + kFixThreads * i), row = f / kD, col = f % kD;
        *reinterpret_cast<half4_t*>(&Eh[row * kFixRow + col]) = hv;
        *reinterpret_cast<half4_t*>(&El[row * kFixRow + col]) = lv;
    }
    half8_t ah[4], al[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const float m8[8] = {mv[ks][0].x, mv[ks][0].y, mv[ks][0].z, mv[ks][0].w,
                             mv[ks][1].x, mv[ks][1].y, mv[ks][1].z, mv[ks][1].w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            ah[ks][q] = (half_t)m8[q];
            al[ks][q] = (half_t)(m8[q] - (float)ah[ks][q]);
        }
    }
    __syncthreads();
    const int t0 = (seg_len + cl) * kC;  // the chunk's first token
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        float4_t acc = {};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int o = (16 * (n0 + nt) + c) * kFixRow + 32 * ks + 8 * g;
            const half8_t bhv = *reinterpret_cast<const half8_t*>(&Eh[o]);
            const half8_t blv = *reinterpret_cast<const half8_t*>(&El[o]);
            acc = mfma16(ah[ks], bhv, acc);
            acc = mfma16(ah[ks], blv, acc);
            acc = mfma16(al[ks], bhv, acc);
        }
        // acc[r]: token 16 w + 4 g + r, column 16 (n0 + nt) + c
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tl = 16 * w + 4 * g + r;
            if (t0 + tl < T)
                out[(((size_t)b * T + t0 + tl) * Hv + h) * kD + 16 * (n0 + nt) + c] = (TIO)(zv[nt][r] + acc[r]);
        }
    }
}

// Clears the ready flags and abort words of a call (n words) before anything reads them.
__global__ void __launch_bounds__(256) gdn_flags_clear(unsigned* __restrict__ w, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) w[i] = 0u;
}

// A positive integer from the environment, or `def` when unset or malformed.
long env_long(const char* name, long def, long hi) {
    const char* e = std::getenv(name);
    if (!e || !*e) return def;
    char* end = nullptr;
    const long v = std::strtol(e, &end, 10);
    return (end && *end == 0 && v >= 0 && v <= hi) ? v : def;
}

// The sequence split of a call: nseg segments of seg_len chunks (nseg == 1: no split).  It pays
// where the carry's workgroups leave most CUs idle (few heads) and the chunk chain is long.
// The call's serial time is about nch / nseg chunk steps (the maps) + nseg - 1 combine steps
// (each about a chunk step) + the fixup, least near nseg = sqrt(nch); the library's plan
// (req = 0) takes the most segments up to sqrt(nch) whose maps launch ((2 nseg - 1) units of 4
// workgroups per head) fits in the 256 CUs of the part, each at least kMinSegChunks chunks
// long: a function of the shapes only, so a workspace sized once serves every call of a shape.
// An explicit request (tsa_gdn_chunked_plan_fwd) replaces it: req = 1 never splits, req >= 2
// asks for req segments (fewer if the sequence has fewer chunks: no segment is empty).
constexpr int kSplitCUs = 256;
constexpr int kMinSegChunks = 8;
struct SegPlan {
    int nseg = 1, seg_len = 0;
};
SegPlan seg_plan(int BHv, int nch, int req) {
    long n = 1;
    if (req >= 2)
        n = std::min<long>(req, nch);
    else if (req == 0 && BHv > 0)
        n = std::min<long>(std::min<long>((kSplitCUs / (4 * BHv) + 1) / 2, nch / kMinSegChunks),
                           (long)std::sqrt((double)nch));
    if (n < 2) return {};
    const int seg_len = (int)((nch + n - 1) / n);
    n = (nch + seg_len - 1) / seg_len;  // no empty segment
    if (n < 2) return {};
    return {(int)n, seg_len};
}

// Byte offset of the split's slots in the workspace: after the chunk workspaces, the ready
// flags and the abort words, rounded up to 256 B.
size_t seg_offset(size_t BHv, size_t nch, bool f32) {
    const size_t end = BHv * nch * ((f32 ? kWsChunkF32 : kWsChunk) + sizeof(unsigned)) +
                       BHv * (kD / (16 * kStrips)) * sizeof(unsigned);
    return (end + 255) & ~(size_t)255;
}
}  // namespace

namespace {
// Workspace bytes of a call under a plan: chunk workspaces, then a ready flag per chunk, then
// an abort word per carry workgroup, then, when the call splits, the slots and the maps' O_Z
// and M rows of the tokens after segment 0
size_t ws_bytes_for(size_t BHv, size_t nch, int T, bool f32, const SegPlan& plan) {
    if (plan.nseg == 1)
        return BHv * nch * ((f32 ? kWsChunkF32 : kWsChunk) + sizeof(unsigned)) +
               BHv * (kD / (16 * kStrips)) * sizeof(unsigned);
    const size_t Tr = (size_t)T - (size_t)plan.seg_len * kC;
    return seg_offset(BHv, nch, f32) + BHv * plan.nseg * kSegSlots * kSegSlotFloats * sizeof(float) +
           2 * BHv * Tr * kD * sizeof(float);
}

// The plan of a call whose workspace holds at most `budget` bytes: the split where it fits,
// else none (the no-allocation entry's fixed scratch).
SegPlan call_plan(int BHv, int nch, int T, bool f32, size_t budget, int req) {
    SegPlan plan = seg_plan(BHv, nch, req);
    if (plan.nseg > 1 && ws_bytes_for((size_t)BHv, (size_t)nch, T, f32, plan) > budget) plan = SegPlan{};
    return plan;
}
}  // namespace

size_t gdn_chunked_ws_bytes(int B, int T, int Hv, bool f32, int nseg) {
    const int nch = (T + kC - 1) / kC, BHv = B * Hv;
    return ws_bytes_for((size_t)BHv, (size_t)nch, T, f32, call_plan(BHv, nch, T, f32, SIZE_MAX, nseg));
}

namespace {

// With TSA_GDN_OVERLAP=1 the prep runs on a second stream of the device so that it overlaps
// the carry: the carry copies a chunk's operands as soon as the prep has published them
// (ready flags), and the chunk-major prep order produces them in the order the carry consumes
// them.  One side stream and its fork / join events per device, created on the first call
// that overlaps on that device and kept until the process ends.
struct SideStream {
    bool tried = false, ok = false;
    int cus = 0;
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kMaxDevices = 64;
std::mutex g_side_mu;
SideStream g_side[kMaxDevices];

// Longest wait of a carry workgroup for a chunk, in ticks of the 100 MHz real-time counter.
unsigned carry_wait_ticks() { return (unsigned)(env_long("TSA_GDN_CARRY_WAIT_US", 2000, 10000000) * 100); }

// The prep and the carry run in order on the caller's stream unless the environment variable
// TSA_GDN_OVERLAP=1 asks for the side-by-side form (the prep on a second stream, the carry
// waiting on its ready flags).  In order is the default: at 32 heads it measured as fast as
// the overlap, and it needs no side stream, events, mutex, flag clear or second carry launch.
bool overlap_requested() { return env_long("TSA_GDN_OVERLAP", 0, 1) != 0; }

template <bool kFused, typename TIO>
hipError_t launch_chunked(const void* q, const void* k, const void* v, const float* g_log,
                          const float* beta, const GdnRawGates& gates, float* state, void* out,
                          int B, int T, int Hq, int Hv, float scale, void* ws, bool may_overlap,
                          hipStream_t stream, size_t ws_budget = SIZE_MAX, int nseg = 0) {
    const int nch = (T + kC - 1) / kC;
    const int BHv = B * Hv;
    const int carry_wgs = BHv * (kD / (16 * kStrips));
    auto Q = static_cast<const TIO*>(q);
    auto K = static_cast<const TIO*>(k);
    auto W = static_cast<unsigned char*>(ws);
    unsigned* flags = reinterpret_cast<unsigned*>(W + (size_t)BHv * nch * ws_chunk<std::is_same<TIO, float>::value>());
    unsigned* aborts = flags + (size_t)BHv * nch;
    const int nflags = BHv * nch + carry_wgs;
    const unsigned wait_ticks = carry_wait_ticks();
    auto clear = [&]() {
        hipLaunchKernelGGL(gdn_flags_clear, dim3((nflags + 255) / 256), dim3(256), 0, stream, flags, nflags);
        return hipGetLastError();
    };
    // In order (the prep, then the carry, on one stream) no ready flags are written or read.
    auto prep = [&](hipStream_t st, bool publish) {
        hipLaunchKernelGGL((gdn_chunk_prep<kFused, TIO>), dim3(BHv * nch), dim3(kThreads), 0, st, Q, K,
                           static_cast<const TIO*>(v), g_log, beta, gates, W, publish ? flags : nullptr, T,
                           Hq, Hv, nch, BHv);
        return hipGetLastError();
    };
    auto carry = [&](int mode, unsigned ticks, int units = 1, CarryJob job = CarryJob{}) {
        hipLaunchKernelGGL(gdn_chunk_carry<TIO>, dim3(units * carry_wgs), dim3(kCarryThreads), 0, stream, Q, K,
                           W, mode == kCarryInOrder ? nullptr : flags, aborts, mode, ticks, state, static_cast<TIO*>(out), T, Hq, Hv, nch, BHv,
                           scale, job);
        return hipGetLastError();
    };

    // Sequence split: in order on the caller's stream (the maps need every chunk's operands)
    const SegPlan plan = call_plan(BHv, nch, T, std::is_same<TIO, float>::value, ws_budget, nseg);
    if (plan.nseg > 1) {
        CarryJob job;
        job.phase = kJobMaps;
        job.nseg = plan.nseg;
        job.seg_len = plan.seg_len;
        job.Tr = T - plan.seg_len * kC;
        job.seg = reinterpret_cast<float*>(W + seg_offset(BHv, nch, std::is_same<TIO, float>::value));
        job.oz = job.seg + (size_t)BHv * plan.nseg * kSegSlots * kSegSlotFloats;
        job.om = job.oz + (size_t)BHv * job.Tr * kD;
        hipError_t e = prep(stream, false);
        if (e == hipSuccess) e = carry(kCarryInOrder, wait_ticks, 2 * plan.nseg - 1, job);
        if (e == hipSuccess) {
            // state columns per combine workgroup: about one workgroup per CU
            const int rows = BHv <= 2 ? 1 : BHv <= 4 ? 2 : BHv <= 8 ? 4 : 8;
            auto combine = rows == 1 ? gdn_seg_combine<1> : rows == 2 ? gdn_seg_combine<2>
                         : rows == 4 ? gdn_seg_combine<4> : gdn_seg_combine<8>;
            hipLaunchKernelGGL(combine, dim3(BHv * (kD / rows)), dim3(kCombThreads), 0, stream, job.seg, state,
                               plan.nseg);
            e = hipGetLastError();
        }
        if (e == hipSuccess) {
            const int nfix = nch - plan.seg_len;
            hipLaunchKernelGGL(gdn_seg_fixup<TIO>, dim3(BHv * nfix), dim3(kFixThreads), 0, stream, job.seg, job.oz,
                               job.om, static_cast<TIO*>(out), T, Hv, plan.nseg, plan.seg_len, job.Tr, nfix);
            e = hipGetLastError();
        }
        return e;
    }

    // The default, and every call that cannot overlap: in order on the caller's stream, with no
    // other runtime call.  The overlap (TSA_GDN_OVERLAP=1) is taken only when it cannot stall:
    // the carry's workgroups (one per CU) must leave at least half the CUs to the prep, and a
    // stream being captured into a graph runs the two kernels in order (a graph does not promise
    // to run sibling nodes concurrently).  The side stream belongs to the device of the caller's
    // stream (the null stream: the current device), which need not be the current device.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusActive;
    int dev = -1;
    SideStream* side = nullptr;
    if (may_overlap && nch > 1 && overlap_requested() && hipStreamIsCapturing(stream, &cap) == hipSuccess &&
        cap == hipStreamCaptureStatusNone &&
        (stream ? hipStreamGetDevice(stream, &dev) == hipSuccess : hipGetDevice(&dev) == hipSuccess) &&
        dev >= 0 && dev < kMaxDevices) {
        std::lock_guard<std::mutex> lock(g_side_mu);
        SideStream& d = g_side[dev];
        if (!d.tried) {  // create the stream and events on that device
            d.tried = true;
            int cur = -1;
            const bool switched = hipGetDevice(&cur) == hipSuccess && cur != dev && hipSetDevice(dev) == hipSuccess;
            d.ok = (cur == dev || switched) &&
                   hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                   hipStreamCreateWithFlags(&d.s, hipStreamNonBlocking) == hipSuccess &&
                   hipEventCreateWithFlags(&d.fork, hipEventDisableTiming) == hipSuccess &&
                   hipEventCreateWithFlags(&d.join, hipEventDisableTiming) == hipSuccess;
            if (switched) (void)hipSetDevice(cur);
        }
        if (d.ok && 2 * carry_wgs <= d.cus) side = &d;
    }
    if (!side) {  // in order: no flag clear needed
        const hipError_t e = prep(stream, false);
        return e != hipSuccess ? e : carry(kCarryInOrder, wait_ticks);
    }
    hipError_t e = clear();
    if (e != hipSuccess) return e;
    // fork: the prep starts after the caller's earlier work (the flag clear included); the
    // carry is queued first so its workgroups take their CUs before the prep fills the rest.
    // join: the caller's stream waits for the prep, then the second carry launch redoes any
    // workgroup that gave up (and otherwise exits at once).  The second launch must stay
    // behind the join: under a scheduler that serialises dispatches it could otherwise run
    // before the prep and wait for flags that cannot come.
    std::lock_guard<std::mutex> lock(g_side_mu);
    e = hipEventRecord(side->fork, stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(side->s, side->fork, 0);
    if (e == hipSuccess) e = carry(kCarryBeside, wait_ticks);
    if (e == hipSuccess) e = prep(side->s, true);
    if (e == hipSuccess) e = hipEventRecord(side->join, side->s);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, side->join, 0);
    if (e == hipSuccess) e = carry(kCarryRetry, kRetryWaitTicks);
    return e;
}
}  // namespace

// ---- the no-allocation variant ----
// `scratch` stands in for the caller's workspace: a file-scope device array that each GPU the
// library runs on holds from the module's load until the process ends.  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in for the symbol):
// the device address comes from hipGetSymbolAddress, once per device, on the first call on
// that device, and is kept in g_scratch.  Every call on a GPU shares that GPU's array and
// leaves its contents behind: the call runs the prep and the carry in order, so it reads no
// ready flags, the carry zeroes the abort words, and the rest of the workspace is written
// before it is read.  Calls that overlap on one GPU race on the
// array.
constexpr size_t kScratchBytes = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

hipError_t scratch_address(hipStream_t stream, void** out) {
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {  // with that device current
        int cur = -1;
        if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return hipSuccess;
}
}  // namespace

size_t gdn_chunked_noalloc_max_bytes() { return kScratchBytes; }

// The no-allocation entry splits the sequence only where the split's workspace fits the scratch.
size_t gdn_chunked_noalloc_ws_bytes(int B, int T, int Hv) {
    const int nch = (T + kC - 1) / kC, BHv = B * Hv;
    return ws_bytes_for((size_t)BHv, (size_t)nch, T, false, call_plan(BHv, nch, T, false, kScratchBytes, 0));
}

hipError_t gdn_chunked_noalloc(const void* q, const void* k, const void* v, const float* g_log,
                               const float* beta, float* state, void* out, int B, int T, int Hq,
                               int Hv, float scale, hipStream_t stream) {
    void* ws = nullptr;
    const hipError_t e = scratch_address(stream, &ws);
    if (e != hipSuccess) return e;
    // in order on the caller's stream: no side stream or event is ever created here
    return launch_chunked<false, half_t>(q, k, v, g_log, beta, GdnRawGates{}, state, out, B, T, Hq, Hv,
                                         scale, ws, false, stream, kScratchBytes);
}

hipError_t gdn_chunked_redo_count(const void* ws, int B, int T, int Hv, bool f32, int* count,
                                  hipStream_t stream) {
    const size_t nch = (size_t)(T + kC - 1) / kC;
    const size_t n = (size_t)B * Hv * (kD / (16 * kStrips));
    const unsigned char* aborts = static_cast<const unsigned char*>(ws) +
                                  (size_t)B * Hv * nch * ((f32 ? kWsChunkF32 : kWsChunk) + sizeof(unsigned));
    unsigned* host = static_cast<unsigned*>(std::malloc(n * sizeof(unsigned)));
    if (!host) return hipErrorOutOfMemory;
    hipError_t e = hipMemcpyAsync(host, aborts, n * sizeof(unsigned), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e == hipSuccess) {
        int c = 0;
        for (size_t i = 0; i < n; ++i) c += host[i] != 0u;
        *count = c;
    }
    std::free(host);
    return e;
}

hipError_t gdn_chunked(const void* q, const void* k, const void* v, const float* g_log,
                       const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                       float scale, void* ws, bool f32, hipStream_t stream, int nseg) {
    if (f32)
        return launch_chunked<false, float>(q, k, v, g_log, beta, GdnRawGates{}, state, out, B, T, Hq,
                                            Hv, scale, ws, true, stream, SIZE_MAX, nseg);
    return launch_chunked<false, half_t>(q, k, v, g_log, beta, GdnRawGates{}, state, out, B, T, Hq, Hv,
                                         scale, ws, true, stream, SIZE_MAX, nseg);
}

hipError_t gdn_chunked_fused(const void* q, const void* k, const void* v, const GdnRawGates& gates,
                             float* state, void* out, int B, int T, int Hq, int Hv, float scale,
                             void* ws, hipStream_t stream) {
    return launch_chunked<true, half_t>(q, k, v, nullptr, nullptr, gates, state, out, B, T, Hq, Hv,
                                        scale, ws, true, stream);
}

}  // namespace tsa
