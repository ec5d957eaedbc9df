// attn_fwd.hip -- softmax flash-attention forward for gfx950 (fp16 MFMA, fp32 softmax).
//
// Same recurrence as flash_attn_sm75_wmma (src/attn_sm75.cu:239-375): stream K/V tiles,
// keep running (m, l, O) per query row, O = O*alpha + P V, finally O / l.  The tiling is
// CDNA4-shaped instead of a 16x16 warp tile:
//   * a workgroup is 4 waves and owns 128 query rows (32 per wave, 8 waves at D = 256);
//     K/V tiles of 64 keys are double-buffered in LDS (64 KiB at D = 128) so two
//     workgroups share a CU, and
//     copied there by LDS-DMA (global_load_lds_dwordx4, per-lane offsets computed once,
//     the bank swizzle applied on the source side), so no register stages them;
//   * each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_f16 (A = K rows from LDS,
//     B = its 32 Q rows held in registers for the whole loop), so a lane owns one query
//     and 16 keys per 32-key block: the row max / row sum are register reductions plus
//     one exchange with lane l^32;
//   * P^T stays in registers (the S^T accumulator converted to fp16 is exactly the B
//     operand layout of the next MFMA) and O^T += V^T P^T reads V^T straight out of the
//     row-major V tile with ds_read_b64_tr_b16 -- no transpose pass;
//   * softmax in the exp2 domain with scale*log2(e) folded into one FMA per score; the
//     running max used for the exponentials is raised only when a tile's max exceeds it
//     by more than 2^8 (then O and l are rescaled), so most tiles skip the O rescale --
//     exact, since O and l always share the same max, with P bounded by 2^8;
//   * causal: tiles above a wave's diagonal are skipped, only diagonal / ragged tiles
//     are masked; heavy (late) query tiles are scheduled first, and all query tiles of
//     one (b, h) land on one XCD so its K/V stay in that XCD's L2;
//   * grouped-query attention and the output gate of gated attention (the D = 256 layers
//     of the reference's target model, docs/qwen38-27b.md:13): query head h reads K/V
//     head h / (Hq / Hkv), and O is multiplied by sigmoid(gate) when a gate is given.
//     At D = 256 a workgroup is 8 waves (256 query rows) sharing one 128 KiB set of K/V
//     tiles, two waves per SIMD at 256 registers each (Q operands 64, O^T 128): LDS
//     addresses are one XOR with an immediate per read and the tile copies need one offset
//     register, so the rest fits.
#include <climits>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

constexpr int kKRows = 64;   // keys per LDS tile

// 16-byte chunk swizzle of an LDS tile row: chunk c of row r lives at c ^ swz<D>(r).
// LDS has 64 banks of 4 bytes; a 256-byte D = 128 row spans all of them, so a chunk's
// banks depend on its position only.  The K operand reads (ds_read_b128, 16 lanes per
// cycle) take 16 consecutive rows at one chunk: swz is a permutation of r % 16.  The
// transposing V reads (ds_read_b64_tr_b16, 32 lanes per cycle) take 4 aligned rows x 4
// chunks of one aligned chunk block: swz moves the 4 rows to 4 different chunk blocks.
// At D = 64 two rows share the 64 banks and the other formula keeps both read patterns
// conflict free.
template <int D>
__device__ __forceinline__ int swz(int r) {
    if (D >= 128) return 4 * (r & 3) + ((r >> 2) & 3);  // D = 256: a row is two bank periods
    return (2 * (r & 3) + ((r >> 2) & 1)) & 7;
}

template <int D>
struct Cfg {
    static constexpr int kChunks = D / 8;                        // 16-B chunks per row
    static constexpr int kTile = kKRows * D;                     // halfs per K or V tile
    static constexpr int kKSteps = D / 16;                       // k-steps of S^T = K Q^T
    static constexpr int kDBlocks = D / 32;                      // 32-row blocks of O^T
    static constexpr int kLdsBytes = 2 * 2 * kTile * 2;          // 2 buffers x (K, V)
};

template <int D>
__device__ __forceinline__ int chunk_pos(int r, int c) {
    return c ^ swz<D>(r);
}

// Map the linear workgroup id to (bh, query tile).  Workgroups are dispatched round
// robin over the 8 XCDs; when BH is a multiple of 8 the heads are spread over the XCDs so
// that all query tiles of a head run on one XCD: with grouped K/V heads (group > 1) XCD x
// runs the contiguous heads x * BH/8 .. (x + 1) * BH/8 - 1, so the query heads of one K/V
// group (adjacent head numbers) read their K/V tiles through the same L2 (gated GQA layer:
// 1.22 -> 0.49 GB of HBM traffic per launch); without groups XCD x runs heads x, x + 8, ...
// (0.48 vs 0.56 GB at B=1 H=32 S=8192 D=128).  Causal runs issue the longest (highest) query
// tiles first.
__device__ __forceinline__ void map_block(int bid, int BH, int n_qt, bool causal, int group,
                                          int& bh, int& qt) {
    int rank;
    if ((BH & 7) == 0) {
        const int xcd = bid & 7, slot = bid >> 3, hpx = BH >> 3;
        bh = group > 1 ? xcd * hpx + slot % hpx : (slot % hpx) * 8 + xcd;
        rank = slot / hpx;
    } else {
        bh = bid % BH;
        rank = bid / BH;
    }
    qt = causal ? (n_qt - 1 - rank) : rank;
}

typedef __attribute__((address_space(3))) void* lds_void_t;

// LDS reads at a byte address held as an integer (so that address arithmetic can be an
// XOR with an immediate plus an offset folded into the instruction).
__device__ __forceinline__ half8_t lds_read_b128(unsigned addr) {
    typedef __attribute__((address_space(3))) const half8_t* p_t;
    return *(p_t)(addr);
}
__device__ __forceinline__ half4_t lds_read_tr16_at(unsigned addr) {
    typedef __attribute__((address_space(3))) fp16x4_t* p_t;
    return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((p_t)(addr)));
}

// K/V tile copy plan.  One LDS-DMA instruction moves 1 KiB (lane l: 16 bytes to M0 + 16*l);
// a tile of 64 rows x D halfs is kTile instructions, K then V, and wave w of kW issues
// instructions w + kW j.  LDS chunk position p of row r holds source chunk p ^ swz(r), so
// the tile lands in the same swizzled layout the operand reads expect.
template <int D, int kW = 4>
struct Dma {
    static constexpr int kTile = kKRows * D * 2 / 1024;  // instructions per K (or V) tile
    static constexpr int kPerWave = 2 * kTile / kW;      // for kW waves per workgroup
    static constexpr int kChunks = D / 8;
    static_assert(kTile % kW == 0, "each wave copies whole groups of K and V blocks");
};
template <int D>
__device__ __forceinline__ unsigned dma_off(int blk, int lane, int lastrow) {
    const int P = blk * 64 + lane;
    const int row = P / Dma<D>::kChunks, cpos = P % Dma<D>::kChunks;
    const int c = cpos ^ swz<D>(row);
    return (unsigned)(min(row, lastrow) * D + c * 8) * 2u;
}
// src = base + off (64-bit base in SGPRs, 32-bit VGPR offset).  Inline asm on purpose:
// the compiler does not track LDS written by DMA per buffer and would wait for every
// copy in flight before the first LDS read of the other buffer; the kernel orders the
// copies itself (vmcnt(0) and a barrier at the end of each tile).
__device__ __forceinline__ void dma_issue(const void* base, unsigned off, unsigned lds_addr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(off), "s"(base), "{m0}"(lds_addr)
                 : "memory");
}
// This wave's share of the copies of K/V rows k0..k0+63 into the buffer at lds_buf, in
// two halves (kPart 0: j < kPerWave/2, kPart 1: the rest) so each can be issued between
// MFMAs.  off0 = dma_off(wave, lane, 63).  Wave w copies blocks w + kW j (K for
// kW j < kTile, V after).  A block is 1 KiB of whole rows and the swizzle reads row bits
// 0-3; when all of a wave's blocks see the same row % 16 pattern -- always at D <= 128
// (blk = w mod 4 fixes it), at D = 256 (two rows per block) when kW is a multiple of 8
// (blk = w mod 8) -- block blk of a full tile sits at off0 + 1024 (blk - w): one register
// for all copies.
template <int D, int kPart, int kW>
__device__ __forceinline__ void copy_tile(unsigned off0, int wave, const half_t* Kh, const half_t* Vh,
                                          int k0, int S, unsigned lds_buf) {
    static_assert(D <= 128 || kW % 8 == 0, "a wave's copy blocks must share one swizzle pattern");
    const half_t* kb = Kh + (size_t)k0 * D;
    const half_t* vb = Vh + (size_t)k0 * D;
    const int lastrow = S - 1 - k0;
    auto issue_all = [&](auto Ragged) {  // a ragged last tile clamps its rows to S - 1
#pragma unroll
        for (int j = kPart * Dma<D, kW>::kPerWave / 2; j < (kPart + 1) * Dma<D, kW>::kPerWave / 2; ++j) {
            constexpr int kT = Dma<D>::kTile;  // a multiple of kW, and wave < kW
            const bool isv = kW * j >= kT;
            const int dblk = kW * j - (isv ? kT : 0);  // blk - wave
            unsigned o;
            if constexpr (!decltype(Ragged)::value) {
                o = off0 + 1024u * (unsigned)dblk;
            } else {  // the same offset with its row clamped to S - 1
                constexpr unsigned kRowB = 2 * D, kRows = 1024 / kRowB;
                // the empty asm keeps this arithmetic inside the ragged branch (hoisted, its
                // values take registers for the whole loop)
                unsigned o0 = off0;
                asm volatile("" : "+v"(o0));
                const int row = (int)(o0 / kRowB) + (int)kRows * dblk;
                o = (unsigned)min(row, lastrow) * kRowB + o0 % kRowB;
            }
            dma_issue(isv ? (const void*)vb : (const void*)kb, o,
                      lds_buf + (unsigned)(isv ? kKRows * D * 2 : 0) + 1024u * (unsigned)(wave + dblk));
        }
    };
    if (lastrow >= kKRows - 1)
        issue_all(std::false_type{});
    else
        issue_all(std::true_type{});
}
__device__ __forceinline__ void dma_wait_barrier() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies have landed
    lds_barrier();
}

// kW waves per workgroup, 32 query rows each: kW = 4 at D <= 128 (two workgroups per CU,
// two waves per SIMD), kW = 8 at D = 256 (one workgroup per CU with the 128 KiB of K/V
// tiles, two waves per SIMD sharing them).
template <int D, bool kCausal, int kW>
__global__ void __launch_bounds__(64 * kW, 2)
attn_fwd_kernel(const half_t* __restrict__ Q, const half_t* __restrict__ K,
                const half_t* __restrict__ V, const half_t* __restrict__ gate,
                half_t* __restrict__ O, int S, int BH, int n_qt, int Hq, int group,
                float c2 /* scale * log2(e) */) {
    using C = Cfg<D>;
    // static and 1 KiB aligned: the XOR address forms below need the buffer's low 10 bits zero
    __shared__ __align__(1024) half_t lds[C::kLdsBytes / 2];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hi = lane >> 5;  // which half of the wave
    int bh, qt;
    map_block(blockIdx.x, BH, n_qt, kCausal, group, bh, qt);
    const size_t head = (size_t)bh * S * D;  // Q, O, gate: query head bh = b * Hq + h
    const size_t kvhead = (size_t)((bh / Hq) * (Hq / group) + (bh % Hq) / group) * S * D;
    const int q0 = qt * (32 * kW);
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

    const int kv_end = kCausal ? min(S, q0 + 32 * kW) : S;
    const int n_tiles = (kv_end + kKRows - 1) / kKRows;
    const int wave_kv_end = kCausal ? min(S, qw0 + 32) : S;

    float16_t o[C::kDBlocks];
#pragma unroll
    for (int i = 0; i < C::kDBlocks; ++i) o[i] = float16_t{};
    float m = -INFINITY;  // max of raw scores (q . k) the exponentials are taken against
    float l = 0.f;        // running sum of this lane's half of the keys

    // Lane-constant parts of the LDS addresses.
    const int krow = lane & 31;            // K operand row within a 32-key block
    const int ksw = swz<D>(krow);
    const int g16 = lane >> 4, i16 = lane & 15;
    const int vj = i16 >> 2, vm = i16 & 3;  // transposed-read source row / column group
    // V^T operand: source row 16*ks + 8*e + 4*hi + vj, columns 32*db + 16*(g16&1) + 4*vm.
    const int vchunk = 2 * (g16 & 1) + (vm >> 1);
    const int vsub = 4 * (vm & 1);

    const unsigned off = dma_off<D>(wave, lane, kKRows - 1);
    const unsigned lds0 = (unsigned)(uintptr_t)(lds_void_t)(void*)lds;
    const unsigned buf_bytes = 2 * C::kTile * 2;
    constexpr unsigned kRowB = 2 * D;  // bytes per K/V row in LDS
    // LDS operand addresses as byte offsets in buffer 0.  A row is 16 * (D / 8) bytes and
    // starts at a multiple of that, so the chunk field (bits 4.. within the row) can be
    // XORed without touching the row bits.  K operand of k-step kk (row krow, chunk
    // (2 kk + hi) ^ swz(krow)): ka ^ (32 kk), since 2 kk + hi = 2 kk ^ hi and swz < 16.
    // V^T operand of key step ks, column block db, half e (rows 16 ks + 4 hi + vj + 8 e,
    // chunk (4 db + vchunk) ^ swz(row), element vsub): swz(row) reads row bits 0-3, which
    // 16 ks leaves alone, so the address is (va[e] ^ 64 db) + 32 D ks.
    unsigned ka = lds0 + krow * kRowB + 16u * (unsigned)(hi ^ ksw);
    unsigned va[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int r = 4 * hi + vj + 8 * e;
        va[e] = lds0 + C::kTile * 2 + r * kRowB + 16u * (unsigned)chunk_pos<D>(r, vchunk) + 2u * vsub;
    }
    copy_tile<D, 0, kW>(off, wave, K + kvhead, V + kvhead, 0, S, lds0);
    copy_tile<D, 1, kW>(off, wave, K + kvhead, V + kvhead, 0, S, lds0);
    dma_wait_barrier();

    if constexpr (D <= 128) {
        // Two tiles per trip: the buffer parity u is then a constant in each copy of the
        // body and the LDS addresses of the two buffers differ by an immediate offset instead
        // of being recomputed every tile (2-3 % at D = 64 and 128).
        for (int t0 = 0; t0 < n_tiles; t0 += 2) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int t = t0 + u;
            if (t >= n_tiles) break;
            const int k0 = t * kKRows;
            const bool more = t + 1 < n_tiles;
            const unsigned nbuf = lds0 + (unsigned)(u ^ 1) * buf_bytes;
            if (k0 >= wave_kv_end) {  // this wave's queries end before the tile: copies only
                if (more) {
                    copy_tile<D, 0, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
                    copy_tile<D, 1, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
                }
            } else {
                const unsigned ubase = (unsigned)u * buf_bytes;
                // The XORed addresses are recomputed next to their reads in each tile (one VALU
                // op each) instead of being held: the empty asm hides that they repeat.
                asm volatile("" : "+v"(ka), "+v"(va[0]), "+v"(va[1]));
                // ---- S^T = K Q^T for two 32-key blocks, the two accumulator chains interleaved;
                // the first half of the next tile's copies goes out halfway ----
                float16_t s[2] = {float16_t{}, float16_t{}};
#pragma unroll
                for (int kk = 0; kk < C::kKSteps; ++kk) {
                    const unsigned a = (ka ^ (32u * kk)) + ubase;
                    s[0] = mfma32(lds_read_b128(a), qf[kk], s[0]);
                    s[1] = mfma32(lds_read_b128(a + 32 * kRowB), qf[kk], s[1]);
                    if (kk == C::kKSteps / 2 - 1 && more)
                        copy_tile<D, 0, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
                }
                // V^T operands of the first key step, read now so that their LDS time runs under
                // the softmax (V does not depend on P); a wave reads transposed V at ~18 B/clk.
                auto read_v = [&](int ks, int db) {
                    const unsigned o = ubase + (unsigned)(32 * D * ks);
                    const half4_t lo = lds_read_tr16_at((va[0] ^ (64u * db)) + o);
                    const half4_t up = lds_read_tr16_at((va[1] ^ (64u * db)) + o);
                    return half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
                };
                half8_t v0[C::kDBlocks];
#pragma unroll
                for (int db = 0; db < C::kDBlocks; ++db) v0[db] = read_v(0, db);
                // ---- masks: causal diagonal and keys past S ----
                if ((kCausal && k0 + kKRows - 1 > qw0) || k0 + kKRows > S) {
                    // register r of block kb holds key k0 + 4 hi + c, c = 32 kb + 8 (r / 4) + r % 4:
                    // compare the constant c against per-lane limits
                    const int base = k0 + 4 * hi;
                    const int lim_q = kCausal ? my_q - base : INT_MAX;  // masked when c > lim_q
                    const int lim_s = S - base;                         // masked when c >= lim_s
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
                            if (c > lim_q || c >= lim_s) s[kb][r] = -INFINITY;
                        }
                }
                // ---- online softmax (exp2 domain), as in the loop below ----
                float mx = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
                mx = max_xor32(mx);
                if (__builtin_amdgcn_ballot_w64((mx - m) * c2 > 8.f)) {
                    const float m_new = fmaxf(m, mx);
                    const float alpha = m_new == -INFINITY ? 1.f : fast_exp2((m - m_new) * c2);
                    m = m_new;
                    l *= alpha;
#pragma unroll
                    for (int db = 0; db < C::kDBlocks; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                }
                const float mc = m == -INFINITY ? 0.f : m * c2;
                half8_t p[4];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        p[2 * kb + (r >> 3)][r & 7] = (half_t)fast_exp2(fmaf(s[kb][r], c2, -mc));
                const half2_t one2 = {(half_t)1.f, (half_t)1.f};
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int w2 = 0; w2 < 4; ++w2)
                        l = __builtin_amdgcn_fdot2(half2_t{p[i][2 * w2], p[i][2 * w2 + 1]}, one2, l, false);
                // ---- O^T += V^T P^T at raised priority, the second copy half among the MFMAs ----
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    if (ks == 1 && more)
                        copy_tile<D, 1, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
#pragma unroll
                    for (int db = 0; db < C::kDBlocks; ++db)
                        o[db] = mfma32(ks == 0 ? v0[db] : read_v(ks, db), p[ks], o[db]);
                }
                __builtin_amdgcn_s_setprio(0);
            }
            dma_wait_barrier();
          }
        }
    } else {
        // D = 256: each 64-key tile is taken as two 32-key halves in turn (S^T of one half: 16
        // registers), which leaves the registers for K and V^T operand read-ahead beside the
        // 128 O^T accumulators and the 64 Q operand registers.
        for (int t = 0; t < n_tiles; ++t) {
            const int k0 = t * kKRows;
            const bool more = t + 1 < n_tiles;
            const unsigned nbuf = lds0 + ((t + 1) & 1) * buf_bytes;
            if (k0 >= wave_kv_end) {  // this wave's queries end before the tile: copies only
                if (more) {
                    copy_tile<D, 0, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
                    copy_tile<D, 1, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
                }
            } else {
                const unsigned ubase = (unsigned)(t & 1) * buf_bytes;
                // the first half of the next tile's copies goes out at the top
                if (more) copy_tile<D, 0, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int kb0 = k0 + 32 * kb;  // first key of this half
                    // a second half wholly past this wave's last query adds nothing
                    if (kCausal && kb == 1 && kb0 > qw0 + 31) break;
                    // The XORed addresses are recomputed next to their reads in each half (one
                    // VALU op each) instead of being held: the empty asm hides that they repeat.
                    asm volatile("" : "+v"(ka), "+v"(va[0]), "+v"(va[1]));
                    // ---- S^T = K Q^T for this half: the K operand reads run kPreK k-steps ahead
                    // of their MFMAs, pinned there by scheduling barriers ----
                    constexpr int kPreK = 3;
                    float16_t sh = float16_t{};
                    half8_t kop[C::kKSteps];
                    auto read_k = [&](int kk) {
                        kop[kk] = lds_read_b128((ka ^ (32u * kk)) + ubase + (unsigned)(32 * kb) * kRowB);
                    };
#pragma unroll
                    for (int kk = 0; kk < kPreK; ++kk) read_k(kk);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int kk = 0; kk < C::kKSteps; ++kk) {
                        if (kk + kPreK < C::kKSteps) read_k(kk + kPreK);
                        sh = mfma32(kop[kk], qf[kk], sh);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    // ---- masks: causal diagonal and keys past S ----
                    if ((kCausal && kb0 + 31 > qw0) || kb0 + 32 > S) {
                        // register r holds key kb0 + 4 hi + c, c = 8 (r / 4) + r % 4: compare the
                        // constant c against per-lane limits
                        const int base = kb0 + 4 * hi;
                        const int lim_q = kCausal ? my_q - base : INT_MAX;  // masked when c > lim_q
                        const int lim_s = S - base;                         // masked when c >= lim_s
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int c = 8 * (r >> 2) + (r & 3);
                            if (c > lim_q || c >= lim_s) sh[r] = -INFINITY;
                        }
                    }
                    // ---- online softmax (exp2 domain) ----
                    float mx = sh[0];
#pragma unroll
                    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sh[r]);
                    mx = max_xor32(mx);
                    // Raise the reference max only when some score would exceed it by 2^8 in the
                    // exp2 domain (always on the first unmasked half: m = -inf).
                    if (__builtin_amdgcn_ballot_w64((mx - m) * c2 > 8.f)) {
                        const float m_new = fmaxf(m, mx);
                        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2((m - m_new) * c2);
                        m = m_new;
                        l *= alpha;
#pragma unroll
                        for (int db = 0; db < C::kDBlocks; ++db)
#pragma unroll
                            for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                    }
                    const float mc = m == -INFINITY ? 0.f : m * c2;
                    half8_t p[2];
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        p[r >> 3][r & 7] = (half_t)fast_exp2(fmaf(sh[r], c2, -mc));
                    // row sum of the fp16 P that multiplies V, on v_dot2_f32_f16
                    const half2_t one2 = {(half_t)1.f, (half_t)1.f};
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            l = __builtin_amdgcn_fdot2(half2_t{p[i][2 * u], p[i][2 * u + 1]}, one2, l, false);
                    // ---- O^T += V^T P^T for this half's two key steps (raised priority: the
                    // other wave of the SIMD is then mostly in its QK^T / softmax part).  The V^T
                    // operand reads run kPreV steps ahead of their MFMAs, pinned there ----
                    auto read_v = [&](int ks, int db) {
                        const unsigned o = ubase + (unsigned)(32 * D * ks);
                        const half4_t lo = lds_read_tr16_at((va[0] ^ (64u * db)) + o);
                        const half4_t up = lds_read_tr16_at((va[1] ^ (64u * db)) + o);
                        return half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
                    };
                    __builtin_amdgcn_sched_barrier(0);
                    __builtin_amdgcn_s_setprio(1);
                    constexpr int kSteps = 2 * C::kDBlocks, kPreV = 2;
                    half8_t vbuf[kSteps];
#pragma unroll
                    for (int i = 0; i < kPreV; ++i) vbuf[i] = read_v(2 * kb + i / C::kDBlocks, i % C::kDBlocks);
#pragma unroll
                    for (int i = 0; i < kSteps; ++i) {
                        const int ks = i / C::kDBlocks, db = i % C::kDBlocks;
                        if (i + kPreV < kSteps)
                            vbuf[i + kPreV] = read_v(2 * kb + (i + kPreV) / C::kDBlocks, (i + kPreV) % C::kDBlocks);
                        if (kb == 0 && i == C::kDBlocks && more)
                            copy_tile<D, 1, kW>(off, wave, K + kvhead, V + kvhead, k0 + kKRows, S, nbuf);
                        o[db] = mfma32(vbuf[i], p[ks], o[db]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    __builtin_amdgcn_s_setprio(0);
                }
            }
            dma_wait_barrier();
        }
    }

    // ---- epilogue: O = O^T / l (times sigmoid(gate)), 4 consecutive d per store ----
    l = sum_xor32(l);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (my_q < S) {
        half_t* orow = O + head + (size_t)my_q * D;
        const half_t* grow = gate ? gate + head + (size_t)my_q * D : nullptr;
#pragma unroll
        for (int db = 0; db < C::kDBlocks; ++db)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int d0 = 32 * db + 8 * rg + 4 * hi;
                float f[4] = {inv, inv, inv, inv};
                if (grow) {
                    const half4_t g4 = *reinterpret_cast<const half4_t*>(grow + d0);
                    // sigmoid by the hardware reciprocal (1 ulp): an IEEE division per element
                    // was ~10 VALU ops, 128 of them per lane at D = 256 in every workgroup's tail
#pragma unroll
                    for (int e = 0; e < 4; ++e) f[e] = inv * __builtin_amdgcn_rcpf(1.f + __expf(-(float)g4[e]));
                }
                const half4_t v4 = {(half_t)(o[db][4 * rg] * f[0]), (half_t)(o[db][4 * rg + 1] * f[1]),
                                    (half_t)(o[db][4 * rg + 2] * f[2]), (half_t)(o[db][4 * rg + 3] * f[3])};
                *reinterpret_cast<half4_t*>(orow + d0) = v4;
            }
    }
}

template <int D, bool kCausal>
hipError_t launch(const half_t* q, const half_t* k, const half_t* v, const half_t* gate, half_t* o,
                  int B, int Hq, int Hkv, int S, float scale, hipStream_t stream) {
    constexpr int kW = D == 256 ? 8 : 4;
    const int BH = B * Hq;
    const int n_qt = (S + 32 * kW - 1) / (32 * kW);
    hipLaunchKernelGGL((attn_fwd_kernel<D, kCausal, kW>), dim3(BH * n_qt), dim3(64 * kW), 0,
                       stream, q, k, v, gate, o, S, BH, n_qt, Hq, Hq / Hkv, scale * kLog2e);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Naive check kernel: one thread per query row (src/attn_sm75.cu:55-94 math), with the
// grouped-query head map and the output gate of attn_fwd_kernel.
// ---------------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(128)
attn_naive_kernel(const half_t* __restrict__ Q, const half_t* __restrict__ K,
                  const half_t* __restrict__ V, const half_t* __restrict__ gate,
                  half_t* __restrict__ O, int S, int Hq, int group, long long rows, float scale,
                  int causal) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows) return;
    const long long bh = idx / S;
    const int qi = (int)(idx % S);
    const size_t off = (size_t)bh * S * D;
    const size_t kvoff = (size_t)((bh / Hq) * (Hq / group) + (bh % Hq) / group) * S * D;
    float qf[D];
#pragma unroll
    for (int d = 0; d < D; ++d) qf[d] = (float)Q[off + (size_t)qi * D + d];
    const int kend = causal ? qi + 1 : S;
    float m = -INFINITY;
    for (int kk = 0; kk < kend; ++kk) {
        const half_t* kr = K + kvoff + (size_t)kk * D;
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
        const half_t* kr = K + kvoff + (size_t)kk * D;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < D; ++d) dot = fmaf(qf[d], (float)kr[d], dot);
        const float p = expf(fmaf(dot, scale, -m));
        l += p;
        const half_t* vr = V + kvoff + (size_t)kk * D;
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = fmaf(p, (float)vr[d], acc[d]);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        float x = acc[d] / l;
        if (gate) x *= 1.f / (1.f + expf(-(float)gate[off + (size_t)qi * D + d]));
        O[off + (size_t)qi * D + d] = (half_t)x;
    }
}

}  // namespace

hipError_t attn_fwd(const void* q, const void* k, const void* v, const void* gate, void* o, int B,
                    int Hq, int Hkv, int S, int D, float scale, int causal, hipStream_t stream) {
    auto Q = static_cast<const half_t*>(q);
    auto K = static_cast<const half_t*>(k);
    auto Vp = static_cast<const half_t*>(v);
    auto G = static_cast<const half_t*>(gate);
    auto Op = static_cast<half_t*>(o);
    if (D == 256)
        return causal ? launch<256, true>(Q, K, Vp, G, Op, B, Hq, Hkv, S, scale, stream)
                      : launch<256, false>(Q, K, Vp, G, Op, B, Hq, Hkv, S, scale, stream);
    if (D == 128)
        return causal ? launch<128, true>(Q, K, Vp, G, Op, B, Hq, Hkv, S, scale, stream)
                      : launch<128, false>(Q, K, Vp, G, Op, B, Hq, Hkv, S, scale, stream);
    return causal ? launch<64, true>(Q, K, Vp, G, Op, B, Hq, Hkv, S, scale, stream)
                  : launch<64, false>(Q, K, Vp, G, Op, B, Hq, Hkv, S, scale, stream);
}

hipError_t attn_naive(const void* q, const void* k, const void* v, const void* gate, void* o,
                      int B, int Hq, int Hkv, int S, int D, float scale, int causal,
                      hipStream_t stream) {
    const long long rows = (long long)B * Hq * S;
    const unsigned blocks = (unsigned)((rows + 127) / 128);
    auto Q = static_cast<const half_t*>(q);
    auto K = static_cast<const half_t*>(k);
    auto Vp = static_cast<const half_t*>(v);
    auto G = static_cast<const half_t*>(gate);
    auto Op = static_cast<half_t*>(o);
    const int group = Hq / Hkv;
    if (D == 256)
        hipLaunchKernelGGL(attn_naive_kernel<256>, dim3(blocks), dim3(128), 0, stream, Q, K, Vp, G,
                           Op, S, Hq, group, rows, scale, causal);
    else if (D == 128)
        hipLaunchKernelGGL(attn_naive_kernel<128>, dim3(blocks), dim3(128), 0, stream, Q, K, Vp, G,
                           Op, S, Hq, group, rows, scale, causal);
    else
        hipLaunchKernelGGL(attn_naive_kernel<64>, dim3(blocks), dim3(128), 0, stream, Q, K, Vp, G,
                           Op, S, Hq, group, rows, scale, causal);
    return hipGetLastError();
}

}  // namespace tsa
