/*
 * oracle.h -- CPU restatement of the reference's naive attention and Gated DeltaNet paths.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * turing-sm75_amd/, its C-ABI, or the drivers) links, loads or calls this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the reference results are compared with / the timed CPU baseline.
 *
 * Every function cites the reference file:line it restates (paths are relative to
 * the cookys/turing-sm75 tree).  Layouts:
 *   attention : Q, K, V, O fp16 bits, [B][H][S][D]            (src/attn_sm75.cu:64,120,254)
 *   GDN       : q, k      [B][T][Hq][dk]                       (src/gdn_sm75.cu:75-77)
 *               v, out    [B][T][Hv][dv]
 *               g_log, beta [B][T][Hv]
 *               state     [B][Hv][dv][dk]  (column c = dv index is contiguous over the
 *                                            dk rows: S[c*dk + i] = S[i][c], :71-72,1094)
 *   V-head h reads QK head h % Hq (src/gdn_sm75.cu:11,68).
 * The reference has no batch dimension; B independent sequences are added here.
 *
 * Pinning (what checks each function beyond retyping it): tests/test_oracle_*.py hold
 * closed forms, invariants and fp64 brute-force checks; see the header of each test.
 */
#ifndef TSA_ORACLE_H
#define TSA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32 (IEEE binary16, round-to-nearest-even, like __float2half) ---- */
void orc_f2h(const float* src, uint16_t* dst, size_t n);
void orc_h2f(const uint16_t* src, float* dst, size_t n);

/* ---- input generators ---------------------------------------------------------- */
/* std::mt19937(seed) + std::normal_distribution<float>(mean, stddev), values rounded to
 * fp16, generated in order into ntensors consecutive tensors of n elements each: the
 * reference's make_tensor sequence Q, K, V (src/attn_sm75.cu:393-406,473-476). */
void orc_mt_normal_half(uint32_t seed, float mean, float stddev, size_t n, int ntensors,
                        uint16_t* out);
/* The GDN driver's LCG (src/gdn_sm75.cu:1270-1279): seed = 1; q, k, v = 0.2*rnd,
 * g_log = -0.2 + 0.05*rnd, beta = 0.4 + 0.4*(rnd + 0.5), generated in that order for
 * one sequence of T tokens with dk = dv = d. */
void orc_gdn_lcg_inputs(int T, int Hq, int Hv, int d, float* q, float* k, float* v,
                        float* g_log, float* beta);

/* ---- attention ------------------------------------------------------------------ */
/* naive_attn_kernel (src/attn_sm75.cu:55-94) for the listed rows.  rows[r] indexes a
 * query row as bh*S + qi.  o_f32 (may be NULL) receives acc/l before fp16 rounding,
 * o_h16 (may be NULL) the fp16 value the reference stores.  Dots are fp32 FMA chains in
 * d order (the reference is device code compiled with FMA contraction), the
 * softmax uses exp in fp32. */
void orc_attn_rows(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int B, int H,
                   int S, int D, float scale, int causal, const int64_t* rows,
                   int64_t nrows, float* o_f32, uint16_t* o_h16, int nthreads);
/* All rows: O = naive attention, fp16 out (the reference's On buffer, :492-497). */
void orc_attn_naive(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O,
                    int B, int H, int S, int D, float scale, int causal, int nthreads);

/* ---- Gated DeltaNet ------------------------------------------------------------- */
/* gdn_cpu (src/gdn_sm75.cu:1078-1106): exact fp32 token-serial recurrence, state updated
 * in place, out written for every token.  Parallel over (b, h) when nthreads > 1; each
 * (b, h) is computed in the reference's order, so results do not depend on nthreads. */
void orc_gdn_serial(const float* q, const float* k, const float* v, const float* g_log,
                    const float* beta, float* state, float* out, int B, int T, int Hq,
                    int Hv, int dk, int dv, float scale, int nthreads);
/* Chunk decomposition of gdn_chunked_cpu (src/gdn_sm75.cu:1109-1244), chunk size C,
 * computed in double (f64) or float (f32).
 *   exact_solve = 1: the exact (I + A)^-1 (the form that equals gdn_cpu in exact
 *                    arithmetic);
 *   exact_solve = 0: the reference's forward-substitution loop as written
 *                    (:1161-1180), which yields I - (I + A)^-1 A^T instead (kept to
 *                    document that finding; never used as the parity target). */
void orc_gdn_chunked_f64(const float* q, const float* k, const float* v, const float* g_log,
                         const float* beta, float* state, float* out, int B, int T, int Hq,
                         int Hv, int dk, int dv, int C, float scale, int exact_solve,
                         int nthreads);
void orc_gdn_chunked_f32(const float* q, const float* k, const float* v, const float* g_log,
                         const float* beta, float* state, float* out, int B, int T, int Hq,
                         int Hv, int dk, int dv, int C, float scale, int exact_solve,
                         int nthreads);
/* The C x C matrix the reference's solve loop produces for one chunk (ggml [i + j*C]
 * order), from kb (same order).  Exposed so a test can check its closed form. */
void orc_ref_solve(const float* kb, float* attn, int C);

#ifdef __cplusplus
}
#endif
#endif
