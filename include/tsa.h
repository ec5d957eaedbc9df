/*
 * tsa.h -- C-ABI of the MI355X (gfx950) attention + Gated DeltaNet kernels.
 *
 * Drop-in boundary for the two hot-path labs of cookys/turing-sm75.  Every entry point
 * takes device pointers to contiguous buffers the caller owns, enqueues work on the
 * given HIP stream (NULL = the default stream) and returns at once: no device memory is
 * allocated and nothing is synchronised (tsa_gdn_chunked_redo_count, a diagnostic, is the
 * one synchronous call).  Every kernel runs on the caller's stream, in order, as the
 * reference's launches run on one stream with caller-owned scratch (src/gdn_sm75.cu:1341-1346).
 * Opt-in only: with the environment variable TSA_GDN_OVERLAP=1 the chunked prefill (not under
 * graph capture) runs its two kernels side by side on the caller's stream and on a second
 * stream of the same device, which it creates with two events on the first such call on that
 * device (under a mutex) and keeps until the process ends.  Errors come back as TSA_* codes,
 * never as exit() or exceptions (the reference's CUDA_CHECK exits, src/attn_sm75.cu:40-48).
 *
 * dtypes: q/k/v/o/out are IEEE fp16 (passed as void*), g_log, beta and the GDN state are
 * fp32; the *_f32 GDN entry points take q/k/v/out in fp32 as well, the reference's own GDN
 * I/O (src/gdn_sm75.cu:57-64).  Layouts follow the reference:
 *   attention : Q, K, V, O                [B][H][S][D]     (src/attn_sm75.cu:64,120,254)
 *   grouped   : Q, gate, O [B][Hq][S][D]; K, V [B][Hkv][S][D]; query head h reads K/V
 *               head h / (Hq / Hkv)
 *   GDN       : q, k                      [B][T][Hq][dk]   (src/gdn_sm75.cu:75-77)
 *               v, out                    [B][T][Hv][dv]
 *               g_log, beta               [B][T][Hv]
 *               state                     [B][Hv][dv][dk]  (S[c*dk + i] = S[i][c], :71-72)
 *   V-head h reads QK head h % Hq (src/gdn_sm75.cu:11,68).  The reference has B = 1.
 */
#ifndef TSA_H
#define TSA_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TSA_OK = 0,
    TSA_ERR_NULL = 1,        /* a required pointer is NULL                           */
    TSA_ERR_SHAPE = 2,       /* a size is < 1, too large, or the shapes disagree      */
    TSA_ERR_UNSUPPORTED = 3, /* a valid shape this library has no kernel for (e.g. D) */
    TSA_ERR_WORKSPACE = 4,   /* workspace NULL or smaller than *_workspace_bytes     */
    TSA_ERR_LAUNCH = 5,      /* the HIP runtime rejected a launch                    */
    TSA_ERR_ARG = 6,         /* a non-shape argument is invalid (scale not finite...) */
    TSA_ERR_SCRATCH = 7      /* the shapes exceed tsa_gdn_chunked_fwd_noalloc's scratch */
};

/* Message for a TSA_* code (static storage). */
const char* tsa_strerror(int code);
/* Library version string, e.g. "tsa 0.1 gfx950". */
const char* tsa_version(void);

/* Softmax flash-attention forward, O = softmax(scale * Q K^T [+ causal mask]) V.
 * Replaces launch_wmma<D> (src/attn_sm75.cu:432-440, dispatched on D at :481-484) and its
 * kernel flash_attn_sm75_wmma (:239-375).  D in {64, 128} as the
 * reference, and 256; any S >= 1 (the reference caps S at 1024 for its naive check only,
 * :457-460); causal 0 or 1 (the reference hard-codes 1, :463).  fp32 softmax statistics,
 * fp16 MFMA. */
int tsa_attn_fwd(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                 int D, float scale, int causal, void* stream);

/* The lab's naive correctness kernel on the device: one thread per query row, fp32 dot
 * products, two-pass exact softmax.  Same math as naive_attn_kernel
 * (src/attn_sm75.cu:55-94) without its per-d recomputation of the dot product and without
 * its S <= 1024 threads-per-block limit.  Used by the attn_sm75 driver's error check. */
int tsa_attn_naive(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                   int D, float scale, int causal, void* stream);

/* The same attention forward on the vector ALUs only (fp32 FMA dots, no MFMA): the
 * same-binary opponent of tsa_attn_fwd, as launch_ffma<D> / flash_attn_sm75_ffma
 * (src/attn_sm75.cu:421-430, :107-233) is of the WMMA kernel in the reference's driver.
 * Same arguments, layouts, shapes and error codes as tsa_attn_fwd. */
int tsa_attn_fwd_valu(const void* q, const void* k, const void* v, void* o, int B, int H, int S,
                      int D, float scale, int causal, void* stream);

/* Gated grouped-query attention: O = softmax(scale * Q K^T [+ causal mask]) V, then
 * O *= sigmoid(gate) element-wise when gate is not NULL.  The attention layer of the
 * reference's target model (24 query / 4 K/V heads, head_dim 256, gate after softmax,
 * docs/qwen38-27b.md:13), which the reference's lab does not implement (:19); no
 * reference kernel is replaced.  Hq % Hkv == 0; D in {64, 128, 256}; q/k are taken after
 * any rotary embedding.  tsa_attn_fwd is this call with Hkv = Hq and no gate. */
int tsa_attn_gqa_fwd(const void* q, const void* k, const void* v, const void* gate, void* o,
                     int B, int Hq, int Hkv, int S, int D, float scale, int causal,
                     void* stream);
/* The same on the naive check kernel (one thread per query row, exact two-pass softmax). */
int tsa_attn_gqa_naive(const void* q, const void* k, const void* v, const void* gate, void* o,
                       int B, int Hq, int Hkv, int S, int D, float scale, int causal,
                       void* stream);

/* Chunked Gated DeltaNet prefill over T tokens for B sequences, state carried in place.
 * Replaces the chunked kernels gdn_wmma_kernel (src/gdn_sm75.cu:361-574),
 * gdn_chunked_kernel (:192-354) and the two-pass gdn_prep_kernel + gdn_apply_kernel
 * (:896-1073), with the exact intra-chunk inverse (I + A)^-1 (the reference's solve loop,
 * :271-292, is only first-order accurate).  dk = dv = 128, chunk = 64.  ws must hold
 * tsa_gdn_chunked_workspace_bytes(...) bytes of device memory, the caller's as the
 * reference driver owns the two-pass scratch (src/gdn_sm75.cu:1341-1346); its contents on
 * entry do not matter (in order the two kernels use no ready flags; a call whose two kernels
 * run side by side, TSA_GDN_OVERLAP=1, clears them first), and calls that share one
 * ws must be ordered on one stream.  With few heads and many chunks (B*Hv <= 21, at least 16
 * chunks) the call splits the sequence into segments (segment state maps with their outputs
 * side by side, a combine, a parallel output fix-up) and the workspace grows by 192 KiB per
 * head and segment and 1 KiB per head and token after the first segment.  The plan, and so
 * the workspace size, is a function of the shapes only; tsa_gdn_chunked_plan_fwd takes an
 * explicit one. */
size_t tsa_gdn_chunked_workspace_bytes(int B, int T, int Hq, int Hv, int dk, int dv,
                                       int chunk);
int tsa_gdn_chunked_fwd(const void* q, const void* k, const void* v, const float* g_log,
                        const float* beta, float* state, void* out, int B, int T, int Hq,
                        int Hv, int dk, int dv, int chunk, float scale, void* ws,
                        size_t ws_bytes, void* stream);

/* The same prefill with fp32 q, k, v, out (the reference's GDN kernels and gdn_cpu take fp32,
 * src/gdn_sm75.cu:57-64,1078-1106): the inputs are converted to the fp16 MFMA operands in
 * registers, never narrowed in memory, and the output is stored in fp32.  Its workspace is
 * larger (the prep leaves fp16 copies of each chunk's K and Q rows there for the state
 * carry): tsa_gdn_chunked_workspace_bytes_f32(...). */
size_t tsa_gdn_chunked_workspace_bytes_f32(int B, int T, int Hq, int Hv, int dk, int dv,
                                           int chunk);
int tsa_gdn_chunked_fwd_f32(const float* q, const float* k, const float* v, const float* g_log,
                            const float* beta, float* state, float* out, int B, int T, int Hq,
                            int Hv, int dk, int dv, int chunk, float scale, void* ws,
                            size_t ws_bytes, void* stream);

/* The chunked prefill with an explicit sequence-split plan (no counterpart in the reference,
 * which carries the state through every chunk in order): nseg = 0 takes the library's plan,
 * the one tsa_gdn_chunked_fwd uses; nseg = 1 never splits; nseg >= 2 asks for nseg segments
 * (fewer when the sequence has fewer chunks, so that no segment is empty).  io_f32 = 1: q, k,
 * v, out are fp32 as in tsa_gdn_chunked_fwd_f32, else fp16.  ws must hold
 * tsa_gdn_chunked_plan_workspace_bytes(..., io_f32, nseg) bytes (0 for invalid arguments).
 * Results equal tsa_gdn_chunked_fwd's whenever the plans agree; otherwise they agree to fp32
 * rounding. */
size_t tsa_gdn_chunked_plan_workspace_bytes(int B, int T, int Hq, int Hv, int dk, int dv,
                                            int chunk, int io_f32, int nseg);
int tsa_gdn_chunked_plan_fwd(const void* q, const void* k, const void* v, const float* g_log,
                             const float* beta, float* state, void* out, int B, int T, int Hq,
                             int Hv, int dk, int dv, int chunk, float scale, int io_f32, int nseg,
                             void* ws, size_t ws_bytes, void* stream);

/* tsa_gdn_chunked_fwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is a fixed 64 MiB device array inside
 * the library, one per GPU, held until the process ends.  The call splits the sequence (as
 * tsa_gdn_chunked_fwd does with few heads) only where the split's larger workspace fits there,
 * and otherwise runs the chunk carry whole; shapes whose workspace exceeds 64 MiB even so
 * return TSA_ERR_SCRATCH (e.g. 32 V-heads up to T = 2240).  Nothing is allocated, no stream
 * or event is created (the kernels run in order on `stream`), and the results equal
 * tsa_gdn_chunked_fwd's bit for bit whenever both take the same plan.  Every call on a GPU
 * uses that GPU's one array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be ordered by the caller. */
int tsa_gdn_chunked_fwd_noalloc(const void* q, const void* k, const void* v, const float* g_log,
                                const float* beta, float* state, void* out, int B, int T, int Hq,
                                int Hv, int dk, int dv, int chunk, float scale, void* stream);

/* Diagnostic, no reference counterpart: after a tsa_gdn_chunked_fwd (fused, or with io_f32 = 1
 * tsa_gdn_chunked_fwd_f32) call on ws with these shapes that ran side by side
 * (TSA_GDN_OVERLAP=1), *count = the number of its state-carrying workgroups that waited longer
 * than the limit for the side-by-side kernel (a scheduler that did not run the two kernels
 * together) and were redone by the call's second launch; 0 when the overlap worked, and after
 * a call in order (the default).  Synchronises `stream` (a device-to-host copy of the call's
 * abort words). */
int tsa_gdn_chunked_redo_count(const void* ws, size_t ws_bytes, int B, int T, int Hq, int Hv,
                               int dk, int dv, int chunk, int io_f32, int* count, void* stream);

/* Token-serial Gated DeltaNet over T tokens (state held on chip for all T).  Replaces the
 * token-serial kernels gdn_serial_kernel, gdn_smem_kernel, gdn_occ/occ2/occ4/occ4p/occ8
 * (src/gdn_sm75.cu:57-188,577-893).  dk = dv = 128. */
int tsa_gdn_recurrent_fwd(const void* q, const void* k, const void* v, const float* g_log,
                          const float* beta, float* state, void* out, int B, int T, int Hq,
                          int Hv, int dk, int dv, float scale, void* stream);

/* The same with fp32 q, k, v, out (the reference's token-serial kernels' own I/O). */
int tsa_gdn_recurrent_fwd_f32(const float* q, const float* k, const float* v, const float* g_log,
                              const float* beta, float* state, float* out, int B, int T, int Hq,
                              int Hv, int dk, int dv, float scale, void* stream);

/* One decode step: one token for each of B sequences, q/k [B][Hq][dk], v/out [B][Hv][dv],
 * g_log/beta [B][Hv], state [B][Hv][dv][dk] updated in place.  The T = 1 case of the
 * token-serial kernels (src/gdn_sm75.cu:744-784 with one iteration). */
int tsa_gdn_decode_step(const void* q, const void* k, const void* v, const float* g_log,
                        const float* beta, float* state, void* out, int B, int Hq, int Hv,
                        int dk, int dv, float scale, void* stream);
/* The same with fp32 q, k, v, out. */
int tsa_gdn_decode_step_f32(const float* q, const float* k, const float* v, const float* g_log,
                            const float* beta, float* state, float* out, int B, int Hq, int Hv,
                            int dk, int dv, float scale, void* stream);

/* ---- The Gated DeltaNet layer's pre / post ops (the target model's layer,
 * docs/qwen38-27b.md:15).  The reference tree has no implementation of them: its inputs
 * assume they were applied (q, k L2-normalised, beta and g_log given), as llama.cpp's graph
 * does around gated_delta_net (the kernels' semantic source, src/gdn_sm75.cu:3).  Here:
 *   q, k    <- x / max(||x||_2, eps) per [dk] row
 *   g_log    = softplus(a + dt_bias[h]) * A[h]   (A = -exp(A_log); softplus passes x > 20)
 *   beta     = sigmoid(b)
 *   post:  y = x / sqrt(mean(x^2) + eps) * w * silu(z) per [dv] row
 * a, b are fp32 [B][T][Hv], dt_bias and A fp32 [Hv], w fp32 [dv]; q/k/x/z/y fp16. ---- */

/* The chunked prefill of tsa_gdn_chunked_fwd with the pre-ops fused: q, k are the raw rows
 * and a, b the raw gate projections.  The norms fold into factors the prefill already
 * applies, so the recurrence reads the raw rows with no extra pass.  Same workspace. */
int tsa_gdn_chunked_fused_fwd(const void* q, const void* k, const void* v, const float* a,
                              const float* b, const float* dt_bias, const float* A, float* state,
                              void* out, int B, int T, int Hq, int Hv, int dk, int dv, int chunk,
                              float scale, float eps, void* ws, size_t ws_bytes, void* stream);

/* tsa_gdn_decode_step with the pre-ops fused (raw q, k rows; raw a, b [B][Hv]). */
int tsa_gdn_decode_fused_step(const void* q, const void* k, const void* v, const float* a,
                              const float* b, const float* dt_bias, const float* A, float* state,
                              void* out, int B, int Hq, int Hv, int dk, int dv, float scale,
                              float eps, void* stream);

/* The pre-ops as their own pass (for tsa_gdn_recurrent_fwd and unfused callers): q_out,
 * k_out fp16 [B][T][Hq][dk]; g_log, beta fp32 [B][T][Hv].  dk = 128. */
int tsa_gdn_preprocess(const void* q, const void* k, const float* a, const float* b,
                       const float* dt_bias, const float* A, void* q_out, void* k_out,
                       float* g_log, float* beta, int B, int T, int Hq, int Hv, int dk,
                       float eps, void* stream);

/* The post-op: gated RMSNorm of the recurrence output x with the gate projection z, both
 * fp16 [B][T][Hv][dv], weight w fp32 [dv], into y (may alias x).  dv = 128. */
int tsa_gdn_gated_rmsnorm(const void* x, const void* z, const float* w, void* y, int B, int T,
                          int Hv, int dv, float eps, void* stream);

/* ---- ggml-layout adapter (the reference's kernels stand in for llama.cpp's
 * gated_delta_net, src/gdn_sm75.cu:3, docs/ggml-turing.md:15-17; ggml is not vendored, so
 * parity with ggml's own op is unpinned).  A tsa_tensor carries the fields of a
 * ggml_tensor view: ne[0] is the innermost dimension, nb[] are byte strides. ---- */
enum { TSA_TYPE_F32 = 0, TSA_TYPE_F16 = 1 }; /* ggml's GGML_TYPE_F32 / GGML_TYPE_F16 */
typedef struct tsa_tensor {
    void* data;
    int type;
    int64_t ne[4];
    size_t nb[4];
} tsa_tensor;

/* Scratch the adapter needs for these shapes (q: [S, Hk, T, B], v: [S, Hv, T, B]); 0 if
 * the shapes are invalid or unsupported. */
size_t tsa_ggml_gdn_workspace_bytes(const tsa_tensor* q, const tsa_tensor* v);

/* The recurrence on ggml views: q, k [S, Hk, T, B]; v, out [S, Hv, T, B] (fp32 or fp16,
 * any strides); g_log, beta [Hv, T, B, 1] and state, state_out [S, S, Hv, B] fp32
 * (state_out may be state itself, the same view).  S = 128; V-head h reads QK head h % Hk.
 * Dispatches on T: the decode step (T = 1), the token-serial kernel, or the chunked
 * prefill.  Dense fp16 / fp32 operands are used in place; others are gathered into ws. */
int tsa_ggml_gated_delta_net(const tsa_tensor* q, const tsa_tensor* k, const tsa_tensor* v,
                             const tsa_tensor* g_log, const tsa_tensor* beta,
                             const tsa_tensor* state, const tsa_tensor* out,
                             const tsa_tensor* state_out, float scale, void* ws,
                             size_t ws_bytes, void* stream);

/* The lab's naive GDN check on the device: one thread per state column, fp32, state read
 * and written in global memory, the order of gdn_cpu (src/gdn_sm75.cu:1078-1106) and
 * gdn_serial_kernel (:57-92).  Used by the gdn driver's error check.  Any dk, dv >= 1. */
int tsa_gdn_naive(const void* q, const void* k, const void* v, const float* g_log,
                  const float* beta, float* state, void* out, int B, int T, int Hq, int Hv,
                  int dk, int dv, float scale, void* stream);
/* The same with fp32 q, k, v, out (the gdn driver's check of its fp32 runs). */
int tsa_gdn_naive_f32(const float* q, const float* k, const float* v, const float* g_log,
                      const float* beta, float* state, float* out, int B, int T, int Hq, int Hv,
                      int dk, int dv, float scale, void* stream);

#ifdef __cplusplus
}
#endif
#endif
