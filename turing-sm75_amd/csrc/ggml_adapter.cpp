// ggml_adapter.cpp -- tsa_ggml_gated_delta_net: the Gated DeltaNet recurrence called with
// ggml-style tensor views, for a llama.cpp / ggml HIP backend (the product the reference's
// kernels stand in for: src/gdn_sm75.cu:3 "matching llama.cpp gated_delta_net.cu",
// docs/ggml-turing.md:15-17).
//
// A view is (data, type, ne[4], nb[4]) with ne[0] innermost and nb[] byte strides, the
// fields of ggml_tensor.  In ggml's order the operands are
//   q, k   [S, Hk, T, B]    v, out  [S, Hv, T, B]    g_log, beta  [Hv, T, B, 1]
//   state, state_out  [S, S, Hv, B]  (ne[0] = the k index: S[b][h][c][i], the reference's
//                                     [Hv][dv][dk] state per sequence, src/gdn_sm75.cu:71-72)
// with S = 128.  q / k / v / out may be fp32 (ggml's op) or fp16 and any strides (views
// into a fused projection); g_log, beta and the states are fp32.  When any of q / k / v / out
// is fp32 the kernels run with fp32 I/O (fp16 operands are widened, exactly), so fp32
// operands are never narrowed; when all four are fp16 they run with fp16 I/O.  Operands
// already in the kernels' dense layout are used in place; the others are gathered into the
// caller's workspace (and the output scattered back) by strided copy kernels.  state_out
// may be the same buffer as state (in place).
//
// Dispatch on the tokens per sequence T: one token -> the decode kernel; T below
// kChunkedMinT -> the token-serial kernel (state on chip for all T); otherwise the chunked
// prefill.  Nothing is allocated: every scratch buffer is carved from `ws`.
#include <climits>
#include <cmath>
#include <cstdint>

#include "../../include/tsa.h"
#include "kernels.h"

namespace {

constexpr int64_t kS = 128;
// Token count from which the chunked prefill is used.  Measured on MI355X at the target
// model's 16 QK / 48 V heads (token-serial vs chunked, us per call): one sequence T=32
// 15.5 vs 17.2, T=48 22.0 vs 16.4; four sequences T=16 17.4 vs 22.5, T=32 30.2 vs 23.5.
// One threshold at 32 costs at most ~2 us against the better kernel on either side.
constexpr int64_t kChunkedMinT = 32;

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

size_t esize(int type) { return type == TSA_TYPE_F16 ? 2 : 4; }

bool dense(const tsa_tensor& t) {
    const size_t e = esize(t.type);
    return t.nb[0] == e && t.nb[1] == e * (size_t)t.ne[0] && t.nb[2] == t.nb[1] * (size_t)t.ne[1] &&
           t.nb[3] == t.nb[2] * (size_t)t.ne[2];
}

tsa::View4 view_of(const tsa_tensor& t) {
    tsa::View4 v;
    for (int i = 0; i < 4; ++i) {
        v.ne[i] = t.ne[i];
        v.nb[i] = (long long)t.nb[i];
    }
    return v;
}

tsa::View4 dense_view(const int64_t (&ne)[4], size_t e) {
    tsa::View4 v;
    long long stride = (long long)e;
    for (int i = 0; i < 4; ++i) {
        v.ne[i] = ne[i];
        v.nb[i] = stride;
        stride *= ne[i];
    }
    return v;
}

bool same_ne(const tsa_tensor& t, int64_t a, int64_t b, int64_t c, int64_t d) {
    return t.ne[0] == a && t.ne[1] == b && t.ne[2] == c && t.ne[3] == d;
}

// Workspace layout: dense q, k, v, out in the I/O type (fp16, or fp32 when f32); dense fp32
// g_log, beta, state; the chunked prefill's workspace.  Each piece is 256-byte aligned and
// sized for the worst case (every operand copied), so the size depends on the shapes only.
struct Plan {
    int64_t B, T, Hk, Hv;
    size_t q, k, v, out, g, beta, state, chunk, total;
};

Plan plan(int64_t B, int64_t T, int64_t Hk, int64_t Hv, bool f32) {
    Plan p{B, T, Hk, Hv, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const size_t e = f32 ? 4 : 2;
    const size_t qk = (size_t)(B * T * Hk * kS) * e, vo = (size_t)(B * T * Hv * kS) * e;
    const size_t gb = (size_t)(B * T * Hv) * 4, st = (size_t)(B * Hv * kS * kS) * 4;
    size_t off = 0;
    p.q = off;     off += align256(qk);
    p.k = off;     off += align256(qk);
    p.v = off;     off += align256(vo);
    p.out = off;   off += align256(vo);
    p.g = off;     off += align256(gb);
    p.beta = off;  off += align256(gb);
    p.state = off; off += align256(st);
    p.chunk = off;
    if (T >= kChunkedMinT) off += tsa::gdn_chunked_ws_bytes((int)B, (int)T, (int)Hv, f32);
    p.total = off;
    return p;
}

bool fits(int64_t B, int64_t T, int64_t Hk, int64_t Hv) {
    // element counts of the largest operand, and the kernels' int workgroup counts
    const int64_t lim = (int64_t)INT_MAX;
    if (B > lim || T > lim || Hk > lim || Hv > lim) return false;
    if (B * Hv > lim / kS || B * T > lim) return false;
    return B * T * (Hk > Hv ? Hk : Hv) <= lim;
}

int check(const tsa_tensor* q, const tsa_tensor* k, const tsa_tensor* v, const tsa_tensor* g,
          const tsa_tensor* beta, const tsa_tensor* state, const tsa_tensor* out,
          const tsa_tensor* state_out, float scale) {
    const tsa_tensor* all[8] = {q, k, v, g, beta, state, out, state_out};
    for (const tsa_tensor* t : all)
        if (!t || !t->data) return TSA_ERR_NULL;
    for (const tsa_tensor* t : all) {
        if (t->type != TSA_TYPE_F32 && t->type != TSA_TYPE_F16) return TSA_ERR_ARG;
        for (int i = 0; i < 4; ++i)
            if (t->ne[i] < 1) return TSA_ERR_SHAPE;
    }
    for (const tsa_tensor* t : {g, beta, state, state_out})
        if (t->type != TSA_TYPE_F32) return TSA_ERR_UNSUPPORTED;
    const int64_t S = q->ne[0], Hk = q->ne[1], T = q->ne[2], B = q->ne[3], Hv = v->ne[1];
    if (!same_ne(*k, S, Hk, T, B) || !same_ne(*v, v->ne[0], Hv, T, B) || !same_ne(*out, v->ne[0], Hv, T, B) ||
        !same_ne(*g, Hv, T, B, 1) || !same_ne(*beta, Hv, T, B, 1) ||
        !same_ne(*state, S, v->ne[0], Hv, B) || !same_ne(*state_out, S, v->ne[0], Hv, B))
        return TSA_ERR_SHAPE;
    if (S != kS || v->ne[0] != kS) return TSA_ERR_UNSUPPORTED;
    // in place means the very same view
    if (state->data == state_out->data)
        for (int i = 0; i < 4; ++i)
            if (state->nb[i] != state_out->nb[i]) return TSA_ERR_ARG;
    if (!std::isfinite(scale)) return TSA_ERR_ARG;
    if (!fits(B, T, Hk, Hv)) return TSA_ERR_SHAPE;
    return TSA_OK;
}

}  // namespace

extern "C" size_t tsa_ggml_gdn_workspace_bytes(const tsa_tensor* q, const tsa_tensor* v) {
    if (!q || !v) return 0;
    for (int i = 0; i < 4; ++i)
        if (q->ne[i] < 1 || v->ne[i] < 1) return 0;
    if (q->ne[0] != kS || v->ne[0] != kS || !fits(q->ne[3], q->ne[2], q->ne[1], v->ne[1])) return 0;
    // the fp32-I/O plan is the larger one: enough whatever the operands' types
    return plan(q->ne[3], q->ne[2], q->ne[1], v->ne[1], true).total;
}

extern "C" int tsa_ggml_gated_delta_net(const tsa_tensor* q, const tsa_tensor* k, const tsa_tensor* v,
                                        const tsa_tensor* g, const tsa_tensor* beta,
                                        const tsa_tensor* state, const tsa_tensor* out,
                                        const tsa_tensor* state_out, float scale, void* ws,
                                        size_t ws_bytes, void* stream) {
    int rc = check(q, k, v, g, beta, state, out, state_out, scale);
    if (rc) return rc;
    const bool f32 = q->type == TSA_TYPE_F32 || k->type == TSA_TYPE_F32 || v->type == TSA_TYPE_F32 ||
                     out->type == TSA_TYPE_F32;
    const Plan p = plan(q->ne[3], q->ne[2], q->ne[1], v->ne[1], f32);
    if (!ws || ws_bytes < p.total) return TSA_ERR_WORKSPACE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    unsigned char* w = static_cast<unsigned char*>(ws);
    hipError_t e = hipSuccess;
    auto ok = [&]() { return e == hipSuccess; };

    // operands in the kernels' layout: used in place when already dense, else gathered
    auto operand = [&](const tsa_tensor& t, size_t off, bool f16) -> void* {
        if (dense(t) && (t.type == TSA_TYPE_F16) == f16) return t.data;
        void* dst = w + off;
        if (ok()) e = tsa::copy4d(t.data, t.type == TSA_TYPE_F16, view_of(t), dst, f16 ? 1 : 0,
                                  dense_view(t.ne, f16 ? 2 : 4), st);
        return dst;
    };
    const void* qd = operand(*q, p.q, !f32);
    const void* kd = operand(*k, p.k, !f32);
    const void* vd = operand(*v, p.v, !f32);
    const float* gd = static_cast<const float*>(operand(*g, p.g, false));
    const float* bd = static_cast<const float*>(operand(*beta, p.beta, false));
    // the state the kernels update in place: state_out itself when it is dense, else scratch
    float* sd = dense(*state_out) ? static_cast<float*>(state_out->data)
                                  : reinterpret_cast<float*>(w + p.state);
    if (ok() && !(state->data == static_cast<void*>(sd) && dense(*state)))
        e = tsa::copy4d(state->data, 0, view_of(*state), sd, 0, dense_view(state->ne, 4), st);
    const bool out_direct = dense(*out) && (out->type == TSA_TYPE_F32) == f32;
    void* od = out_direct ? out->data : static_cast<void*>(w + p.out);
    if (!ok()) return TSA_ERR_LAUNCH;

    const int B = (int)p.B, T = (int)p.T, Hk = (int)p.Hk, Hv = (int)p.Hv;
    if (T >= kChunkedMinT)
        e = tsa::gdn_chunked(qd, kd, vd, gd, bd, sd, od, B, T, Hk, Hv, scale, w + p.chunk, f32, st);
    else  // T == 1 takes the decode kernel inside gdn_recurrent
        e = tsa::gdn_recurrent(qd, kd, vd, gd, bd, sd, od, B, T, Hk, Hv, scale, f32, st);
    if (ok() && !out_direct)
        e = tsa::copy4d(od, f32 ? 0 : 1, dense_view(out->ne, f32 ? 4 : 2), out->data,
                        out->type == TSA_TYPE_F16, view_of(*out), st);
    if (ok() && sd != state_out->data)
        e = tsa::copy4d(sd, 0, dense_view(state_out->ne, 4), state_out->data, 0, view_of(*state_out), st);
    return ok() ? TSA_OK : TSA_ERR_LAUNCH;
}
