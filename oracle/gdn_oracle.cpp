// gdn_oracle.cpp -- CPU restatement of the reference's Gated DeltaNet host paths.
// TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the product.
//
//   orc_gdn_serial      : gdn_cpu          (src/gdn_sm75.cu:1078-1106)
//   orc_gdn_chunked_*   : gdn_chunked_cpu  (src/gdn_sm75.cu:1109-1244), chunk size C,
//                         with either the exact (I + A)^-1 or the reference's solve loop.
//
// Recurrence (src/gdn_sm75.cu:6-11): per token, g = exp(g_log);
//   kv = S^T k;  d = (v - g*kv)*beta;  S = g*S + k (x) d;  out = scale * S^T q.
// The host reference is compiled without FMA contraction, so this file is built with
// -ffp-contract=off and keeps the reference's summation order.
#include <cmath>
#include <vector>

#include "oracle.h"

extern "C" void orc_gdn_serial(const float* q, const float* k, const float* v,
                               const float* g_log, const float* beta, float* state, float* out,
                               int B, int T, int Hq, int Hv, int dk, int dv, float scale,
                               int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
    for (int bh = 0; bh < B * Hv; ++bh) {
        const int b = bh / Hv, h = bh % Hv;
        const int hq = h % Hq;  // :1085
        float* Sg = state + (size_t)bh * dv * dk;
        std::vector<float> S(Sg, Sg + (size_t)dv * dk);  // :1086-1087
        for (int t = 0; t < T; ++t) {
            const size_t bt = (size_t)b * T + t;
            const float* qt = q + (bt * Hq + hq) * dk;   // :1089
            const float* kt = k + (bt * Hq + hq) * dk;   // :1090
            const float* vt = v + (bt * Hv + h) * dv;    // :1091
            const float g = std::exp(g_log[bt * Hv + h]);  // :1092
            const float bb = beta[bt * Hv + h];            // :1093
            for (int c = 0; c < dv; ++c) {
                float* Sc = S.data() + (size_t)c * dk;
                float kv = 0.f;
                for (int i = 0; i < dk; ++i) kv += Sc[i] * kt[i];  // :1095-1096
                const float d = (vt[c] - g * kv) * bb;              // :1097
                float attn = 0.f;
                for (int i = 0; i < dk; ++i) {                      // :1098-1101
                    Sc[i] = g * Sc[i] + kt[i] * d;
                    attn += Sc[i] * qt[i];
                }
                out[(bt * Hv + h) * dv + c] = attn * scale;  // :1102
            }
        }
        for (size_t i = 0; i < (size_t)dv * dk; ++i) Sg[i] = S[i];  // :1104
    }
}

namespace {

// The reference's solve (src/gdn_sm75.cu:1161-1180) written out: lhs = I + strict part
// of kb (ggml [i + j*C] order), forward substitution column by column, attn = X + I.
template <typename R>
void ref_solve(const R* kb, R* attn, int C) {
    std::vector<R> lhs((size_t)C * C), X((size_t)C * C);
    for (int j = 0; j < C; ++j)
        for (int i = 0; i < C; ++i)
            lhs[i + j * C] = ((i < j) ? kb[i + j * C] : R(0)) + (i == j ? R(1) : R(0));
    for (int colj = 0; colj < C; ++colj) {
        for (int r = 0; r < C; ++r) {
            R sum = 0;
            for (int p = 0; p < r; ++p) sum += lhs[p + r * C] * X[p + colj * C];
            const R bb = (r < colj) ? -kb[r + colj * C] : R(0);
            X[r + colj * C] = (bb - sum) / lhs[r + r * C];
        }
    }
    for (int j = 0; j < C; ++j)
        for (int i = 0; i < C; ++i) attn[i + j * C] = X[i + j * C] + (i == j ? R(1) : R(0));
}

// Exact solve in the same storage: attn[i + t*C] = Tm[t][i] with Tm = (I + A)^-1 and
// A[t][s] = kb[s + t*C] for s < t (strictly lower, unit diagonal after adding I).  This is
// what makes the chunk form equal to the serial recurrence (derivation in the header of
// tests/test_oracle_gdn.py).
template <typename R>
void exact_solve(const R* kb, R* attn, int C) {
    // Forward substitution on rows: Tm[t][i] = delta_ti - sum_{i<=s<t} A[t][s] Tm[s][i].
    std::vector<R> Tm((size_t)C * C, R(0));
    for (int t = 0; t < C; ++t) {
        Tm[(size_t)t * C + t] = 1;
        for (int i = 0; i < t; ++i) {
            R acc = 0;
            for (int s = i; s < t; ++s) acc += kb[s + t * C] * Tm[(size_t)s * C + i];
            Tm[(size_t)t * C + i] = -acc;
        }
    }
    for (int t = 0; t < C; ++t)
        for (int i = 0; i < C; ++i) attn[i + t * C] = Tm[(size_t)t * C + i];
}

template <typename R>
void gdn_chunked(const float* q, const float* k, const float* v, const float* g_log,
                 const float* beta, float* state, float* out, int B, int T, int Hq, int Hv,
                 int dk, int dv, int C, float scale, int exact, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    const int nch = (T + C - 1) / C;  // :1112
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
    for (int bh = 0; bh < B * Hv; ++bh) {
        const int b = bh / Hv, h = bh % Hv;
        const int hq = h % Hq;
        float* Sg = state + (size_t)bh * dv * dk;
        std::vector<R> S(Sg, Sg + (size_t)dv * dk);  // S[c*dk + i]
        std::vector<R> qc((size_t)C * dk), kc((size_t)C * dk), vc((size_t)C * dv);
        std::vector<R> gl(C), bt(C), gcs(C), kb((size_t)C * C), kq((size_t)C * C),
            attn((size_t)C * C);
        std::vector<R> vmix((size_t)C * dv), kcd((size_t)C * dk), vnew((size_t)C * dv),
            Sn((size_t)dv * dk);
        for (int ch = 0; ch < nch; ++ch) {
            const int t0 = ch * C;
            // Gather the chunk; tokens past T are zero (:1121-1137).
            for (int t = 0; t < C; ++t) {
                const int tt = t0 + t;
                const bool ok = tt < T;
                const size_t bt_ = (size_t)b * T + tt;
                for (int i = 0; i < dk; ++i) {
                    qc[(size_t)t * dk + i] = ok ? q[(bt_ * Hq + hq) * dk + i] : 0.f;
                    kc[(size_t)t * dk + i] = ok ? k[(bt_ * Hq + hq) * dk + i] : 0.f;
                }
                for (int c = 0; c < dv; ++c) vc[(size_t)t * dv + c] = ok ? v[(bt_ * Hv + h) * dv + c] : 0.f;
                gl[t] = ok ? g_log[bt_ * Hv + h] : 0.f;
                bt[t] = ok ? beta[bt_ * Hv + h] : 0.f;
            }
            gcs[0] = gl[0];  // :1139-1141
            for (int t = 1; t < C; ++t) gcs[t] = gcs[t - 1] + gl[t];
            // kb[i + j*C] = (k_i.k_j) beta_j exp(G_j - G_i), kq[i + j*C] = (k_i.q_j) exp(G_j - G_i),
            // both for i <= j (:1143-1158).
            for (int j = 0; j < C; ++j) {
                for (int i = 0; i < C; ++i) {
                    const R mask = (i <= j) ? std::exp(gcs[j] - gcs[i]) : R(0);
                    R dkk = 0, dq = 0;
                    for (int d = 0; d < dk; ++d) {
                        dkk += kc[(size_t)i * dk + d] * kc[(size_t)j * dk + d];
                        dq += kc[(size_t)i * dk + d] * qc[(size_t)j * dk + d];
                    }
                    kb[i + j * C] = dkk * bt[j] * mask;
                    kq[i + j * C] = (i <= j) ? dq * mask : R(0);
                }
            }
            if (exact) exact_solve<R>(kb.data(), attn.data(), C);
            else ref_solve<R>(kb.data(), attn.data(), C);
            // vmix_t = sum_i attn[i + t*C] beta_i v_i ; kcd_t = sum_i attn[i + t*C] beta_i e^{G_i} k_i
            // (:1182-1195)
            for (int t = 0; t < C; ++t) {
                for (int c = 0; c < dv; ++c) {
                    R vm = 0;
                    for (int i = 0; i < C; ++i) vm += vc[(size_t)i * dv + c] * bt[i] * attn[i + t * C];
                    vmix[(size_t)t * dv + c] = vm;
                }
                for (int d = 0; d < dk; ++d) {
                    R kk = 0;
                    for (int i = 0; i < C; ++i)
                        kk += kc[(size_t)i * dk + d] * bt[i] * std::exp(gcs[i]) * attn[i + t * C];
                    kcd[(size_t)t * dk + d] = kk;
                }
            }
            const R g_last = gcs[C - 1];
            // vnew_t[c] = vmix_t[c] - sum_i kcd_t[i] S[c][i]   (:1209-1216)
            for (int t = 0; t < C; ++t)
                for (int c = 0; c < dv; ++c) {
                    R vp = 0;
                    for (int i = 0; i < dk; ++i) vp += kcd[(size_t)t * dk + i] * S[(size_t)c * dk + i];
                    vnew[(size_t)t * dv + c] = vmix[(size_t)t * dv + c] - vp;
                }
            // out_t[c] = scale*(sum_i S[c][i] q_t[i] e^{G_t} + sum_i vnew_i[c] kq[i + t*C])  (:1218-1228)
            for (int t = 0; t < C; ++t) {
                const int tt = t0 + t;
                if (tt >= T) continue;
                const R eg = std::exp(gcs[t]);
                for (int c = 0; c < dv; ++c) {
                    R va = 0, ai = 0;
                    for (int i = 0; i < C; ++i) va += vnew[(size_t)i * dv + c] * kq[i + t * C];
                    for (int i = 0; i < dk; ++i) ai += S[(size_t)c * dk + i] * (qc[(size_t)t * dk + i] * eg);
                    out[(((size_t)b * T + tt) * Hv + h) * dv + c] = (float)((ai + va) * scale);
                }
            }
            // S[c][a] = e^{G_last} S[c][a] + sum_t k_t[a] e^{G_last - G_t} vnew_t[c]  (:1230-1241)
            const R ge = std::exp(g_last);
            for (int c = 0; c < dv; ++c)
                for (int a = 0; a < dk; ++a) {
                    R add = 0;
                    for (int t = 0; t < C; ++t)
                        add += kc[(size_t)t * dk + a] * std::exp(g_last - gcs[t]) * vnew[(size_t)t * dv + c];
                    Sn[(size_t)c * dk + a] = ge * S[(size_t)c * dk + a] + add;
                }
            S.swap(Sn);
        }
        for (size_t i = 0; i < (size_t)dv * dk; ++i) Sg[i] = (float)S[i];
    }
}

}  // namespace

extern "C" void orc_gdn_chunked_f64(const float* q, const float* k, const float* v,
                                    const float* g_log, const float* beta, float* state,
                                    float* out, int B, int T, int Hq, int Hv, int dk, int dv,
                                    int C, float scale, int exact_solve, int nthreads) {
    gdn_chunked<double>(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, C, scale,
                        exact_solve, nthreads);
}

extern "C" void orc_gdn_chunked_f32(const float* q, const float* k, const float* v,
                                    const float* g_log, const float* beta, float* state,
                                    float* out, int B, int T, int Hq, int Hv, int dk, int dv,
                                    int C, float scale, int exact_solve, int nthreads) {
    gdn_chunked<float>(q, k, v, g_log, beta, state, out, B, T, Hq, Hv, dk, dv, C, scale,
                       exact_solve, nthreads);
}

extern "C" void orc_ref_solve(const float* kb, float* attn, int C) {
    ref_solve<float>(kb, attn, C);
}
