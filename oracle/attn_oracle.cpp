// attn_oracle.cpp -- CPU restatement of naive_attn_kernel (src/attn_sm75.cu:55-94).
// TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the product.
//
// The reference kernel computes, per (bh, query row q):
//   m   = max_k scale*(q . k)              over k <= q when causal   (:67-76)
//   l   = sum_k exp(scale*(q . k) - m)                                (:78-90)
//   acc = sum_k exp(scale*(q . k) - m) * V[k][d]     for each d
//   O   = half(acc / l)                                               (:91)
// It recomputes the dot product inside the d loop (:84-87); every recomputation yields
// the same fp32 value, so this restatement computes each dot once (O(S*D) per row)
// and produces the same numbers.  The kernel is device code built with nvcc's default
// FMA contraction, so the dot is a chain of fmaf in d order and the exponent argument
// is fmaf(dot, scale, -m).
#include <cmath>
#include <vector>

#include "oracle.h"

namespace {

inline float h2f(uint16_t h) {
    float f;
    orc_h2f(&h, &f, 1);
    return f;
}

void attn_row(const float* Qf_row, const float* Kf, const float* Vf, int S, int D, int qi,
              float scale, int causal, float* scores, float* acc_out) {
    const int kend = causal ? (qi + 1 < S ? qi + 1 : S) : S;
    float m = -INFINITY;
    for (int k = 0; k < kend; ++k) {
        const float* kr = Kf + (size_t)k * D;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot = std::fma(Qf_row[d], kr[d], dot);
        scores[k] = dot;
        m = std::fmax(m, dot * scale);
    }
    float l = 0.f;
    for (int d = 0; d < D; ++d) acc_out[d] = 0.f;
    // The reference accumulates l and acc in k order for every d; l is the same sum for
    // each d, so it is accumulated once here.
    for (int k = 0; k < kend; ++k) {
        const float p = std::exp(std::fma(scores[k], scale, -m));
        l += p;
        const float* vr = Vf + (size_t)k * D;
        for (int d = 0; d < D; ++d) acc_out[d] = std::fma(p, vr[d], acc_out[d]);
    }
    for (int d = 0; d < D; ++d) acc_out[d] = acc_out[d] / l;
}

}  // namespace

extern "C" void orc_attn_rows(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int B,
                              int H, int S, int D, float scale, int causal,
                              const int64_t* rows, int64_t nrows, float* o_f32,
                              uint16_t* o_h16, int nthreads) {
    (void)B;
    (void)H;
    if (nthreads < 1) nthreads = 1;
    // Rows are grouped by head so each head's K/V are converted once per group.
    int64_t start = 0;
    while (start < nrows) {
        const int64_t bh = rows[start] / S;
        int64_t end = start;
        while (end < nrows && rows[end] / S == bh) ++end;
        const size_t off = (size_t)bh * S * D;
        std::vector<float> Kf((size_t)S * D), Vf((size_t)S * D);
        orc_h2f(K + off, Kf.data(), (size_t)S * D);
        orc_h2f(V + off, Vf.data(), (size_t)S * D);
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 4)
        for (int64_t r = start; r < end; ++r) {
            const int qi = (int)(rows[r] % S);
            std::vector<float> qf(D), scores(S), acc(D);
            for (int d = 0; d < D; ++d) qf[d] = h2f(Q[off + (size_t)qi * D + d]);
            attn_row(qf.data(), Kf.data(), Vf.data(), S, D, qi, scale, causal, scores.data(),
                     acc.data());
            if (o_f32)
                for (int d = 0; d < D; ++d) o_f32[(size_t)r * D + d] = acc[d];
            if (o_h16) orc_f2h(acc.data(), o_h16 + (size_t)r * D, (size_t)D);
        }
        start = end;
    }
}

extern "C" void orc_attn_naive(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                               uint16_t* O, int B, int H, int S, int D, float scale, int causal,
                               int nthreads) {
    const int64_t n = (int64_t)B * H * S;
    std::vector<int64_t> rows(n);
    for (int64_t i = 0; i < n; ++i) rows[i] = i;
    orc_attn_rows(Q, K, V, B, H, S, D, scale, causal, rows.data(), n, nullptr, O, nthreads);
}
