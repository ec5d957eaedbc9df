// attn_sm75 -- the attention lab driver, rebuilt over the tsa C-ABI.
//
//   attn_sm75 [B H S D] [--causal 0|1] [--std X] [--outlier P] [--seed N] [--iters N]
//             [--hkv N] [--gate 0|1]
//
// Mirrors main() of src/attn_sm75.cu:442-554: positional B H S D (default 2 8 512 128),
// D in {64, 128} (usage error -> exit 2), scale 1/sqrt(D), std::mt19937(seed) with
// normal_distribution(0, std) rounded to fp16 for Q, K, V in that order (seed 42, std 0.5 as
// in :398,473-476), the MFMA kernel checked against the naive kernel by max-abs error with
// the 0.02 gate, 20 timed iterations, TFLOP/s in the dense-equivalent (4 B H S^2 D) and
// causal-executed (2 B H S (S+1) D) conventions (:531-535), exit 0 iff the MFMA kernel's
// check passes.  The VALU kernel (tsa_attn_fwd_valu) is checked and timed beside it for plain
// attention, as the reference's FFMA kernel is (:486-489,500-502,521-528).
// Differences: causal is a flag (the reference hard-codes 1, :463) and S is not capped at
// 1024 (the naive check here is O(S^2 D), not O(S^2 D^2)).  --outlier P multiplies each
// element by 8 with probability P (independent mt19937(seed + 1) stream).  D = 256 is
// accepted as well.  --hkv N (H % N == 0) runs grouped-query attention with N K/V heads and
// --gate 1 multiplies the output by sigmoid(gate), gate ~ N(0, 1) drawn after V: the gated
// attention layer of the reference's target model (docs/qwen38-27b.md:13), through
// tsa_attn_gqa_fwd and checked against tsa_attn_gqa_naive.
#include "driver_util.h"

int main(int argc, char** argv) {
    Opts opt(argc, argv);
    int B = 2, H = 8, S = 512, D = 128;
    if (opt.bad || !opt.known({"causal", "std", "outlier", "seed", "iters", "hkv", "gate"}) ||
        (opt.pos.size() != 0 && opt.pos.size() != 4)) {
        std::fprintf(stderr, "usage: %s [B H S D] [--causal 0|1] [--std X] [--outlier P] [--seed N] [--iters N] [--hkv N] [--gate 0|1]\n", argv[0]);
        return 2;
    }
    if (opt.pos.size() == 4) {
        B = std::atoi(opt.pos[0].c_str());
        H = std::atoi(opt.pos[1].c_str());
        S = std::atoi(opt.pos[2].c_str());
        D = std::atoi(opt.pos[3].c_str());
    }
    const int causal = std::atoi(opt.get("causal", "1").c_str());
    const float stdv = (float)std::atof(opt.get("std", "0.5").c_str());
    const double outlier = std::atof(opt.get("outlier", "0").c_str());
    const unsigned seed = (unsigned)std::strtoul(opt.get("seed", "42").c_str(), nullptr, 10);
    const int iters = std::atoi(opt.get("iters", "20").c_str());
    const int Hkv = std::atoi(opt.get("hkv", std::to_string(H).c_str()).c_str());
    const int gate_flag = std::atoi(opt.get("gate", "0").c_str());
    const bool gated = gate_flag == 1;
    if (D != 64 && D != 128 && D != 256) {
        std::fprintf(stderr, "kernels instantiate D=64, D=128 and D=256 only\n");
        return 2;
    }
    if (B < 1 || H < 1 || S < 1 || Hkv < 1 || H % Hkv != 0 || (causal != 0 && causal != 1) ||
        (gate_flag != 0 && gate_flag != 1) || iters < 1) {
        std::fprintf(stderr, "invalid shape or option\n");
        return 2;
    }
    const float scale = 1.f / std::sqrt((float)D);
    const size_t elems = (size_t)B * H * S * D;
    const size_t kv_elems = (size_t)B * Hkv * S * D;

    print_gpu();
    std::printf("shape           : B=%d H=%d S=%d D=%d  causal=%d", B, H, S, D, causal);
    if (Hkv != H || gated) std::printf("  K/V heads=%d  gate=%d", Hkv, (int)gated);
    std::printf("\n");
    std::printf("tile            : 128 q rows x 64 keys per LDS tile, 4 waves, v_mfma_f32_32x32x16_f16\n");

    std::vector<f16> hq(elems), hk(kv_elems), hv(kv_elems), hg(gated ? elems : 0);
    {
        std::mt19937 rng(seed);
        std::mt19937 rng_o(seed + 1);
        std::uniform_real_distribution<double> u01(0.0, 1.0);
        for (std::vector<f16>* t : {&hq, &hk, &hv}) {
            std::normal_distribution<float> dist(0.f, stdv);
            for (size_t i = 0; i < t->size(); ++i) {
                float x = dist(rng);
                if (outlier > 0 && u01(rng_o) < outlier) x *= 8.f;
                (*t)[i] = (f16)x;
            }
        }
        std::normal_distribution<float> gd(0.f, 1.f);
        for (size_t i = 0; i < hg.size(); ++i) hg[i] = (f16)gd(rng);
    }
    DevBuf<f16> Q(elems), K(kv_elems), V(kv_elems), G(gated ? elems : 1), Om(elems), On(elems);
    DevBuf<f16> Of(gated || Hkv != H ? 1 : elems);
    Q.upload(hq);
    K.upload(hk);
    V.upload(hv);
    if (gated) G.upload(hg);
    const bool gqa = Hkv != H || gated;
    const void* gp = gated ? G.d : nullptr;
    auto run_mfma = [&] {
        if (gqa) DRV_TSA(tsa_attn_gqa_fwd(Q.d, K.d, V.d, gp, Om.d, B, H, Hkv, S, D, scale, causal, nullptr));
        else DRV_TSA(tsa_attn_fwd(Q.d, K.d, V.d, Om.d, B, H, S, D, scale, causal, nullptr));
    };
    // the VALU opponent (no MFMA), as the reference's launch_ffma (src/attn_sm75.cu:486-489);
    // plain attention only (the reference's lab has no grouped-query or gated variant)
    auto run_valu = [&] { DRV_TSA(tsa_attn_fwd_valu(Q.d, K.d, V.d, Of.d, B, H, S, D, scale, causal, nullptr)); };
    auto run_naive = [&] {
        if (gqa) DRV_TSA(tsa_attn_gqa_naive(Q.d, K.d, V.d, gp, On.d, B, H, Hkv, S, D, scale, causal, nullptr));
        else DRV_TSA(tsa_attn_naive(Q.d, K.d, V.d, On.d, B, H, S, D, scale, causal, nullptr));
    };

    run_mfma();
    if (!gqa) run_valu();
    run_naive();
    DRV_HIP(hipDeviceSynchronize());
    std::vector<f16> om, on, of;
    Om.download(om);
    On.download(on);
    auto max_err = [&](const std::vector<f16>& a) {
        float e = 0.f;
        for (size_t i = 0; i < elems; ++i) {
            const float d = std::fabs((float)a[i] - (float)on[i]);
            e = (d > e || d != d) ? d : e;
        }
        return e;
    };
    const float err = max_err(om);
    std::printf("max |mfma-naive| : %.5f   %s\n", err, err < 2e-2f ? "OK" : "FAIL");
    if (!gqa) {
        Of.download(of);
        const float err_v = max_err(of);
        std::printf("max |valu-naive| : %.5f   %s\n", err_v, err_v < 2e-2f ? "OK" : "FAIL");
    }

    const float mfma_ms = time_ms(run_mfma, iters);
    const float valu_ms = gqa ? 0.f : time_ms(run_valu, iters);
    const int naive_iters = S > 2048 ? 1 : iters;
    const float naive_ms = time_ms(run_naive, naive_iters);

    const double flops_dense = 4.0 * B * H * (double)S * S * D;
    const double flops_exec = causal ? 2.0 * B * H * (double)S * (S + 1.0) * D : flops_dense;
    auto tflops = [](double f, float ms) { return f / (ms * 1e-3) / 1e12; };
    std::printf("mfma  (gfx950)  : %8.4f ms   %7.1f TFLOP/s dense-eq   %7.1f %s\n", mfma_ms,
                tflops(flops_dense, mfma_ms), tflops(flops_exec, mfma_ms),
                causal ? "causal-exec" : "executed");
    if (!gqa)
        std::printf("valu  (gfx950)  : %8.4f ms   %7.1f TFLOP/s dense-eq   %7.1f %s\n", valu_ms,
                    tflops(flops_dense, valu_ms), tflops(flops_exec, valu_ms),
                    causal ? "causal-exec" : "executed");
    std::printf("naive oracle    : %8.4f ms   (not a realistic fallback)\n", naive_ms);
    if (!gqa) std::printf("mfma vs valu    : %.2fx  (same FLOP convention both sides)\n", valu_ms / mfma_ms);
    std::printf("mfma vs naive   : %.2fx\n", naive_ms / mfma_ms);
    return err < 2e-2f ? 0 : 1;
}
