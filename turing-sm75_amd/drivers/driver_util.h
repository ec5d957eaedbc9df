// driver_util.h -- small helpers shared by the attn_sm75 and gdn lab drivers.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "tsa.h"

// HIP runtime failures in a driver: message and exit(1), as CUDA_CHECK does in the
// reference drivers (src/attn_sm75.cu:40-48).
#define DRV_HIP(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess) {                                                           \
            std::fprintf(stderr, "HIP %s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

// Library failures: message and exit(1).
#define DRV_TSA(expr)                                                                     \
    do {                                                                                  \
        int rc_ = (expr);                                                                 \
        if (rc_ != TSA_OK) {                                                              \
            std::fprintf(stderr, "tsa %s:%d: %s\n", __FILE__, __LINE__, tsa_strerror(rc_)); \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

typedef _Float16 f16;

template <typename T>
struct DevBuf {
    T* d = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t n_) : n(n_) { DRV_HIP(hipMalloc(&d, n * sizeof(T) + 16)); }
    ~DevBuf() { (void)hipFree(d); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    void upload(const std::vector<T>& h) { DRV_HIP(hipMemcpy(d, h.data(), n * sizeof(T), hipMemcpyHostToDevice)); }
    void download(std::vector<T>& h) const {
        h.resize(n);
        DRV_HIP(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    }
};

inline void print_gpu() {
    hipDeviceProp_t prop{};
    DRV_HIP(hipGetDeviceProperties(&prop, 0));
    std::printf("GPU             : %s  (%s, %d CUs)\n", prop.name, prop.gcnArchName,
                prop.multiProcessorCount);
}

// Average milliseconds per call of fn over iters calls, timed with HIP events on the
// default stream after one untimed call.
template <typename F>
float time_ms(F&& fn, int iters) {
    fn();
    hipEvent_t e0, e1;
    DRV_HIP(hipEventCreate(&e0));
    DRV_HIP(hipEventCreate(&e1));
    DRV_HIP(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i) fn();
    DRV_HIP(hipEventRecord(e1, nullptr));
    DRV_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    DRV_HIP(hipEventElapsedTime(&ms, e0, e1));
    DRV_HIP(hipEventDestroy(e0));
    DRV_HIP(hipEventDestroy(e1));
    return ms / iters;
}

// "--name value" options after the positional arguments.
struct Opts {
    std::vector<std::string> pos;
    std::vector<std::pair<std::string, std::string>> kv;
    bool bad = false;
    Opts(int argc, char** argv) {
        for (int i = 1; i < argc; ++i) {
            if (std::strncmp(argv[i], "--", 2) == 0) {
                if (i + 1 >= argc) { bad = true; return; }
                kv.emplace_back(argv[i] + 2, argv[i + 1]);
                ++i;
            } else {
                pos.emplace_back(argv[i]);
            }
        }
    }
    std::string get(const char* name, const char* def) const {
        for (auto& p : kv)
            if (p.first == name) return p.second;
        return def;
    }
    bool known(std::initializer_list<const char*> names) const {
        for (auto& p : kv) {
            bool ok = false;
            for (auto n : names) ok = ok || p.first == n;
            if (!ok) return false;
        }
        return true;
    }
};
