// common.h -- shared device helpers for the gfx950 kernels (CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsa {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __fp16 fp16x4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

// D(32x32 fp32) += A(32x16 fp16) * B(16x32 fp16).  Lane l holds A[l%32][8*(l/32)+s] and
// B[8*(l/32)+s][l%32] in slot s, and D[8*(r/4) + 4*(l/32) + r%4][l%32] in register r.
__device__ __forceinline__ float16_t mfma32(const half8_t& a, const half8_t& b, const float16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// D(16x16 fp32) += A(16x32 fp16) * B(32x16 fp16).  Lane l holds A[l%16][8*(l/16)+s],
// B[8*(l/16)+s][l%16] in slot s, and D[4*(l/16) + r][l%16] in register r.
__device__ __forceinline__ float4_t mfma16(const half8_t& a, const half8_t& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D(16x16 fp32) += A(16x4 fp32) * B(4x16 fp32).  Lane l holds A[l%16][l/16], B[l/16][l%16],
// and D[4*(l/16) + r][l%16] in register r.
__device__ __forceinline__ float4_t mfma16f32(float a, float b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes, source lane
// s supplies the address of 4 consecutive fp16 values; result lane i, slot j receives
// element i%4 of source lane 4*j + i/4.
__device__ __forceinline__ half4_t lds_read_tr16(const half_t* p) {
    typedef __attribute__((address_space(3))) fp16x4_t* lds_ptr_t;
    fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_ptr_t)(p));
    return __builtin_bit_cast(half4_t, v);
}

// DPP lane moves within a row of 16 lanes (row_mask / bank_mask all enabled).
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- lane 7-i within each group of 8
constexpr int kDppRowMirror = 0x140;  // lane i <- lane 15-i within each row of 16

// Sum over each aligned group of 8 lanes; every lane of the group receives the total.
__device__ __forceinline__ float sum8(float x) {
    x += dpp_mov<kDppXor1>(x);
    x += dpp_mov<kDppXor2>(x);
    x += dpp_mov<kDppHalfMirror>(x);
    return x;
}

// Values of lanes l and l ^ 32 on every lane, from v_permlane32_swap (a VALU exchange of the
// two wave halves; __shfl_xor goes through ds_bpermute, an LDS round trip): on return lane l
// holds the pair as {x[l % 32], x[l % 32 + 32]}.  Inline asm, not the builtin: this compiler
// folds the builtin's second result into its first (r0 + r1 becomes r0 + r0).  The s_nop
// gives the wait states the compiler puts between a VALU write and this instruction.
__device__ __forceinline__ void halves32(float x, float& lo, float& hi) {
    unsigned a = __builtin_bit_cast(unsigned, x), b = a;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    lo = __builtin_bit_cast(float, a);
    hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_xor32(float x) {
    float a, b;
    halves32(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor32(float x) {
    float a, b;
    halves32(x, a, b);
    return a + b;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The gates of the target model's Gated DeltaNet layer: softplus(x) = log(1 + e^x), with x
// above 20 passed through (the threshold ggml and torch use), and the logistic sigmoid.
__device__ __forceinline__ float gdn_softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float gdn_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every
// outstanding global load and store of the wave (vmcnt counts both), which would drain
// prefetches issued for later iterations; use this one where no global memory written
// by one wave is read by another wave of the workgroup.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace tsa
