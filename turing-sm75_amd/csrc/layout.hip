// layout.hip -- strided 4-D copies with a type change, for the ggml-layout adapter
// (ggml_adapter.cpp).  A ggml tensor view is (ne[4], nb[4]): ne[0] is the innermost
// dimension, nb[i] the byte stride of dimension i.  These kernels move a view into a dense
// buffer of the kernels' own layout or back, converting fp32 <-> fp16 on the way.  One
// thread per element (row-major over ne[3..0]); the index arithmetic is 64-bit.  They are
// HBM-bound passes that exist only when the caller's tensors are not already in the
// kernels' dense fp16 layout.
#include "common.h"
#include "kernels.h"

namespace tsa {
namespace {

template <typename Tin, typename Tout>
__global__ void __launch_bounds__(256)
copy4d_kernel(const unsigned char* __restrict__ src, unsigned char* __restrict__ dst, View4 s,
              View4 d, long long n) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const long long i0 = i % s.ne[0];
    const long long r1 = i / s.ne[0];
    const long long i1 = r1 % s.ne[1];
    const long long r2 = r1 / s.ne[1];
    const long long i2 = r2 % s.ne[2];
    const long long i3 = r2 / s.ne[2];
    const Tin x = *reinterpret_cast<const Tin*>(src + i0 * s.nb[0] + i1 * s.nb[1] + i2 * s.nb[2] + i3 * s.nb[3]);
    *reinterpret_cast<Tout*>(dst + i0 * d.nb[0] + i1 * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3]) = (Tout)x;
}

}  // namespace

hipError_t copy4d(const void* src, int src_f16, const View4& s, void* dst, int dst_f16,
                  const View4& d, hipStream_t stream) {
    const long long n = s.ne[0] * s.ne[1] * s.ne[2] * s.ne[3];
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    auto S = static_cast<const unsigned char*>(src);
    auto D = static_cast<unsigned char*>(dst);
    if (src_f16 && dst_f16)
        hipLaunchKernelGGL((copy4d_kernel<half_t, half_t>), grid, dim3(256), 0, stream, S, D, s, d, n);
    else if (src_f16)
        hipLaunchKernelGGL((copy4d_kernel<half_t, float>), grid, dim3(256), 0, stream, S, D, s, d, n);
    else if (dst_f16)
        hipLaunchKernelGGL((copy4d_kernel<float, half_t>), grid, dim3(256), 0, stream, S, D, s, d, n);
    else
        hipLaunchKernelGGL((copy4d_kernel<float, float>), grid, dim3(256), 0, stream, S, D, s, d, n);
    return hipGetLastError();
}

}  // namespace tsa
