// ffn_kernels.hip -- the float steps around the ternary matmuls of a BitNet-style feed-forward block
// on gfx950: RMSNorm (optionally fused with the int8 activation quantisation that feeds the
// up-projection) and SwiGLU.
//
// Semantics follow the reference's CPU routines (src/simd_math.cpp): RMSNorm
//   out[i] = in[i] * inv * w[i],  inv = 1 / sqrt(sum(in^2) / size + eps)          (:7-12, :14-38)
// and SwiGLU over interleaved pairs out[i] = silu(in[2i]) * in[2i+1],
//   silu(g) = g / (1 + exp(-g))                                                     (:40-46).
// The sum of squares is a parallel tree here (the reference sums sequentially, or in 8 AVX2 lanes),
// so results agree to float rounding, not bit for bit -- the reference's own test tolerance between
// its scalar and AVX2 versions is 1e-4 relative (tests/test_simd_math.cpp:17-27).
// Both kernels are HBM streams: one workgroup per row for RMSNorm (two reads of the row, the second
// from cache), a flat grid for SwiGLU.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "row_stats.h"
#include "ternary_kernels.h"

namespace ternix_hip {
namespace {

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ X, const float* __restrict__ W,
                                                      float eps, float* __restrict__ out, int8_t* __restrict__ Q,
                                                      float* __restrict__ row_scale, int K) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* x = X + (size_t)m * (size_t)K;
    const float inv = row_rms_inv(x, K, eps, red);
    if (Q == nullptr) {
        float* o = out + (size_t)m * (size_t)K;
        for (int k = threadIdx.x; k < K; k += 256) o[k] = row_value(x, W, inv, k);
        return;
    }
    // Fused quantisation of the normalised row (the rule of quantize_rows_kernel).
    const float a = fmaxf(row_absmax(x, W, inv, K, red), 1e-5f);
    const float s = 127.0f / a;
    if (threadIdx.x == 0) row_scale[m] = a / 127.0f;
    int8_t* q = Q + (size_t)m * (size_t)K;
    for (int k = threadIdx.x; k < K; k += 256) q[k] = (int8_t)quantize_value(row_value(x, W, inv, k), s);
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                     size_t pairs) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pairs) return;
    const float g = in[2 * i], u = in[2 * i + 1];
    out[i] = (g / (1.0f + expf(-g))) * u;
}

}  // namespace

hipError_t launch_rmsnorm(const float* X, const float* W, float eps, float* out, int8_t* Q, float* row_scale, int M,
                          int K, hipStream_t st) {
    if (M == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)M), dim3(256), 0, st, X, W, eps, out, Q, row_scale, K);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* in, float* out, size_t pairs, hipStream_t st) {
    if (pairs == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, st, in, out, pairs);
    return hipGetLastError();
}

}  // namespace ternix_hip
