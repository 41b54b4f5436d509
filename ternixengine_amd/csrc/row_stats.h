// row_stats.h -- per-row statistics of fp32 activations shared by every kernel that normalises or
// quantises a row (ffn_kernels.hip, quantize_rows_kernel in layer_kernels.hip, and the skinny GEMVs'
// fused activation prologue in skinny_kernels.hip).  All of them run 256-thread workgroups and use
// exactly these loops, so the same row gives the same bits whichever kernel computes it:
//   sum of squares: per-thread fmaf over k = tid, tid + 256, ..., then a fixed butterfly and a fixed
//   4-wave combine; RMSNorm inv = 1 / sqrt(ss / K + eps) (reference src/simd_math.cpp:7-12);
//   absmax of the (optionally normalised) row: a max-reduction, exact in any order;
//   quantisation a = max(absmax, 1e-5), s = 127 / a, q = clamp(rint(v * s), -128, 127), row scale a / 127.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

namespace ternix_hip {

// Sum over a 256-thread workgroup; every thread gets the result.  red: 4 floats of LDS.
__device__ __forceinline__ float row_block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();  // red may still be read from a previous call
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float row_block_max(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// 1 / sqrt(mean(x^2) + eps) of one row of K floats.
__device__ __forceinline__ float row_rms_inv(const float* x, int K, float eps, float* red) {
    float ss = 0.0f;
    for (int k = threadIdx.x; k < K; k += 256) ss = fmaf(x[k], x[k], ss);
    ss = row_block_sum(ss, red);
    return 1.0f / sqrtf(ss / (float)K + eps);
}

// Normalised value of element k (w == nullptr: the raw value).
__device__ __forceinline__ float row_value(const float* x, const float* w, float inv, int k) {
    return w ? x[k] * inv * w[k] : x[k];
}

// max |row_value| over the row.
__device__ __forceinline__ float row_absmax(const float* x, const float* w, float inv, int K, float* red) {
    float amax = 0.0f;
    for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(row_value(x, w, inv, k)));
    return row_block_max(amax, red);
}

__device__ __forceinline__ int quantize_value(float v, float s) {
    const float r = rintf(v * s);
    return (int)fminf(fmaxf(r, -128.0f), 127.0f);
}

}  // namespace ternix_hip
