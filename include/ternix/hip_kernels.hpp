// hip_kernels.hpp -- C++ face of libternix_hip.so with the shape of the reference's
// include/ternix/cuda_kernels.cuh:1-23 (same names with `hip` for `cuda`, same argument order and
// meaning, hipError_t for cudaError_t).  Header-only: every function forwards to the C-ABI in
// ternix_hip.h, so C++ callers link only libternix_hip.so.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "ternix/ternix_hip.h"

namespace ternix {

// C[M,N] (int32) = A[M,K] (int8) x W[K,N] (ternary, packed 4 per byte as K x N/4).
// Device-pointer variants are asynchronous on `stream`; they return the launch status.

// Reference: mul_mat_ternary_cuda_naive (cuda_kernels.cuh:10-12).  Any M, K; N % 4 == 0.
inline hipError_t mul_mat_ternary_hip_naive(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N,
                                            hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(ternix_hip_mul_mat_ternary_naive(dA, dB, dC, M, K, N, stream));
}

// Reference: mul_mat_ternary_cuda_tiled (cuda_kernels.cuh:14-17).  Same contract: M, N, K multiples
// of 64 (hipErrorInvalidValue otherwise, before any pointer is used); computed by the int8-MFMA GEMM.
inline hipError_t mul_mat_ternary_hip_tiled(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N,
                                            hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(ternix_hip_mul_mat_ternary_tiled(dA, dB, dC, M, K, N, stream));
}

// Any shape (N % 4 == 0), automatic kernel choice (skinny split-K for small M, MFMA GEMM otherwise).
inline hipError_t mul_mat_ternary_hip(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K,
                                      int64_t N, hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(ternix_hip_mul_mat_ternary(dA, dB, dC, M, K, N, stream));
}

// Reference: mul_mat_ternary_cuda_host (cuda_kernels.cuh:19-21): host pointers, allocates, copies,
// runs, copies back, frees on every path.  tiled selects the tiled contract, else the naive kernel.
inline hipError_t mul_mat_ternary_hip_host(const int8_t* A, const uint8_t* B_packed, int32_t* C, int M, int K, int N,
                                           bool tiled) {
    return static_cast<hipError_t>(
        ternix_hip_mul_mat_ternary_host(A, B_packed, C, M, K, N, tiled ? TERNIX_HIP_TILED : TERNIX_HIP_NAIVE));
}

// Opt-in tile-64 weights (no reference counterpart; the offline re-layout interleave_weights_offline
// reserves, bitpack.cpp:29-33): convert once, then call the tile-64 matmul with the converted buffer.
// K % 64 == 0 and N % 64 == 0 for the conversion; K % 128 == 0 and N % 256 == 0 for the matmul.
inline hipError_t interleave_weights_tile64_hip(uint8_t* dOut, const uint8_t* dPacked, int64_t K, int64_t N,
                                                hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(ternix_hip_interleave_weights_tile64(dOut, dPacked, K, N, stream));
}
inline hipError_t mul_mat_ternary_hip_tile64(const int8_t* dA, const uint8_t* dWt, int32_t* dC, int64_t M, int64_t K,
                                             int64_t N, hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(ternix_hip_mul_mat_ternary_tile64(dA, dWt, dC, M, K, N, stream));
}

}  // namespace ternix
