// ternary_kernels.h -- internal launch functions of libternix_hip.so (not part of the public ABI).
#pragma once
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace ternix_hip {

// Largest number of k-rows one accumulator may sum (a multiple of 64) without int32 overflow of the
// scaled MFMA partial sums.  The worst per-row term is the out-of-domain code 10 in a field decoded
// as a signed byte of -128 times an activation of -128 (+16384), so K rows stay exact while
// 16384 * K < 2^31, i.e. K < 2^17.  (In-domain codes reach at most 8192 per row.)
constexpr int kMaxKPerAccumulator = (1 << 17) - 64;

hipError_t launch_zero(int32_t* C, size_t n, hipStream_t st);
// Skinny split-K kernel; M <= 32.  splits > 1 zeroes C first and accumulates atomically.
hipError_t launch_skinny(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int splits,
                         int steps_per_split, hipStream_t st);
// LDS-tiled MFMA GEMM over k-rows [k_begin, k_end); accumulate != 0 adds into C instead of storing.
hipError_t launch_gemm(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int k_begin,
                       int k_end, int accumulate, hipStream_t st);
hipError_t launch_naive(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, hipStream_t st);

}  // namespace ternix_hip
