// ternary_kernels.h -- internal launch functions of libternix_hip.so (not part of the public ABI).
#pragma once
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace ternix_hip {

// Largest number of k-rows one accumulator may sum without risking int32 overflow of the
// scaled (x64) MFMA partial sums: 64 * 128 * 2^18 = 2^31.
constexpr int kMaxKPerAccumulator = 1 << 18;

hipError_t launch_zero(int32_t* C, size_t n, hipStream_t st);
// Skinny split-K kernel; M <= 32.  splits > 1 zeroes C first and accumulates atomically.
hipError_t launch_skinny(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int splits,
                         int steps_per_split, hipStream_t st);
// LDS-tiled MFMA GEMM over k-rows [k_begin, k_end); accumulate != 0 adds into C instead of storing.
hipError_t launch_gemm(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int k_begin,
                       int k_end, int accumulate, hipStream_t st);
hipError_t launch_naive(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, hipStream_t st);

}  // namespace ternix_hip
