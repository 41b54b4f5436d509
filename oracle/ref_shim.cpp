// ref_shim.cpp -- C-ABI wrappers around the reference's own CPU sources
// (/root/reference/src/mul_mat_ternary.cpp, src/bitpack.cpp, src/simd_math.cpp), compiled
// unchanged by oracle/Makefile into oracle/_ref/libternix_ref.so.
// TEST INFRASTRUCTURE ONLY: used to write golden vectors (tests/golden) and as
// bench.py's "reference" CPU baseline; the product never loads it.
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

#include "ternix/bitpack.hpp"
#include "ternix/mul_mat_ternary.h"
#include "ternix/simd_math.hpp"

extern "C" {

void ref_pack_ternary(uint8_t* p, const int8_t* u, size_t n) { ternix::pack_ternary_weights(p, u, n); }
void ref_unpack_ternary(int8_t* u, const uint8_t* p, size_t n) { ternix::unpack_ternary_weights(u, p, n); }
void ref_mm_naive(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K, size_t N) {
    ternix::mul_mat_ternary_naive(A, B, C, M, K, N);
}
void ref_mm_scalar(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K, size_t N) {
    ternix::mul_mat_ternary_scalar(A, B, C, M, K, N);
}
void ref_mm_avx2(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K, size_t N) {
    ternix::mul_mat_ternary_avx2(A, B, C, M, K, N);
}
void ref_rms_norm_scalar(float* out, const float* in, const float* w, size_t n, float eps) {
    ternix::rms_norm_scalar(out, in, w, n, eps);
}
void ref_rms_norm_avx2(float* out, const float* in, const float* w, size_t n, float eps) {
    ternix::rms_norm_avx2(out, in, w, n, eps);
}
void ref_swiglu(float* out, const float* in, size_t n) { ternix::swiglu(out, in, n); }
void ref_mm_avx2_blocked(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K, size_t N) {
    ternix::mul_mat_ternary_avx2_blocked(A, B, C, M, K, N);
}

// Rows are independent in every reference kernel, so row blocks (multiples of
// 4, the blocked kernel's MR) may run on separate threads.  impl: 0 scalar,
// 1 avx2, 2 avx2_blocked.
void ref_mm_rows_mt(int impl, const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K, size_t N,
                    int nthreads) {
    using Fn = void (*)(const int8_t*, const uint8_t*, int32_t*, size_t, size_t, size_t);
    const Fn fn = impl == 0 ? ternix::mul_mat_ternary_scalar
                            : (impl == 1 ? ternix::mul_mat_ternary_avx2 : ternix::mul_mat_ternary_avx2_blocked);
    if (nthreads < 1) nthreads = 1;
    const size_t blocks = (M + 3) / 4;
    if ((size_t)nthreads > blocks) nthreads = (int)(blocks ? blocks : 1);
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) {
        const size_t r0 = 4 * (blocks * t / nthreads), r1e = 4 * (blocks * (t + 1) / nthreads);
        const size_t r1 = r1e < M ? r1e : M;
        if (r0 >= r1) continue;
        pool.emplace_back([=] { fn(A + r0 * K, B, C + r0 * N, r1 - r0, K, N); });
    }
    for (auto& th : pool) th.join();
}

}  // extern "C"
