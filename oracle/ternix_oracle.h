/*
 * ternix_oracle.h -- CPU restatement of TernixEngine's ternary matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (ternixengine_amd/, include/)
 * may include, link or call this code.  It is used by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
 *
 * Every function restates one reference function (paths relative to the
 * reference repository root) in plain C, with no intrinsics, so that its
 * semantics can be read line by line:
 *
 *   oracle_pack_ternary        src/bitpack.cpp:5-15
 *   oracle_unpack_ternary      src/bitpack.cpp:17-27
 *   oracle_interleave          src/bitpack.cpp:29-33
 *   oracle_mm_naive            src/mul_mat_ternary.cpp:8-36
 *   oracle_mm_scalar           src/mul_mat_ternary.cpp:38-58
 *   oracle_mm_avx2             src/mul_mat_ternary.cpp:60-105
 *   oracle_mm_avx2_blocked     src/mul_mat_ternary.cpp:107-152
 *   oracle_gemm_unpacked       tests/test_ternary_matmul.cpp:31-39 (the
 *                              closed-form int32 GEMM on unpacked weights)
 *
 * Parity pinning (how each function is checked, tests/test_oracle.py):
 *   - pack/unpack: known answer {1,0,-1,1,-1,0,1,0} -> {0x71,0x13}
 *     (tests/test_bitpack.cpp:6), exhaustive 81-pattern round trip, and the
 *     golden vectors written by the compiled reference (tests/golden/).
 *   - all matmuls: equality with oracle_gemm_unpacked on the reference test
 *     shapes, closed forms (W==0 -> 0, W==+1 -> row sums, A==-128 & W==-1 ->
 *     128*K), and the golden vectors and SHA-256 digests computed by the
 *     compiled reference sources (oracle/_ref).
 *   - invalid code 0b10 (outside the domain): naive -> 0, scalar -> -2a,
 *     avx2 -> -a, each checked against the compiled reference's output.
 */
#ifndef TERNIX_ORACLE_H
#define TERNIX_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void oracle_pack_ternary(uint8_t* packed, const int8_t* unpacked, size_t size);
void oracle_unpack_ternary(int8_t* unpacked, const uint8_t* packed, size_t size);
void oracle_interleave(uint8_t* out, const uint8_t* packed, size_t size);

void oracle_mm_naive(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N);
void oracle_mm_scalar(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N);
/* Return 0 on success, -1 if the AVX2 precondition N % 8 == 0 is violated
 * (the reference leaves that case undefined; mul_mat_ternary.h:41-42). */
int oracle_mm_avx2(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N);
int oracle_mm_avx2_blocked(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N);

void oracle_gemm_unpacked(const int8_t* A, const int8_t* W, int32_t* C, size_t M, size_t K, size_t N);

/* Row-parallel driver over oracle_mm_scalar (rows split over nthreads). */
void oracle_mm_scalar_mt(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N,
                         int nthreads);

#ifdef __cplusplus
}
#endif
#endif
