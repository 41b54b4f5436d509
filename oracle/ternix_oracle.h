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
 *   oracle_rms_norm            src/simd_math.cpp:7-12 (rms_norm_scalar)
 *   oracle_swiglu              src/simd_math.cpp:40-46
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
 *   - rms_norm / swiglu: the reference's known values (tests/test_simd_math.cpp:7-15,
 *     :29-35) and bit equality with the compiled reference's rms_norm_scalar and
 *     swiglu (oracle/_ref) on random inputs.
 *
 * Quantised layer boundary (no reference implementation: the reference leaves
 * weight and activation quantisation as a stub, scripts/quantize.py:5,
 * README.md:203; these restate the BitNet b1.58 formulas the library documents
 * in include/ternix/ternix_hip.h, step for step in IEEE fp32):
 *   oracle_quantize_rows_absmax      per-row absmax int8 activation quantisation
 *   oracle_dequant                   y = (float)c * (row_scale[m] * w_scale)
 *   oracle_quantize_weights_absmean  absmean ternary weight quantisation
 * Pinned in tests/test_quant.py by closed forms that a wrong sign, index, scale
 * or rounding mode breaks: zero rows (q = 0, scale = 1e-5/127), a row whose
 * absmax element maps to exactly +-127, constant rows, ties rounding to even,
 * row independence (permuting rows permutes outputs), int32 values that are
 * exact in fp32 times power-of-two scales (exact products), and a float64 numpy
 * evaluation of the same formulas within one fp32 rounding.
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

void oracle_rms_norm(float* out, const float* in, const float* weight, size_t size, float eps);
void oracle_swiglu(float* out, const float* in, size_t size);

void oracle_quantize_rows_absmax(const float* X, int8_t* Q, float* row_scale, size_t M, size_t K);
void oracle_dequant(const int32_t* C, float* Y, const float* row_scale, float w_scale, size_t M, size_t N);
float oracle_quantize_weights_absmean(int8_t* Wq, const float* W, size_t size);

/* Row-parallel driver over oracle_mm_scalar (rows split over nthreads). */
void oracle_mm_scalar_mt(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N,
                         int nthreads);

#ifdef __cplusplus
}
#endif
#endif
