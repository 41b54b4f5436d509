/*
 * ternix_oracle.c -- plain-C restatement of TernixEngine's CPU ternary matmul
 * path.  TEST INFRASTRUCTURE ONLY (see ternix_oracle.h): the product never
 * links this file; tests, smoke() and bench.py's cpu_baseline use it as the
 * checker.
 */
#include "ternix_oracle.h"

#include <math.h>

#include <pthread.h>
#include <string.h>

/* src/bitpack.cpp:5-15 -- value at flat index 4i+j goes to bits 2j..2j+1 of
 * byte i, with +1 -> 01, -1 -> 11 and everything else -> 00. */
void oracle_pack_ternary(uint8_t* packed, const int8_t* unpacked, size_t size) {
    for (size_t i = 0; i < size / 4; ++i) {
        unsigned byte = 0;
        for (unsigned j = 0; j < 4; ++j) {
            const int8_t v = unpacked[4 * i + j];
            const unsigned code = v == 1 ? 1u : (v == -1 ? 3u : 0u);
            byte |= code << (2 * j);
        }
        packed[i] = (uint8_t)byte;
    }
}

/* src/bitpack.cpp:17-27 -- 01 -> +1, 11 -> -1, anything else (00 and the
 * invalid 10) -> 0. */
void oracle_unpack_ternary(int8_t* unpacked, const uint8_t* packed, size_t size) {
    for (size_t i = 0; i < size / 4; ++i) {
        for (unsigned j = 0; j < 4; ++j) {
            const unsigned code = (packed[i] >> (2 * j)) & 3u;
            unpacked[4 * i + j] = code == 1 ? 1 : (code == 3 ? -1 : 0);
        }
    }
}

/* src/bitpack.cpp:29-33 -- identity copy of size/4 bytes. */
void oracle_interleave(uint8_t* out, const uint8_t* packed, size_t size) {
    memcpy(out, packed, size / 4);
}

/* src/mul_mat_ternary.cpp:8-36 -- i-j-k order, branching decode (10 -> 0). */
void oracle_mm_naive(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N) {
    const size_t nb = N / 4;
    for (size_t i = 0; i < M; ++i) {
        for (size_t j = 0; j < N; ++j) {
            int32_t sum = 0;
            for (size_t k = 0; k < K; ++k) {
                const unsigned code = (Bp[k * nb + j / 4] >> ((j % 4) * 2)) & 3u;
                int w = 0;
                if (code == 1) w = 1;
                else if (code == 3) w = -1;
                sum += (int32_t)A[i * K + k] * w;
            }
            C[i * N + j] = sum;
        }
    }
}

/* src/mul_mat_ternary.cpp:38-58 -- i-k-j order, zero C first, decode
 * w = (b & 1) - (b & 2), so the invalid code 10 contributes -2a. */
void oracle_mm_scalar(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N) {
    const size_t nb = N / 4;
    for (size_t i = 0; i < M; ++i) {
        int32_t* c = C + i * N;
        for (size_t j = 0; j < N; ++j) c[j] = 0;
        for (size_t k = 0; k < K; ++k) {
            const int32_t a = A[i * K + k];
            const uint8_t* b = Bp + k * nb;
            for (size_t j = 0; j < N; ++j) {
                const int code = (b[j >> 2] >> ((j & 3) * 2)) & 3;
                c[j] += a * ((code & 1) - (code & 2));
            }
        }
    }
}

/* The AVX2 kernels' per-lane arithmetic (mul_mat_ternary.cpp:90-98): the
 * 2-bit field is sign-extended from bit 1 (slli 30 / srai 30), giving
 * {00,01,10,11} -> {0,+1,-2,-1}, and _mm256_sign_epi32(a, w) yields -a, 0 or a
 * by the sign of w alone (so the invalid code 10 gives -a). */
static inline int32_t avx2_lane(int32_t a, unsigned code) {
    const int32_t w = (int32_t)((uint32_t)code << 30) >> 30;
    return w < 0 ? -a : (w == 0 ? 0 : a);
}

/* Eight consecutive fields starting at column j are read as one little-endian
 * uint16 at byte j/4 (mul_mat_ternary.cpp:85-87); lane t takes bits 2t..2t+1
 * (shift vector {0,2,...,14}, :71,:90). */
static inline unsigned load_u16(const uint8_t* p) { return (unsigned)p[0] | ((unsigned)p[1] << 8); }

static void avx2_rows(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N) {
    const size_t nb = N / 4;
    for (size_t i = 0; i < M; ++i) {
        for (size_t j = 0; j < N; j += 8) {
            int32_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (size_t k = 0; k < K; ++k) {
                const int32_t a = A[i * K + k];
                const unsigned packed_w = load_u16(&Bp[k * nb + j / 4]);
                for (unsigned t = 0; t < 8; ++t) acc[t] += avx2_lane(a, (packed_w >> (2 * t)) & 3u);
            }
            for (unsigned t = 0; t < 8; ++t) C[i * N + j + t] = acc[t];
        }
    }
}

/* src/mul_mat_ternary.cpp:60-105 */
int oracle_mm_avx2(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N) {
    if (N % 8 != 0) return -1;
    avx2_rows(A, Bp, C, M, K, N);
    return 0;
}

/* src/mul_mat_ternary.cpp:107-152 -- blocks of MR=4 rows share one decode of
 * each 8-weight group; leftover rows (M % 4) go through the one-row kernel
 * (:149-151).  Integer addition is exact, so the blocking changes only the
 * order of work, not the result. */
int oracle_mm_avx2_blocked(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N) {
    enum { MR = 4 };
    if (N % 8 != 0) return -1;
    const size_t nb = N / 4;
    size_t i = 0;
    for (; i + MR <= M; i += MR) {
        for (size_t j = 0; j < N; j += 8) {
            int32_t acc[MR][8];
            memset(acc, 0, sizeof(acc));
            for (size_t k = 0; k < K; ++k) {
                const unsigned packed_w = load_u16(&Bp[k * nb + j / 4]);
                unsigned code[8];
                for (unsigned t = 0; t < 8; ++t) code[t] = (packed_w >> (2 * t)) & 3u;
                for (unsigned r = 0; r < MR; ++r) {
                    const int32_t a = A[(i + r) * K + k];
                    for (unsigned t = 0; t < 8; ++t) acc[r][t] += avx2_lane(a, code[t]);
                }
            }
            for (unsigned r = 0; r < MR; ++r)
                for (unsigned t = 0; t < 8; ++t) C[(i + r) * N + j + t] = acc[r][t];
        }
    }
    if (i < M) avx2_rows(A + i * K, Bp, C + i * N, M - i, K, N);
    return 0;
}

/* tests/test_ternary_matmul.cpp:31-39 -- plain i-k-j int32 GEMM on the
 * unpacked weights; shares no decode with any kernel. */
void oracle_gemm_unpacked(const int8_t* A, const int8_t* W, int32_t* C, size_t M, size_t K, size_t N) {
    memset(C, 0, M * N * sizeof(int32_t));
    for (size_t i = 0; i < M; ++i)
        for (size_t k = 0; k < K; ++k) {
            const int32_t a = A[i * K + k];
            const int8_t* w = W + k * N;
            int32_t* c = C + i * N;
            for (size_t j = 0; j < N; ++j) c[j] += a * (int32_t)w[j];
        }
}

/* ---- multi-threaded driver (rows, or 4-column slices when M is small) ---- */

typedef struct {
    const int8_t* A;
    const uint8_t* Bp;
    int32_t* C;
    size_t M, K, N;
    size_t r0, r1;   /* row range */
    size_t c0, c1;   /* column range, multiples of 4 */
} mt_job;

static void* mt_run(void* arg) {
    const mt_job* j = (const mt_job*)arg;
    const size_t nb = j->N / 4;
    for (size_t i = j->r0; i < j->r1; ++i) {
        int32_t* c = j->C + i * j->N;
        for (size_t col = j->c0; col < j->c1; ++col) c[col] = 0;
        for (size_t k = 0; k < j->K; ++k) {
            const int32_t a = j->A[i * j->K + k];
            const uint8_t* b = j->Bp + k * nb;
            for (size_t col = j->c0; col < j->c1; ++col) {
                const int code = (b[col >> 2] >> ((col & 3) * 2)) & 3;
                c[col] += a * ((code & 1) - (code & 2));
            }
        }
    }
    return NULL;
}

void oracle_mm_scalar_mt(const int8_t* A, const uint8_t* Bp, int32_t* C, size_t M, size_t K, size_t N,
                         int nthreads) {
    enum { MAXT = 64 };
    if (nthreads < 1) nthreads = 1;
    if (nthreads > MAXT) nthreads = MAXT;
    pthread_t tid[MAXT];
    mt_job job[MAXT];
    const int by_rows = M >= (size_t)nthreads;
    for (int t = 0; t < nthreads; ++t) {
        mt_job* j = &job[t];
        j->A = A; j->Bp = Bp; j->C = C; j->M = M; j->K = K; j->N = N;
        if (by_rows) {
            j->r0 = M * t / nthreads; j->r1 = M * (t + 1) / nthreads;
            j->c0 = 0; j->c1 = N;
        } else {
            const size_t nq = N / 4;
            j->r0 = 0; j->r1 = M;
            j->c0 = 4 * (nq * t / nthreads); j->c1 = 4 * (nq * (t + 1) / nthreads);
        }
        pthread_create(&tid[t], NULL, mt_run, j);
    }
    for (int t = 0; t < nthreads; ++t) pthread_join(tid[t], NULL);
}

/* ---- quantised layer boundary (see the header: no reference counterpart) ---- */

/* a = max(absmax, 1e-5); s = 127 / a; q = clamp(rint(x * s), -128, 127); row_scale = a / 127. */
void oracle_quantize_rows_absmax(const float* X, int8_t* Q, float* row_scale, size_t M, size_t K) {
    for (size_t m = 0; m < M; ++m) {
        const float* x = X + m * K;
        float amax = 0.0f;
        for (size_t k = 0; k < K; ++k) {
            const float v = fabsf(x[k]);
            if (v > amax) amax = v;
        }
        const float a = amax > 1e-5f ? amax : 1e-5f;
        const float s = 127.0f / a;
        row_scale[m] = a / 127.0f;
        for (size_t k = 0; k < K; ++k) {
            float r = rintf(x[k] * s);
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            Q[m * K + k] = (int8_t)r;
        }
    }
}

/* f = row_scale[m] * w_scale (one rounding), y = (float)c * f (one rounding). */
void oracle_dequant(const int32_t* C, float* Y, const float* row_scale, float w_scale, size_t M, size_t N) {
    for (size_t m = 0; m < M; ++m) {
        const float f = row_scale[m] * w_scale;
        for (size_t n = 0; n < N; ++n) Y[m * N + n] = (float)C[m * N + n] * f;
    }
}

/* gamma = max(mean|W|, 1e-5) (sum in double, index order); w = clamp(rint(W / gamma), -1, 1). */
float oracle_quantize_weights_absmean(int8_t* Wq, const float* W, size_t size) {
    double sum = 0.0;
    for (size_t i = 0; i < size; ++i) sum += fabs((double)W[i]);
    float gamma = size ? (float)(sum / (double)size) : 0.0f;
    if (!(gamma >= 1e-5f)) gamma = 1e-5f;
    for (size_t i = 0; i < size; ++i) {
        const float r = rintf(W[i] / gamma);
        Wq[i] = (int8_t)(r > 1.0f ? 1 : (r < -1.0f ? -1 : (int)r));
    }
    return gamma;
}

/* src/simd_math.cpp:7-12 -- sequential float sum of squares, inv = 1 / sqrt(mean + eps). */
void oracle_rms_norm(float* out, const float* in, const float* weight, size_t size, float eps) {
    float sum_sq = 0.0f;
    for (size_t i = 0; i < size; ++i) sum_sq += in[i] * in[i];
    const float inv = 1.0f / sqrtf(sum_sq / (float)size + eps);
    for (size_t i = 0; i < size; ++i) out[i] = in[i] * inv * weight[i];
}

/* src/simd_math.cpp:40-46 -- interleaved (gate, up) pairs. */
void oracle_swiglu(float* out, const float* in, size_t size) {
    for (size_t i = 0; i + 1 < size; i += 2) {
        const float x = in[i], y = in[i + 1];
        out[i / 2] = (x / (1.0f + expf(-x))) * y;
    }
}
