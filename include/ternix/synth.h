/*
 * synth.h -- deterministic synthetic inputs for benches and tests (libternix_hip.so).
 *
 * Not part of the reference API: the reference draws its test data from std::mt19937 with
 * std::uniform_int_distribution, whose output is standard-library specific.  These generators are
 * fully specified integer functions, so every platform produces the same bytes:
 *
 *   u64(seed, stream, i) = splitmix64 finaliser of
 *       (seed ^ (stream * 0xD1B54A32D192ED03)) + (i + 1) * 0x9E3779B97F4A7C15
 *
 * Element i of an array always uses draw i (Gaussian: draws 3i..3i+2), so any slice can be
 * generated independently and large arrays are filled by several threads.
 */
#ifndef TERNIX_SYNTH_H
#define TERNIX_SYNTH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint64_t ternix_synth_u64(uint64_t seed, uint64_t stream, uint64_t index);

/* a[i] = low byte of u64(i), read as int8: uniform on [-128, 127]. */
void ternix_synth_act_uniform(int8_t* a, size_t n, uint64_t seed, uint64_t stream);

/* Rounded Gaussian, clipped to [-128, 127]: s = sum of the twelve 16-bit halves of draws 3i..3i+2
 * minus 393210 (Irwin-Hall, mean 0, standard deviation ~65536), a = clip((s * sigma + 32768) >> 16). */
void ternix_synth_act_gauss(int8_t* a, size_t n, uint64_t seed, uint64_t stream, int sigma);

/* Ternary weights: u = top 32 bits of u64(i); u < p_neg -> -1, u < p_neg + p_pos -> +1, else 0.
 * p_neg, p_pos are probabilities scaled by 2^32 (p_neg + p_pos <= 2^32). */
void ternix_synth_ternary(int8_t* w, size_t n, uint64_t seed, uint64_t stream, uint64_t p_neg, uint64_t p_pos);

/* Same weights as ternix_synth_ternary(n), written directly in the packed 2-bit layout (n % 4 == 0,
 * n/4 bytes): equal to pack(ternix_synth_ternary(...)). */
void ternix_synth_ternary_packed(uint8_t* wp, size_t n, uint64_t seed, uint64_t stream, uint64_t p_neg,
                                 uint64_t p_pos);

#ifdef __cplusplus
}
#endif
#endif
