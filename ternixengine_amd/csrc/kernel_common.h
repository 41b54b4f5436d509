// kernel_common.h -- shared device helpers of the gfx950 (CDNA4) kernels for
// C[M,N] int32 = A[M,K] int8 x W[K,N] ternary (skinny_kernels.hip, gemm_kernels.hip, layer_kernels.hip).
//
// Weight layout (the contract, reference src/bitpack.cpp:5-15): row-major K x NB bytes, NB = N/4,
// weight (k, n) in bits 2*(n%4) of byte k*NB + n/4; 00 = 0, 01 = +1, 11 = -1 (10 decodes as -2,
// like the reference's scalar and CUDA decode, src/mul_mat_ternary.cpp:53, src/cuda_kernels.cu:40).
//
// Every matmul kernel here feeds v_mfma_i32_16x16x64_i8.  The int8 MFMA reduces along K inside a
// lane (lane l holds 16 K-consecutive bytes of one row of A and of one column of B, K-block l/16),
// while the packed layout runs along N.  The kernels therefore
//   1. gather, per lane, one packed byte-column (= 4 output columns) over 16 consecutive k-rows:
//      with the gfx950 transposing LDS read ds_read_b64_tr_b8 from a row-major LDS stage (the
//      DMA-staged and wave-pipelined GEMVs, the pipelined GEMM), or with a 4x4 byte transpose in
//      registers (v_perm_b32; the register-staged GEMVs and the older GEMM kernels);
//   2. split every dword into four MFMA B-operand dwords, one per 2-bit field j, without any
//      per-weight work (a handful of bitwise ops per 16 weights, see "Field decode" below);
//   3. run one MFMA per field: MFMA column i of field j is output column 4*(byte-col_i) + j.
// Which k-rows a lane's 16 bytes hold only has to agree between A and B, so the natural row order
// is used for both and A fragments are plain 16-byte loads.
//
// Kernel families (the launch layer, ternix_hip.cpp, picks one per call):
//   skinny_wave_kernel    M <= 32: 16-byte weight strips, per-wave DMA rings, one launch for K <= 4096
//   skinny_dma_kernel     M <= 16, long K: 256-byte strips staged by DMA, split-K + reduce
//   skinny_short/fast/generic_kernel  register-staged GEMVs (fallbacks, fused FFN prologue)
//   gemm_pipe_kernel / gemm_fast_kernel / gemm_kernel  LDS-tiled MFMA GEMMs (M > 32)
//   splitk_reduce_kernel, pad_rows_kernel, quantize / dequant kernels: the steps around them
//
// Field decode.  Let x be 4 bytes (4 k-rows), each holding fields f0..f3 (bits 0-1 .. 6-7).
//   * "shift" form: (x << (6-2j)) & 0xC0C0C0C0 puts field j in the top two bits of each byte, so
//     the signed byte is 64*w (01 -> 0x40 = +64, 11 -> 0xC0 = -64, 10 -> 0x80 = -128 = -2*64).
//     MFMA then yields 64*(A.W); the result is an exact arithmetic shift right by 6.
//   * "complement" form (fields 0..2): z = x ^ 0x55555555 flips each field's low bit, so
//     z & (3 << 2j) per byte equals 4^j * (1 - w) (00 -> 1, 01 -> 0, 11 -> 2, 10 -> 3).  MFMA gives
//     4^j * (R - A.W) with R the row sum of A over the same k range, so A.W = R - (S >> 2j).
//     One shared XOR plus one AND per field; field 3 uses the shift form with shift 0 (one AND).
//     R itself comes from one extra MFMA against an all-ones B per k-step, shared by all tiles.
// The complement form costs 5 VALU ops per 16 weights and needs R; the shift form costs 7 ops and
// needs nothing else.  The register-staged GEMVs use the complement form; the DMA-staged and
// wave-pipelined GEMVs and the GEMMs use the shift form (the decode is not what limits them, and the
// R MFMA per m-tile would add a quarter to a GEMM wave's MFMA issue).
// Accumulator bound: each k-row adds at most 64*128 = 8192 in magnitude to a scaled accumulator
// (16384 for the out-of-domain code 10, byte -128 times activation -128); the launch layer splits K
// so that no accumulator sums more than kMaxKPerAccumulator = 2^17 - 128 k-rows.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ternary_kernels.h"

// Device helpers shared by the kernel files; each translation unit gets its own (inline) copy.
namespace ternix_hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// 4x4 byte transpose.  r0..r3 are four rows (byte b of r_i = byte-column b of row i); on return
// c_b holds byte-column b of the four rows, row i in byte i.  v_perm_b32 picks bytes of {S0,S1}:
// selector 0-3 = bytes of the second operand, 4-7 = bytes of the first.
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                             uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3) {
    const uint32_t t01l = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
    const uint32_t t01h = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
    const uint32_t t23l = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
    const uint32_t t23h = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    c0 = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
    c1 = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
    c2 = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
    c3 = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
}

// Block ids are dealt round-robin over the 8 XCDs (XCD = id % 8).  xcd_linear(id, total) renumbers
// them so that each XCD's blocks get consecutive numbers: XCD x holds ids x, x+8, ... and receives
// the numbers [prefix(x), prefix(x) + count(x)).  A bijection on [0, total) for any total; it only
// steers which blocks share an XCD's L2 and does not affect results.
__device__ __forceinline__ int xcd_linear(int id, int total) {
    const int q = total >> 3, r = total & 7, x = id & 7;
    return x * q + min(x, r) + (id >> 3);
}

// Dequantising store of four consecutive outputs of one row: y = (float)c * (rs[row] * ws), the scale
// product rounded once, then one rounding per output (the CPU oracle uses the same two steps).
// With os.swiglu the four values are two interleaved (gate, up) pairs and the stored row is N/2 wide:
// h[col/2 + p] = silu(y[2p]) * y[2p+1], silu(g) = g / (1 + exp(-g)) (reference src/simd_math.cpp:40-46).
typedef float v2f __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float store_scaled_f(const OutScale& os, float f, int row, int N, int col, v4i c, int vec);
__device__ __forceinline__ void store_scaled(const OutScale& os, int row, int N, int col, v4i c, int vec) {
    store_scaled_f(os, os.rs[row] * os.ws, row, N, col, c, vec);
}
// As store_scaled with the combined scale f = row_scale * w_scale given.  Returns the largest |value|
// stored (fmaxf from 0, as the absmax of the row statistics takes it).
__device__ __forceinline__ float store_scaled_f(const OutScale& os, float f, int row, int N, int col, v4i c, int vec) {
    const v4f y = {(float)c[0] * f, (float)c[1] * f, (float)c[2] * f, (float)c[3] * f};
    if (os.swiglu) {
        const v2f h = {(y[0] / (1.0f + expf(-y[0]))) * y[1], (y[2] / (1.0f + expf(-y[2]))) * y[3]};
        float* out = os.Y + (size_t)row * (size_t)(N / 2) + col / 2;
        if (vec) {
            __builtin_nontemporal_store(h, reinterpret_cast<v2f*>(out));
        } else {
            out[0] = h[0];
            out[1] = h[1];
        }
        return fmaxf(fmaxf(0.0f, fabsf(h[0])), fabsf(h[1]));
    }
    float* out = os.Y + (size_t)row * (size_t)N + col;
    if (vec) {
        __builtin_nontemporal_store(y, reinterpret_cast<v4f*>(out));
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = y[j];
    }
    return fmaxf(fmaxf(fmaxf(fmaxf(0.0f, fabsf(y[0])), fabsf(y[1])), fabsf(y[2])), fabsf(y[3]));
}

// The same for two consecutive outputs c0, c1 of one row (an even column `col`), with the same two
// roundings per output; with os.swiglu they are one (gate, up) pair and the one value h[col / 2] is
// stored.  Returns the largest |value| stored (fmaxf from 0).
__device__ __forceinline__ float store_scaled_pair(const OutScale& os, float f, int row, int N, int col, int c0, int c1) {
    const float y0 = (float)c0 * f, y1 = (float)c1 * f;
    if (os.swiglu) {
        const float h = (y0 / (1.0f + expf(-y0))) * y1;
        os.Y[(size_t)row * (size_t)(N / 2) + col / 2] = h;
        return fmaxf(0.0f, fabsf(h));
    }
    float* out = os.Y + (size_t)row * (size_t)N + col;
    out[0] = y0;
    out[1] = y1;
    return fmaxf(fmaxf(0.0f, fabsf(y0)), fabsf(y1));
}

// ------------------------------------------------------------------------------------------------
// Loads with optional bounds / alignment handling.
// ------------------------------------------------------------------------------------------------

// Four packed bytes of row `row` starting at byte-column `bc` (bc % 4 == 0).  ALIGNED: NB % 4 == 0
// and B is 4-byte aligned, so the dword is entirely inside or entirely outside the row.
template <bool ALIGNED>
__device__ __forceinline__ uint32_t load_w4(const uint8_t* __restrict__ B, int row, int bc, int K, int NB) {
    if (row >= K) return 0u;
    const uint8_t* p = B + (size_t)row * (size_t)NB + bc;
    if (ALIGNED) {
        return bc < NB ? *reinterpret_cast<const uint32_t*>(p) : 0u;
    } else {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b)
            if (bc + b < NB) v |= (uint32_t)p[b] << (8 * b);
        return v;
    }
}

// 16 activation bytes of row m starting at k (k % 16 == 0).  ALIGNED: K % 16 == 0 and A is 16-byte
// aligned, so the chunk is entirely inside or outside the row.
template <bool ALIGNED>
__device__ __forceinline__ v4i load_a16(const int8_t* __restrict__ A, int m, int k, int M, int K) {
    v4i r = {0, 0, 0, 0};
    if (m >= M) return r;
    const int8_t* p = A + (size_t)m * (size_t)K + k;
    if (ALIGNED) {
        if (k < K) r = *reinterpret_cast<const v4i*>(p);
    } else {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int b = 0; b < 16; ++b)
            if (k + b < K) w[b >> 2] |= (uint32_t)(uint8_t)p[b] << (8 * (b & 3));
        r = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
    return r;
}

// As load_a16 but rows end at k_end <= K (k_end % 64 == 0 or k_end == K, so an aligned chunk is
// still entirely inside or outside).
template <bool ALIGNED>
__device__ __forceinline__ v4i load_a16_range(const int8_t* __restrict__ A, int m, int k, int M, int K, int k_end) {
    if (k >= k_end) return v4i{0, 0, 0, 0};
    if (ALIGNED || k + 16 <= k_end) return load_a16<ALIGNED>(A, m, k, M, K);
    v4i r = {0, 0, 0, 0};
    if (m >= M) return r;
    const int8_t* p = A + (size_t)m * (size_t)K + k;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < 16; ++b)
        if (k + b < k_end) w[b >> 2] |= (uint32_t)(uint8_t)p[b] << (8 * (b & 3));
    return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

#define TX_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (7 << 4) | (0xF << 8))
#define TX_LGKMCNT0() __builtin_amdgcn_s_waitcnt((0xF) | (3 << 14) | (7 << 4) | (0 << 8))

// 16 bytes per lane from global memory straight into LDS: lane l of the wave writes lds + 16*l.
// (A plain device function, so the kernel templates that call it instantiate cleanly for the host.)
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds) {
    __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// The same with a non-temporal load (streamed past the caches: weight streams far larger than L2).
__device__ __forceinline__ void lds_dma16_nt(const void* gsrc, void* lds) {
    __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)lds, 16, 0, 2);
}

// Transposing 8-byte LDS read (ds_read_b64_tr_b8: within each 16-lane group, result lane j byte i
// is byte j % 8 of the 8 bytes addressed by lane 2i + j/8).  Issued as inline assembly: the compiler then neither
// waits for the LDS DMA in flight into other stage buffers before it (it cannot tell they do not
// alias) nor for its own result -- the caller waits with lgkmcnt before using the value.
__device__ __forceinline__ uint64_t lds_read_tr8(const void* lds) {
    uint64_t v;
    const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
    __asm__ volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

__device__ __forceinline__ v4i lds_read_b128_asm(uint32_t addr) {
    v4i v;
    __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ uint64_t lds_read_tr8_asm(uint32_t addr) {
    uint64_t v;
    __asm__ volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ uint32_t lds_read_b32_asm(uint32_t addr) {
    uint32_t v;
    __asm__ volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
// LDS byte store as inline assembly (no compiler-placed wait for LDS DMA in flight); the caller waits
// with lgkmcnt before anything reads it.
__device__ __forceinline__ void lds_write_b8_asm(uint32_t addr, uint32_t v) {
    __asm__ volatile("ds_write_b8 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_b32_asm(uint32_t addr, uint32_t v) {
    __asm__ volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Tile-64 weight layout (opt-in, written by ternix_hip_interleave_weights): the K x NB packed matrix
// as 1 KB blocks of 64 k-rows x 16 bytes; block (strip c, k-step s) starts at byte (c * K/64 + s) * 1024
// and row r of the block sits at 16-byte position r ^ (8 * ((r / 16) % 2)) (the map is its own
// inverse).  A wave's 64-lane DMA of one block is 1 KB contiguous and lands in LDS already in the
// bank-spread order the transposing reads want.
__device__ __forceinline__ int tile64_pos(int r) { return r ^ (((r >> 4) & 1) << 3); }
__device__ __forceinline__ uint32_t tile64_offset(int strip, int row, int nK) {
    return ((uint32_t)strip * (uint32_t)nK + (uint32_t)(row >> 6)) * 1024u + (uint32_t)tile64_pos(row & 63) * 16u;
}

}  // namespace
}  // namespace ternix_hip
