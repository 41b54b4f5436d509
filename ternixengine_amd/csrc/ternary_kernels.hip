// ternary_kernels.hip -- gfx950 (CDNA4) kernels for C[M,N] int32 = A[M,K] int8 x W[K,N] ternary.
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

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <atomic>

#include "row_stats.h"
#include "ternary_kernels.h"

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
__device__ __forceinline__ void store_scaled_f(const OutScale& os, float f, int row, int N, int col, v4i c, int vec);
__device__ __forceinline__ void store_scaled(const OutScale& os, int row, int N, int col, v4i c, int vec) {
    store_scaled_f(os, os.rs[row] * os.ws, row, N, col, c, vec);
}
// As store_scaled with the combined scale f = row_scale * w_scale given.
__device__ __forceinline__ void store_scaled_f(const OutScale& os, float f, int row, int N, int col, v4i c, int vec) {
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
        return;
    }
    float* out = os.Y + (size_t)row * (size_t)N + col;
    if (vec) {
        __builtin_nontemporal_store(y, reinterpret_cast<v4f*>(out));
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = y[j];
    }
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

// ------------------------------------------------------------------------------------------------
// Skinny split-K kernels (decode shapes, M <= 32).
//
// MFMA mapping.  A wave owns a column slab of 64*TB packed bytes (256*TB output columns).  Lane
// (q = l%16, kb = l/16) owns dwords q + 16h (h < TB) of the slab -- byte-columns g = 4h..4h+3 of the
// lane -- and k-rows 16kb..16kb+15 of every 64-row k-step.  Per k-step it transposes its 16 rows x
// 4*TB byte-columns (v_perm) and drives 16*TB MFMAs per m-tile (4*TB byte-columns x 4 fields) plus
// one row-sum MFMA for the complement decode.
//
// Fast kernel (K % 64 == 0, NB % 64 == 0, 16-byte aligned A and W): weights are read with coalesced
// 16-byte loads -- one wave instruction covers 16/TB rows x 64*TB bytes, whole 128-byte lines when
// TB == 2 -- into registers, two k-steps in flight per wave, and go through a per-wave LDS block to
// come back in the transposed lane layout.  The workgroup's activation slice (its rows x its
// k-range) is copied to LDS once, so activation fragments never wait behind weight loads.
// Generic kernel (any shape / alignment): branch-free clamped dword loads, no LDS staging.
//
// Split-K.  A workgroup has 4 waves: 4/KW column slabs x KW waves per slab; the KW waves of a slab
// take alternate k-steps and are summed in LDS.  blockIdx.y splits K further over `splits`
// workgroups: each stores its partial tile with plain stores in the workspace P[split][M][N] and
// splitk_reduce_kernel (the next launch on the stream) adds the partials.  Cross-workgroup exchange
// inside one launch would need device-scope release/acquire fences, which on this multi-XCD part
// write back and invalidate a whole L2 per workgroup, and same-address device-scope atomics from
// several XCDs serialise at the memory side; the kernel boundary gives the ordering for free.
// (SK_ATOMIC, used only when no workspace is available, accumulates into a pre-zeroed C instead.)
// LOW_M: at most 4 rows in this m-group, all held by lanes 0-15 (rows 4*kb + i of an MFMA tile), so
// only those lanes take part in the LDS exchange and the epilogue.
// ------------------------------------------------------------------------------------------------

constexpr int SK_WAVES = 4;
constexpr int kRowRegs = 32;  // fused activation quantisation: row elements per thread (K <= 8192)

enum SkinnyMode { SK_STORE = 0, SK_ATOMIC = 1, SK_PARTIAL = 2 };

struct SkinnyArgs {
    const int8_t* A;
    const uint8_t* B;
    int32_t* C;
    int32_t* P;           // workspace partials [splits][M][N] (SK_PARTIAL)
    int M, K, N;
    int steps_per_split;
    int splits;
    int mode;             // SkinnyMode
    int vec_store;        // C is 16-byte aligned
    int aligned_w;        // generic kernel: NB % 4 == 0 and W 4-byte aligned
    int aligned_a;        // generic kernel: K % 16 == 0 and A 16-byte aligned
    OutScale os;          // SK_STORE: dequantised float output instead of C when os.Y is set
    // Fused activation quantisation (skinny_short_kernel with AQ > 0): A is produced from the fp32
    // rows X (optionally RMS-normalised with weight G), and rs_out receives the row scales.
    const float* X;
    const float* G;
    float eps;
    float* rs_out;
    int n_out;            // skinny_wave_kernel, store mode: C / os.Y has n_out <= N columns (0: N)
    int line_units;       // skinny_wave_kernel: block -> strip mapping by 128-byte line units
};

// One k-step of MFMA work for one 16-row x 4-byte-column block: raw[r] is the dword of row r.
// Byte-column g of the block feeds tiles acc[t][gbase + g][0..3] (one per 2-bit field).
template <int MT, int G>
__device__ __forceinline__ void skinny_mfma_block(const uint32_t (&raw)[16], const v4i (&a)[MT], int gbase,
                                                  v4i (&acc)[MT][G][4]) {
    uint32_t T[4][4];  // T[g][rq]: byte-column g, rows 4rq..4rq+3
#pragma unroll
    for (int rq = 0; rq < 4; ++rq)
        transpose4x4(raw[4 * rq], raw[4 * rq + 1], raw[4 * rq + 2], raw[4 * rq + 3], T[0][rq], T[1][rq], T[2][rq],
                     T[3][rq]);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        v4i b0, b1, b2, b3;
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
            const uint32_t x = T[g][rq];
            const uint32_t z = x ^ 0x55555555u;
            b0[rq] = (int)(z & 0x03030303u);
            b1[rq] = (int)(z & 0x0C0C0C0Cu);
            b2[rq] = (int)(z & 0x30303030u);
            b3[rq] = (int)(x & 0xC0C0C0C0u);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            acc[t][gbase + g][0] = mfma_i8(a[t], b0, acc[t][gbase + g][0]);
            acc[t][gbase + g][1] = mfma_i8(a[t], b1, acc[t][gbase + g][1]);
            acc[t][gbase + g][2] = mfma_i8(a[t], b2, acc[t][gbase + g][2]);
            acc[t][gbase + g][3] = mfma_i8(a[t], b3, acc[t][gbase + g][3]);
        }
    }
}

// Finishes a wave's accumulators: complement decode, LDS sum over the KW waves of the slab, and the
// store / partial store / atomic add of the slab's outputs.  Must be reached by every wave.
// bcol(g) = byte-column of lane value g = tile_bc + 64*(g/4) + 4q + g%4.
template <int MT, int G, int KW, int TILES, bool LOW_M>
__device__ __forceinline__ void skinny_epilogue(const SkinnyArgs& args, int32_t* red, v4i (&acc)[MT][G][4],
                                                const v4i (&accR)[MT], int tw, int kw, int tile_bc, int m0,
                                                int split) {
    constexpr int NV = MT * 16 * G;
    constexpr int XL = LOW_M ? 16 : 64;
    const int lane = threadIdx.x & 63;
    const int q = lane & 15, kb = lane >> 4;
    const int M = args.M, N = args.N, NB = N >> 2;

    // w = R - S_j / 4^j (j < 3), S_3 / 64.  MFMA tile layout: lane l holds column l%16 and rows
    // 4*(l/16) + i in element i.
    int val[MT][G][4][4];  // [t][g][j][i]
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int R = accR[t][i];
                val[t][g][0][i] = R - acc[t][g][0][i];
                val[t][g][1][i] = R - (acc[t][g][1][i] >> 2);
                val[t][g][2][i] = R - (acc[t][g][2][i] >> 4);
                val[t][g][3][i] = acc[t][g][3][i] >> 6;
            }

    const bool xlane = !LOW_M || kb == 0;
    const int xl = LOW_M ? q : lane;
    if (KW > 1) {
        // Halving tree over the KW waves of the slab: the upper half writes, the lower half adds.
        __syncthreads();  // the buffer may alias the staging blocks still in use by other waves
#pragma unroll
        for (int h = KW / 2; h >= 1; h >>= 1) {
            if (kw >= h && kw < 2 * h && xlane) {
                int32_t* dst = red + ((kw - h) * TILES + tw) * NV * XL + xl;
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (m0 + 16 * t + 4 * kb + i >= M) continue;
#pragma unroll
                        for (int g = 0; g < G; ++g)
#pragma unroll
                            for (int j = 0; j < 4; ++j) dst[(((t * 4 + i) * G + g) * 4 + j) * XL] = val[t][g][j][i];
                    }
            }
            __syncthreads();
            if (kw < h && xlane) {
                const int32_t* src = red + (kw * TILES + tw) * NV * XL + xl;
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (m0 + 16 * t + 4 * kb + i >= M) continue;
#pragma unroll
                        for (int g = 0; g < G; ++g)
#pragma unroll
                            for (int j = 0; j < 4; ++j) val[t][g][j][i] += src[(((t * 4 + i) * G + g) * 4 + j) * XL];
                    }
            }
            if (h > 1) __syncthreads();
        }
    }
    if (kw != 0 || !xlane) return;

    int32_t* out_base = args.mode == SK_PARTIAL ? args.P + (size_t)split * (size_t)M * (size_t)N : args.C;
    const bool vec = args.mode == SK_PARTIAL || args.vec_store;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m0 + 16 * t + 4 * kb + i;
            if (row >= M) continue;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int bcol = tile_bc + 64 * (g >> 2) + 4 * q + (g & 3);
                if (bcol >= NB) continue;
                if (args.mode == SK_STORE && args.os.Y) {
                    store_scaled(args.os, row, N, 4 * bcol,
                                 v4i{val[t][g][0][i], val[t][g][1][i], val[t][g][2][i], val[t][g][3][i]},
                                 args.vec_store);
                    continue;
                }
                int32_t* out = out_base + (size_t)row * (size_t)N + 4 * bcol;
                if (args.mode == SK_ATOMIC) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (val[t][g][j][i] != 0) atomicAdd(out + j, val[t][g][j][i]);
                } else if (vec) {
                    *reinterpret_cast<v4i*>(out) = v4i{val[t][g][0][i], val[t][g][1][i], val[t][g][2][i], val[t][g][3][i]};
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = val[t][g][j][i];
                }
            }
        }
}

template <int MT, int TB, int KW, bool LOW_M>
struct SkinnyFastGeometry {
    static constexpr int G = 4 * TB;                  // byte-columns per lane
    static constexpr int TILES = SK_WAVES / KW;       // column slabs per workgroup
    static constexpr int ROW_DW = 16 * TB;            // dwords per staged row
    static constexpr int STAGE_DW = 64 * ROW_DW + 4 * 16;  // + 64-byte pad per 16 rows
    static constexpr int RED_DW = TILES * (KW / 2) * MT * 16 * G * (LOW_M ? 16 : 64);
    static constexpr int SMEM_DW = (SK_WAVES * STAGE_DW > RED_DW) ? SK_WAVES * STAGE_DW : RED_DW;
};

template <int MT, int TB, int KW, int PD, bool LOW_M>
__global__ __launch_bounds__(64 * SK_WAVES) __attribute__((amdgpu_waves_per_eu((TB == 1 && MT == 1) ? 2 : 1)))
void skinny_fast_kernel(SkinnyArgs args) {
    using Geo = SkinnyFastGeometry<MT, TB, KW, LOW_M>;
    constexpr int G = Geo::G, TILES = Geo::TILES, ROW_DW = Geo::ROW_DW, STAGE_DW = Geo::STAGE_DW;
    constexpr int RPI = 16 / TB;        // rows per load instruction
    constexpr int NLD = 4 * TB;         // load instructions per k-step
    constexpr int BS = 64 * SK_WAVES;
    __shared__ __attribute__((aligned(16))) int32_t smem[Geo::SMEM_DW];
    // this workgroup's activation slice, row pitch a_pitch bytes (k-range + 16, so the 16 rows read by
    // one ds_read_b128 fall on distinct banks)
    extern __shared__ __attribute__((aligned(16))) int8_t a_lds[];

    const int8_t* __restrict__ A = args.A;
    const uint8_t* __restrict__ B = args.B;
    const int M = args.M, K = args.K, NB = args.N >> 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
    const int tw = wave % TILES, kw = wave / TILES;
    const int q = lane & 15, kb = lane >> 4;
    // (column workgroup, split) from the block id, XCD-aware: block ids are dealt round-robin over
    // the 8 XCDs, so renumber them such that the workgroups of one split that sit next to each other
    // along N run on the same XCD and share the cache lines that straddle their column ranges.
    int cx, sy;
    {
        const int lin = xcd_linear(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
        cx = lin % gridDim.x;
        sy = lin / gridDim.x;
    }
    const int tile_bc = (cx * TILES + tw) * 64 * TB;
    const int m0 = blockIdx.z * (16 * MT);
    const int nsteps = K >> 6;
    const int s_begin = sy * args.steps_per_split;
    const int s_stop = min(nsteps, s_begin + args.steps_per_split);
    const int s_end = tile_bc < NB ? s_stop : s_begin;  // a slab past the last column loads nothing
    const int s0 = s_begin + kw;

    v4i acc[MT][G][4];
    v4i accR[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        accR[t] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][g][j] = v4i{0, 0, 0, 0};
    }
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};

    // Weight loads: lane (rr, cc) reads 16-byte chunk cc of row h*RPI + rr of the slab.
    const int rr = lane / (4 * TB), cc = lane % (4 * TB);
    const uint32_t goff = (uint32_t)rr * (uint32_t)NB + (uint32_t)(tile_bc + cc * 16);
    auto gload = [&](int s, v4i (&g4)[NLD]) {
        const uint8_t* rowbase = B + (size_t)s * 64 * (size_t)NB;  // wave-uniform
#pragma unroll
        for (int h = 0; h < NLD; ++h)
            g4[h] = *reinterpret_cast<const v4i*>(rowbase + goff + (uint32_t)(RPI * h) * (uint32_t)NB);
    };

    // Activation slice: first batch of loads, then the weight prologue, then the LDS stores.
    const int a_rows = min(16 * MT, M - m0);
    const int n16 = (s_stop - s_begin) * 4;  // 16-byte chunks per activation row
    const int a_total = a_rows * n16;
    const int a_pitch = args.steps_per_split * 64 + 16;
    auto a_src = [&](int c) {
        return reinterpret_cast<const v4i*>(A + (size_t)(m0 + c / n16) * (size_t)K + (size_t)s_begin * 64 +
                                            (c % n16) * 16);
    };
    auto a_dst = [&](int c) { return reinterpret_cast<v4i*>(a_lds + (c / n16) * a_pitch + (c % n16) * 16); };
    v4i areg[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) areg[u] = *a_src(min((int)threadIdx.x + u * BS, a_total - 1));

    // Ring of PD steps in flight: slot p holds step s0 + (it + p) * KW.  The prologue loads are
    // unconditional (clamped to the wave's last step) so that the same number of loads is in flight
    // on every path into the steady-state loop and the compiler waits for exactly the slot it uses.
    const bool has_steps = s0 < s_end;  // wave-uniform
    v4i gbuf[PD][NLD];
    if (has_steps) {
#pragma unroll
        for (int p = 0; p < PD; ++p) gload(min(s0 + p * KW, s_end - 1), gbuf[p]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
        if ((int)threadIdx.x + u * BS < a_total) *a_dst(threadIdx.x + u * BS) = areg[u];
    for (int c = threadIdx.x + 2 * BS; c < a_total; c += BS) *a_dst(c) = *a_src(c);
    __syncthreads();

    int a_off[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) a_off[t] = min(16 * t + q, a_rows - 1) * a_pitch + kb * 16;
    int32_t* stage = smem + wave * STAGE_DW;

    // One k-step: weights through the wave's LDS block into the transposed layout, activations from
    // the slice, then the MFMAs.
    auto consume = [&](int cur, v4i (&g4)[NLD], uint32_t (&raw)[TB][16], v4i (&a)[MT]) {
#pragma unroll
        for (int h = 0; h < NLD; ++h) {
            const int R = RPI * h + rr;
            *reinterpret_cast<v4i*>(stage + R * ROW_DW + (R >> 4) * 16 + cc * 4) = g4[h];
        }
        __asm__ volatile("" ::: "memory");  // LDS is in order within a wave; keep the compiler so
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                raw[tb][r] = (uint32_t)stage[(16 * kb + r) * ROW_DW + 16 * kb + q + 16 * tb];
#pragma unroll
        for (int t = 0; t < MT; ++t) a[t] = *reinterpret_cast<const v4i*>(a_lds + a_off[t] + (cur - s_begin) * 64);
        __asm__ volatile("" ::: "memory");
    };
    auto compute = [&](const uint32_t (&raw)[TB][16], const v4i (&a)[MT]) {
#pragma unroll
        for (int t = 0; t < MT; ++t) accR[t] = mfma_i8(a[t], ones, accR[t]);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) skinny_mfma_block<MT, G>(raw[tb], a, 4 * tb, acc);
    };

    if (has_steps) {
        int it = 0;
        // steady state: every slot consumed and refilled, no conditions
        for (; s0 + (it + 2 * PD - 1) * KW < s_end; it += PD) {
#pragma unroll
            for (int p = 0; p < PD; ++p) {
                const int cur = s0 + (it + p) * KW;
                uint32_t raw[TB][16];
                v4i a[MT];
                consume(cur, gbuf[p], raw, a);
                gload(cur + PD * KW, gbuf[p]);
                compute(raw, a);
                // keep the next slot's LDS stores (and their wait for its loads) after this math
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // tail: fewer than 2*PD steps left
        for (; s0 + it * KW < s_end; it += PD) {
#pragma unroll
            for (int p = 0; p < PD; ++p) {
                const int cur = s0 + (it + p) * KW;
                if (cur < s_end) {
                    uint32_t raw[TB][16];
                    v4i a[MT];
                    consume(cur, gbuf[p], raw, a);
                    if (cur + PD * KW < s_end) gload(cur + PD * KW, gbuf[p]);
                    compute(raw, a);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
    skinny_epilogue<MT, G, KW, TILES, LOW_M>(args, smem, acc, accR, tw, kw, tile_bc, m0, sy);
}

// Short-range skinny kernel: the fast kernel's column geometry (4 waves, one 64-byte slab each) for
// workgroups whose k-range is at most SPS k-steps, the decode case where K is split over the whole
// chip.  Every weight and activation load of the workgroup is issued up front (no ring, no LDS copy
// of the activations, no barrier), so the code a workgroup runs is short and its loads all overlap.
// AQ selects the activation source: 0 the int8 A; 1 fp32 rows X quantised on the fly (absmax, the
// rule of quantize_rows_kernel); 2 fp32 rows X RMS-normalised with weight G, then quantised (the rule
// of rmsnorm_kernel).  With AQ > 0 every workgroup computes the statistics of its m-group's rows with
// the shared row_stats.h loops (the rows are small and cached; the weight loads are already in flight),
// so its int8 fragments are bit-identical to the standalone kernels' output; workgroup (0, 0) also
// stores the row scales for the launch that applies them (split-K reduce or dequant), which is why the
// launcher only uses AQ > 0 with splits > 1.
template <int SPS, bool LOW_M, int AQ>
__global__ __launch_bounds__(64 * SK_WAVES) void skinny_short_kernel(SkinnyArgs args) {
    using Geo = SkinnyFastGeometry<1, 1, 1, LOW_M>;
    constexpr int ROW_DW = Geo::ROW_DW, STAGE_DW = Geo::STAGE_DW;
    __shared__ __attribute__((aligned(16))) int32_t smem[Geo::SMEM_DW];
    const int8_t* __restrict__ A = args.A;
    const uint8_t* __restrict__ B = args.B;
    const int M = args.M, K = args.K, NB = args.N >> 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane & 15, kb = lane >> 4;
    int cx, sy;
    {
        const int lin = xcd_linear(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
        cx = lin % gridDim.x;
        sy = lin / gridDim.x;
    }
    const int tile_bc = (cx * SK_WAVES + wave) * 64;
    const int m0 = blockIdx.z * 16;
    const int s_begin = sy * args.steps_per_split;
    const int cnt = tile_bc < NB ? min(min(SPS, args.steps_per_split), (K >> 6) - s_begin) : 0;  // wave-uniform
    const int s_last = s_begin + max(cnt, 1) - 1;

    // Weights: lane (rr, cc) reads 16 bytes at column 16cc of rows 16h + rr of each step; addresses
    // clamped into the matrix, so every load is unconditional.
    const int rr = lane >> 2, cc = lane & 3;
    const uint8_t* wbase = B + (size_t)rr * (size_t)NB + (size_t)(min(tile_bc, NB - 64) + cc * 16);
    v4i g4[SPS][4];
#pragma unroll
    for (int u = 0; u < SPS; ++u) {
        const uint8_t* sb = wbase + (size_t)min(s_begin + u, s_last) * 64 * (size_t)NB;
#pragma unroll
        for (int h = 0; h < 4; ++h) g4[u][h] = *reinterpret_cast<const v4i*>(sb + (size_t)(16 * h) * (size_t)NB);
    }
    // Activations: row m0 + q (clamped; rows >= M are never stored), bytes 16kb.. of each step.
    v4i a[SPS][1];
    if constexpr (AQ == 0) {
        const int8_t* abase = A + (size_t)min(m0 + q, M - 1) * (size_t)K + kb * 16;
#pragma unroll
        for (int u = 0; u < SPS; ++u)
            a[u][0] = *reinterpret_cast<const v4i*>(abase + (size_t)min(s_begin + u, s_last) * 64);
    } else {
        // Each thread loads its elements k = tid + 256 j of a row once (K <= 256 * kRowRegs), the row
        // statistics come from registers (same accumulation order as row_stats.h), and the int8 values
        // of this workgroup's k-range go through LDS to the lanes that feed them to the MFMAs.
        __shared__ float red[4];
        __shared__ __attribute__((aligned(16))) int8_t qbuf[16][SPS * 64];
        const int rows = min(16, M - m0);
        const int kbase = s_begin * 64;
        // the workgroup's k-range (cnt is per wave: 0 for a slab past the last column)
        const int krange = max(min(min(SPS, args.steps_per_split), (K >> 6) - s_begin), 1) * 64;
        for (int r = 0; r < rows; ++r) {  // uniform: every thread takes part in the reductions
            const float* x = args.X + (size_t)(m0 + r) * (size_t)K;
            float xv[kRowRegs], gv[AQ == 2 ? kRowRegs : 1];
#pragma unroll
            for (int j = 0; j < kRowRegs; ++j) {
                const int k = (int)threadIdx.x + 256 * j;
                xv[j] = k < K ? x[k] : 0.0f;
                if constexpr (AQ == 2) gv[j] = k < K ? args.G[k] : 0.0f;
            }
            float inv = 1.0f;
            if constexpr (AQ == 2) {
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < kRowRegs; ++j) ss = fmaf(xv[j], xv[j], ss);  // +0 past K changes nothing
                ss = row_block_sum(ss, red);
                inv = 1.0f / sqrtf(ss / (float)K + args.eps);
            }
            auto val = [&](int j) {
                if constexpr (AQ == 2) return xv[j] * inv * gv[j];
                else return xv[j];
            };
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < kRowRegs; ++j) amax = fmaxf(amax, fabsf(val(j)));
            const float am = fmaxf(row_block_max(amax, red), 1e-5f);
            const float sc = 127.0f / am;
            if (threadIdx.x == 0 && cx == 0 && sy == 0) args.rs_out[m0 + r] = am / 127.0f;
#pragma unroll
            for (int j = 0; j < kRowRegs; ++j) {
                const int kk = (int)threadIdx.x + 256 * j - kbase;
                if (kk >= 0 && kk < krange) qbuf[r][kk] = (int8_t)quantize_value(val(j), sc);
            }
        }
        __syncthreads();
        const int row = min(m0 + q, M - 1) - m0;
#pragma unroll
        for (int u = 0; u < SPS; ++u)
            a[u][0] = *reinterpret_cast<const v4i*>(&qbuf[row][min(u, max(cnt, 1) - 1) * 64 + kb * 16]);
    }

    v4i acc[1][4][4];
    v4i accR[1] = {v4i{0, 0, 0, 0}};
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[0][g][j] = v4i{0, 0, 0, 0};
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    int32_t* stage = smem + wave * STAGE_DW;
#pragma unroll
    for (int u = 0; u < SPS; ++u) {
        if (u < cnt) {
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int R = 16 * h + rr;
                *reinterpret_cast<v4i*>(stage + R * ROW_DW + (R >> 4) * 16 + cc * 4) = g4[u][h];
            }
            __asm__ volatile("" ::: "memory");  // LDS is in order within a wave; keep the compiler so
            uint32_t raw[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) raw[r] = (uint32_t)stage[(16 * kb + r) * ROW_DW + 16 * kb + q];
            __asm__ volatile("" ::: "memory");
            accR[0] = mfma_i8(a[u][0], ones, accR[0]);
            skinny_mfma_block<1, 4>(raw, a[u], 0, acc);
        }
    }
    skinny_epilogue<1, 4, 1, SK_WAVES, LOW_M>(args, smem, acc, accR, wave, 0, tile_bc, m0, sy);
}

// Four packed bytes at (row, bc), 0 outside the K x NB matrix; clamped indices, masked value.
__device__ __forceinline__ uint32_t ld_w4(const uint8_t* __restrict__ B, int row, int bc, int K, int NB, bool aligned) {
    const int rc = min(row, K - 1);
    if (aligned) {
        const int bcc = min(bc, NB - 4);
        const uint32_t v = *reinterpret_cast<const uint32_t*>(B + (size_t)rc * (size_t)NB + bcc);
        return (bc < NB && row < K) ? v : 0u;
    }
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int c = min(bc + b, NB - 1);
        const uint32_t byte = B[(size_t)rc * (size_t)NB + c];
        v |= ((bc + b < NB) ? byte : 0u) << (8 * b);
    }
    return row < K ? v : 0u;
}

// Generic skinny kernel: any K, N % 4 == 0, any alignment.  TB = 1, 2 slabs x 2 waves.  AW / AA:
// weights / activations aligned for dword / 16-byte loads (template parameters, so every load is
// straight-line code).  The next k-step's loads are issued before the current step's MFMAs (two
// register sets, clamped indices, so the number of loads in flight is the same on every path).
template <int MT, bool LOW_M, bool AW, bool AA>
__global__ __launch_bounds__(64 * SK_WAVES) void skinny_generic_kernel(SkinnyArgs args) {
    constexpr int KW = 2, TILES = 2, G = 4;
    __shared__ __attribute__((aligned(16))) int32_t smem[TILES * (KW / 2) * MT * 16 * G * (LOW_M ? 16 : 64)];
    const int8_t* __restrict__ A = args.A;
    const uint8_t* __restrict__ B = args.B;
    const int M = args.M, K = args.K, NB = args.N >> 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tw = wave % TILES, kw = wave / TILES;
    const int q = lane & 15, kb = lane >> 4;
    const int tile_bc = (blockIdx.x * TILES + tw) * 64;
    const int bc = tile_bc + 4 * q;
    const int m0 = blockIdx.z * (16 * MT);
    const int nsteps = (K + 63) >> 6;
    const int s_begin = blockIdx.y * args.steps_per_split;
    const int s_end = tile_bc < NB ? min(nsteps, s_begin + args.steps_per_split) : s_begin;

    v4i acc[MT][G][4];
    v4i accR[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        accR[t] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][g][j] = v4i{0, 0, 0, 0};
    }
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    auto load_step = [&](int st, uint32_t (&raw)[16], v4i (&a)[MT]) {
        const int k0 = st * 64 + kb * 16;
#pragma unroll
        for (int r = 0; r < 16; ++r) raw[r] = ld_w4(B, k0 + r, bc, K, NB, AW);
#pragma unroll
        for (int t = 0; t < MT; ++t) a[t] = load_a16<AA>(A, min(m0 + 16 * t + q, M - 1), k0, M, K);
    };
    auto compute = [&](const uint32_t (&raw)[16], const v4i (&a)[MT]) {
#pragma unroll
        for (int t = 0; t < MT; ++t) accR[t] = mfma_i8(a[t], ones, accR[t]);
        skinny_mfma_block<MT, G>(raw, a, 0, acc);
    };
    const int s0 = s_begin + kw;
    if (s0 < s_end) {
        const int s_last = s0 + ((s_end - 1 - s0) / KW) * KW;  // this wave's last step
        uint32_t raw0[16], raw1[16];
        v4i a0[MT], a1[MT];
        load_step(s0, raw0, a0);
        for (int st = s0;;) {
            load_step(min(st + KW, s_last), raw1, a1);
            compute(raw0, a0);
            st += KW;
            if (st >= s_end) break;
            load_step(min(st + KW, s_last), raw0, a0);
            compute(raw1, a1);
            st += KW;
            if (st >= s_end) break;
        }
    }
    skinny_epilogue<MT, G, KW, TILES, LOW_M>(args, smem, acc, accR, tw, kw, tile_bc, m0, blockIdx.y);
}

// ------------------------------------------------------------------------------------------------
// LDS-tiled GEMM (prefill shapes).
//
// Workgroup tile BM x (4*BNB) outputs, BNB packed byte-columns, k-step 64.  4 waves in a 2 x 2 grid,
// wave tile (BM/2) rows x (BNB/2) byte-columns; per k-step a wave issues (BM/32) x (BNB/32) x 4
// MFMAs.  A tile in LDS: BM rows x 64 bytes, 16-byte chunks XOR-swizzled by (row/4)%4 so the 16 rows
// read by one ds_read_b128 land on distinct banks.  W tile in LDS is stored transposed (byte-column
// major, the 64 k-rows of a byte-column contiguous, pitch 80 bytes) so a lane's B fragment is one
// ds_read_b128; the transpose is done in registers (v_perm) between the global load and the LDS
// store.  Two LDS stages: global loads of step s+1 are issued before the MFMAs of step s.
// ------------------------------------------------------------------------------------------------

constexpr int GM_THREADS = 256;
constexpr int WT_PITCH = 80;  // bytes per transposed byte-column (64 k-rows + 16 pad)

template <int BM, int BNB, bool ALIGNED_W, bool ALIGNED_A>
__global__ __launch_bounds__(GM_THREADS) void gemm_kernel(const int8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                          int32_t* __restrict__ C, int M, int K, int N,
                                                          int tiles_n, int k_begin, int k_end, int accumulate,
                                                          int vec_store, int k_split, OutScale os) {
    if (gridDim.y > 1) {  // split-K: this workgroup's k-range, partial tile in slab blockIdx.y
        k_begin += (int)blockIdx.y * k_split;
        k_end = min(k_end, k_begin + k_split);
        C += (size_t)blockIdx.y * (size_t)M * (size_t)N;
    }
    constexpr int WM = BM / 2;            // rows per wave
    constexpr int WB = BNB / 2;           // byte-columns per wave
    constexpr int MT = WM / 16;           // m-tiles per wave
    constexpr int GT = WB / 16;           // 16-byte-column groups per wave
    constexpr int A_CHUNKS = BM * 4;      // 16-byte chunks per A stage
    constexpr int A_PER_T = A_CHUNKS / GM_THREADS;
    constexpr int W_JOBS = (BNB / 4) * 16;  // (dword column, row quad) jobs per W stage
    constexpr int W_PER_T = (W_JOBS + GM_THREADS - 1) / GM_THREADS;
    static_assert(A_CHUNKS % GM_THREADS == 0, "A tile must split evenly");

    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * 64];
    __shared__ __attribute__((aligned(16))) uint8_t sW[2][BNB * WT_PITCH];

    const int NB = N >> 2;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int q = lane & 15, kb = lane >> 4;

    // Block -> tile: consecutive block ids are dealt round-robin over the 8 XCDs; regroup so that
    // each XCD works on a contiguous run of tiles (neighbouring tiles share A rows / W columns in
    // that XCD's L2).
    const int nblocks = gridDim.x;
    const int bid = blockIdx.x;
    const int per_xcd = (nblocks + 7) >> 3;
    const int xcd = bid & 7, slot = bid >> 3;
    int tile = xcd * per_xcd + slot;
    if ((nblocks & 7) != 0) tile = bid;  // uneven split: keep the plain order
    const int tm = tile / tiles_n, tn = tile % tiles_n;
    const int row0 = tm * BM;
    const int bc0 = tn * BNB;
    // k-steps cover [k_begin, k_end); k_begin % 64 == 0.  Loads treat k >= k_end as zero.
    const int nsteps = (k_end - k_begin + 63) >> 6;

    v4i areg[A_PER_T];
    uint32_t wreg[W_PER_T][4];

    auto gload = [&](int s) {
        const int k0 = k_begin + s * 64;
#pragma unroll
        for (int p = 0; p < A_PER_T; ++p) {
            const int c = tid + p * GM_THREADS;
            const int r = c >> 2, ch = c & 3;
            areg[p] = load_a16_range<ALIGNED_A>(A, row0 + r, k0 + ch * 16, M, K, k_end);
        }
#pragma unroll
        for (int p = 0; p < W_PER_T; ++p) {
            const int job = tid + p * GM_THREADS;
            if (job < W_JOBS) {
                const int dc = job % (BNB / 4), rq = job / (BNB / 4);
#pragma unroll
                for (int r = 0; r < 4; ++r) wreg[p][r] = load_w4<ALIGNED_W>(B, k0 + 4 * rq + r, bc0 + 4 * dc, k_end, NB);
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < A_PER_T; ++p) {
            const int c = tid + p * GM_THREADS;
            const int r = c >> 2, ch = c & 3;
            const int sw = ch ^ ((r >> 2) & 3);
            *reinterpret_cast<v4i*>(&sA[buf][r * 64 + sw * 16]) = areg[p];
        }
#pragma unroll
        for (int p = 0; p < W_PER_T; ++p) {
            const int job = tid + p * GM_THREADS;
            if (job < W_JOBS) {
                const int dc = job % (BNB / 4), rq = job / (BNB / 4);
                uint32_t c0, c1, c2, c3;
                transpose4x4(wreg[p][0], wreg[p][1], wreg[p][2], wreg[p][3], c0, c1, c2, c3);
                uint8_t* base = &sW[buf][(4 * dc) * WT_PITCH + 4 * rq];
                *reinterpret_cast<uint32_t*>(base) = c0;
                *reinterpret_cast<uint32_t*>(base + WT_PITCH) = c1;
                *reinterpret_cast<uint32_t*>(base + 2 * WT_PITCH) = c2;
                *reinterpret_cast<uint32_t*>(base + 3 * WT_PITCH) = c3;
            }
        }
    };

    v4i acc[MT][GT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g = 0; g < GT; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][g][j] = v4i{0, 0, 0, 0};

    if (nsteps > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();

    for (int s = 0; s < nsteps; ++s) {
        const int buf = s & 1;
        if (s + 1 < nsteps) gload(s + 1);

        // B fragments for this wave: GT groups of 16 byte-columns, 16 k-rows each.
        v4i bfr[GT][4];
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            const int col = wn * WB + g * 16 + q;
            const v4i x4 = *reinterpret_cast<const v4i*>(&sW[buf][col * WT_PITCH + kb * 16]);
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const uint32_t x = (uint32_t)x4[rq];
                bfr[g][0][rq] = (int)((x << 6) & 0xC0C0C0C0u);
                bfr[g][1][rq] = (int)((x << 4) & 0xC0C0C0C0u);
                bfr[g][2][rq] = (int)((x << 2) & 0xC0C0C0C0u);
                bfr[g][3][rq] = (int)(x & 0xC0C0C0C0u);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int r = wm * WM + t * 16 + q;
            const int sw = kb ^ ((r >> 2) & 3);
            const v4i a = *reinterpret_cast<const v4i*>(&sA[buf][r * 64 + sw * 16]);
#pragma unroll
            for (int g = 0; g < GT; ++g)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][g][j] = mfma_i8(a, bfr[g][j], acc[t][g][j]);
        }

        if (s + 1 < nsteps) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: element i of tile (t, g, j) is row 4*kb + i of m-tile t, column 4*(byte-col) + j.
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + wm * WM + t * 16 + 4 * kb + i;
            if (row >= M) continue;
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const int bcol = bc0 + wn * WB + g * 16 + q;
                if (bcol >= NB) continue;
                v4i v = {acc[t][g][0][i] >> 6, acc[t][g][1][i] >> 6, acc[t][g][2][i] >> 6, acc[t][g][3][i] >> 6};
                if (os.Y) {  // dequantised float output: y = c * (row_scale[row] * w_scale)
                    store_scaled(os, row, N, 4 * bcol, v, vec_store);
                    continue;
                }
                int32_t* out = C + (size_t)row * (size_t)N + 4 * bcol;
                if (vec_store) {
                    if (accumulate) v += *reinterpret_cast<const v4i*>(out);
                    __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(out));  // streamed, not re-read
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = accumulate ? out[j] + v[j] : v[j];
                }
            }
        }
}

// ------------------------------------------------------------------------------------------------
// Pipelined LDS-tiled GEMM (prefill shapes; K % 128 == 0, NB % 64 == 0, aligned A and W).
//
// Workgroup = 8 waves (8/WGN along M x WGN along N) on a BM x 64-byte-column tile (BM x 256
// outputs); wave tile BM*WGN/8 rows x 64/WGN byte-columns, i.e. m-tiles x 16-byte-column groups x
// 4 fields of 16x16 MFMA outputs.  Each decoded weight fragment feeds all m-tiles of the wave.
// K advances in stages of 128 (two MFMA k-steps), NS LDS stages deep.
//   * A and W both go global -> LDS with direct 16-byte loads (global_load_lds_dwordx4): no
//     registers held, so NS-1 stages are in flight while one is consumed.  Each wave instruction
//     fills 64 consecutive 16-byte LDS slots; the bank-conflict swizzles are applied by choosing
//     which global chunk each lane loads.
//   * A rows (128 bytes per stage): chunk c of row r at position c ^ ((r/2) % 8), so the 16 rows of
//     one ds_read_b128 fragment read fall on distinct banks.
//   * W rows stay row-major (64 bytes = 4 chunks per stage row): chunk c of row r at position
//     c ^ ((r/2) % 4) ^ ((r/16) % 2).  The first term spreads the 8 rows one 16-lane group reads over
//     32 banks; the second gives the group of the next 16 rows (the other half of the wave's k-block,
//     read in the same pass) the other 32 banks (measured: no LDS bank conflicts left).
//     B fragments are read with ds_read_b64_tr_b8, which transposes bytes within
//     each 16-lane group: result lane j, byte i = byte (j % 8) of the 8 bytes addressed by lane
//     2i + j/8.  Lane x addresses k-row (x/2) at byte offset 8*(x%2) of its 16-byte-column group,
//     so lane q receives byte-column q of 8 consecutive k-rows; two reads give the 16 k-rows of its
//     MFMA B operand, with no VALU transpose and no transposed stores.
// Stage s: wait until stage s has landed (vmcnt with a static count: every thread issues the same
// loads each stage, tails are clamped), raw s_barrier, issue stage s+NS-1, then the MFMAs of stage
// s.  A buffer is refilled only after the barrier that follows its last read.
// ------------------------------------------------------------------------------------------------

#define TX_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (7 << 4) | (0xF << 8))
#define TX_LGKMCNT0() __builtin_amdgcn_s_waitcnt((0xF) | (3 << 14) | (7 << 4) | (0 << 8))

// 16 bytes per lane from global memory straight into LDS: lane l of the wave writes lds + 16*l.
// (A plain device function, so the kernel templates that call it instantiate cleanly for the host.)
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds) {
    __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// Transposing 8-byte LDS read (see above).  Issued as inline assembly: the compiler then neither
// waits for the LDS DMA in flight into other stage buffers before it (it cannot tell they do not
// alias) nor for its own result -- the caller waits with lgkmcnt before using the value.
__device__ __forceinline__ uint64_t lds_read_tr8(const void* lds) {
    uint64_t v;
    const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
    __asm__ volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

constexpr int GF_THREADS = 512;
constexpr int GF_BK = 128;
constexpr int GF_BNB = 64;

__device__ __forceinline__ int gf_swz_a(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int gf_swz_w(int r) { return ((r >> 1) & 3) ^ ((r >> 4) & 1); }
// W swizzle for a given stage-row width: 64-byte rows as gf_swz_w; 32-byte rows (two chunks) keep the
// 8 rows of one transposing read on distinct banks by their pitch alone and flip the chunk for the
// second 16-row half of a wave's k-block, which is read in the same pass.
template <int BNB>
__device__ __forceinline__ int swz_w(int r) { return BNB == 64 ? gf_swz_w(r) : (BNB == 32 ? ((r >> 4) & 1) : 0); }

template <int BM, int WGN, int NS, int BK>
__global__ __launch_bounds__(GF_THREADS) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_fast_kernel(const int8_t* __restrict__ A, const uint8_t* __restrict__ B, int32_t* __restrict__ C, int M,
                      int K, int N, int tiles_n, int k_begin, int k_end, int accumulate, int vec_store,
                      int k_split, OutScale os) {
    if (gridDim.y > 1) {  // split-K: this workgroup's k-range, partial tile in slab blockIdx.y
        k_begin += (int)blockIdx.y * k_split;
        k_end = min(k_end, k_begin + k_split);
        C += (size_t)blockIdx.y * (size_t)M * (size_t)N;
    }
    constexpr int WGM = 8 / WGN;             // waves along M
    constexpr int WM = BM / WGM;             // rows per wave
    constexpr int MT = WM / 16;              // m-tiles per wave
    constexpr int GT = 4 / WGN;              // 16-byte-column groups per wave
    constexpr int KS = BK / 64;              // MFMA k-steps per stage
    constexpr int CPR = BK / 16;             // 16-byte A chunks per row per stage
    constexpr int A_STAGE = BM * BK;         // bytes
    constexpr int W_STAGE = BK * GF_BNB;     // bytes
    constexpr int NA = A_STAGE / 16 / GF_THREADS;  // A loads per thread per stage
    constexpr int NW = W_STAGE / 16 / GF_THREADS;  // W loads per thread per stage
    // Separate arrays per stage: the compiler tracks in-flight LDS DMA per array, so reads of one
    // stage do not wait for loads into the others.
    __shared__ __attribute__((aligned(16))) int8_t sA0[A_STAGE];
    __shared__ __attribute__((aligned(16))) int8_t sA1[A_STAGE];
    __shared__ __attribute__((aligned(16))) int8_t sA2[A_STAGE];
    __shared__ __attribute__((aligned(16))) int8_t sA3[NS > 3 ? A_STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t sW0[W_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW1[W_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW2[W_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW3[NS > 3 ? W_STAGE : 16];
    auto stage_a = [&](int i) -> int8_t* { return i == 0 ? sA0 : (i == 1 ? sA1 : (i == 2 ? sA2 : sA3)); };
    auto stage_w = [&](int i) -> uint8_t* { return i == 0 ? sW0 : (i == 1 ? sW1 : (i == 2 ? sW2 : sW3)); };

    const int NB = N >> 2;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int q = lane & 15, kb = lane >> 4;

    // Block -> tile, XCD-aware: each XCD gets a contiguous run of tile numbers (xcd_linear).
    // Grouped order: consecutive tile numbers walk 4 row bands before moving to the next column
    // band, so each XCD's contiguous run of tiles is a ~4 x 8 block (A read by ~2 XCDs and W by
    // ~4, instead of W by all 8).
    int tm, tn;
    {
        const int t = xcd_linear(blockIdx.x, gridDim.x);
        const int tiles_m = gridDim.x / tiles_n;
        constexpr int GM = 4;
        const int first_m = (t / (GM * tiles_n)) * GM;
        const int gm = min(tiles_m - first_m, GM);
        const int local = t % (GM * tiles_n);
        tm = first_m + local % gm;
        tn = local / gm;
    }
    const int row0 = tm * BM;
    const int bc0 = tn * GF_BNB;
    const int nst = (k_end - k_begin) / BK;  // stages

    // Load geometry.  Instruction p of wave w fills 16-byte slots (p*8 + w)*64 + lane.  32-bit lane
    // offsets (M*K and K*NB < 2^32, checked by the launcher) from wave-uniform bases.
    uint32_t a_off[NA];
#pragma unroll
    for (int p = 0; p < NA; ++p) {
        const int slot = (p * 8 + wave) * 64 + lane;
        const int r = slot / CPR, pos = slot % CPR;
        const int grow = min(row0 + r, M - 1);  // rows past M load row M-1; never stored
        a_off[p] = (uint32_t)grow * (uint32_t)K + (uint32_t)(((pos & ~7) | ((pos & 7) ^ gf_swz_a(r))) * 16);
    }
    uint32_t w_off[NW];
#pragma unroll
    for (int p = 0; p < NW; ++p) {
        const int slot = (p * 8 + wave) * 64 + lane;
        const int r = slot >> 2, pos = slot & 3;
        w_off[p] = (uint32_t)r * (uint32_t)NB + (uint32_t)(bc0 + (pos ^ gf_swz_w(r)) * 16);
    }
    auto issue = [&](int st, int buf) {
        const int sc = min(st, nst - 1);  // clamped: keeps the per-stage load count static
        const int8_t* abase = A + k_begin + (size_t)sc * BK;
        int8_t* adst = stage_a(buf);
#pragma unroll
        for (int p = 0; p < NA; ++p) lds_dma16(abase + a_off[p], adst + (p * 8 + wave) * 1024);
        const uint8_t* wbase = B + (size_t)(k_begin + sc * BK) * (size_t)NB;
        uint8_t* wdst = stage_w(buf);
#pragma unroll
        for (int p = 0; p < NW; ++p) lds_dma16(wbase + w_off[p], wdst + (p * 8 + wave) * 1024);
    };

    v4i acc[MT][GT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g = 0; g < GT; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][g][j] = v4i{0, 0, 0, 0};

    auto compute = [&](int buf) {
        const int8_t* a_st = stage_a(buf);
        const uint8_t* w_st = stage_w(buf);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            v4i a[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int r = wm * WM + t * 16 + q;
                const int c = kk * 4 + kb;  // chunk; the swizzle permutes within groups of 8
                a[t] = *reinterpret_cast<const v4i*>(a_st + r * BK + 16 * ((c & ~7) | ((c & 7) ^ gf_swz_a(r))));
            }
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const int cg = wn * GT + g;  // 16-byte column group within the tile
                const int r0 = kk * 64 + kb * 16 + (q >> 1);
                const int r1 = r0 + 8;
                uint64_t lo = lds_read_tr8(w_st + r0 * GF_BNB + 16 * (cg ^ gf_swz_w(r0)) + 8 * (q & 1));
                uint64_t hi = lds_read_tr8(w_st + r1 * GF_BNB + 16 * (cg ^ gf_swz_w(r1)) + 8 * (q & 1));
                // The wait names the results, so no use of them can be scheduled before it.
                __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo), "+v"(hi));
                const uint32_t x4[4] = {(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
                v4i bfr[4];
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const uint32_t x = x4[r4];
                    bfr[0][r4] = (int)((x << 6) & 0xC0C0C0C0u);
                    bfr[1][r4] = (int)((x << 4) & 0xC0C0C0C0u);
                    bfr[2][r4] = (int)((x << 2) & 0xC0C0C0C0u);
                    bfr[3][r4] = (int)(x & 0xC0C0C0C0u);
                }
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[t][g][j] = mfma_i8(a[t], bfr[j], acc[t][g][j]);
            }
        }
    };

    // Prologue: stages 0 .. NS-2 in flight.
#pragma unroll
    for (int p = 0; p < NS - 1; ++p) issue(p, p);

    // h is always a literal at the call sites, so after inlining every buffer index is a constant;
    // the main loop has no conditions, so the compiler counts the loads in flight exactly as the
    // waits assume.
    auto stage = [&](int st, int h) {
        TX_VMCNT((NS - 2) * (NA + NW));  // stage st has landed (the NS-2 later stages may not)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(st + NS - 1, (h + NS - 1) % NS);
        compute(h % NS);
        TX_LGKMCNT0();  // this stage's LDS reads are done before the next barrier
        __builtin_amdgcn_sched_barrier(0);
    };
    int s = 0;
    for (; s + NS <= nst; s += NS) {
        stage(s + 0, 0);
        stage(s + 1, 1);
        stage(s + 2, 2);
        if (NS > 3) stage(s + 3, 3);
    }
    if (s + 0 < nst) stage(s + 0, 0);
    if (s + 1 < nst) stage(s + 1, 1);
    if (NS > 3 && s + 2 < nst) stage(s + 2, 2);
    TX_VMCNT(0);  // no LDS DMA may land after the workgroup exits

    // Epilogue: element i of tile (t, g, j) is row 4*kb + i of m-tile t, column 4*(byte-col) + j.
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + wm * WM + t * 16 + 4 * kb + i;
            if (row >= M) continue;
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const int bcol = bc0 + (wn * GT + g) * 16 + q;
                v4i v = {acc[t][g][0][i] >> 6, acc[t][g][1][i] >> 6, acc[t][g][2][i] >> 6, acc[t][g][3][i] >> 6};
                if (os.Y) {  // dequantised float output: y = c * (row_scale[row] * w_scale)
                    store_scaled(os, row, N, 4 * bcol, v, vec_store);
                    continue;
                }
                int32_t* out = C + (size_t)row * (size_t)N + 4 * bcol;
                if (vec_store) {
                    if (accumulate) v += *reinterpret_cast<const v4i*>(out);
                    __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(out));  // streamed, not re-read
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = accumulate ? out[j] + v[j] : v[j];
                }
            }
        }
}

// ------------------------------------------------------------------------------------------------
// Software-pipelined variant of the LDS-tiled GEMM.  Same tiles, LDS layouts and DMA as
// gemm_fast_kernel; the difference is the order of work inside a wave:
//   * every LDS fragment read is inline assembly, so the only LDS waits are the explicit ones;
//   * the fragments of the next MFMA k-step are read while the MFMAs of the current one run
//     (two register sets, alternating);
//   * the stage barrier (stage s+1 landed everywhere, stage s free for reuse) and the DMA issue of
//     stage s+NS happen before the last k-step's MFMAs of stage s, and the first fragments of
//     stage s+1 are read right after it, so the MFMA pipe never waits for a fresh stage's reads.
// NS stages are in flight: NS-1 DMA stages ahead of the one being read.
// ------------------------------------------------------------------------------------------------
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
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

template <int MT, int GT>
struct PipeFrag {
    v4i a[MT];
    uint64_t lo[GT], hi[GT];
};

template <int BM, int WGN, int NS, int BK, int NWV, int BNB>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_pipe_kernel(const int8_t* __restrict__ A, const uint8_t* __restrict__ B, int32_t* __restrict__ C, int M,
                      int K, int N, int tiles_n, int k_begin, int k_end, int accumulate, int vec_store,
                      int k_split, OutScale os) {
    if (gridDim.y > 1) {  // split-K: this workgroup's k-range, partial tile in slab blockIdx.y
        k_begin += (int)blockIdx.y * k_split;
        k_end = min(k_end, k_begin + k_split);
        C += (size_t)blockIdx.y * (size_t)M * (size_t)N;
    }
    constexpr int THR = 64 * NWV;           // threads per workgroup
    constexpr int CW = BNB / 16;            // 16-byte chunks per W stage row
    constexpr int WGM = NWV / WGN;
    constexpr int WM = BM / WGM;
    constexpr int MT = WM / 16;
    constexpr int GT = CW / WGN;
    constexpr int KS = BK / 64;
    constexpr int CPR = BK / 16;
    constexpr int A_STAGE = BM * BK;
    constexpr int W_STAGE = BK * BNB;
    constexpr int NA = A_STAGE / 16 / THR;
    constexpr int NW = W_STAGE / 16 / THR;
    static_assert(KS % 2 == 0, "fragment sets alternate per k-step");
    static_assert(NA >= 1 && NW >= 1 && GT >= 1, "tile too small for the workgroup");
    __shared__ __attribute__((aligned(16))) int8_t sA0[A_STAGE];
    __shared__ __attribute__((aligned(16))) int8_t sA1[A_STAGE];
    __shared__ __attribute__((aligned(16))) int8_t sA2[A_STAGE];
    __shared__ __attribute__((aligned(16))) int8_t sA3[NS > 3 ? A_STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t sW0[W_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW1[W_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW2[W_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW3[NS > 3 ? W_STAGE : 16];
    auto stage_a = [&](int i) -> int8_t* { return i == 0 ? sA0 : (i == 1 ? sA1 : (i == 2 ? sA2 : sA3)); };
    auto stage_w = [&](int i) -> uint8_t* { return i == 0 ? sW0 : (i == 1 ? sW1 : (i == 2 ? sW2 : sW3)); };

    const int NB = N >> 2;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int q = lane & 15, kb = lane >> 4;

    const int tiles_m = (M + BM - 1) / BM;
    int tm, tn;
    {
        const int t = xcd_linear(blockIdx.x, gridDim.x);
        constexpr int GM = 4;
        const int first_m = (t / (GM * tiles_n)) * GM;
        const int gm = min(tiles_m - first_m, GM);
        const int local = t % (GM * tiles_n);
        tm = first_m + local % gm;
        tn = local / gm;
    }
    const int row0 = tm * BM;
    const int bc0 = tn * BNB;
    const int nst = (k_end - k_begin) / BK;

    uint32_t a_off[NA];
#pragma unroll
    for (int p = 0; p < NA; ++p) {
        const int slot = (p * NWV + wave) * 64 + lane;
        const int r = slot / CPR, pos = slot % CPR;
        const int grow = min(row0 + r, M - 1);
        a_off[p] = (uint32_t)grow * (uint32_t)K + (uint32_t)(((pos & ~7) | ((pos & 7) ^ gf_swz_a(r))) * 16);
    }
    uint32_t w_off[NW];
#pragma unroll
    for (int p = 0; p < NW; ++p) {
        const int slot = (p * NWV + wave) * 64 + lane;
        const int r = slot / CW, pos = slot % CW;
        w_off[p] = (uint32_t)r * (uint32_t)NB + (uint32_t)(bc0 + (pos ^ swz_w<BNB>(r)) * 16);
    }
    auto issue = [&](int st, int buf) {
        const int sc = min(st, nst - 1);
        const int8_t* abase = A + k_begin + (size_t)sc * BK;
        int8_t* adst = stage_a(buf);
#pragma unroll
        for (int p = 0; p < NA; ++p) lds_dma16(abase + a_off[p], adst + (p * NWV + wave) * 1024);
        const uint8_t* wbase = B + (size_t)(k_begin + sc * BK) * (size_t)NB;
        uint8_t* wdst = stage_w(buf);
#pragma unroll
        for (int p = 0; p < NW; ++p) lds_dma16(wbase + w_off[p], wdst + (p * NWV + wave) * 1024);
    };

    // Per-lane fragment offsets inside a stage.  A: row wm*WM + 16t + q, chunk kk*4 + kb (the swizzle
    // depends on the row only through (row/2) % 8, the same for all t).  W: k-row 64kk + 16kb + q/2
    // (+8 for the second read), 16-byte group wn*GT + g (swizzle through (row/2) % 4, the same for all
    // kk and for the +8 row).
    uint32_t a_lane[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        const int r = wm * WM + q;
        const int c = kk * 4 + kb;
        a_lane[kk] = (uint32_t)(r * BK + 16 * ((c & ~7) | ((c & 7) ^ gf_swz_a(r))));
    }
    uint32_t w_lane[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        const int cg = wn * GT + g;
        const int r0 = kb * 16 + (q >> 1);
        w_lane[g] = (uint32_t)(r0 * BNB + 16 * (cg ^ swz_w<BNB>(r0)) + 8 * (q & 1));
    }
    auto read = [&](PipeFrag<MT, GT>& f, int buf, int kk) {
        const uint32_t ab = lds_u32(stage_a(buf)) + a_lane[kk];
#pragma unroll
        for (int t = 0; t < MT; ++t) f.a[t] = lds_read_b128_asm(ab + (uint32_t)(t * 16 * BK));
        const uint32_t wb = lds_u32(stage_w(buf)) + (uint32_t)(kk * 64 * BNB);
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            f.lo[g] = lds_read_tr8_asm(wb + w_lane[g]);
            f.hi[g] = lds_read_tr8_asm(wb + w_lane[g] + 8 * BNB);
        }
    };
    // All LDS reads issued so far have returned; the empty asm statements tie each fragment register
    // to that point, so no use of them is scheduled before it.
    auto wait_frag = [&](PipeFrag<MT, GT>& f) {
        TX_LGKMCNT0();
#pragma unroll
        for (int t = 0; t < MT; ++t) __asm__ volatile("" : "+v"(f.a[t]));
#pragma unroll
        for (int g = 0; g < GT; ++g) __asm__ volatile("" : "+v"(f.lo[g]), "+v"(f.hi[g]));
    };

    v4i acc[MT][GT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g = 0; g < GT; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][g][j] = v4i{0, 0, 0, 0};

    auto mfmas = [&](const PipeFrag<MT, GT>& f) {
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            const uint32_t x4[4] = {(uint32_t)f.lo[g], (uint32_t)(f.lo[g] >> 32), (uint32_t)f.hi[g],
                                    (uint32_t)(f.hi[g] >> 32)};
            v4i bfr[4];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const uint32_t x = x4[r4];
                bfr[0][r4] = (int)((x << 6) & 0xC0C0C0C0u);
                bfr[1][r4] = (int)((x << 4) & 0xC0C0C0C0u);
                bfr[2][r4] = (int)((x << 2) & 0xC0C0C0C0u);
                bfr[3][r4] = (int)(x & 0xC0C0C0C0u);
            }
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][g][j] = mfma_i8(f.a[t], bfr[j], acc[t][g][j]);
        }
    };

    PipeFrag<MT, GT> f0, f1;
    // Prologue: all NS stages in flight, wait for stage 0, first fragments.
#pragma unroll
    for (int p = 0; p < NS; ++p) issue(p, p);
    TX_VMCNT((NS - 1) * (NA + NW));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read(f0, 0, 0);

    // One stage in buffer h (a literal at every call site).  Fragment set f0 serves even k-steps.
    auto stage = [&](int st, int h) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            PipeFrag<MT, GT>& cur = (kk & 1) ? f1 : f0;
            PipeFrag<MT, GT>& nxt = (kk & 1) ? f0 : f1;
            wait_frag(cur);
            __builtin_amdgcn_sched_barrier(0);
            if (kk + 1 < KS) {
                read(nxt, h, kk + 1);
            } else if (st + 1 < nst) {
                TX_VMCNT((NS - 2) * (NA + NW));  // stage st+1 has landed (NS-2 later stages may not)
                __builtin_amdgcn_s_barrier();     // ... everywhere, and every wave is done reading stage st
                __builtin_amdgcn_sched_barrier(0);
                issue(st + NS, h);
                read(nxt, (h + 1) % NS, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            mfmas(cur);
            // keep the next k-step's wait below these MFMAs (it would otherwise be hoisted among them
            // and wait for the reads just issued)
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int s = 0;
    for (; s + NS <= nst; s += NS) {
        stage(s + 0, 0);
        stage(s + 1, 1);
        stage(s + 2, 2);
        if (NS > 3) stage(s + 3, 3);
    }
    if (s + 0 < nst) stage(s + 0, 0);
    if (s + 1 < nst) stage(s + 1, 1);
    if (NS > 3 && s + 2 < nst) stage(s + 2, 2);
    TX_VMCNT(0);  // no LDS DMA may land after the workgroup exits

#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + wm * WM + t * 16 + 4 * kb + i;
            if (row >= M) continue;
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const int bcol = bc0 + (wn * GT + g) * 16 + q;
                v4i v = {acc[t][g][0][i] >> 6, acc[t][g][1][i] >> 6, acc[t][g][2][i] >> 6, acc[t][g][3][i] >> 6};
                if (os.Y) {  // dequantised float output: y = c * (row_scale[row] * w_scale)
                    store_scaled(os, row, N, 4 * bcol, v, vec_store);
                    continue;
                }
                int32_t* out = C + (size_t)row * (size_t)N + 4 * bcol;
                if (vec_store) {
                    if (accumulate) v += *reinterpret_cast<const v4i*>(out);
                    __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(out));  // streamed, not re-read
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = accumulate ? out[j] + v[j] : v[j];
                }
            }
        }
}

// ------------------------------------------------------------------------------------------------
// DMA-staged skinny kernel (M <= 16 per m-group, long weight streams).
//
// The register-staged skinny kernels read each weight row as 64-byte pieces, one per wave, so every
// load instruction touches 16 rows x half a cache line and only PD k-steps fit in a wave's registers.
// Here the workgroup's weight strip (256 bytes of each row, 1024 outputs) goes global -> LDS with
// global_load_lds_dwordx4: one instruction reads 4 whole rows of the strip (full 128-byte lines),
// no registers hold data in flight, and NS-1 k-steps (16 KB each) are in flight per workgroup, small
// enough for two workgroups per CU.  The activation slice of the k-range (16 rows, clamped, up to
// 16*NAD 16-byte chunks per row) is DMA'd once at the start in k-chunk-major order, so the 16 rows
// one fragment read touches are 256 contiguous bytes.
//   * Stage layout: 64 rows x 16 chunks of 16 bytes; chunk c of row r sits at position
//     c ^ sd_swz(r), chosen per lane when the DMA address is formed.  sd_swz spreads the 8 rows that
//     one 16-lane group of a transposing read touches over 8 positions (32 banks) and gives the next
//     16-row group the other 32 banks.
//   * B fragments: ds_read_b64_tr_b8 as in gemm_pipe_kernel -- lane q gets byte-column q of its
//     16-byte group for 16 k-rows (two reads); wave w owns groups 4w..4w+3 (a 64-byte slab).
//   * Decode: shift form, field j of every byte moved to bits 6-7 (values 64*w), result >> 6.
// Step it: wait for this wave's DMAs of step it (static vmcnt while later steps are in flight,
// vmcnt(0) in the last NS-1 steps), barrier, issue step it+NS-1 into the buffer read at step it-1,
// read fragments, MFMAs.  Outputs and modes are those of the other skinny kernels.
// ------------------------------------------------------------------------------------------------
constexpr int SD_BNB = 256;                  // strip bytes per row (per workgroup)
constexpr int SD_STAGE = 64 * SD_BNB;        // one k-step
constexpr int SD_NL = SD_STAGE / 16 / 256;   // DMA instructions per thread per k-step

__device__ __forceinline__ int sd_swz(int r) { return (r & 7) | (((r >> 4) & 1) << 3); }

template <int NS, int NAD, bool LOW_M, int AQ = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void skinny_dma_kernel(SkinnyArgs args) {
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    __shared__ __attribute__((aligned(16))) uint8_t sW0[SD_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW1[SD_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW2[NS > 2 ? SD_STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t sW3[NS > 3 ? SD_STAGE : 16];
    __shared__ __attribute__((aligned(16))) int8_t sA[NAD * 256 * 16];
    auto stage_w = [&](int i) -> uint8_t* { return i == 0 ? sW0 : (i == 1 ? sW1 : (i == 2 ? sW2 : sW3)); };

    const int8_t* __restrict__ A = args.A;
    const uint8_t* __restrict__ B = args.B;
    const int M = args.M, K = args.K, NB = args.N >> 2;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane & 15, kb = lane >> 4;
    int cx, sy;
    {
        const int lin = xcd_linear(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
        cx = lin % gridDim.x;
        sy = lin / gridDim.x;
    }
    const int bc0 = cx * SD_BNB;
    const int m0 = blockIdx.z * 16;
    const int s_begin = sy * args.steps_per_split;
    const int nst = min(K >> 6, s_begin + args.steps_per_split) - s_begin;  // >= 1 (planner)

    // Activation slice: position j = 16 c + r holds 16-byte chunk c of row r (rows clamped to the
    // m-group, chunks to the k-range).  AQ > 0: built below from the fp32 rows instead.
    const int a_rows = min(16, M - m0);
    float xv[AQ ? kRowRegs : 1], gv[AQ == 2 ? kRowRegs : 1];
    auto load_row = [&](int r) {  // elements k = tid + 256 j of row m0 + r (K <= 256 * kRowRegs)
        const float* x = args.X + (size_t)(m0 + r) * (size_t)K;
#pragma unroll
        for (int j = 0; j < (AQ ? kRowRegs : 0); ++j) {
            const int k = tid + 256 * j;
            xv[j] = k < K ? x[k] : 0.0f;
            if constexpr (AQ == 2) gv[j] = k < K ? args.G[k] : 0.0f;
        }
    };
    if constexpr (AQ != 0) {
        load_row(0);  // before the weight DMAs, so waiting for it does not wait for them
    } else {
        const int8_t* abase = A + (size_t)m0 * (size_t)K + (size_t)s_begin * 64;
#pragma unroll
        for (int u = 0; u < NAD; ++u) {
            const int j = u * 256 + tid;
            const int c = min(j >> 4, nst * 4 - 1), r = min(j & 15, a_rows - 1);
            lds_dma16(abase + (size_t)r * (size_t)K + c * 16, sA + (u * 256 + wave * 64) * 16);
        }
    }
    uint32_t w_off[SD_NL];
#pragma unroll
    for (int p = 0; p < SD_NL; ++p) {
        const int slot = (p * 4 + wave) * 64 + lane;
        const int r = slot >> 4, pos = slot & 15;
        const int col = min(bc0 + (pos ^ sd_swz(r)) * 16, NB - 16);  // past the last column: re-read, unused
        w_off[p] = (uint32_t)r * (uint32_t)NB + (uint32_t)col;
    }
    auto issue = [&](int st, int buf) {
        const uint8_t* wbase = B + (size_t)(s_begin + st) * 64 * (size_t)NB;
        uint8_t* wdst = stage_w(buf);
#pragma unroll
        for (int p = 0; p < SD_NL; ++p) lds_dma16(wbase + w_off[p], wdst + (p * 4 + wave) * 1024);
    };
    uint32_t w_lane[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int r0 = kb * 16 + (q >> 1);
        w_lane[g] = (uint32_t)(r0 * SD_BNB + 16 * ((wave * 4 + g) ^ sd_swz(r0)) + 8 * (q & 1));
    }
    const uint32_t a_lane = lds_u32(sA) + (uint32_t)((kb * 16 + q) * 16);

    v4i acc[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[g][j] = v4i{0, 0, 0, 0};

    auto step = [&](int it, int buf) {
        const uint32_t wb = lds_u32(stage_w(buf));
        uint64_t lo[4], hi[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            lo[g] = lds_read_tr8_asm(wb + w_lane[g]);
            hi[g] = lds_read_tr8_asm(wb + w_lane[g] + 8 * SD_BNB);
        }
        v4i a = lds_read_b128_asm(a_lane + (uint32_t)(it * 64 * 16));
        TX_LGKMCNT0();
        __asm__ volatile("" : "+v"(a));
#pragma unroll
        for (int g = 0; g < 4; ++g) __asm__ volatile("" : "+v"(lo[g]), "+v"(hi[g]));
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t x4[4] = {(uint32_t)lo[g], (uint32_t)(lo[g] >> 32), (uint32_t)hi[g], (uint32_t)(hi[g] >> 32)};
            v4i bfr[4];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const uint32_t x = x4[r4];
                bfr[0][r4] = (int)((x << 6) & 0xC0C0C0C0u);
                bfr[1][r4] = (int)((x << 4) & 0xC0C0C0C0u);
                bfr[2][r4] = (int)((x << 2) & 0xC0C0C0C0u);
                bfr[3][r4] = (int)(x & 0xC0C0C0C0u);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[g][j] = mfma_i8(a, bfr[j], acc[g][j]);
        }
    };

    // Prologue: NS-1 steps in flight (the activation slice DMA went first).
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
        if (p < nst) issue(p, p);
    if constexpr (AQ != 0) {
        // Fused activation quantisation (the rule and accumulation order of quantize_rows_kernel /
        // rmsnorm_kernel, from row_stats.h, so the int8 values are bit-identical to theirs): every
        // workgroup computes its rows' statistics from registers and writes the int8 values of its
        // own k-range into the slice layout; workgroup (0, 0) stores the row scales for the reduce.
        __shared__ float red[4];
        const int kbase = s_begin * 64, krange = nst * 64;
        for (int r = 0; r < a_rows; ++r) {  // uniform: every thread takes part in the reductions
            if (r > 0) load_row(r);
            float inv = 1.0f;
            if constexpr (AQ == 2) {
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < kRowRegs; ++j) ss = fmaf(xv[j], xv[j], ss);  // +0 past K changes nothing
                ss = row_block_sum(ss, red);
                inv = 1.0f / sqrtf(ss / (float)K + args.eps);
            }
            auto val = [&](int j) {
                if constexpr (AQ == 2) return xv[j] * inv * gv[j];
                else return xv[j];
            };
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < kRowRegs; ++j) amax = fmaxf(amax, fabsf(val(j)));
            const float am = fmaxf(row_block_max(amax, red), 1e-5f);
            const float sc = 127.0f / am;
            if (tid == 0 && cx == 0 && sy == 0) args.rs_out[m0 + r] = am / 127.0f;
#pragma unroll
            for (int j = 0; j < kRowRegs; ++j) {
                const int kk = tid + 256 * j - kbase;
                if (kk >= 0 && kk < krange) sA[((kk >> 4) * 16 + r) * 16 + (kk & 15)] = (int8_t)quantize_value(val(j), sc);
            }
        }
        TX_LGKMCNT0();  // this thread's slice bytes are written; the first step's barrier publishes them
    }
    int it = 0;
    // Steady state: step it+NS-1 exists, so exactly NS-1 steps are outstanding at each wait.
    for (; it + NS - 1 < nst; ++it) {
        TX_VMCNT((NS - 2) * SD_NL);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(it + NS - 1, (it + NS - 1) % NS);
        step(it, it % NS);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (; it < nst; ++it) {
        TX_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        step(it, it % NS);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Epilogue: lane (q, kb) holds rows 4kb+i of byte-columns bc0 + 16(4 wave + g) + q.
    if (LOW_M && kb != 0) return;
    int32_t* out_base = args.mode == SK_PARTIAL ? args.P + (size_t)sy * (size_t)M * (size_t)args.N : args.C;
    const bool vec = args.mode == SK_PARTIAL || args.vec_store;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 4 * kb + i;
        if (row >= M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int bcol = bc0 + (wave * 4 + g) * 16 + q;
            if (bcol >= NB) continue;
            const v4i v = {acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            if (args.mode == SK_STORE && args.os.Y) {
                store_scaled(args.os, row, args.N, 4 * bcol, v, args.vec_store);
                continue;
            }
            int32_t* out = out_base + (size_t)row * (size_t)args.N + 4 * bcol;
            if (args.mode == SK_ATOMIC) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (v[j] != 0) atomicAdd(out + j, v[j]);
            } else if (vec) {
                *reinterpret_cast<v4i*>(out) = v;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = v[j];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Wave-pipelined skinny kernel (M <= 16 per m-group): no barrier in the k-loop.
//
// A workgroup owns SW bytes of every weight row (4 * SW outputs) and its four waves take alternate
// 64-row k-steps of the workgroup's k-range.  Each wave streams its own steps global -> LDS with
// global_load_lds_dwordx4 into a private ring of NSW slots (64 x SW bytes each) and reads them back
// with ds_read_b64_tr_b8 itself, so only the wave's own vmcnt orders the ring: no workgroup barrier
// until the four waves' sums are combined at the end.  The activation fragment of a step (16 rows,
// clamped, 16 bytes per lane) is loaded with the step's DMAs.  Narrow strips give many workgroups
// without a K split, so a wide-N GEMV can store C directly (one launch, no reduce).
//   * SW = 32: chunk c of row r at position c ^ ((r / 16) % 2) (the two 16-lane groups of a
//     transposing read use different banks); SW = 16: row r at position r ^ (8 ((r / 16) % 2)).
// Loads are issued for the same number of steps on every wave (clamped addresses past the range, no
// MFMAs for them), so the vmcnt waits are static.
// ------------------------------------------------------------------------------------------------
template <int SW, int NSW, bool LOW_M, int AQ = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void skinny_wave_kernel(SkinnyArgs args) {
    static_assert(SW == 16 || SW == 32, "16- or 32-byte strips");
    constexpr int QK = 4096;                   // AQ: whole rows of K <= QK quantised into LDS
    constexpr int G = SW / 16;                 // 16-byte column groups per strip
    constexpr int SLOT = 64 * SW;              // bytes per ring slot (one k-step)
    constexpr int NL = SLOT / 1024;            // DMA instructions per step per wave
    constexpr int RED = 3 * 64 * 16 * G * 4;   // cross-wave reduction buffer (waves 1-3)
    constexpr int RING = 4 * NSW * SLOT;
    __shared__ __attribute__((aligned(16))) uint8_t lds[RING > RED ? RING : RED];
    __shared__ __attribute__((aligned(16))) int8_t qbuf[AQ ? 16 : 1][AQ ? QK : 16];
    __shared__ float rscale[16];

    const int8_t* __restrict__ A = args.A;
    const uint8_t* __restrict__ B = args.B;
    const int M = args.M, K = args.K, NB = args.N >> 2;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane & 15, kb = lane >> 4;
    // Block -> (strip, split): the hardware deals block ids round-robin to the 8 XCDs (XCD = id % 8).
    // The 128 / SW strips that share each 128-byte line of a weight row form one unit, and all
    // blocks of a unit sit on one XCD, so the line is fetched into one L2 only; ids past the last
    // unit, or strips past the last column, have no work.
    constexpr int SPL = 128 / SW;  // strips per 128-byte line
    const int n_strips = NB / SW, lines = (n_strips + SPL - 1) / SPL;
    int cx, sy;
    if (args.line_units) {
        const int b = blockIdx.x, t = b >> 3;
        const int u = (b & 7) + 8 * (t / SPL);  // unit: (split, line group)
        sy = u / lines;
        cx = (u % lines) * SPL + t % SPL;
        if (sy >= args.splits || cx >= n_strips) return;  // whole workgroup: no barrier reached yet
    } else {
        // contiguous strip ranges per XCD (balanced; lines at range ends are fetched by two L2s)
        const int total = n_strips * args.splits;
        if ((int)blockIdx.x >= total) return;
        const int lin = xcd_linear(blockIdx.x, total);
        cx = lin % n_strips;
        sy = lin / n_strips;
    }
    const int bc0 = cx * SW;
    const int m0 = blockIdx.z * 16;
    const int s_begin = sy * args.steps_per_split;
    const int nst = min(K >> 6, s_begin + args.steps_per_split) - s_begin;  // >= 1
    const int iters = ((nst + 3) / 4 + NSW - 1) / NSW * NSW;                  // per wave, padded
    uint8_t* ring = lds + wave * NSW * SLOT;

    // DMA lane mapping: instruction p, lane l -> LDS byte 1024 p + 16 l of the slot.
    uint32_t w_off[NL];
#pragma unroll
    for (int p = 0; p < NL; ++p) {
        const int pos = p * 64 + lane;  // 16-byte position in the slot
        int r, c;
        if (SW == 32) {
            r = pos >> 1;
            c = (pos & 1) ^ ((r >> 4) & 1);
        } else {
            r = pos ^ (((pos >> 4) & 1) << 3);
            c = 0;
        }
        w_off[p] = (uint32_t)r * (uint32_t)NB + (uint32_t)(bc0 + 16 * c);
    }
    const int a_rows = min(16, M - m0);
    const int8_t* a_row = A + (size_t)(m0 + min(q, a_rows - 1)) * (size_t)K + kb * 16;
    const int s_last = s_begin + nst - 1;
    v4i a_ring[NSW];
    auto issue = [&](int it, int slot_c, v4i& a_dst) {
        const int s = min(s_begin + wave + 4 * it, s_last);
        const uint8_t* wbase = B + (size_t)s * 64 * (size_t)NB;
        uint8_t* dst = ring + slot_c * SLOT;
#pragma unroll
        for (int p = 0; p < NL; ++p) lds_dma16(wbase + w_off[p], dst + p * 1024);
        if constexpr (AQ == 0) a_dst = *reinterpret_cast<const v4i*>(a_row + (size_t)s * 64);
    };
    // AQ > 0 (one launch, whole rows): every workgroup quantises its m-group's fp32 rows itself (the
    // rule and accumulation order of quantize_rows_kernel / rmsnorm_kernel, from row_stats.h, so the
    // int8 values and scales are bit-identical to theirs) into qbuf, and dequantises its outputs with
    // its own copy of the row scales; workgroup 0 also stores them to rs_out.
    constexpr int QR = AQ ? QK / 256 : 1;
    float xv[QR], gv[AQ == 2 ? QR : 1];
    auto load_row = [&](int r) {
        const float* x = args.X + (size_t)(m0 + r) * (size_t)K;
#pragma unroll
        for (int j = 0; j < (AQ ? QR : 0); ++j) {
            const int k = tid + 256 * j;
            xv[j] = k < K ? x[k] : 0.0f;
            if constexpr (AQ == 2) gv[j] = k < K ? args.G[k] : 0.0f;
        }
    };
    if constexpr (AQ != 0) load_row(0);  // before the weight DMAs, so waiting for it does not wait for them
    // Transposing-read addresses: lane q reads byte-column q of group g, rows 16 kb + q/2 (+8).
    uint32_t w_lo[G], w_hi[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int r = kb * 16 + (q >> 1), r8 = r + 8;
        if (SW == 32) {
            w_lo[g] = (uint32_t)(r * 32 + 16 * (g ^ ((r >> 4) & 1)) + 8 * (q & 1));
            w_hi[g] = (uint32_t)(r8 * 32 + 16 * (g ^ ((r8 >> 4) & 1)) + 8 * (q & 1));
        } else {
            w_lo[g] = (uint32_t)((r ^ (((r >> 4) & 1) << 3)) * 16 + 8 * (q & 1));
            w_hi[g] = (uint32_t)((r8 ^ (((r8 >> 4) & 1) << 3)) * 16 + 8 * (q & 1));
        }
    }

    v4i acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[g][j] = v4i{0, 0, 0, 0};

#pragma unroll
    for (int p = 0; p < NSW - 1; ++p) issue(p, p, a_ring[p]);
    if constexpr (AQ != 0) {
        __shared__ float red[4];
        for (int r = 0; r < a_rows; ++r) {  // uniform: every thread takes part in the reductions
            if (r > 0) load_row(r);
            float inv = 1.0f;
            if constexpr (AQ == 2) {
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < QR; ++j) ss = fmaf(xv[j], xv[j], ss);  // +0 past K changes nothing
                ss = row_block_sum(ss, red);
                inv = 1.0f / sqrtf(ss / (float)K + args.eps);
            }
            auto val = [&](int j) {
                if constexpr (AQ == 2) return xv[j] * inv * gv[j];
                else return xv[j];
            };
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < QR; ++j) amax = fmaxf(amax, fabsf(val(j)));
            const float am = fmaxf(row_block_max(amax, red), 1e-5f);
            const float sc = 127.0f / am;
            if (tid == 0) {
                rscale[r] = am / 127.0f;
                if (cx == 0 && sy == 0) args.rs_out[m0 + r] = am / 127.0f;
            }
#pragma unroll
            for (int j = 0; j < QR; ++j) {
                const int k = tid + 256 * j;
                if (k < K) qbuf[r][k] = (int8_t)quantize_value(val(j), sc);
            }
        }
        __syncthreads();  // qbuf and rscale complete
    }
    constexpr int VPS = NL + (AQ ? 0 : 1);  // vector memory operations per step and wave
    for (int it0 = 0; it0 < iters; it0 += NSW) {
#pragma unroll
        for (int p = 0; p < NSW; ++p) {
            const int it = it0 + p;
            issue(it + NSW - 1, (p + NSW - 1) % NSW, a_ring[(p + NSW - 1) % NSW]);
            TX_VMCNT((NSW - 1) * VPS);       // step `it` (DMAs and activation load) has landed
            if (wave + 4 * it < nst) {       // wave-uniform
                const uint32_t base = lds_u32(ring + p * SLOT);
                uint64_t lo[G], hi[G];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    lo[g] = lds_read_tr8_asm(base + w_lo[g]);
                    hi[g] = lds_read_tr8_asm(base + w_hi[g]);
                }
                TX_LGKMCNT0();
#pragma unroll
                for (int g = 0; g < G; ++g) __asm__ volatile("" : "+v"(lo[g]), "+v"(hi[g]));
                v4i a;
                if constexpr (AQ != 0)
                    a = *reinterpret_cast<const v4i*>(&qbuf[min(q, a_rows - 1)][(s_begin + wave + 4 * it) * 64 + kb * 16]);
                else
                    a = a_ring[p];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const uint32_t x4[4] = {(uint32_t)lo[g], (uint32_t)(lo[g] >> 32), (uint32_t)hi[g],
                                            (uint32_t)(hi[g] >> 32)};
                    v4i bfr[4];
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        const uint32_t x = x4[r4];
                        bfr[0][r4] = (int)((x << 6) & 0xC0C0C0C0u);
                        bfr[1][r4] = (int)((x << 4) & 0xC0C0C0C0u);
                        bfr[2][r4] = (int)((x << 2) & 0xC0C0C0C0u);
                        bfr[3][r4] = (int)(x & 0xC0C0C0C0u);
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[g][j] = mfma_i8(a, bfr[j], acc[g][j]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    TX_VMCNT(0);  // the padding loads into the ring have landed before the ring is reused

    // Sum the four waves: waves 1-3 put, wave 0 adds and stores.
    __syncthreads();
    if (wave > 0) {
        v4i* r = reinterpret_cast<v4i*>(lds) + (wave - 1) * 64 * 4 * G;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) r[(g * 4 + j) * 64 + lane] = acc[g][j];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
        const v4i* r = reinterpret_cast<const v4i*>(lds) + w * 64 * 4 * G;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[g][j] += r[(g * 4 + j) * 64 + lane];
    }
    if (LOW_M && kb != 0) return;
    int32_t* out_base = args.mode == SK_PARTIAL ? args.P + (size_t)sy * (size_t)M * (size_t)args.N : args.C;
    const bool vec = args.mode == SK_PARTIAL || args.vec_store;
    // Store mode writes n_out columns at pitch n_out (a padded problem's real columns).
    const int NO = (args.mode == SK_STORE && args.n_out > 0) ? args.n_out : args.N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 4 * kb + i;
        if (row >= M) continue;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int bcol = bc0 + 16 * g + q;
            if (4 * bcol >= NO) continue;
            const v4i v = {acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            if (args.mode == SK_STORE && args.os.Y) {
                if constexpr (AQ != 0) store_scaled_f(args.os, rscale[row - m0] * args.os.ws, row, NO, 4 * bcol, v, args.vec_store);
                else store_scaled(args.os, row, NO, 4 * bcol, v, args.vec_store);
                continue;
            }
            int32_t* out = out_base + (size_t)row * (size_t)NO + 4 * bcol;
            if (args.mode == SK_ATOMIC) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (v[j] != 0) atomicAdd(out + j, v[j]);
            } else if (vec) {
                *reinterpret_cast<v4i*>(out) = v;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = v[j];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Naive kernel: one work-item per output, weights decoded per k from global memory with
// w = (b & 1) - (b & 2) (the reference decode2, src/cuda_kernels.cu:40-54).
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void naive_kernel(const int8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                    int32_t* __restrict__ C, int M, int K, int N) {
    const int col = blockIdx.x * 64 + (threadIdx.x & 63);
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (row >= M || col >= N) return;
    const int NB = N >> 2;
    const int shift = (col & 3) * 2;
    int acc = 0;
    for (int k = 0; k < K; ++k) {
        const unsigned bits = (B[(size_t)k * NB + (col >> 2)] >> shift) & 3u;
        acc += (int)A[(size_t)row * K + k] * ((int)(bits & 1u) - (int)(bits & 2u));
    }
    C[(size_t)row * N + col] = acc;
}

__global__ __launch_bounds__(256) void zero_kernel(int32_t* __restrict__ C, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * 256;
    for (; i < n; i += stride) C[i] = 0;
}

// C[m][n] = sum over splits of P[s][m][n].  A workgroup owns 64 consecutive groups of 4 outputs
// (lane = group); its 4 waves take splits s = w, w+4, ... with all their loads issued at once (one
// memory round trip for up to 64 splits), then add in LDS.  Integer addition is exact, so the order
// does not change the result.
// P: [splits][M][n_in] int32 (slab stride slab4 16-byte units); C / os.Y: M x N (N <= n_in: the
// columns past N of a padded problem are dropped).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const int32_t* __restrict__ P, int32_t* __restrict__ C,
                                                            size_t n4, int splits, int vec_store, OutScale os,
                                                            int N, int n_in, size_t slab4) {
    __shared__ v4i part[3][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t i = (size_t)blockIdx.x * 64 + lane;
    const size_t ic = i < n4 ? i : n4 - 1;
    const size_t si = n_in == N ? ic : (4 * ic / (size_t)N) * (size_t)(n_in / 4) + (4 * ic % (size_t)N) / 4;
    const v4i* src = reinterpret_cast<const v4i*>(P) + si;
    v4i sum = {0, 0, 0, 0};
    for (int s0 = wave; s0 < splits; s0 += 64) {
        v4i v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int s = s0 + 4 * u;
            v[u] = s < splits ? src[(size_t)s * slab4] : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) sum += v[u];
    }
    if (wave > 0) part[wave - 1][lane] = sum;
    __syncthreads();
    if (wave != 0 || i >= n4) return;
    sum += part[0][lane] + part[1][lane] + part[2][lane];
    if (os.Y) {
        const size_t e = 4 * i;  // N % 4 == 0: the four outputs share a row
        store_scaled(os, (int)(e / (size_t)N), N, (int)(e % (size_t)N), sum, vec_store);
        return;
    }
    if (vec_store) {
        reinterpret_cast<v4i*>(C)[i] = sum;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) C[4 * i + j] = sum[j];
    }
}

template <int MT, bool LOW_M>
hipError_t launch_generic(const SkinnyArgs& a, dim3 grid, hipStream_t st) {
    const dim3 block(64 * SK_WAVES);
    if (a.aligned_w && a.aligned_a) hipLaunchKernelGGL((skinny_generic_kernel<MT, LOW_M, true, true>), grid, block, 0, st, a);
    else if (a.aligned_w) hipLaunchKernelGGL((skinny_generic_kernel<MT, LOW_M, true, false>), grid, block, 0, st, a);
    else if (a.aligned_a) hipLaunchKernelGGL((skinny_generic_kernel<MT, LOW_M, false, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((skinny_generic_kernel<MT, LOW_M, false, false>), grid, block, 0, st, a);
    return hipGetLastError();
}

template <int NS, bool LOW_M, int AQ = 0>
void launch_dma_ns(const SkinnyArgs& a, dim3 grid, hipStream_t st) {
    const int sps = a.steps_per_split;
    if (sps <= 4) hipLaunchKernelGGL((skinny_dma_kernel<NS, 1, LOW_M, AQ>), grid, dim3(256), 0, st, a);
    else if (sps <= 8) hipLaunchKernelGGL((skinny_dma_kernel<NS, 2, LOW_M, AQ>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((skinny_dma_kernel<NS, 4, LOW_M, AQ>), grid, dim3(256), 0, st, a);
}

// Fused activation quantisation (aq 1 or 2) runs with 3 stages only.
hipError_t launch_dma(const SkinnyArgs& a, dim3 grid, int ns, int aq, hipStream_t st) {
    const bool low = a.M <= 4;
    if (aq == 1) low ? launch_dma_ns<3, true, 1>(a, grid, st) : launch_dma_ns<3, false, 1>(a, grid, st);
    else if (aq == 2) low ? launch_dma_ns<3, true, 2>(a, grid, st) : launch_dma_ns<3, false, 2>(a, grid, st);
    else if (ns == 2) low ? launch_dma_ns<2, true>(a, grid, st) : launch_dma_ns<2, false>(a, grid, st);
    else if (ns == 3) low ? launch_dma_ns<3, true>(a, grid, st) : launch_dma_ns<3, false>(a, grid, st);
    else low ? launch_dma_ns<4, true>(a, grid, st) : launch_dma_ns<4, false>(a, grid, st);
    return hipGetLastError();
}

template <int AQ>
void launch_short_aq(const SkinnyArgs& a, dim3 grid, hipStream_t st) {
    const int sps = a.steps_per_split;
    const dim3 block(64 * SK_WAVES);
    if (a.M <= 4) {
        if (sps == 1) hipLaunchKernelGGL((skinny_short_kernel<1, true, AQ>), grid, block, 0, st, a);
        else if (sps == 2) hipLaunchKernelGGL((skinny_short_kernel<2, true, AQ>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((skinny_short_kernel<4, true, AQ>), grid, block, 0, st, a);
    } else {
        if (sps == 1) hipLaunchKernelGGL((skinny_short_kernel<1, false, AQ>), grid, block, 0, st, a);
        else if (sps == 2) hipLaunchKernelGGL((skinny_short_kernel<2, false, AQ>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((skinny_short_kernel<4, false, AQ>), grid, block, 0, st, a);
    }
}

hipError_t launch_short(const SkinnyArgs& a, dim3 grid, int aq, hipStream_t st) {
    if (aq == 2) launch_short_aq<2>(a, grid, st);
    else if (aq == 1) launch_short_aq<1>(a, grid, st);
    else launch_short_aq<0>(a, grid, st);
    return hipGetLastError();
}

template <int MT, int TB, int KW, int PD, bool LOW_M>
hipError_t launch_fast_t(const SkinnyArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((skinny_fast_kernel<MT, TB, KW, PD, LOW_M>), grid, dim3(64 * SK_WAVES),
                       skinny_a_lds_bytes(a.M, a.steps_per_split), st, a);
    return hipGetLastError();
}

// PD (k-steps in flight per wave): 2 (measured on MI355X: 17.9 us vs 18.8 us with 4 on cfg5 big; the
// smaller ring also frees registers).
template <int MT, int TB, bool LOW_M>
hipError_t launch_fast_kw(const SkinnyArgs& a, int kw, dim3 grid, hipStream_t st) {
    constexpr int PD = 2;
    if (kw >= 4) return launch_fast_t<MT, TB, 4, PD, LOW_M>(a, grid, st);
    if (kw == 2) return launch_fast_t<MT, TB, 2, PD, LOW_M>(a, grid, st);
    return launch_fast_t<MT, TB, 1, PD, LOW_M>(a, grid, st);
}

template <int BM, int BNB>
hipError_t launch_gemm_t(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, bool aw, bool aa,
                         int kb, int ke, int acc, hipStream_t st, const OutScale& os, int splits, int k_split) {
    const int NB = N >> 2;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (NB + BNB - 1) / BNB;
    const dim3 grid(tiles_m * tiles_n, splits), block(GM_THREADS);
    const int vs = ((uintptr_t)(os.Y ? (const void*)os.Y : (const void*)C) % 16) == 0;
    if (aw && aa)
        hipLaunchKernelGGL((gemm_kernel<BM, BNB, true, true>), grid, block, 0, st, A, B, C, M, K, N, tiles_n, kb, ke, acc, vs, k_split, os);
    else if (aw)
        hipLaunchKernelGGL((gemm_kernel<BM, BNB, true, false>), grid, block, 0, st, A, B, C, M, K, N, tiles_n, kb, ke, acc, vs, k_split, os);
    else if (aa)
        hipLaunchKernelGGL((gemm_kernel<BM, BNB, false, true>), grid, block, 0, st, A, B, C, M, K, N, tiles_n, kb, ke, acc, vs, k_split, os);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, BNB, false, false>), grid, block, 0, st, A, B, C, M, K, N, tiles_n, kb, ke, acc, vs, k_split, os);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Activation quantisation and dequantisation (the steps either side of the matmul in a BitNet b1.58
// layer; the reference leaves them as a stub, scripts/quantize.py:5, README.md:203).
//   quantize_rows_kernel: one workgroup per row; absmax by a max-reduction (exact, order-free),
//     s = 127 / max(absmax, 1e-5), q = clamp(rint(x * s), -128, 127) (round half to even),
//     row_scale = max(absmax, 1e-5) / 127 -- IEEE division and multiplication, no contraction, so the
//     CPU restatement reproduces every bit.
//   dequant_kernel: y = (float)c * (row_scale[m] * w_scale) for an int32 C (Y may alias C: each
//     element is read before the same element is written by the same thread).
// Both are HBM streams (quantise: 4 bytes read + 1 written per element, twice over the row if it
// does not stay in cache; dequantise: 4 + 4 bytes per output).
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_kernel(const int32_t* C, OutScale os, int N, size_t items, int vec) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= items) return;
    const size_t e = 4 * i;
    const int row = (int)(e / (size_t)N), col = (int)(e % (size_t)N);
    v4i c;
    if (vec) {
        c = reinterpret_cast<const v4i*>(C)[i];
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = C[e + j];
    }
    store_scaled(os, row, N, col, c, vec);
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ X, int8_t* __restrict__ Q,
                                                            float* __restrict__ row_scale, int K, int vec) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* x = X + (size_t)m * (size_t)K;
    int8_t* q = Q + (size_t)m * (size_t)K;
    float amax = 0.0f;
    if (vec) {
        for (int c = threadIdx.x; c < K / 4; c += 256) {
            const v4f v = reinterpret_cast<const v4f*>(x)[c];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
    } else {
        for (int c = threadIdx.x; c < K; c += 256) amax = fmaxf(amax, fabsf(x[c]));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float a = fmaxf(amax, 1e-5f);
    const float s = 127.0f / a;
    if (threadIdx.x == 0) row_scale[m] = a / 127.0f;
    auto qz = [&](float v) -> int {
        const float r = rintf(v * s);
        return (int)fminf(fmaxf(r, -128.0f), 127.0f);
    };
    if (vec) {
        for (int c = threadIdx.x; c < K / 16; c += 256) {
            const v4f* src = reinterpret_cast<const v4f*>(x) + 4 * c;
            v4i out;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const v4f v = src[u];
                out[u] = (int)((uint32_t)(qz(v[0]) & 0xFF) | ((uint32_t)(qz(v[1]) & 0xFF) << 8) |
                               ((uint32_t)(qz(v[2]) & 0xFF) << 16) | ((uint32_t)(qz(v[3]) & 0xFF) << 24));
            }
            reinterpret_cast<v4i*>(q)[c] = out;
        }
    } else {
        for (int c = threadIdx.x; c < K; c += 256) q[c] = (int8_t)qz(x[c]);
    }
}

}  // namespace

hipError_t launch_zero(int32_t* C, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, C, n);
    return hipGetLastError();
}

// Fused activation quantisation on the DMA kernel: whole rows in registers (K <= 256 * kRowRegs) and a
// split, whose reduce launch applies the row scales the kernel stores.
bool skinny_dma_aq_ok(int aq_mode, int K, int splits) {
    return aq_mode == 0 || (K <= 256 * kRowRegs && splits > 1);
}

// skinny_dma_kernel: one m-group of <= 16 rows, whole 64-row k-steps, 16-byte aligned operands, an
// activation slice of <= 16 steps per split.
bool skinny_dma_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int steps_per_split) {
    const int NB = N >> 2;
    return M <= 16 && (K % 64 == 0) && (NB % 64 == 0) && ((uintptr_t)B % 16 == 0) && ((uintptr_t)A % 16 == 0) &&
           steps_per_split >= 1 && steps_per_split <= 16 && (NB < (1 << 26));
}

bool skinny_fast_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int steps_per_split) {
    const int NB = N >> 2;
    return (K % 64 == 0) && (NB % 64 == 0) && ((uintptr_t)B % 16 == 0) && ((uintptr_t)A % 16 == 0) &&
           (NB < (1 << 26)) && skinny_a_lds_bytes(M, steps_per_split) <= kSkinnyALdsMax;
}

bool skinny_short_ok(const uint8_t* B, int M, int K, int N, int steps_per_split, int splits) {
    const int NB = N >> 2;
    return M <= 16 && steps_per_split <= 4 && splits > 1 && (K % 64 == 0) && (NB % 64 == 0) &&
           ((uintptr_t)B % 16 == 0) && (NB < (1 << 26)) && K <= 256 * kRowRegs;
}

hipError_t launch_skinny(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int tb, int kw,
                         int splits, int steps_per_split, int32_t* partials, hipStream_t st, const OutScale& os,
                         const ActQuant& aq, int dma_ns, int n_out) {
    const int NB = N >> 2;
    const int mode = splits <= 1 ? SK_STORE : (partials ? SK_PARTIAL : SK_ATOMIC);
    if (n_out > 0 && (mode != SK_PARTIAL || n_out > N || n_out % 4 != 0)) return hipErrorInvalidValue;
    if (mode == SK_ATOMIC && C == nullptr) return hipErrorInvalidValue;  // scaled call without int scratch
    if (aq.mode != 0 && !skinny_short_ok(B, M, K, N, steps_per_split, splits)) return hipErrorInvalidValue;
    if (mode == SK_ATOMIC) {
        const hipError_t e = launch_zero(C, (size_t)M * (size_t)N, st);
        if (e != hipSuccess) return e;
    }
    const bool scaled = os.Y != nullptr;
    const int vec_store = ((uintptr_t)(scaled ? (const void*)os.Y : (const void*)C) % 16) == 0;
    const int aw = (NB % 4 == 0) && ((uintptr_t)B % 4 == 0);
    const int aa = (K % 16 == 0) && ((uintptr_t)A % 16 == 0);
    SkinnyArgs a{A, B, C, partials, M, K, N, steps_per_split, splits, mode, vec_store, aw, aa,
                 mode == SK_STORE ? os : OutScale{}};
    const int mt = M <= 16 ? 1 : 2;
    const int mgroups = (M + 16 * mt - 1) / (16 * mt);
    hipError_t e;
    static const bool no_short = [] {
        const char* e = std::getenv("TERNIX_SKINNY_SHORT");
        return e && e[0] == '0';
    }();
    if (dma_ns != 0 && (!skinny_dma_aq_ok(aq.mode, K, splits) || dma_ns < 2 || dma_ns > 4 ||
                        !skinny_dma_ok(A, B, M, K, N, steps_per_split)))
        return hipErrorInvalidValue;
    if (dma_ns != 0) {
        const dim3 grid((NB + SD_BNB - 1) / SD_BNB, splits, mgroups);
        a.X = aq.X;
        a.G = aq.G;
        a.eps = aq.eps;
        a.rs_out = aq.rs_out;
        e = launch_dma(a, grid, aq.mode != 0 ? 3 : dma_ns, aq.mode, st);
    } else if (aq.mode != 0) {
        // Fused activation quantisation: only on the short kernel with a split (see skinny_short_kernel).
        a.X = aq.X;
        a.G = aq.G;
        a.eps = aq.eps;
        a.rs_out = aq.rs_out;
        const dim3 grid((NB + 255) / 256, splits, mgroups);
        e = launch_short(a, grid, aq.mode, st);
    } else if (mt == 1 && tb == 1 && kw == 1 && steps_per_split <= 4 && !no_short &&
               skinny_fast_ok(A, B, M, K, N, steps_per_split)) {
        const dim3 grid((NB + 255) / 256, splits, mgroups);
        e = launch_short(a, grid, 0, st);
    } else if (skinny_fast_ok(A, B, M, K, N, steps_per_split)) {
        if (mt == 2) tb = 1;
        const int slab = 64 * tb * (SK_WAVES / (kw >= 4 ? 4 : (kw == 2 ? 2 : 1)));  // bytes per workgroup
        const dim3 grid((NB + slab - 1) / slab, splits, mgroups);
        if (M <= 4) e = tb == 2 ? launch_fast_kw<1, 2, true>(a, kw, grid, st) : launch_fast_kw<1, 1, true>(a, kw, grid, st);
        else if (M <= 16) e = tb == 2 ? launch_fast_kw<1, 2, false>(a, kw, grid, st) : launch_fast_kw<1, 1, false>(a, kw, grid, st);
        else e = launch_fast_kw<2, 1, false>(a, kw, grid, st);
    } else {
        const dim3 grid((NB + 127) / 128, splits, mgroups);
        if (M <= 4) e = launch_generic<1, true>(a, grid, st);
        else if (M <= 16) e = launch_generic<1, false>(a, grid, st);
        else e = launch_generic<2, false>(a, grid, st);
    }
    if (e != hipSuccess) return e;
    if (mode == SK_ATOMIC && scaled) return launch_dequant(C, os, M, N, st);  // C: alias of os.Y or scratch
    if (mode != SK_PARTIAL) return e;
    const size_t n4 = (size_t)M * (size_t)N / 4;
    const int n_c = n_out > 0 ? n_out : N;
    const size_t n4c = (size_t)M * (size_t)n_c / 4;
    const int vec_c = n_out > 0 ? ((uintptr_t)(scaled ? (const void*)os.Y : (const void*)C) % 16) == 0 : vec_store;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n4c + 63) / 64)), dim3(256), 0, st, partials, C, n4c,
                       splits, vec_c, os, n_c, N, n4);
    return hipGetLastError();
}

// Compute units of the current device, read once per device (the attribute query is not free).
int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Narrow 64 x 64 tiles for M <= 64 when they alone fill at most one workgroup per CU (measured on
// MI355X: cfg3 M=64 up 18.0 -> 13.4 us with no K split, 4096^2 at M=64 16.2 -> 9.9 us; with more
// tiles than CUs, e.g. N = 28672, the 256-column tiles are faster).  TERNIX_GEMM_NARROW=0 / 1 turns
// the choice off / on regardless (experiments).
bool gemm_narrow_wanted(int M, int K, int N) {
    static const int env = [] {
        const char* e = std::getenv("TERNIX_GEMM_NARROW");
        return e ? std::atoi(e) : -1;
    }();
    const int NB = N >> 2;
    if (env == 0 || M > 64 || NB % 16 != 0 || K % 256 != 0) return false;
    if (env > 0) return true;
    return (long)((M + 63) / 64) * (NB / 16) <= device_cu_count();
}

bool gemm_narrow_ok(int M, int K, int N, int k_len, int splits, int k_split) {
    return gemm_narrow_wanted(M, K, N) && k_len % 256 == 0 && (splits == 1 || k_split % 256 == 0);
}

bool skinny_wave_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int sw) {
    const int NB = N >> 2;
    return M <= 32 && (sw == 16 || sw == 32) && K % 64 == 0 && NB % sw == 0 && (uintptr_t)B % 16 == 0 &&
           (uintptr_t)A % 16 == 0 && NB < (1 << 26);
}

hipError_t launch_skinny_wave(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int sw, int nsw,
                              int splits, int steps_per_split, int32_t* partials, hipStream_t st, const OutScale& os,
                              int n_out, const ActQuant& aq) {
    if (!skinny_wave_ok(A, B, M, K, N, sw) || nsw < 2 || nsw > 4 || steps_per_split < 1) return hipErrorInvalidValue;
    // Fused activation quantisation: one launch over whole rows (K <= 4096), 16-byte strips, 2 slots.
    if (aq.mode != 0 && (splits != 1 || K > 4096 || sw != 16 || nsw != 2 || n_out > 0 || aq.X == nullptr ||
                         aq.rs_out == nullptr || (aq.mode == 2 && aq.G == nullptr)))
        return hipErrorInvalidValue;
    const int NB = N >> 2;
    const int mode = splits <= 1 ? SK_STORE : (partials ? SK_PARTIAL : SK_ATOMIC);
    if (n_out > 0 && (mode == SK_ATOMIC || n_out > N || n_out % 4 != 0)) return hipErrorInvalidValue;
    if (mode == SK_ATOMIC && C == nullptr) return hipErrorInvalidValue;
    if (mode == SK_ATOMIC) {
        const hipError_t e = launch_zero(C, (size_t)M * (size_t)N, st);
        if (e != hipSuccess) return e;
    }
    const bool scaled = os.Y != nullptr;
    const int vec_store = ((uintptr_t)(scaled ? (const void*)os.Y : (const void*)C) % 16) == 0;
    SkinnyArgs a{A, B, C, partials, M, K, N, steps_per_split, splits, mode, vec_store, 1, 1,
                 mode == SK_STORE ? os : OutScale{}};
    a.n_out = n_out;
    a.X = aq.X;
    a.G = aq.G;
    a.eps = aq.eps;
    a.rs_out = aq.rs_out;
    // Line units: 8 XCDs x (128 / sw) strips x enough rounds for every (split, line-group) unit.
    // Measured on MI355X (cold weights): line units help the one-launch shapes (cfg1 5.76 -> 5.24 us,
    // cfg2 up 6.75 -> 6.5, ragged 17x4093x1028 13.1 -> 11.5) and cost 2 % with a K split.
    static const int lu_env = [] {
        const char* e = std::getenv("TERNIX_WAVE_LINES");  // experiments: 0 / 1 forces the mapping
        return e ? std::atoi(e) : -1;
    }();
    a.line_units = lu_env >= 0 ? lu_env : (splits == 1);
    const int spl = 128 / sw, units = splits * ((NB / sw + spl - 1) / spl);
    const unsigned gx = a.line_units ? (unsigned)(8 * spl * ((units + 7) / 8)) : (unsigned)((NB / sw) * splits);
    const dim3 grid(gx, 1, (M + 15) / 16), block(256);
    const bool low = M <= 4;
#define TX_SW_LAUNCH(SW_, NSW_)                                                              \
    do {                                                                                      \
        if (low) hipLaunchKernelGGL((skinny_wave_kernel<SW_, NSW_, true>), grid, block, 0, st, a);  \
        else hipLaunchKernelGGL((skinny_wave_kernel<SW_, NSW_, false>), grid, block, 0, st, a);     \
    } while (0)
    if (aq.mode == 1) {
        if (low) hipLaunchKernelGGL((skinny_wave_kernel<16, 2, true, 1>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((skinny_wave_kernel<16, 2, false, 1>), grid, block, 0, st, a);
    } else if (aq.mode == 2) {
        if (low) hipLaunchKernelGGL((skinny_wave_kernel<16, 2, true, 2>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((skinny_wave_kernel<16, 2, false, 2>), grid, block, 0, st, a);
    } else if (sw == 32 && nsw == 4) TX_SW_LAUNCH(32, 4);
    else if (sw == 32) TX_SW_LAUNCH(32, 2);
    else if (nsw == 4) TX_SW_LAUNCH(16, 4);
    else if (nsw == 3) TX_SW_LAUNCH(16, 3);
    else TX_SW_LAUNCH(16, 2);
#undef TX_SW_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (mode == SK_ATOMIC && scaled) return launch_dequant(C, os, M, N, st);
    if (mode != SK_PARTIAL) return e;
    return n_out > 0 ? launch_splitk_reduce(partials, C, M, n_out, splits, os, st, N)
                     : launch_splitk_reduce(partials, C, M, N, splits, os, st);
}

hipError_t launch_gemm(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int k_begin, int k_end,
                       int accumulate, hipStream_t st, const OutScale& os, int splits, int k_split) {
    const int NB = N >> 2;
    // Experiment switches, read once per process.
    static const char* const force_generic = std::getenv("TERNIX_GEMM_GENERIC");
    if (splits < 1) splits = 1;
    const bool fast = (K % GF_BK == 0) && ((k_end - k_begin) % GF_BK == 0) && (k_begin % GF_BK == 0) &&
                      (splits == 1 || k_split % GF_BK == 0) &&
                      (NB % GF_BNB == 0) && ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0) &&
                      k_end > k_begin && (size_t)M * (size_t)K < ((size_t)1 << 32) &&
                      (size_t)GF_BK * (size_t)NB < ((size_t)1 << 32) && !(force_generic && force_generic[0] == '1');
    if (fast) {
        const int vs = ((uintptr_t)(os.Y ? (const void*)os.Y : (const void*)C) % 16) == 0;
        const int tiles_n = NB / GF_BNB;
        static const char* const bm_env = std::getenv("TERNIX_GEMM_BM");
        static const char* const wgn_env = std::getenv("TERNIX_GEMM_WGN");
        static const char* const bk_env = std::getenv("TERNIX_GEMM_BK");
        // Measured on MI355X (cfg4 shapes): 256-row tiles only when they still give >= 1.5 tiles per
        // CU, else 128-row tiles; 8 waves as 2 (M) x 4 (N); 128-deep stages.
        const int cus = device_cu_count();
        int bm = (splits == 1 && (long)((M + 255) / 256) * tiles_n * 2 >= 3L * cus) ? 256 : 128;
        if (bm_env) bm = std::atoi(bm_env) == 128 ? 128 : 256;
        const int wgn = wgn_env && std::atoi(wgn_env) == 2 ? 2 : 4;
        int bk = 128;
        if (bk_env && std::atoi(bk_env) == 256 && bm == 128 && (k_end - k_begin) % 256 == 0) bk = 256;
        const dim3 grid(((M + bm - 1) / bm) * tiles_n, splits);
        // 128-row tiles run the software-pipelined kernel (measured faster on MI355X); 256-row tiles
        // keep gemm_fast_kernel, whose wave tile leaves no registers for a second fragment set.
        static const int pipe_env = [] {
            const char* e = std::getenv("TERNIX_GEMM_PIPE");
            return e ? std::atoi(e) : -1;
        }();
        const int pipe = pipe_env >= 0 ? (pipe_env == 1 && bm == 256 ? 0 : pipe_env) : (bm == 128 ? 1 : 0);
        static const int pipe_ns = [] {
            const char* e = std::getenv("TERNIX_GEMM_NS");
            return e && std::atoi(e) == 4 ? 4 : 3;
        }();
        static const int small_m_max = [] {
            const char* e = std::getenv("TERNIX_GEMM_SMALLM");  // experiments only
            return e ? std::atoi(e) : 64;
        }();
        if (M <= small_m_max && gemm_narrow_ok(M, K, N, k_end - k_begin, splits, k_split)) {
            // 64 x 64 output tiles (16 bytes of every weight row): enough workgroups without a K
            // split where the 256-column tiles would need one; one m-tile per wave, 256-deep stages.
            const dim3 gridn((unsigned)(((M + 63) / 64) * (NB / 16)), splits);
            hipLaunchKernelGGL((gemm_pipe_kernel<64, 1, 3, 256, 4, 16>), gridn, dim3(256), 0, st, A, B, C, M, K, N,
                               NB / 16, k_begin, k_end, accumulate, vs, k_split, os);
            return hipGetLastError();
        }
        // One round of 128-row tiles with a short k-range (cfg4 4096^2): two co-resident workgroups
        // of 64-row tiles per CU instead, whose barriers and final stores overlap each other's work
        // (measured on MI355X: 29.5 -> 27.9 us; with long K or several rounds the 128-row tiles win).
        const long tiles128 = (long)((M + 127) / 128) * tiles_n;
        const bool short_round = splits == 1 && bm == 128 && !bm_env && tiles128 <= cus &&
                                 2 * tiles128 >= cus && (k_end - k_begin) <= 4096;
        if (M <= small_m_max || short_round) {
            // Small M (64 rows or fewer): four-wave workgroups on 64-row tiles, so no MFMA row or A
            // byte is spent on padding rows; the caller splits K to fill the chip.
            const dim3 grid64((unsigned)(((M + 63) / 64) * tiles_n), splits);
            hipLaunchKernelGGL((gemm_pipe_kernel<64, 4, 3, 128, 4, 64>), grid64, dim3(256), 0, st, A, B, C, M, K, N,
                               tiles_n, k_begin, k_end, accumulate, vs, k_split, os);
            return hipGetLastError();
        }
        if (pipe) {
#define TX_GP_LAUNCH(BM_, WGN_, NS_, BK_)                                                                      \
    hipLaunchKernelGGL((gemm_pipe_kernel<BM_, WGN_, NS_, BK_, 8, GF_BNB>), grid, dim3(GF_THREADS), 0, st, A, B, C, M, \
                       K, N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os)
            if (bk == 256 && wgn == 4) TX_GP_LAUNCH(128, 4, 3, 256);
            else if (bk == 256) TX_GP_LAUNCH(128, 2, 3, 256);
            else if (wgn == 4 && pipe_ns == 4) TX_GP_LAUNCH(128, 4, 4, 128);
            else if (wgn == 4) TX_GP_LAUNCH(128, 4, 3, 128);
            else if (pipe_ns == 4) TX_GP_LAUNCH(128, 2, 4, 128);
            else TX_GP_LAUNCH(128, 2, 3, 128);
#undef TX_GP_LAUNCH
            return hipGetLastError();
        }
#define TX_GF_LAUNCH(BM_, WGN_, NS_, BK_)                                                                         \
    hipLaunchKernelGGL((gemm_fast_kernel<BM_, WGN_, NS_, BK_>), grid, dim3(GF_THREADS), 0, st, A, B, C, M, K, N, \
                       tiles_n, k_begin, k_end, accumulate, vs, k_split, os)
        if (bm == 256 && wgn == 4) TX_GF_LAUNCH(256, 4, 3, 128);
        else if (bm == 256) TX_GF_LAUNCH(256, 2, 3, 128);
        else if (bk == 256 && wgn == 4) TX_GF_LAUNCH(128, 4, 3, 256);
        else if (bk == 256) TX_GF_LAUNCH(128, 2, 3, 256);
        else if (wgn == 4) TX_GF_LAUNCH(128, 4, 4, 128);
        else TX_GF_LAUNCH(128, 2, 4, 128);
#undef TX_GF_LAUNCH
        return hipGetLastError();
    }
    const bool aw = (NB % 4 == 0) && ((uintptr_t)B % 4 == 0);
    const bool aa = (K % 16 == 0) && ((uintptr_t)A % 16 == 0);
    return launch_gemm_t<128, 64>(A, B, C, M, K, N, aw, aa, k_begin, k_end, accumulate, st, os, splits, k_split);
}

hipError_t launch_splitk_reduce(const int32_t* P, int32_t* C, int M, int N, int splits, const OutScale& os,
                                hipStream_t st, int n_in) {
    if (n_in <= 0) n_in = N;
    const size_t n4 = (size_t)M * (size_t)N / 4;
    if (n4 == 0) return hipSuccess;
    const int vec = ((uintptr_t)(os.Y ? (const void*)os.Y : (const void*)C) % 16) == 0;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n4 + 63) / 64)), dim3(256), 0, st, P, C, n4, splits, vec,
                       os, N, n_in, (size_t)M * (size_t)n_in / 4);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Padded copy for ragged shapes: rows of `len` bytes at pitch src_pitch (any alignment) into rows of
// dst_pitch bytes (16-byte aligned, dst_pitch % 16 == 0), zero-filled past len and for the rows
// rows..dst_rows-1.  Each thread writes one 16-byte chunk from five aligned dword loads and
// v_alignbyte; an aligned dword holding at least one byte of the source buffer never crosses a page
// the buffer does not touch, so loads stay within the buffer's pages (dwords starting past its last
// byte are not loaded).
// ------------------------------------------------------------------------------------------------
struct PadJob {
    const uint8_t* src;
    uint8_t* dst;
    int rows, dst_rows, src_pitch, len, dst_pitch;
    size_t chunks;  // dst_rows * dst_pitch / 16
};

__device__ __forceinline__ void pad_chunk(const PadJob& j, size_t idx) {
    const int cpr = j.dst_pitch >> 4;
    const int r = (int)(idx / (size_t)cpr), c = (int)(idx % (size_t)cpr);
    v4i out = {0, 0, 0, 0};
    const int n = min(max(j.len - 16 * c, 0), 16);  // source bytes in this chunk
    if (r < j.rows && n > 0) {
        const uint8_t* p = j.src + (size_t)r * (size_t)j.src_pitch + 16 * c;
        const uint8_t* end = j.src + (size_t)(j.rows - 1) * (size_t)j.src_pitch + j.len;
        const uint32_t* pa = reinterpret_cast<const uint32_t*>((uintptr_t)p & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
        uint32_t d[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) d[k] = reinterpret_cast<const uint8_t*>(pa + k) < end ? pa[k] : 0u;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t v = __builtin_amdgcn_alignbyte(d[m + 1], d[m], sh);
            const int keep = min(max(n - 4 * m, 0), 4);  // bytes of this dword inside the row
            v = keep >= 4 ? v : (keep == 0 ? 0u : (v & ((1u << (8 * keep)) - 1u)));
            out[m] = (int)v;
        }
    }
    *reinterpret_cast<v4i*>(j.dst + (size_t)r * (size_t)j.dst_pitch + 16 * c) = out;
}

__global__ __launch_bounds__(256) void pad_rows_kernel(PadJob j0, PadJob j1) {
    const size_t total = j0.chunks + j1.chunks;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        if (i < j0.chunks) pad_chunk(j0, i);
        else pad_chunk(j1, i - j0.chunks);
    }
}

hipError_t launch_pad_rows(const uint8_t* src0, uint8_t* dst0, int rows0, int dst_rows0, int src_pitch0, int len0,
                           int dst_pitch0, const uint8_t* src1, uint8_t* dst1, int rows1, int dst_rows1,
                           int src_pitch1, int len1, int dst_pitch1, hipStream_t st) {
    if (dst_pitch0 % 16 != 0 || (uintptr_t)dst0 % 16 != 0 || len0 > dst_pitch0 || rows0 > dst_rows0 ||
        (dst1 && (dst_pitch1 % 16 != 0 || (uintptr_t)dst1 % 16 != 0 || len1 > dst_pitch1 || rows1 > dst_rows1)))
        return hipErrorInvalidValue;
    const PadJob j0{src0, dst0, rows0, dst_rows0, src_pitch0, len0, dst_pitch0,
                    (size_t)dst_rows0 * (size_t)dst_pitch0 / 16};
    const PadJob j1{src1, dst1, rows1, dst_rows1, src_pitch1, len1, dst_pitch1,
                    dst1 ? (size_t)dst_rows1 * (size_t)dst_pitch1 / 16 : 0};
    const size_t total = j0.chunks + j1.chunks;
    if (total == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(pad_rows_kernel, dim3(blocks), dim3(256), 0, st, j0, j1);
    return hipGetLastError();
}

hipError_t launch_dequant(const int32_t* C, const OutScale& os, int M, int N, hipStream_t st) {
    const size_t n = (size_t)M * (size_t)N;
    if (n == 0) return hipSuccess;
    const int vec = ((uintptr_t)C % 16 == 0) && ((uintptr_t)os.Y % 16 == 0);
    const size_t items = n / 4;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, C, os, N, items, vec);
    return hipGetLastError();
}

hipError_t launch_quantize_rows(const float* X, int8_t* Q, float* row_scale, int M, int K, hipStream_t st) {
    if (M == 0) return hipSuccess;
    const int vec = (K % 16 == 0) && ((uintptr_t)X % 16 == 0) && ((uintptr_t)Q % 16 == 0);
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)M), dim3(256), 0, st, X, Q, row_scale, K, vec);
    return hipGetLastError();
}

hipError_t launch_naive(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, hipStream_t st) {
    const dim3 grid((N + 63) / 64, (M + 3) / 4);
    hipLaunchKernelGGL(naive_kernel, grid, dim3(256), 0, st, A, B, C, M, K, N);
    return hipGetLastError();
}

}  // namespace ternix_hip
