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
constexpr int kMaxKPerAccumulator = (1 << 17) - 128;

// Optional dequantised output of a matmul launch: when Y is set the kernels write
// Y[m][n] = (float)C[m][n] * (rs[m] * ws) (fp32, row-major M x N) instead of the int32 C.
// With swiglu set, Y is M x N/2: each interleaved (gate, up) column pair of the dequantised product
// becomes silu(gate) * up (reference swiglu, src/simd_math.cpp:40-46); Y must not alias C then.
struct OutScale {
    float* Y = nullptr;
    const float* rs = nullptr;  // per-row activation scale [M]
    float ws = 0.0f;            // weight scale
    int swiglu = 0;
};

// Test and tuning switches (set only through ternix_hip_debug_set; never read from the environment).
// Each key holds up to four ints; debug_get returns -1 for a value that is not set, and the planners
// then make their normal choice.
enum DebugKey : int {
    DBG_WAVE_LAST = 0,   // [0] largest split count summed inside the wave GEMV launch (0: never)
    DBG_SKINNY_WAVE,     // [0] == 0: no wave-pipelined GEMV; else (sw, nsw, splits) forced
    DBG_WAVE_SW,         // [0] strip width of the wave-pipelined GEMV on row-major weights (16 / 32);
                         //     with [1] > 1 also the atomic split plan's strip width and split count;
                         //     [2] 1 / 0: column waves (M <= 4) forced on / off in that plan
    DBG_SKINNY_DMA,      // [0] == 0: no DMA-staged GEMV; 2..4: its stage count; [1] > 0: its split count
    DBG_SKINNY_SHORT,    // [0] == 0: no register-staged short GEMV
    DBG_RAGGED_PAD,      // [0] == 0: ragged shapes run the generic kernels instead of a padded copy
    DBG_GEMM_NARROW,     // [0] 0 / 1: 64 x 64 GEMM tiles for M <= 64 off / forced
    DBG_GEMM_GENERIC,    // [0] == 1: the generic (register-staged) GEMM for every GEMM call
    DBG_GEMM_SPLITS,     // [0] GEMM split-K count forced
    DBG_GEMM_BM,         // [0] 64 / 128 / 256: GEMM tile height forced
    DBG_DEEP,            // [0] == 0: no whole-K deep GEMV; else (sw, nw, nsw, splits) forced
    DBG_SK_ORDER,        // [0] 1: release/acquire (agent scope) for the in-launch split sums
    DBG_M1_ATOMIC,       // [0] 0: no zero-fill + atomic split plan for M = 1 GEMVs; [1] / [2] largest M of
                         //     the self-zeroing atomic plan on row-major / tile-64 weights (default 64 / 16)
    DBG_GEMM_GM,         // [0] > 0: row tiles per group in the tile order of the 64/128-row GEMM kernels
    DBG_SELF_ZERO,       // [0] 0: no in-launch zeroing of C for M = 1 (fill launch or reduce launch instead)
    DBG_NT,              // [0] DMA-staged GEMV, [1] wave-pipelined GEMV: 1 non-temporal weight loads, 0 plain
    DBG_WAVE_TICKET,     // [0] 1 / 0: wave-pipelined GEMV waits for its split ticket in the first step / before it
    DBG_LINE,            // [0] 0: no whole-line GEMV; > 0: its k-steps per workgroup forced; [1] its data waves (4 / 8)
    DBG_FFN_AMAX,        // [0] == 0: the decode FFN block's down GEMV takes whole rows of h, not the maxima
    DBG_COUNT
};
int debug_get(DebugKey key, int idx = 0);

hipError_t launch_zero(int32_t* C, size_t n, hipStream_t st);
// Ticket words of the self-zeroing GEMVs: a strip's {T, Z} pair sits tk_stride 64-bit words after the
// previous strip's, one 256-byte line apart when there are at most kTicketSpreadMax strips, so that
// different strips' ticket atomics never queue on one line (measured on MI355X, whole-line GEMV, cfg2
// up: 8.2 -> 5.1 us).  ticket_units: 16-byte units of the library's ticket region the strips need.
constexpr size_t kTicketSpreadMax = 1024;
inline int ticket_stride(size_t strips) { return strips <= kTicketSpreadMax ? 32 : 2; }
inline size_t ticket_units(size_t strips) { return strips * (size_t)ticket_stride(strips) / 2; }
// Bits of the device fault word (skinny_kernels.hip); the same values as TERNIX_FAULT_* in ternix_hip.h.
constexpr unsigned kFaultZeroWait = 1u;  // a bounded wait for a strip's zeroed word gave up
// Synchronises the current device, returns the fault word's bits in *bits and clears them.
hipError_t take_faults(unsigned* bits);
hipError_t take_line_faults(unsigned* bits);
// Bare streaming read of `bytes` (rounded down to 16) at p (16-byte aligned): the HBM floor reference.
hipError_t launch_stream_read(const void* p, size_t bytes, int* out, hipStream_t st);
// LDS bytes the skinny fast kernel uses for one workgroup's activation slice (the rows of one
// m-group x steps_per_split * 64 bytes, each row padded by 16 bytes); the fast kernel runs only up
// to kSkinnyALdsMax, so planners keep steps_per_split small enough for it.
constexpr size_t kSkinnyALdsMax = 32 * 1024;
inline size_t skinny_a_lds_bytes(int M, int steps_per_split) {
    const int rows = M <= 16 ? M : 32;
    return (size_t)rows * ((size_t)steps_per_split * 64 + 16);
}
// True when launch_skinny takes the fast kernel for this call.
bool skinny_fast_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int steps_per_split);
// Skinny split-K GEMV/GEMM for M <= 32.  tb: 64-byte (1) or 128-byte (2) column slab per wave (fast
// kernel, M <= 16); kw: waves per slab inside a workgroup (1, 2 or 4; fast kernel).  With
// splits > 1 each split's partial C goes to `partials` ([splits][M][N] int32, 16-byte aligned) and a
// reduce kernel sums them into C; without a workspace C is zeroed and accumulated with atomics.
// With os.Y set, the store and partial-sum modes write the dequantised floats (fused into the store or
// the reduce); the atomic mode accumulates int32 in C, which the caller converts afterwards.
// Fused activation quantisation for the skinny path (mode 1: quantise fp32 rows X; mode 2: RMSNorm
// with weight G and eps, then quantise); the int8 A argument is then unused and the row scales go to
// rs_out.  Only valid when skinny_short_ok() holds for the plan (launch_skinny returns
// hipErrorInvalidValue otherwise, before launching anything).
struct ActQuant {
    int mode = 0;
    const float* X = nullptr;
    const float* G = nullptr;
    float eps = 0.0f;
    float* rs_out = nullptr;
    // Whole-line GEMV only.  Producer (float output): per row and strip the largest |value| stored,
    // at amax_out[row * amax_stride + strip].  Consumer (mode 3): X's rows quantised with the absmax
    // taken from amax_in[row * amax_stride + i], i < amax_n (a producer's per-strip maxima of X).
    float* amax_out = nullptr;
    const float* amax_in = nullptr;
    int amax_stride = 0;
    int amax_n = 0;
};
// Whole-line decode GEMV (line_gemv.hip): M <= 16, K % 64 == 0, N/4 % 16 == 0, 16-byte aligned A and W
// (or, int32 output only, any K, N % 4 == 0 and any A / W address: the ragged form); 8-byte aligned C;
// S k-steps per workgroup, NW data waves (4 or 8); K splits added with int32 atomics into C zeroed by
// each strip's split 0 (tickets: two 64-bit words per 128-byte strip, persistent).  tiled: W in the
// tile-64 layout (K % 128 == 0, N % 256 == 0), read in the same pieces.
bool line_gemv_ok(const int8_t* A, const uint8_t* B, int M, int K, int N);
bool line_gemv_ragged_ok(int M, int K, int N);  // the ragged-operand form (int32 output)
int line_gemv_splits(int K, int S);
hipError_t launch_line_gemv(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int S, int NW,
                            unsigned long long* tk, int tk_stride, hipStream_t st, const OutScale& os = OutScale{},
                            const ActQuant& aq = ActQuant{}, int xcd_chunks = 0, int tiled = 0);
// (os.Y set: float output through the last-arriving split of each strip, C then being the int32 buffer
// of the sums, tickets spread one line per strip; aq.mode 1 / 2: fused activation quantisation of
// fp32 rows aq.X with M <= 4 and M * K <= 8192, only with os.Y; mode 3: any K, from a producer's
// per-strip maxima.)
bool skinny_short_ok(const uint8_t* B, int M, int K, int N, int steps_per_split, int splits);
// True when the DMA-staged skinny kernel can run this call: M <= 16, K % 64 == 0, N % 256 == 0,
// 16-byte aligned A and W, 1..16 k-steps per split.
bool skinny_dma_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int steps_per_split);
// ... and can also quantise the activations in its prologue (aq_mode 1 or 2): K <= 8192, splits > 1.
bool skinny_dma_aq_ok(int aq_mode, int K, int splits);
// dma_ns (2..4) selects the DMA-staged kernel with that many LDS stages (its own plan: tb and kw are
// ignored; skinny_dma_ok and skinny_dma_aq_ok must hold, hipErrorInvalidValue otherwise; with aq set
// it runs 3 stages).
hipError_t launch_skinny(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int tb, int kw,
                         int splits, int steps_per_split, int32_t* partials, hipStream_t st,
                         const OutScale& os = OutScale{}, const ActQuant& aq = ActQuant{}, int dma_ns = 0,
                         int n_out = 0, unsigned long long* tickets = nullptr);
// (tickets, with the DMA-staged kernel and no partials: the splits add into C with int32 atomics,
// each strip's first split zeroing its outputs inside the launch instead of a fill launch.)
// (n_out > 0: a padded problem -- N is the padded column count of A x W, and C / os.Y has n_out <= N
// columns; only with a split-K workspace, whose reduce drops the padding.)
// Compute units of the current device (cached per device).
int device_cu_count();
// Wave-pipelined skinny kernel (M <= 32, K % 64 == 0, N/4 % sw == 0, aligned A and W): sw = 16 or
// 32 bytes of weight row per workgroup, nsw = 2 or 4 ring slots per wave; splits == 1 stores C
// directly, splits > 1 goes through `partials` and the reduce launch like launch_skinny.
bool skinny_wave_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int sw);
hipError_t launch_skinny_wave(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int sw, int nsw,
                              int splits, int steps_per_split, int32_t* partials, hipStream_t st,
                              const OutScale& os = OutScale{}, int n_out = 0, const ActQuant& aq = ActQuant{},
                              int tiled = 0, int* counters = nullptr, unsigned long long* tickets = nullptr,
                              int column_waves = 0);
// (tiled != 0: W is in the tile-64 layout of launch_interleave_weights, sw must be 16.
// n_out > 0: a padded problem -- C / os.Y has n_out <= N columns; not with the atomic mode.
// aq set: the activations are quantised in the kernel from aq.X (splits == 1, K <= 4096, sw 16,
// nsw 2); the dequantising epilogue then uses the kernel's own row scales.)
// True when launch_gemm runs this M <= 64 shape on 64 x 64 tiles (K % 256 == 0, N/4 % 16 == 0, at
// most one tile per CU); split-K k-ranges must then be multiples of 256.
bool gemm_narrow_wanted(int M, int K, int N, int tiled = 0);
// Tile height (64 or 128 rows) launch_gemm uses for this shape when K is split.
int gemm_split_rows(int M, int K, int N);
// The GEMM kernel launch_gemm runs for these arguments (Invalid: it would return hipErrorInvalidValue).
enum class GemmChoice { Invalid, Narrow64, Pipe64, Pipe128, Fast256, Generic };
GemmChoice gemm_choice(const int8_t* A, const uint8_t* B, int M, int K, int N, int k_begin, int k_end, int splits,
                       int k_split, int tiled);
const char* gemm_choice_name(GemmChoice c);
// LDS-tiled MFMA GEMM over k-rows [k_begin, k_end); accumulate != 0 adds into C instead of storing.
// With os.Y set the tile epilogue writes the dequantised floats instead (accumulate must be 0).
// splits > 1: split-K over gridDim.y, each workgroup row of the grid covering k_split k-rows (a
// multiple of 64, of 128 for the fast kernels) and writing its partial tile to C + y * M * N
// (accumulate must be 0 and os unset; launch_splitk_reduce finishes the sum).
hipError_t launch_gemm(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int k_begin,
                       int k_end, int accumulate, hipStream_t st, const OutScale& os = OutScale{}, int splits = 1,
                       int k_split = 0, int tiled = 0);
// (tiled != 0: W in the tile-64 layout; needs K % 128 == 0, N/4 % 64 == 0, aligned operands, k-ranges
// of whole 128-row stages, K * N/4 < 2^32; hipErrorInvalidValue otherwise.)
// C (or os.Y) = sum over `splits` slabs of P ([splits][M][N] int32).
hipError_t launch_splitk_reduce(const int32_t* P, int32_t* C, int M, int N, int splits, const OutScale& os,
                                hipStream_t st, int n_in = 0);
// (n_in > N: the partials have n_in columns per row, of which the first N are summed into C.)
// Whole-K decode GEMV (skinny_deep.hip): sw = 16 / 32-byte strips, nw = 8 / 16 waves per workgroup,
// nsw ring slots per wave (skinny_deep_config_ok lists the built combinations).  splits == 1 stores C
// (or os.Y, n_out columns when n_out > 0) directly; splits > 1 writes [splits][M][N] partials and the
// reduce launch sums them.  Needs K % 64 == 0, N/4 % sw == 0, 16-byte aligned A and W.
bool skinny_deep_config_ok(int sw, int nw, int nsw);
bool skinny_deep_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int sw);
hipError_t launch_skinny_deep(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int sw, int nw,
                              int nsw, int splits, int steps_per_split, int32_t* partials, hipStream_t st,
                              const OutScale& os = OutScale{}, int n_out = 0, int tiled = 0);
// Tile-64 weight layout (opt-in; kernel_common.h): Wt = the K x N/4 packed W as 1 KB blocks of 64
// k-rows x 16 bytes.  K % 64 == 0, N/4 % 16 == 0, 16-byte aligned, Wt != W.
hipError_t launch_tile64(const uint8_t* W, uint8_t* Wt, int K, int N, hipStream_t st);
// Padded copy of up to two row sets in one launch (ragged shapes): rows of len bytes at src_pitch
// into dst rows of dst_pitch bytes (dst 16-byte aligned, dst_pitch % 16 == 0), zero-filled past len
// and for rows rows..dst_rows-1.  dst1 == nullptr: one set only.
hipError_t launch_pad_rows(const uint8_t* src0, uint8_t* dst0, int rows0, int dst_rows0, int src_pitch0, int len0,
                           int dst_pitch0, const uint8_t* src1, uint8_t* dst1, int rows1, int dst_rows1,
                           int src_pitch1, int len1, int dst_pitch1, hipStream_t st);
// In-place-capable conversion of an int32 C to the dequantised float Y (Y may alias C).
hipError_t launch_dequant(const int32_t* C, const OutScale& os, int M, int N, hipStream_t st);
// Per-row RMSNorm (reference rms_norm_scalar, src/simd_math.cpp:7-12): out = x * inv * w with
// inv = 1 / sqrt(sum(x^2) / K + eps); with Q set, the normalised row is quantised like
// launch_quantize_rows instead of stored (out may then be NULL).
hipError_t launch_rmsnorm(const float* X, const float* W, float eps, float* out, int8_t* Q, float* row_scale, int M,
                          int K, hipStream_t st);
// Reference swiglu (src/simd_math.cpp:40-46) over each row of interleaved (gate, up) pairs:
// out[m][i] = silu(in[m][2i]) * in[m][2i+1], `pairs` outputs per row.
hipError_t launch_swiglu(const float* in, float* out, size_t pairs, hipStream_t st);
// Per-row absmax int8 quantisation of fp32 activations: row_scale[m] = max(absmax_m, 1e-5) / 127,
// Q = clamp(rint(X * (127 / max(absmax_m, 1e-5))), -128, 127).
hipError_t launch_quantize_rows(const float* X, int8_t* Q, float* row_scale, int M, int K, hipStream_t st);
hipError_t launch_naive(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, hipStream_t st);
// 2-bit weight format on the device (bitpack_kernels.hip): `size` weights <-> size/4 packed bytes.
hipError_t launch_pack(uint8_t* packed, const int8_t* w, size_t size, hipStream_t st);
hipError_t launch_unpack(int8_t* w, const uint8_t* packed, size_t size, hipStream_t st);

}  // namespace ternix_hip
