/*
 * ternix_hip.h -- C-ABI of the MI355X (gfx950) ternary matmul library
 * (libternix_hip.so).
 *
 *   C[M,N] int32 = A[M,K] int8 x W[K,N],  W in {-1,0,+1}
 *
 * W is passed packed: a row-major K x (N/4) byte array, four weights per byte
 * along N, weight (k, n) in bits 2*(n%4)..2*(n%4)+1 of byte k*(N/4) + n/4, with
 * 00 = 0, 01 = +1, 11 = -1 (reference: src/bitpack.cpp:5-15, README.md:46-53).
 * The undefined code 10 is decoded as -2 by every kernel here, which is what
 * the reference's scalar CPU kernel and CUDA kernels do
 * (src/mul_mat_ternary.cpp:53, src/cuda_kernels.cu:40).
 *
 * Every function returns an int that is a hipError_t value: 0 (hipSuccess),
 * 1 (hipErrorInvalidValue) when an argument is rejected -- always before any
 * pointer is touched or any work is queued -- or the runtime error of the
 * failing HIP call.  This mirrors the cudaError_t contract of the reference
 * (include/ternix/cuda_kernels.cuh:8-21, src/cuda_kernels.cu:126-156).
 *
 * Device-pointer entry points are asynchronous on `stream` (a hipStream_t, or
 * NULL for the default stream).  The caller owns A, B and C; C is fully
 * overwritten (never accumulated into).  Shapes are int64; N must be a
 * multiple of 4; M, K or N may be 0.
 * Workspace.  Some plans need device scratch besides A, B and C:
 *   - split-K partial sums [splits][M][N] int32 of the small-M GEMVs (M = 2..32,
 *     and M = 1 on wide matrices) and of GEMMs whose output tiles alone cannot fill
 *     the chip (mid-size M against K > 4096);
 *   - padded copies of W (K' x N'/4) and A (M x K') for ragged shapes (K % 64,
 *     N/4 % 64) and misaligned operands, at any M;
 *   - 64 K int32 arrival counters of the GEMVs that add a few K splits inside one
 *     launch (zero between calls), and in the same 512 KiB buffer 16 K pairs of
 *     64-bit per-strip tickets of the M = 1 GEMVs below (advanced by every call,
 *     never reset).
 * M = 1 GEMVs on all but wide matrices need no workspace: the K splits add into C
 * with int32 atomics; with the library's tickets each strip's first split zeroes
 * its outputs inside the same launch, else (caller-owned workspace, the allocation-
 * free entry point, or capture before the tickets exist) a fill kernel zeroes C
 * first.  By default the library owns this
 * scratch per (device, stream): allocated the first time a shape needs more than
 * the current size (at most 256 MiB unless one call needs more), kept until the
 * process ends or ternix_hip_release_stream, outgrown buffers retired but not
 * freed.  No allocation happens while the stream is being captured into a hipGraph:
 * a call that would need one then takes a plan that needs none (GEMV splits zero C
 * and add with atomics, ragged shapes run the generic kernels), with identical
 * results.  A graph captured with library calls on a stream uses that stream's
 * buffers, so it must not run concurrently with any other library work issued on
 * that stream (every call on one stream is ordered, so ordinary use is safe).
 * Callers that must not allocate on the call pass their own workspace
 * (ternix_hip_mul_mat_ternary_ws, sized by ..._workspace_size) or use
 * ternix_hip_mul_mat_ternary_noalloc.
 * Calls are thread-safe; calls that share an output buffer race as any two
 * kernels writing one buffer do.
 *
 * Kernels are written for gfx950 only; on any other device the entry points
 * return hipErrorInvalidDeviceFunction (98) from the launch.
 */
#ifndef TERNIX_HIP_H
#define TERNIX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Automatic dispatch: the skinny split-K MFMA kernel for small M, the
 * LDS-tiled MFMA GEMM for large M.  Any M, K >= 0; N % 4 == 0.
 * Replaces: ternix::mul_mat_ternary_cuda_tiled / _naive
 * (reference include/ternix/cuda_kernels.cuh:11-17) for callers that do not
 * want to pick a kernel. */
int ternix_hip_mul_mat_ternary(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                               int64_t M, int64_t K, int64_t N, void* stream);

/* Forced skinny (decode) path: M <= 32 (returns hipErrorInvalidValue above).
 * Weights decoded in registers, int8 MFMA, split-K over the grid (see
 * Workspace above).
 * New in this library; its reference counterpart is the M=1 use of
 * mul_mat_ternary_cuda_naive (reference src/cuda_kernels.cu:126-132). */
int ternix_hip_mul_mat_ternary_gemv(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                                    int64_t M, int64_t K, int64_t N, void* stream);

/* Forced LDS-tiled int8-MFMA GEMM path: any M, K; N % 4 == 0.
 * Replaces the computation of mul_mat_ternary_cuda_tiled (reference
 * src/cuda_kernels.cu:71-122, 134-140) without its M,N,K % 64 restriction. */
int ternix_hip_mul_mat_ternary_gemm(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                                    int64_t M, int64_t K, int64_t N, void* stream);

/* Drop-in for mul_mat_ternary_cuda_tiled (reference
 * include/ternix/cuda_kernels.cuh:14-17, src/cuda_kernels.cu:134-140): the same
 * shape contract -- M, N and K multiples of 64, else hipErrorInvalidValue
 * before any pointer is used -- computed by the MFMA GEMM. */
int ternix_hip_mul_mat_ternary_tiled(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                                     int64_t M, int64_t K, int64_t N, void* stream);

/* Drop-in for mul_mat_ternary_cuda_naive (reference
 * include/ternix/cuda_kernels.cuh:10-12, src/cuda_kernels.cu:42-54, 126-132):
 * one work-item per output element, any M, K; N % 4 == 0. */
int ternix_hip_mul_mat_ternary_naive(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                                     int64_t M, int64_t K, int64_t N, void* stream);

/* ---- workspace contract of the automatic path ----
 * Some plans need device scratch beyond A, B and C: split-K partial sums
 * ([splits][M][N] int32, K split over workgroups when the output alone cannot fill the
 * chip: mid-size M against long K, decode shapes with very long K) and, for ragged or
 * misaligned operands, padded copies of W (K' x N'/4) and A (M x K').  By default the
 * library owns it (see Workspace above).  Callers that must not allocate on the hot path
 * size it once with ternix_hip_mul_mat_ternary_workspace_size and pass it in.
 * No reference counterpart: the reference's device-pointer kernels need no scratch
 * (src/cuda_kernels.cu:126-140). */

/* Bytes of workspace ternix_hip_mul_mat_ternary_ws needs so that it takes exactly the
 * plan ternix_hip_mul_mat_ternary would, for 16-byte aligned A and W (as hipMalloc
 * returns them); 0 when the plan uses none, and for a rejected shape.  The _for form
 * gives the need for the given operand addresses (only their alignment is used:
 * misaligned operands are worked on through padded copies, which need more). */
size_t ternix_hip_mul_mat_ternary_workspace_size(int64_t M, int64_t K, int64_t N);
size_t ternix_hip_mul_mat_ternary_workspace_size_for(const int8_t* dA, const uint8_t* dB,
                                                     int64_t M, int64_t K, int64_t N);

/* ternix_hip_mul_mat_ternary with a caller-owned workspace (dWorkspace: 256-byte
 * aligned, workspace_bytes long; may be NULL with 0 bytes).  Never allocates device
 * memory.  With at least ternix_hip_mul_mat_ternary_workspace_size(M, K, N) bytes it runs
 * the automatic plan (except that split sums are never done inside one launch: a
 * reduce launch adds them); with less it takes a plan that needs no more than given
 * (for a GEMV with a K split: C is zeroed and the splits add into it with int32 atomics,
 * exact and order-independent; a ragged shape runs the generic kernels).  Results are
 * identical either way.  The workspace holds no state between calls; calls sharing one
 * workspace must be ordered (same stream, or synchronised), as for any buffer two
 * kernels write.  hipErrorInvalidValue (before any work) for a misaligned workspace. */
int ternix_hip_mul_mat_ternary_ws(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                                  int64_t M, int64_t K, int64_t N,
                                  void* dWorkspace, size_t workspace_bytes, void* stream);

/* ternix_hip_mul_mat_ternary that allocates nothing: its scratch is a fixed device
 * array of ternix_hip_noalloc_scratch_bytes() (32 MiB) inside the library, one per
 * GPU, held until the process ends.  Same results and status contract as
 * ternix_hip_mul_mat_ternary; hipErrorOutOfMemory (2), before any work, when the
 * shape needs more scratch than that (ternix_hip_mul_mat_ternary_workspace_size).
 * Every call on one GPU shares that GPU's array and nothing in it carries over
 * between calls: calls that overlap in time on one GPU (two streams, two host
 * threads) race and must be serialised by the caller.
 * No reference counterpart: for callers that cannot allocate device memory
 * (code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
int ternix_hip_mul_mat_ternary_noalloc(const int8_t* dA, const uint8_t* dB, int32_t* dC,
                                       int64_t M, int64_t K, int64_t N, void* stream);
size_t ternix_hip_noalloc_scratch_bytes(void);

/* Frees the library-owned workspace of (current device, stream) after synchronising
 * the stream.  The caller guarantees that no hipGraph captured on that stream with
 * library calls runs again afterwards (it would reference the freed buffers).  The next
 * call on the stream allocates afresh.  Returns 0 or the hipStreamSynchronize error. */
int ternix_hip_release_stream(void* stream);

/* Writes a one-line description of the kernel(s) the automatic path would launch for
 * this call (operand addresses matter only through their alignment; nothing is read or
 * launched) into buf (len bytes, NUL-terminated).  0, or hipErrorInvalidValue for a
 * rejected shape or buffer. */
int ternix_hip_plan_describe(const int8_t* dA, const uint8_t* dB, int64_t M, int64_t K, int64_t N,
                             char* buf, size_t len);

/* Kernel choice for ternix_hip_mul_mat_ternary_host. */
enum ternix_hip_variant {
    TERNIX_HIP_AUTO = 0,
    TERNIX_HIP_NAIVE = 1,
    TERNIX_HIP_GEMV = 2,
    TERNIX_HIP_GEMM = 3,
    TERNIX_HIP_TILED = 4
};

/* Synchronous host-pointer convenience wrapper: allocates device buffers,
 * copies A and B in, runs `variant` on the default stream, synchronises,
 * copies C out and frees every buffer on every path.
 * Replaces mul_mat_ternary_cuda_host (reference
 * include/ternix/cuda_kernels.cuh:19-21, src/cuda_kernels.cu:142-156), whose
 * bool `tiled` maps to TERNIX_HIP_TILED / TERNIX_HIP_NAIVE. */
int ternix_hip_mul_mat_ternary_host(const int8_t* A, const uint8_t* B_packed, int32_t* C,
                                    int64_t M, int64_t K, int64_t N, int variant);

/* hipGetErrorString of a status returned above (never NULL). */
const char* ternix_hip_error_string(int status);

/* Library version as an integer, major*10000 + minor*100 + patch. */
int ternix_hip_version(void);

/* Number of HIP devices visible to the process (0 when there is none or no
 * driver); the reference binding's has_cuda probe (pybind11_wrapper.cpp:86-90)
 * becomes has_hip = ternix_hip_device_count() > 0. */
int ternix_hip_device_count(void);

/* Test and tuning switches.  The library never reads the environment: its
 * kernel choice depends only on the call's arguments and the device, unless a
 * caller sets a switch here.  `key` names a switch and v0..v3 its values (-1:
 * unset); ternix_hip_debug_reset() clears all of them.  Keys (the planner's
 * choice is used for an unset value):
 *   "wave_last" v0      most K splits summed inside one wave-GEMV launch (0: none)
 *   "skinny_wave" v0..2 0: no wave-pipelined GEMV; else force (strip bytes,
 *                       ring slots, splits)
 *   "wave_sw" v0..v2    v0 16: 16-byte wave strips on row-major weights; with v1 > 1 the
 *                       strip width (16 / 32) and split count of the atomic split plan;
 *                       v2 1 / 0: column waves (M <= 4) on / off in that plan
 *   "skinny_dma" v0,v1  v0 0: no DMA-staged GEMV; 2..4: its stage count; v1: its
 *                       split count forced
 *   "skinny_short" v0   0: no register-staged short GEMV
 *   "ragged_pad" v0     0: ragged shapes run the generic kernels, not a padded copy
 *   "gemm_narrow" v0    0 / 1: 64 x 64 GEMM tiles for M <= 64 off / forced
 *   "gemm_generic" v0   1: the generic GEMM for every GEMM call
 *   "gemm_splits" v0    GEMM split-K count forced
 *   "gemm_bm" v0        64 / 128 / 256: GEMM tile height forced
 *   "gemm_gm" v0        row tiles per group in the tile order of the 64/128-row GEMMs
 *   "deep" v0..3        0: no whole-K deep GEMV; else force (strip bytes, waves
 *                       per workgroup, ring slots, splits)
 *   "sk_order" v0       1: release/acquire form of the in-launch split sums
 *   "m1_atomic" v0..2   v0 0: M = 1 GEMVs without the zero-fill + int32-atomic split plan;
 *                       v1 / v2: largest M of the self-zeroing atomic split plan on
 *                       row-major (<= 64) / tile-64 (<= 16) weights
 *   "self_zero" v0      0: M = 1 GEMVs never zero C inside the launch (the wave plan
 *                       zeroes it with a fill kernel, wide ones use the reduce launch)
 *   "nt" v0,v1          1 / 0: non-temporal weight loads on / off in the DMA-staged
 *                       (v0) and the wave-pipelined (v1) GEMVs
 *   "wave_ticket" v0    1 / 0: the wave-pipelined GEMV's self-zeroing splits wait
 *                       for their ticket in the first k-step / right after the
 *                       first weight loads (default: 1 for k-ranges of >= 9 steps)
 * Returns 0, or 1 (hipErrorInvalidValue) for an unknown key.  Switches are
 * process-wide; a call running concurrently sees the old or the new value.
 * No reference counterpart (test hook of this library). */
int ternix_hip_debug_set(const char* key, int v0, int v1, int v2, int v3);
void ternix_hip_debug_reset(void);
/* Measurement hook: one launch that only streams `bytes` (rounded down to a multiple
 * of 16) from dSrc (16-byte aligned); dFlag (one int) is written only in a case that
 * does not occur in practice.  Benchmarks time it as the bare HBM read floor of a
 * matmul that reads the same number of bytes. */
int ternix_hip_debug_stream_read(const void* dSrc, size_t bytes, int* dFlag, void* stream);
/* Device fault word of the current GPU: the kernels' bounded in-launch waits never
 * hang, and a wave whose wait gives up records it here instead (the call that hit
 * it still returned hipSuccess, and its output is not trustworthy).  This
 * synchronises the device, stores the recorded TERNIX_FAULT_* bits in *bits (0 when
 * none) and clears them.  Returns 0, hipErrorInvalidValue for a null pointer, or
 * the runtime's error.  No reference counterpart (the reference's kernels have no
 * in-launch waits, cuda_kernels.cu:42-122). */
#define TERNIX_FAULT_ZERO_WAIT 1u /* a K split's wait for its strip's zeroed outputs gave up */
int ternix_hip_take_faults(unsigned int* bits);
/* Number of device allocations the library has made in this process (workspace
 * buffers, split counters, the host wrapper's temporaries); a test hook. */
long long ternix_hip_debug_alloc_count(void);

/* ---- weight format (host), C-ABI of reference include/ternix/bitpack.hpp:6-8 ---- */

/* pack_ternary_weights (reference src/bitpack.cpp:5-15): `size` elements of
 * {-1,0,+1} -> size/4 bytes; values outside {-1,+1} encode as 00. */
void ternix_pack_ternary_weights(uint8_t* packed, const int8_t* unpacked, size_t size);
/* unpack_ternary_weights (reference src/bitpack.cpp:17-27): 01 -> +1,
 * 11 -> -1, 00 and 10 -> 0. */
void ternix_unpack_ternary_weights(int8_t* unpacked, const uint8_t* packed, size_t size);
/* interleave_weights_offline (reference src/bitpack.cpp:29-33): identity copy
 * of size/4 bytes (the K x N/4 layout is consumed as is by every kernel). */
void ternix_interleave_weights_offline(uint8_t* interleaved, const uint8_t* packed, size_t size);
/* Opt-in pre-permuted layout ("tile-64"), the MI355X form of the offline
 * interleave the reference reserves (src/bitpack.cpp:29-33 keeps it the identity;
 * no reference kernel reads a permuted layout).  The K x N/4 packed matrix is cut
 * into 16-byte column strips c (64 weight columns) and 64-row k-steps s; block
 * (c, s) is 1 KB at byte offset (c * K/64 + s) * 1024 and holds row r of the step
 * at 16-byte position r ^ (8 * ((r / 16) % 2)).  Requires K % 64 == 0,
 * (N/4) % 16 == 0, out != packed; returns 0, or 1 (hipErrorInvalidValue). */
int ternix_interleave_weights_tile64(uint8_t* out, const uint8_t* packed, size_t K, size_t N);

/* ---- quantised layer boundary (BitNet b1.58 scheme; no reference counterpart: the
 *      reference leaves weight and activation quantisation as a stub, scripts/quantize.py:5,
 *      README.md:203) ---- */

/* Per-row absmax int8 quantisation of fp32 activations X[M][K] (row-major), asynchronous:
 *   a_m = max(max_k |X[m][k]|, 1e-5),  Q[m][k] = clamp(rint(X[m][k] * (127 / a_m)), -128, 127),
 *   dRowScale[m] = a_m / 127  (IEEE fp32 division and multiplication, round half to even).
 * NaN and infinite inputs are outside the domain. */
int ternix_hip_quantize_activations(const float* dX, int8_t* dQ, float* dRowScale, int64_t M, int64_t K,
                                    void* stream);

/* ternix_hip_mul_mat_ternary with the dequantisation fused into the output:
 *   Y[m][n] = (float)C[m][n] * (dRowScale[m] * w_scale)    (fp32, row-major M x N)
 * (the scale product rounded once, then one rounding per output), where C is the exact int32
 * product.  Same shapes, dispatch and status contract as ternix_hip_mul_mat_ternary; dRowScale must
 * not be NULL when M > 0. */
int ternix_hip_mul_mat_ternary_dequant(const int8_t* dA, const uint8_t* dB, float* dY, int64_t M, int64_t K,
                                       int64_t N, const float* dRowScale, float w_scale, void* stream);

/* Host, offline: absmean ternary quantisation of fp32 weights W (size elements, K x N row-major,
 * size % 4 == 0) straight into the packed format:
 *   gamma = max(mean |W|, 1e-5) (summed in double in index order),
 *   w = clamp(rint(W / gamma), -1, 1), packed as ternix_pack_ternary_weights; *w_scale = gamma.
 * Returns 0, or 1 for a size that is not a multiple of 4 or a NULL pointer. */
int ternix_quantize_weights_absmean(uint8_t* packed, float* w_scale, const float* W, size_t size);

/* ---- feed-forward block on the device (asynchronous on `stream`) ---- */

/* rms_norm_avx2 / rms_norm_scalar of reference include/ternix/simd_math.hpp:8-10
 * (src/simd_math.cpp:7-38) applied to each of `rows` rows of `size` floats:
 * out = in * inv * weight, inv = 1 / sqrt(sum(in^2) / size + eps).  The sum of squares is
 * a parallel reduction: results match the reference to float rounding (its own
 * scalar-vs-AVX2 tolerance is 1e-4 relative). */
int ternix_hip_rms_norm(float* dOut, const float* dIn, const float* dWeight, int64_t rows, int64_t size, float eps,
                        void* stream);
/* swiglu of reference include/ternix/simd_math.hpp:11-12 (src/simd_math.cpp:40-46):
 * out[i] = silu(in[2i]) * in[2i+1], silu(g) = g / (1 + exp(-g)), for i < size / 2. */
int ternix_hip_swiglu(float* dOut, const float* dIn, int64_t size, void* stream);
/* RMSNorm fused with ternix_hip_quantize_activations: each normalised row is quantised
 * straight to int8 (no float output). */
int ternix_hip_rms_norm_quantize(int8_t* dQ, float* dRowScale, const float* dIn, const float* dWeight, int64_t rows,
                                 int64_t size, float eps, void* stream);
/* Up-projection with dequantisation and SwiGLU fused into its output: the N output columns
 * are interleaved (gate, up) pairs, dH is M x N/2 fp32 with
 *   dH[m][i] = silu(y[m][2i]) * y[m][2i+1],  y = (float)C * (dRowScale[m] * w_scale).
 * dScratch (M x N int32, may be NULL) is used only when the split-K or K-chunk path cannot
 * fuse the epilogue (first use of a shape inside graph capture, K > 131008); such a call
 * with dScratch == NULL returns hipErrorInvalidValue. */
int ternix_hip_mul_mat_ternary_swiglu(const int8_t* dA, const uint8_t* dB, float* dH, int64_t M, int64_t K,
                                      int64_t N, const float* dRowScale, float w_scale, int32_t* dScratch,
                                      void* stream);
/* Bytes of device workspace ternix_hip_ffn_forward needs for M rows, hidden size H and
 * intermediate size F. */
size_t ternix_hip_ffn_workspace_size(int64_t M, int64_t H, int64_t F);
/* One BitNet-style feed-forward block, four launches on `stream`:
 *   q1, rs1 = rms_norm_quantize(dX, dNormWeight, eps)                  [M x H]
 *   h       = swiglu matmul(q1, dWgu: H x 2F packed, interleaved gate/up columns, ws_gu)
 *   q2, rs2 = quantize_activations(h)                                  [M x F]
 *   dY      = dequant matmul(q2, dWd: F x H packed, ws_d)              [M x H] fp32
 * H % 4 == 0, F % 2 == 0; dWorkspace is 256-byte aligned with at least
 * ternix_hip_ffn_workspace_size(M, H, F) bytes.  No reference counterpart (the reference's
 * TransformerLayer::forward is a stub, README.md:204); its pieces mirror simd_math.hpp and the
 * matmul entry points above. */
int ternix_hip_ffn_forward(float* dY, const float* dX, const float* dNormWeight, float eps, const uint8_t* dWgu,
                           float ws_gu, const uint8_t* dWd, float ws_d, int64_t M, int64_t H, int64_t F,
                           void* dWorkspace, size_t workspace_bytes, void* stream);

/* ---- weight format on the device (asynchronous on `stream`) ---- */

/* pack_ternary_weights on device memory (reference src/bitpack.cpp:5-15, same
 * semantics as ternix_pack_ternary_weights): `size` int8 weights at dW ->
 * size/4 bytes at dPacked.  hipErrorInvalidValue for a null pointer when
 * size/4 > 0. */
int ternix_hip_pack_ternary_weights(uint8_t* dPacked, const int8_t* dW, size_t size, void* stream);
/* unpack_ternary_weights on device memory (reference src/bitpack.cpp:17-27):
 * size/4 bytes at dPacked -> 4*(size/4) int8 weights at dW. */
int ternix_hip_unpack_ternary_weights(int8_t* dW, const uint8_t* dPacked, size_t size, void* stream);
/* interleave_weights_offline on device memory (reference src/bitpack.cpp:29-33):
 * the identity, a device-to-device copy of size/4 bytes (none when dOut == dPacked). */
int ternix_hip_interleave_weights_offline(uint8_t* dOut, const uint8_t* dPacked, size_t size, void* stream);
/* ternix_interleave_weights_tile64 on device memory (one coalesced permutation copy);
 * K % 64 == 0, (N/4) % 16 == 0, 16-byte aligned, dOut != dPacked, K * N/4 < 2^32. */
int ternix_hip_interleave_weights_tile64(uint8_t* dOut, const uint8_t* dPacked, int64_t K, int64_t N, void* stream);
/* ternix_hip_mul_mat_ternary on tile-64 weights dWt (same C = A x W, same status
 * contract); K % 128 == 0, N % 256 == 0, dA and dWt 16-byte aligned, K * N/4 < 2^32.
 * Each wave's weight read is one contiguous 1 KB block, which the LDS transposing
 * reads consume without a swizzle: the decode-shaped calls (M <= 32) run faster than
 * on the row-major layout. */
int ternix_hip_mul_mat_ternary_tile64(const int8_t* dA, const uint8_t* dWt, int32_t* dC, int64_t M, int64_t K,
                                      int64_t N, void* stream);
/* ternix_hip_mul_mat_ternary_dequant on tile-64 weights: Y = (float)C * (dRowScale[m] * w_scale),
 * fp32 M x N, the scaling fused into the output; same contract as ternix_hip_mul_mat_ternary_tile64. */
int ternix_hip_mul_mat_ternary_tile64_dequant(const int8_t* dA, const uint8_t* dWt, float* dY, int64_t M, int64_t K,
                                              int64_t N, const float* dRowScale, float w_scale, void* stream);
/* ternix_hip_ffn_forward with both weight matrices in the tile-64 layout (dWguT: H x 2F, interleaved
 * (gate, up) columns, dWdT: F x H, each converted by ternix_hip_interleave_weights_tile64): the same
 * results bit for bit, the same workspace (ternix_hip_ffn_workspace_size).  H % 256 == 0,
 * F % 128 == 0; no reference counterpart. */
int ternix_hip_ffn_forward_tile64(float* dY, const float* dX, const float* dNormWeight, float eps,
                                  const uint8_t* dWguT, float ws_gu, const uint8_t* dWdT, float ws_d, int64_t M,
                                  int64_t H, int64_t F, void* dWorkspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TERNIX_HIP_H */
