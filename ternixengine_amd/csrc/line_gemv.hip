// line_gemv.hip -- gfx950 whole-line decode GEMV (M <= 16; ragged operands M <= 32) for the ternary
// matmul, and its launcher.
// Shared helpers, the weight layout and the decode forms are described in kernel_common.h.
//
// Work unit: one 128-byte strip of the packed weight rows (one whole cache line per row, 512 output
// columns) over S consecutive 64-row k-steps.  Unit (strip s, split t) is workgroup t * strips + s,
// so every strip's split 0 is dispatched before any other split of it; or, when the rows share cache
// lines between strips and the whole grid is resident at once, the units are taken in 8 contiguous
// chunks, one per XCD (xcd_chunks).
//
//   * Weights: the unit's S x 8 KB go global -> LDS with global_load_lds_dwordx4, all issued at
//     once (S instructions per wave for 8 data waves); one wave instruction moves 8 whole 128-byte
//     lines.  Stage row r keeps chunk c at 16-byte position c ^ swz(r), swz(r) = ((r/2) % 4) ^
//     4 * ((r/16) % 2): the 8 rows one 16-lane group of a transposing read touches cover 32 banks,
//     and the next 16-row group (read in the same instruction) the other 32.
//   * Data wave w owns the strip's w-th 16-byte column group (GW = 8 / NW groups per wave): per k-step
//     two ds_read_b64_tr_b8 give lane q byte-column q of 16 k-rows, the shift-form decode makes four
//     B operands, and v_mfma_i32_16x16x64_i8 against the activation fragment (row q < M, 16 bytes of
//     k-block kb, loaded straight from global memory; MG = 2: a second fragment for rows 16 .. 31)
//     accumulates 64 output columns.
//   * K splits add into C with int32 atomics (exact, order-free).  C is zeroed inside the launch by
//     each strip's split 0, with no wait in any data wave: the workgroup's extra protocol wave takes
//     the call's ticket and, in split 0, zeroes the strip's outputs with agent-scope (write-through)
//     stores, waits for them and publishes the call's number in the strip's "zeroed" word at once
//     (the other splits read it when their own weights have landed, by which time it is there); in
//     the other splits it waits for that word.  The data waves only meet it at the barrier before their
//     atomics.
//
// Ticket protocol (per strip: a 64-bit ticket counter T and a 64-bit zeroed word Z that persist
// across calls in the library's per-stream counter buffer; the same words and rules as the
// self-zeroing wave-pipelined GEMV in skinny_kernels.hip, so the two may alternate on one stream):
// every call adds exactly 64 to T (split 0 adds 64 - (splits - 1), every other split 1, each with
// one returning atomic add), so T is a multiple of 64 between calls and every split of a call reads
// back a value whose quotient by 64 is the number of calls before it.  Split 0 writes that number + 1
// to Z after its zeroing stores have completed; the other splits add into C only after reading it
// there.  The waited-for split was dispatched first (lower workgroup id, in-order dispatch), so it
// runs while any other split of its strip waits.  The wait is still bounded; a wave that gives up
// records kFaultZeroWait in the library's fault word (ternix_hip_take_faults) and adds anyway.
//
// Fused forms (the decode feed-forward block's GEMVs, and dequantising calls):
//   * AQ = 1 / 2: the int8 activations are made inside the kernel from fp32 rows X (absmax
//     quantisation; AQ = 2 RMS-normalises with weight G first), with the loops and rounding of
//     row_stats.h, so they are bit-identical to quantize_rows_kernel / rmsnorm_kernel.  In every
//     workgroup, data wave r < M loads row r (and G) ahead of its weights -- into its registers for
//     rows up to 3072 wide, else by DMA into LDS --, computes the row's statistics alone (no barrier,
//     DPP row exchanges instead of LDS shuffles) and quantises the unit's activations of the row.
//     AQ = 3: the absmax comes from a producer's per-strip maxima of the rows (amax_in, written by
//     an EPI launch with amax_out), so only the unit's slice of each row is read.
//   * EPI: a float output Y = C * (row scale * weight scale), optionally with the SwiGLU of
//     interleaved (gate, up) column pairs.  The splits add their sums, still scaled by 64, a column
//     pair at a time as one 64-bit integer with a returning atomic into the int32 buffer C (zeroed as
//     above); the low 6 bits of the even column count the splits added, so each pair's last adder
//     knows it, recovers both sums and writes Y.  One launch, no dequantisation launch, no arrival
//     counter.  With amax_out the per-strip maxima of |Y| are folded into zeroed entries.
//   * RG: ragged operands (K not a multiple of 64, N/4 not a multiple of 16, A or W at any address),
//     int32 output: the weights are staged through registers from aligned dwords instead of the
//     DMA, the last k-step is partial (zero rows past K), and the outputs past N are not written --
//     no padded copy of the operands, one launch.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kernel_common.h"
#include "row_stats.h"
#include "ternary_kernels.h"

namespace ternix_hip {

// This file's device fault word (its kernels cannot see the one in skinny_kernels.hip: every .hip
// file is its own device code object).  Read and cleared with the other by take_faults.
__device__ unsigned int g_line_fault_word;

namespace {

constexpr int kLineSpinLimit = 1 << 20;  // tries of the zeroed-word wait (about a second)
constexpr int kLineQK = 8192;            // fused quantisation: M x K <= kLineQK fp32 activations (in LDS)

struct LineArgs {
    const int8_t* A;
    const uint8_t* B;
    int32_t* C;                    // int32 sums (the output, or with EPI the int32 buffer of the sums)
    int M, K, N;
    int strips;                    // ceil(N/4 / 128)
    int splits;                    // workgroups per strip (<= 64)
    unsigned long long* tk;        // per strip {T, Z, arrivals}
    int tk_stride;                 // 64-bit words between consecutive strips' words
    const float* X;                // AQ: fp32 rows (M x K)
    const float* G;                // AQ == 2: RMSNorm weight (K)
    float eps;
    float* rs_out;                 // AQ: row scales (M), written by workgroup 0
    OutScale os;                   // EPI: float output
    int vec_y;                     // EPI: Y 16-byte aligned
    int xcd_chunks;                // unit order: 0 split-major by workgroup id, 1 in 8 contiguous chunks
    float* amax_out;               // EPI: per row and strip, the largest |value| the strip stored (or null)
    int amax_stride;               // floats between rows of amax_out / amax_in (a multiple of 4)
    const float* amax_in;          // AQ == 3: the producer's per-strip maxima of the rows of X
    int amax_n;                    // AQ == 3: entries per row of amax_in
};

__device__ __forceinline__ int line_swz(int r) { return ((r >> 1) & 3) ^ (((r >> 4) & 1) << 2); }

// v from lane l ^ m of the same 16-lane row (m = 1, 2, 4, 8), through DPP (no LDS): quad
// permutations for 1 and 2; for 4 and 8 the row shifts up and down, each lane taking the one that
// reaches its partner.
template <int m>
__device__ __forceinline__ float row_xor(float v, int lane) {
    const int x = __float_as_int(v);
    if constexpr (m == 1) return __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));
    if constexpr (m == 2) return __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));
    const int up = __builtin_amdgcn_update_dpp(x, x, 0x100 + m, 0xF, 0xF, false);    // row_shl: lane l + m
    const int down = __builtin_amdgcn_update_dpp(x, x, 0x110 + m, 0xF, 0xF, false);  // row_shr: lane l - m
    return __int_as_float((lane & m) ? down : up);
}

// Four dwords at a 4-byte aligned address, read by one 16-byte load; global-memory pointers to
// dwords and to such groups (addresses rebuilt from integers would otherwise be flat accesses).
typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
typedef __attribute__((address_space(1))) const uint32_t g_u32;
typedef __attribute__((address_space(1))) const u4a g_u4a;

template <int S, int NW, int AQ, bool EPI, bool RG, int MG = 1, bool T64 = false>
__global__ __launch_bounds__(64 * (NW + 1)) void line_gemv_kernel(const uint8_t* Bp, const void* Ap, const void* Gp, int32_t* Cp,
                                                         unsigned long long* tkp, int Kp, int Np, unsigned shape_p,
                                                         unsigned aux_p, LineArgs args) {
    // Leading scalars (preloaded into SGPRs by the command processor): Ap is A, or X with fused
    // quantisation; Gp is G (AQ 2) or the producer's maxima (AQ 3); tkp the strips' tickets; shape_p
    // packs the strip count (bits 0-15), the split count (16-22), the XCD-chunked order (23) and M
    // (24-31); aux_p the tickets' stride (bits 0-5) and the maxima's row stride (6-31).
    static_assert(NW == 4 || NW == 8, "4 or 8 data waves");
    static_assert(AQ == 0 || EPI, "fused quantisation comes with the float output");
    static_assert(!RG || (AQ == 0 && !EPI), "ragged operands: int32 output from int8 activations");
    static_assert(MG == 1 || (MG == 2 && RG), "two 16-row groups (17-32 rows) on ragged operands only");
    static_assert(!(T64 && RG), "tile-64 weights are aligned by contract");
    constexpr int GW = 8 / NW;  // 16-byte column groups per data wave
    constexpr int STEP = 8192;  // bytes per k-step of the strip (64 rows x 128 bytes)
    __shared__ __attribute__((aligned(16))) uint8_t lds[S * STEP];
    // rows of X at a 1 KB-aligned pitch (AQ 3: the unit's slices), G's copies (AQ 3: the row maxima)
    __shared__ __attribute__((aligned(16))) float xl[AQ ? kLineQK + 1024 : 4];
    __shared__ __attribute__((aligned(16))) float gl[AQ == 2 ? kLineQK + 1024 : (AQ == 3 ? 2048 : 4)];
    __shared__ __attribute__((aligned(16))) int8_t qbuf[AQ ? 4 * S * 64 : 16];  // AQ: the unit's int8 rows
    __shared__ float rscale[4];
    __shared__ float wmax[16 * 4];  // EPI with amax_out: per wave and row, the largest |value| written

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int strips = (int)(shape_p & 0xFFFFu), splits_p = (int)((shape_p >> 16) & 0x7Fu);
    const int xcd_p = (int)((shape_p >> 23) & 1u), Mp = (int)(shape_p >> 24);
    const int tk_stride_p = (int)(aux_p & 63u), amax_stride_p = (int)(aux_p >> 6);
    // Workgroup g runs on XCD g mod 8.  With xcd_chunks the split-major unit sequence is cut into 8
    // contiguous chunks, chunk x taken by the workgroups of XCD x in order, so that neighbouring strips
    // of one split share an L2 (rows whose length is not a multiple of 128 bytes put one cache line
    // in two strips).
    // Without it the grid is (strips, splits): dispatched in the same split-major order, with no
    // division to find the unit's strip and split.
    int split = (int)blockIdx.y, s = (int)blockIdx.x;
    if (xcd_p) {
        const int unit0 = (int)blockIdx.x;
        const int G = strips * splits_p, q = G >> 3, r = G & 7, x = unit0 & 7;
        const int unit = x * q + min(x, r) + (unit0 >> 3);
        split = unit / strips;
        s = unit - split * strips;
    }
    const int M = Mp, K = Kp, N = Np, NB = N >> 2;
    const int s0 = split * S;                 // first k-step
    const int nst = min(S, ((K + 63) >> 6) - s0);  // k-steps of this unit (>= 1; RG: the last may be partial)
    const int bc0 = s * 128;                  // first byte-column of the strip
    const bool zeroer = split == 0;
    unsigned long long* tk = tkp + (size_t)tk_stride_p * (size_t)s;

    // AQ: wave r < M stages what row r needs, global -> LDS ahead of its weights, 1 KB per instruction
    // (the last chunk's lanes past the end re-read valid bytes into the row's padding), so that
    // waiting for it leaves the weight DMAs in flight and involves no other wave:
    //   AQ 1 / 2: the whole row of X (and, AQ 2, a copy of G) at a 1 KB-aligned row pitch;
    //   AQ 3: the unit's slice of the row (64 nst activations) and the producer's maxima of the row.
    const int xpitch = AQ == 3 ? ((S * 256 + 1023) & ~1023) : ((K * 4 + 1023) & ~1023);  // bytes per row
    const int apitch = (amax_stride_p * 4 + 1023) & ~1023;
    // AQ 1 / 2 with K <= 256 KJ: row r and G go straight into wave r's registers instead (lane l: k =
    // 256 j + 4 l .. + 3), with this unit's 64 nst values of each (lane l: k = 64 (s0 + u) + l).
    constexpr int KJ = (AQ == 1 || AQ == 2) ? 12 : 1;
    const bool regs = (AQ == 1 || AQ == 2) && K <= 256 * KJ;
    v4i xr[KJ], gr[KJ];
    uint32_t xs[S], gs[S];
    if constexpr (AQ == 1 || AQ == 2) {
        if (wave < M && regs) {
            const float* xrow = reinterpret_cast<const float*>(Ap) + (size_t)wave * (size_t)K;
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                const int k = 256 * j + 4 * lane;
                xr[j] = k < K ? *reinterpret_cast<const v4i*>(xrow + k) : v4i{0, 0, 0, 0};
                gr[j] = AQ == 2 && k < K ? *reinterpret_cast<const v4i*>(reinterpret_cast<const float*>(Gp) + k) : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < S; ++u) {
                const int k = 64 * (s0 + min(u, nst - 1)) + lane;
                xs[u] = __float_as_uint(xrow[k]);
                gs[u] = AQ == 2 ? __float_as_uint(reinterpret_cast<const float*>(Gp)[k]) : 0u;
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // these loads ahead of the weights' DMAs (in-order counter)
    }
    if constexpr (AQ != 0) {
        if (wave < M && !regs) {
            const uint8_t* xb = reinterpret_cast<const uint8_t*>(Ap);
            uint8_t* xd = reinterpret_cast<uint8_t*>(xl) + wave * xpitch;
            if constexpr (AQ == 3) {
                const int n = nst * 256;
                const uint8_t* src = xb + ((size_t)wave * (size_t)K + (size_t)s0 * 64) * 4;
                for (int c = 0; c * 1024 < n; ++c) lds_dma16(src + min(c * 1024 + lane * 16, n - 16), xd + c * 1024);
                const int na = amax_stride_p * 4;
                const uint8_t* asrc = reinterpret_cast<const uint8_t*>(reinterpret_cast<const float*>(Gp) + (size_t)wave * amax_stride_p);
                uint8_t* ad = reinterpret_cast<uint8_t*>(gl) + wave * apitch;
                for (int c = 0; c * 1024 < na; ++c) lds_dma16(asrc + min(c * 1024 + lane * 16, na - 16), ad + c * 1024);
            } else {
                const int n = K * 4;
                const uint8_t* src = xb + (size_t)wave * (size_t)n;
                for (int c = 0; c * 1024 < n; ++c) lds_dma16(src + min(c * 1024 + lane * 16, n - 16), xd + c * 1024);
                if constexpr (AQ == 2) {
                    const uint8_t* gb = reinterpret_cast<const uint8_t*>(reinterpret_cast<const float*>(Gp));
                    uint8_t* gd = reinterpret_cast<uint8_t*>(gl) + wave * xpitch;
                    for (int c = 0; c * 1024 < n; ++c) lds_dma16(gb + min(c * 1024 + lane * 16, n - 16), gd + c * 1024);
                }
            }
        }
    }

    auto issue_weights = [&]() {
        const int r_in = lane >> 3, pos = lane & 7;
        if constexpr (RG) {
            // Ragged operands (K % 64, N/4 % 16 or the weights' address arbitrary): register loads of
            // the same 16-byte pieces as the DMA below, from 4-byte aligned dwords (no load leaves the
            // rows' 4-byte aligned extent), funnel-shifted into place; rows past K are zeros, bytes past
            // the row end are the next row's or zeros (their outputs are not written).  Then written
            // to LDS in the DMA's layout.  (Measured on MI355X against loading each of the five dwords
            // on its own: 1x1000x3076 4.23 -> 3.53 us, 1x8191x2052 5.95 -> 5.16, 17x4093x1028 8.59 -> 7.89.)
            constexpr int NP = (S * 8 + NW - 1) / NW;
            // end of the 4-byte aligned extent of the weight rows
            const uintptr_t w_hull = (reinterpret_cast<uintptr_t>(Bp) + (size_t)K * (size_t)NB + 3) & ~uintptr_t(3);
            uint32_t d[NP][5];
            int sh[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = wave + NW * i;
                sh[i] = 0;
#pragma unroll
                for (int u = 0; u < 5; ++u) d[i][u] = 0;
                if (p < S * 8) {
                    const int step = p >> 3, r = (p & 7) * 8 + r_in;
                    const int c = pos ^ line_swz(r), col = bc0 + 16 * c;
                    const int kr = (s0 + step) * 64 + r;
                    const int v = (step < nst && kr < K) ? min(16, NB - col) : 0;  // bytes of the piece
                    if (v > 0) {
                        const uintptr_t src = reinterpret_cast<uintptr_t>(Bp) + (size_t)kr * (size_t)NB + (size_t)col;
                        const uintptr_t wa = src & ~uintptr_t(3);
                        sh[i] = (int)(src & 3);
                        // Where the four dwords from the piece's first one lie inside the rows' aligned
                        // extent: one 16-byte load (4-byte aligned), and the fifth dword when the piece
                        // needs it; near the extent's end, only the dwords holding a byte of the piece.
                        g_u32* w = (g_u32*)wa;
                        if (wa + 16 <= w_hull) {
                            const u4a x = *(g_u4a*)wa;
#pragma unroll
                            for (int u = 0; u < 4; ++u) d[i][u] = x[u];
                            if (sh[i] + v > 16) d[i][4] = w[4];
                        } else {
#pragma unroll
                            for (int u = 0; u < 5; ++u)
                                if (4 * u < sh[i] + v) d[i][u] = w[u];
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = wave + NW * i;
                if (p < S * 8) {
                    const uint32_t b = (uint32_t)sh[i] * 8u;
                    v4i o;
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        o[u] = (int)(uint32_t)((((uint64_t)d[i][u + 1] << 32) | d[i][u]) >> b);
                    *reinterpret_cast<v4i*>(lds + (p >> 3) * STEP + (p & 7) * 1024 + lane * 16) = o;
                }
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < (S * 8 + NW - 1) / NW; ++i) {
            const int p = wave + NW * i;
            if (p < S * 8) {  // compile-time per (i, wave-uniform p): all waves issue ceil(8S / NW) or fewer
                const int step = min(p >> 3, nst - 1), r = (p & 7) * 8 + r_in;
                int c = pos ^ line_swz(r);
                if (bc0 + 16 * c >= NB) c = 0;  // past the last column (a partial last strip): a valid chunk, unused
                // T64: the same piece in the tile-64 layout (the 8 rows of one chunk that an instruction
                // reads are one contiguous 128-byte line of their block)
                // (row-major: a wave-uniform base for the instruction's 8 rows, a 32-bit lane offset)
                const uint8_t* src =
                    T64 ? Bp + tile64_offset((bc0 >> 4) + c, (s0 + step) * 64 + r, K >> 6)
                        : Bp + (size_t)((s0 + step) * 64 + (p & 7) * 8) * (size_t)NB +
                              (uint32_t)(r_in * NB + bc0 + 16 * c);
                lds_dma16(src, lds + (p >> 3) * STEP + (p & 7) * 1024);
            }
        }
    };

    unsigned long long old = 0, saved_exec;
    if (wave == NW) {
        // Protocol wave.  Split 0 first issues the zeroing stores (they need no ticket).
        if (zeroer) {
            const int n8 = 2 * min(128, NB - bc0);  // 8-byte units of the strip's outputs in one row
            for (int r = 0; r < M; ++r) {
                unsigned long long* z = reinterpret_cast<unsigned long long*>(Cp + (size_t)r * (size_t)N + 4 * bc0);
                for (int u = lane; u < n8; u += 64) __hip_atomic_store(z + u, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if constexpr (EPI) {  // the strip's maxima start at 0 too (published with the zeroed word)
                if (args.amax_out != nullptr && lane < M)
                    __hip_atomic_store(reinterpret_cast<unsigned int*>(args.amax_out) + (size_t)lane * amax_stride_p + s,
                                       0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // T += 64 - (splits - 1) (no return needed).  Lane 0 alone enabled; nothing waited for here.
            const unsigned long long inc = (unsigned long long)(64 - (splits_p - 1));
            __asm__ volatile(
                "s_mov_b64 %0, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add_x2 %1, %2, off\n\t"
                "s_mov_b64 exec, %0"
                : "=&s"(saved_exec)
                : "v"(tk), "v"(inc)
                : "memory");
        } else {
            // The returning T += 1 (its value / 64 + 1 names this call), lane 0 alone enabled, not
            // waited for here: `old` is only read after the wait below, which names it.
            __asm__ volatile(
                "s_mov_b64 %1, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add_x2 %0, %2, %3, off sc0\n\t"
                "s_mov_b64 exec, %1"
                : "=&v"(old), "=&s"(saved_exec)
                : "v"(tk), "v"(1ull)
                : "memory");
        }
    } else {
        // Data waves.  DMA instruction p (k-step p / 8, rows 8 (p % 8) .. +7) is issued by wave p % NW;
        // lane l fills 16-byte position l % 8 of row 8 (p % 8) + l / 8.  Steps past the unit's last
        // re-read its last step into their own (unused) stage slot, so every wave issues the same number
        // of DMAs on every path.
        issue_weights();
    }

    // AQ: wave r < M makes row r's int8 activations for this unit, with no barrier and no other wave.
    // The row statistics follow row_stats.h exactly (a 256-thread workgroup, thread t summing
    // k = t + 256 j in increasing j, the xor butterfly 32 .. 1 over each wave's 64 threads, then
    // (w0 + w1) + (w2 + w3)): lane l plays threads 4 l .. 4 l + 3 (one 16-byte LDS read each j), the
    // butterfly's offsets 32 .. 4 are lane offsets 8 .. 1 and 2, 1 are within the lane, and the four
    // waves' sums sit in lanes 0, 16, 32, 48.  The absmax is a maximum (exact in any order); AQ 3
    // takes it over the producer's per-strip maxima.  The unit's M x 64 nst values are quantised into
    // qbuf; rscale[r] (and, in workgroup 0, rs_out[r]) gets the row scale.  LDS is read and written
    // with inline assembly: a compiler-placed LDS access would first wait for every LDS DMA in flight.
    if constexpr (AQ != 0) {
        if (wave < M) {
            TX_VMCNT((S * 8 + NW - 1) / NW);  // this wave's row data have landed (its weights may not)
            const int r = wave;
            const uint32_t xa = lds_u32(xl) + (uint32_t)(r * xpitch);
            const uint32_t ga = lds_u32(gl) + (uint32_t)(r * (AQ == 3 ? apitch : xpitch));
            float inv = 1.0f, m = 0.0f;
            if constexpr (AQ == 3) {
                for (int i0 = 0; i0 < args.amax_n; i0 += 64) {
                    uint32_t v = lds_read_b32_asm(ga + 4 * min(i0 + lane, args.amax_n - 1));
                    TX_LGKMCNT0();
                    __asm__ volatile("" : "+v"(v));
                    if (i0 + lane < args.amax_n) m = fmaxf(m, __uint_as_float(v));
                }
            } else if (regs) {
                if constexpr (AQ == 2) {
                    float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < KJ; ++j)
                        if (256 * j + 4 * lane < K) {
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                const float x = __int_as_float(xr[j][c]);
                                ss[c] = fmaf(x, x, ss[c]);
                            }
                        }
#pragma unroll
                    for (int c = 0; c < 4; ++c) ss[c] += row_xor<8>(ss[c], lane);
#pragma unroll
                    for (int c = 0; c < 4; ++c) ss[c] += row_xor<4>(ss[c], lane);
#pragma unroll
                    for (int c = 0; c < 4; ++c) ss[c] += row_xor<2>(ss[c], lane);
#pragma unroll
                    for (int c = 0; c < 4; ++c) ss[c] += row_xor<1>(ss[c], lane);
                    const float w = (ss[0] + ss[2]) + (ss[1] + ss[3]);
                    const float w0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 0));
                    const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 16));
                    const float w2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 32));
                    const float w3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 48));
                    inv = 1.0f / sqrtf(((w0 + w1) + (w2 + w3)) / (float)K + args.eps);
                }
#pragma unroll
                for (int j = 0; j < KJ; ++j)
                    if (256 * j + 4 * lane < K) {
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const float x = __int_as_float(xr[j][c]);
                            m = fmaxf(m, fabsf(AQ == 2 ? x * inv * __int_as_float(gr[j][c]) : x));
                        }
                    }
            } else {
                if constexpr (AQ == 2) {
                    float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    for (int j0 = 0; j0 < K; j0 += 256 * 8) {
                        v4i xb[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) xb[u] = lds_read_b128_asm(xa + 4 * min(j0 + 256 * u + 4 * lane, K - 4));
                        TX_LGKMCNT0();
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            __asm__ volatile("" : "+v"(xb[u]));
                            if (j0 + 256 * u + 4 * lane < K) {
#pragma unroll
                                for (int c = 0; c < 4; ++c) {
                                    const float x = __int_as_float(xb[u][c]);
                                    ss[c] = fmaf(x, x, ss[c]);
                                }
                            }
                        }
                    }
#pragma unroll
                    for (int off = 8; off >= 1; off >>= 1)
#pragma unroll
                        for (int c = 0; c < 4; ++c) ss[c] += __shfl_xor(ss[c], off);
                    // offsets 2 and 1: thread 4 l + c holds (ss[c] + ss[c ^ 2]) + (ss[c ^ 1] + ss[c ^ 3]) in
                    // the same order for c = 0 (the value lanes 16 w pass on as wave w's sum)
                    const float w = (ss[0] + ss[2]) + (ss[1] + ss[3]);
                    const float w0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 0));
                    const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 16));
                    const float w2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 32));
                    const float w3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 48));
                    inv = 1.0f / sqrtf(((w0 + w1) + (w2 + w3)) / (float)K + args.eps);
                }
                for (int j0 = 0; j0 < K; j0 += 256 * 4) {
                    v4i xb[4], gb[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const uint32_t o = 4 * min(j0 + 256 * u + 4 * lane, K - 4);
                        xb[u] = lds_read_b128_asm(xa + o);
                        gb[u] = AQ == 2 ? lds_read_b128_asm(ga + o) : v4i{0, 0, 0, 0};
                    }
                    TX_LGKMCNT0();
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        __asm__ volatile("" : "+v"(xb[u]), "+v"(gb[u]));
                        if (j0 + 256 * u + 4 * lane < K) {
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                const float x = __int_as_float(xb[u][c]);
                                m = fmaxf(m, fabsf(AQ == 2 ? x * inv * __int_as_float(gb[u][c]) : x));
                            }
                        }
                    }
                }
            }
            m = fmaxf(m, row_xor<8>(m, lane));
            m = fmaxf(m, row_xor<4>(m, lane));
            m = fmaxf(m, row_xor<2>(m, lane));
            m = fmaxf(m, row_xor<1>(m, lane));
            m = fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16))),
                      fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)),
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48))));
            const float am = fmaxf(m, 1e-5f), sc = 127.0f / am;
            if (lane == 0) {
                lds_write_b32_asm(lds_u32(rscale) + 4 * r, __float_as_uint(am / 127.0f));
                if (blockIdx.x == 0 && blockIdx.y == 0) args.rs_out[r] = am / 127.0f;
            }
            // this unit's values of the row: k = 64 s0 + i, i < 64 nst, lane i % 64
            const uint32_t qa = lds_u32(qbuf) + (uint32_t)(r * (S * 64));
            uint32_t xv[S], gv[S];
            if (regs) {
#pragma unroll
                for (int u = 0; u < S; ++u) {
                    xv[u] = xs[u];
                    gv[u] = gs[u];
                }
            } else {
#pragma unroll
                for (int u = 0; u < S; ++u) {
                    const int i = min(u, nst - 1) * 64 + lane;
                    const int k = AQ == 3 ? i : s0 * 64 + i;
                    xv[u] = lds_read_b32_asm(xa + 4 * k);
                    gv[u] = AQ == 2 ? lds_read_b32_asm(ga + 4 * k) : 0u;
                }
                TX_LGKMCNT0();
            }
#pragma unroll
            for (int u = 0; u < S; ++u) {
                __asm__ volatile("" : "+v"(xv[u]), "+v"(gv[u]));
                if (u < nst) {
                    const float x = __uint_as_float(xv[u]);
                    const float v = AQ == 2 ? x * inv * __uint_as_float(gv[u]) : x;
                    lds_write_b8_asm(qa + (uint32_t)(u * 64 + lane), (uint32_t)quantize_value(v, sc) & 0xFFu);
                }
            }
        }
    }

    if (wave == NW) {
        if (zeroer) {
            // As soon as the zeroing stores have completed (not at barrier (1), which waits for this
            // workgroup's weights): Z += 1 (lane 0 alone enabled), so the other splits find it there
            // when their own weights have landed.
            const unsigned long long one = 1;
            __asm__ volatile(
                "s_waitcnt vmcnt(0)\n\t"
                "s_mov_b64 %0, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add_x2 %1, %2, off\n\t"
                "s_mov_b64 exec, %0"
                : "=&s"(saved_exec)
                : "v"(tk + 1), "v"(one)
                : "memory");
            __builtin_amdgcn_s_barrier();  // (1)
        } else {
            __builtin_amdgcn_s_barrier();  // (1) the data waves' weights have landed
            // the coherent (sc1) load of Z, lane 0 alone enabled, then the wait for it and the ticket
            unsigned long long zw;
            __asm__ volatile(
                "s_mov_b64 %2, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_load_dwordx2 %0, %3, off sc1\n\t"
                "s_mov_b64 exec, %2\n\t"
                "s_waitcnt vmcnt(0)"
                : "=&v"(zw), "+v"(old), "=&s"(saved_exec)
                : "v"(tk + 1)
                : "memory");
            // lane 0's values (the other lanes' registers were not written)
            const unsigned long long old0 =
                ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(old >> 32)) << 32) |
                (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)old);
            unsigned long long zw0 =
                ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(zw >> 32)) << 32) |
                (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)zw);
            const unsigned long long call1 = (old0 >> 6) + 1;
            if (lane == 0) {
                for (int n = 0; zw0 != call1 && n < kLineSpinLimit; ++n) {
                    __builtin_amdgcn_s_sleep(1);
                    zw0 = __hip_atomic_load(tk + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (zw0 != call1)
                    __hip_atomic_fetch_or(&g_line_fault_word, kFaultZeroWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __builtin_amdgcn_s_barrier();  // (2) the strip's outputs are zeroed for this call
        return;
    }

    // Activation fragments: lane (q, kb) feeds row 16 mg + q of m-group mg, activations 16 kb .. 16 kb
    // + 15 of each k-step.
    const int q = lane & 15, kb = lane >> 4;
    v4i a[MG][S];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
        for (int st = 0; st < S; ++st) a[mg][st] = v4i{0, 0, 0, 0};
    if constexpr (RG) {
        // 16 activations at an arbitrary address, from 4-byte aligned dwords; those past K (the next
        // row's or zeros) multiply the zero rows above.
        const uintptr_t a_hull = (reinterpret_cast<uintptr_t>(Ap) + (size_t)M * (size_t)K + 3) & ~uintptr_t(3);
#pragma unroll
        for (int mg = 0; mg < MG; ++mg)
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const int row = 16 * mg + q;
                const int k0 = (s0 + st) * 64 + kb * 16, v = st < nst && row < M ? min(16, K - k0) : 0;
                if (v > 0) {
                    const uintptr_t src = reinterpret_cast<uintptr_t>(Ap) + (size_t)row * (size_t)K + (size_t)k0;
                    const uintptr_t wa = src & ~uintptr_t(3);
                    const uint32_t b = (uint32_t)(src & 3) * 8u;
                    // as for the weights: one 16-byte load inside the rows' aligned extent
                    g_u32* w = (g_u32*)wa;
                    uint32_t d[5] = {0u, 0u, 0u, 0u, 0u};
                    if (wa + 16 <= a_hull) {  // as for the weights
                        const u4a x = *(g_u4a*)wa;
#pragma unroll
                        for (int u = 0; u < 4; ++u) d[u] = x[u];
                        if ((int)(b / 8) + v > 16) d[4] = w[4];
                    } else {
#pragma unroll
                        for (int u = 0; u < 5; ++u) d[u] = 4 * u < (int)(b / 8) + v ? w[u] : 0u;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        a[mg][st][u] = (int)(uint32_t)((((uint64_t)d[u + 1] << 32) | d[u]) >> b);
                }
            }
    } else if constexpr (AQ == 0) {
        const int8_t* arow = reinterpret_cast<const int8_t*>(Ap) + (size_t)min(q, M - 1) * (size_t)K + (size_t)s0 * 64 + kb * 16;
#pragma unroll
        for (int st = 0; st < S; ++st)
            if (st < nst && q < M) a[0][st] = *reinterpret_cast<const v4i*>(arow + st * 64);
    }
    TX_LGKMCNT0();  // AQ: the int8 rows are in LDS; RG: the weights' LDS writes
    TX_VMCNT(0);
    if constexpr (RG) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_barrier();  // (1) every data wave's weights are in LDS
    if constexpr (RG) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (AQ != 0) {
#pragma unroll
        for (int st = 0; st < S; ++st)
            if (st < nst && q < M) a[0][st] = *reinterpret_cast<const v4i*>(qbuf + q * (S * 64) + st * 64 + kb * 16);
    }

    v4i acc[MG][GW][4];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
        for (int gi = 0; gi < GW; ++gi)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[mg][gi][j] = v4i{0, 0, 0, 0};
    // Every fragment read of the unit first (two transposing reads per k-step and group), one wait,
    // then the decode and the MFMAs: the LDS latency is paid once, not once per k-step.
    const int r0 = kb * 16 + (q >> 1), r1 = r0 + 8;
    uint64_t lo[S][GW], hi[S][GW];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int gi = 0; gi < GW; ++gi) {
            const int g = wave * GW + gi;
            const uint8_t* base = lds + st * STEP + 8 * (q & 1);
            if (st < nst) {
                lo[st][gi] = lds_read_tr8(base + r0 * 128 + 16 * (g ^ line_swz(r0)));
                hi[st][gi] = lds_read_tr8(base + r1 * 128 + 16 * (g ^ line_swz(r1)));
            } else {
                lo[st][gi] = hi[st][gi] = 0;
            }
        }
    TX_LGKMCNT0();
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int gi = 0; gi < GW; ++gi) __asm__ volatile("" : "+v"(lo[st][gi]), "+v"(hi[st][gi]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < S; ++st) {
        if (st < nst) {
#pragma unroll
            for (int gi = 0; gi < GW; ++gi) {
                const uint32_t x4[4] = {(uint32_t)lo[st][gi], (uint32_t)(lo[st][gi] >> 32), (uint32_t)hi[st][gi],
                                        (uint32_t)(hi[st][gi] >> 32)};
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
                for (int mg = 0; mg < MG; ++mg)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[mg][gi][j] = mfma_i8(a[mg][st], bfr[j], acc[mg][gi][j]);
            }
        }
    }
    __builtin_amdgcn_s_barrier();  // (2) every wave is done with the stage buffers; C is zeroed
    __builtin_amdgcn_sched_barrier(0);

    // Epilogue: lane (q, kb) holds rows 4 kb + i (i < 4) of columns 4 (bc0 + 16 g + q) + j.  Each wave
    // lays a row's 64 outputs of a group out in column order in its own 256 bytes of the idle stage
    // buffer, then adds them to C:
    //   * int32 output: one column per lane, 64 consecutive int32 per atomic instruction;
    //   * EPI: the sums still scaled by 64 (the decode's factor), so their low 6 bits are free; lane l
    //     adds column pair l as one 64-bit integer (2^32 (odd column) + even column + 1) with a
    //     returning atomic.  The even column's low 6 bits count the splits added so far, and the
    //     64-bit sum is exact, so the split that sees splits - 1 there is the pair's last adder: it
    //     recovers both sums (even = (low half - splits) / 64, odd = (sum - low half) / 2^32 / 64) and
    //     writes the float output (dequantised, optionally the SwiGLU of the pair) -- no arrival
    //     counter and no second pass over the sums.
    int32_t* rb = reinterpret_cast<int32_t*>(lds) + wave * 64;
    float lm[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // EPI with amax_out: per row, the largest |value| this lane wrote
#pragma unroll
    for (int gi = 0; gi < GW; ++gi) {
        const int g = wave * GW + gi;
        if (bc0 + 16 * g >= NB) continue;  // wave-uniform
        const int col0 = 4 * (bc0 + 16 * g);  // the group's first column
        int32_t* out = Cp + col0 + lane;
        const bool in_row = !RG || col0 + lane < N;  // RG: a partial last group
#pragma unroll
        for (int mg = 0; mg < MG; ++mg)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 16 * mg + 4 * i4 + ii;
                if (i < M) {  // workgroup-uniform
                    if (kb == i4) {
                        const int sh = EPI ? 0 : 6;
                        const v4i v = {acc[mg][gi][0][ii] >> sh, acc[mg][gi][1][ii] >> sh, acc[mg][gi][2][ii] >> sh,
                                       acc[mg][gi][3][ii] >> sh};
                        *reinterpret_cast<v4i*>(rb + 4 * q) = v;
                    }
                    __builtin_amdgcn_wave_barrier();
                    if constexpr (EPI) {
                        const int32_t e = rb[2 * (lane & 31)], o = rb[2 * (lane & 31) + 1];
                        __builtin_amdgcn_wave_barrier();
                        const int c = col0 + 2 * lane;
                        if (lane < 32 && c < N) {
                            const unsigned long long add =
                                ((unsigned long long)(uint32_t)o << 32) + (unsigned long long)(long long)(e + 1);
                            unsigned long long* word = reinterpret_cast<unsigned long long*>(Cp + (size_t)i * (size_t)N + c);
                            const unsigned long long prev = __hip_atomic_fetch_add(word, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            if ((int)((uint32_t)prev & 63u) == splits_p - 1) {
                                const long long tot = (long long)(prev + add);
                                const int lo = (int)(uint32_t)tot;
                                const int ce = (lo - splits_p) >> 6;
                                const int co = (int)((tot - (long long)lo) >> 38);
                                const float f = (AQ != 0 ? rscale[i] : args.os.rs[i]) * args.os.ws;
                                const float mx = store_scaled_pair(args.os, f, i, N, c, ce, co);
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (r == i) lm[r] = fmaxf(lm[r], mx);
                            }
                        }
                    } else {
                        const int32_t v = rb[lane];
                        __builtin_amdgcn_wave_barrier();
                        if (in_row)
                            __hip_atomic_fetch_add(out + (size_t)i * (size_t)N, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
    }
    if constexpr (EPI) {
        if (args.amax_out != nullptr) {
            // The strip's largest |value| per row (M <= 4), for the consumer's quantisation: a maximum
            // over the pairs this wave finished, folded into the strip's entry (non-negative floats
            // order as their bit patterns).
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (r >= M) break;  // workgroup-uniform
                float m = lm[r];
                m = fmaxf(m, row_xor<8>(m, lane));
                m = fmaxf(m, row_xor<4>(m, lane));
                m = fmaxf(m, row_xor<2>(m, lane));
                m = fmaxf(m, row_xor<1>(m, lane));
                m = fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16))),
                          fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)),
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48))));
                if (lane == 0) wmax[wave * 4 + r] = m;
            }
            __syncthreads();  // the data waves only (the protocol wave has left)
            if (tid < M) {
                float m = 0.0f;
                for (int w = 0; w < NW; ++w) m = fmaxf(m, wmax[w * 4 + tid]);
                if (m > 0.0f)  // one atomic per workgroup and row: the strip's entry is shared by its splits
                    __hip_atomic_fetch_max(reinterpret_cast<unsigned int*>(args.amax_out) + (size_t)tid * amax_stride_p + s,
                                           __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

}  // namespace

bool line_gemv_ok(const int8_t* A, const uint8_t* B, int M, int K, int N) {
    const int NB = N / 4;
    return M >= 1 && M <= 16 && K >= 64 && K % 64 == 0 && N % 4 == 0 && NB % 16 == 0 && (uintptr_t)A % 16 == 0 &&
           (uintptr_t)B % 16 == 0 && (size_t)K * (size_t)NB < ((size_t)1 << 40);
}

bool line_gemv_ragged_ok(int M, int K, int N) {
    return M >= 1 && M <= 32 && K >= 1 && N >= 4 && N % 4 == 0 && (size_t)K * (size_t)(N / 4) < ((size_t)1 << 40);
}

int line_gemv_splits(int K, int S) { return ((K + 63) / 64 + S - 1) / S; }


hipError_t launch_line_gemv(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int S, int NW,
                            unsigned long long* tk, int tk_stride, hipStream_t st, const OutScale& os,
                            const ActQuant& aq, int xcd_chunks, int tiled) {
    const bool ragged = !line_gemv_ok(A, B, M, K, N);
    // tile-64 weights: aligned operands (K % 128, N % 256 by the layout's contract), 4 GiB at most
    if (tiled && (ragged || K % 128 != 0 || N % 256 != 0 || (size_t)K * (size_t)(N / 4) >= ((size_t)1 << 32)))
        return hipErrorInvalidValue;
    const bool epi = os.Y != nullptr;
    if ((ragged && (!line_gemv_ragged_ok(M, K, N) || epi || aq.mode != 0)) || tk == nullptr || C == nullptr ||
        (uintptr_t)C % 8 != 0 || (M > 4 && aq.mode != 0))
        return hipErrorInvalidValue;
    if (aq.mode != 0 && (!epi || M > 4 || (aq.mode != 3 && (size_t)M * (size_t)K > (size_t)kLineQK) ||
                         aq.X == nullptr || aq.rs_out == nullptr || (aq.mode == 2 && aq.G == nullptr) ||
                         (uintptr_t)aq.X % 16 != 0 || (aq.mode == 2 && (uintptr_t)aq.G % 16 != 0)))
        return hipErrorInvalidValue;
    if (aq.mode == 3 && (aq.amax_in == nullptr || (uintptr_t)aq.amax_in % 16 != 0 || aq.amax_n < 1 ||
                         aq.amax_stride < aq.amax_n || aq.amax_stride % 4 != 0 || M * aq.amax_stride * 4 > 8192))
        return hipErrorInvalidValue;
    if (aq.amax_out != nullptr && (!epi || M > 4 || aq.amax_stride < (N / 4 + 127) / 128))
        return hipErrorInvalidValue;
    if (epi && ((aq.mode == 0 && os.rs == nullptr) || (os.swiglu && N % 8 != 0) || K > 65536))
        return hipErrorInvalidValue;
    LineArgs a;
    a.A = A;
    a.B = B;
    a.C = C;
    a.M = M;
    a.K = K;
    a.N = N;
    a.strips = (N / 4 + 127) / 128;
    a.splits = line_gemv_splits(K, S);
    a.tk = tk;
    a.tk_stride = tk_stride;
    a.X = aq.X;
    a.G = aq.G;
    a.eps = aq.eps;
    a.rs_out = aq.rs_out;
    a.os = os;
    a.vec_y = epi && (uintptr_t)os.Y % 16 == 0;
    a.xcd_chunks = xcd_chunks;
    a.amax_out = aq.amax_out;
    a.amax_stride = aq.amax_stride;
    a.amax_in = aq.amax_in;
    a.amax_n = aq.amax_n;

    if (a.splits > 64 || a.strips > 0xFFFF || M > 255 || a.tk_stride > 63 || a.amax_stride > (1 << 25) ||
        (size_t)S * 64 > (size_t)kMaxKPerAccumulator)
        return hipErrorInvalidValue;
    const dim3 grid = xcd_chunks ? dim3((unsigned)(a.strips * a.splits)) : dim3((unsigned)a.strips, (unsigned)a.splits);
    // 0 int32 out, 1 dequantised, 2 / 3 / 4 with fused quantisation, 5 / 6 int32 out from ragged
    // operands in one / two 16-row groups
    const int mode = ragged ? (M > 16 ? 6 : 5) : (epi ? 1 + aq.mode : 0);
    const unsigned aux = (unsigned)a.tk_stride | ((unsigned)a.amax_stride << 6);
    const unsigned shape = (unsigned)a.strips | ((unsigned)a.splits << 16) | ((a.xcd_chunks ? 1u : 0u) << 23) |
                           ((unsigned)a.M << 24);
#define TX_LINE_ARGS a.B, aq.mode ? (const void*)a.X : (const void*)a.A, aq.mode == 3 ? (const void*)a.amax_in : (const void*)a.G, \
    a.C, a.tk, a.K, a.N, shape, aux, a
#define TX_LINE(SS, WW, AQQ, EE, RR)                                                                         \
    if (S == SS && NW == WW && mode == (RR ? 5 : (EE ? 1 + AQQ : 0))) {                                      \
        if (tiled)                                                                                           \
            hipLaunchKernelGGL((line_gemv_kernel<SS, WW, AQQ, EE, false, 1, true>), grid, dim3(64 * (WW + 1)), \
                               0, st, TX_LINE_ARGS);                                                         \
        else                                                                                                 \
            hipLaunchKernelGGL((line_gemv_kernel<SS, WW, AQQ, EE, RR>), grid, dim3(64 * (WW + 1)), 0, st,     \
                               TX_LINE_ARGS);                                                                \
        return hipGetLastError();                                                                            \
    }
#define TX_LINE_RG2(SS)                                                                                      \
    if (S == SS && NW == 8 && mode == 6) {                                                                   \
        hipLaunchKernelGGL((line_gemv_kernel<SS, 8, 0, false, true, 2>), grid, dim3(64 * 9), 0, st, TX_LINE_ARGS); \
        return hipGetLastError();                                                                            \
    }
#define TX_LINE_S(SS)                   \
    TX_LINE(SS, 8, 0, false, false)     \
    TX_LINE(SS, 8, 0, true, false)      \
    TX_LINE(SS, 8, 1, true, false)      \
    TX_LINE(SS, 8, 2, true, false)      \
    TX_LINE(SS, 8, 3, true, false)      \
    TX_LINE(SS, 8, 0, false, true)
    TX_LINE(1, 8, 0, false, false)
    TX_LINE_S(2)
    TX_LINE_S(3)
    TX_LINE_S(4)
    TX_LINE_S(6)
    TX_LINE_S(8)
    TX_LINE_RG2(2)  // two 16-row groups: up to 6 k-steps (8 would spill)
    TX_LINE_RG2(3)
    TX_LINE_RG2(4)
    TX_LINE_RG2(6)
    TX_LINE(2, 4, 0, false, false)
    TX_LINE(4, 4, 0, false, false)
#undef TX_LINE_S
#undef TX_LINE_RG2
#undef TX_LINE
#undef TX_LINE_ARGS
    return hipErrorInvalidValue;
}


hipError_t take_line_faults(unsigned* bits) {
    unsigned v = 0;
    hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_line_fault_word), sizeof(v), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    if (v != 0) {
        const unsigned zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_line_fault_word), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
    }
    *bits = v;
    return e;
}

}  // namespace ternix_hip
