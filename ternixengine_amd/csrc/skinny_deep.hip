// skinny_deep.hip -- gfx950 decode GEMV with the whole K range of a column strip in one workgroup,
// for weights in the tile-64 layout (kernel_common.h).
//
// The decode shapes (M <= 16 per m-group) are too small to fill 256 CUs unless K is split across
// workgroups, and a K split needs a cross-workgroup exchange: either a second (reduce) launch or
// partial sums published through memory plus a same-address arrival counter, each costing whole
// memory round trips after the last k-step.  This kernel has no exchange at all: a workgroup owns a
// strip of 16 bytes of every weight row (64 output columns) over the whole of K (or over a long
// k-range when the host does split, see below), and its NW waves (8 or 16, up to 1024 threads)
// take alternate 64-row k-steps.  On tile-64 weights a strip is one contiguous run of 1 KB blocks,
// so every request is for whole 128-byte lines and one CU streams its strip fast enough.  (On the
// row-major layout each row piece is 16 bytes of a 128-byte line: measured on MI355X the CU's
// request rate then caps it at a fraction of the bandwidth -- cfg2 up 7.6 us against 6.6 for the
// split wave kernel, cfg5 big 30 us against 15.6 -- so the automatic path never uses it there.)
// The waves  Every wave streams its own steps global -> LDS with
// global_load_lds_dwordx4 into a private ring of NSW slots and reads them back with the transposing
// ds_read_b64_tr_b8, so the k-loop has no workgroup barrier and NW * (NSW - 1) steps of weights are
// in flight per CU (up to ~112 KB: enough to cover HBM latency at a CU's share of the bandwidth).
// The waves' int32 sums meet once in LDS at the end and the workgroup writes C (optionally
// dequantised) with 16-byte stores.
//
// MFMA mapping and decode are those of the wave-pipelined kernel (kernel_common.h): lane
// (q = l % 16, kb = l / 16) receives byte-column q of k-rows 16 kb .. 16 kb + 15 of the step from
// two transposing reads, each dword splits into four B-operand dwords by the shift-form decode
// (64 * w per signed byte), and one v_mfma_i32_16x16x64_i8 per 2-bit field accumulates 16 output
// columns for the 16 rows of the m-group; the final >> 6 is exact.
//
// LDS layout of a slot (64 rows x 16 bytes): row r at 16-byte position r ^ 8 ((r / 16) % 2), which is
// the order of a tile-64 block, so the two 16-lane halves of a transposing read hit different banks.
//
// splits > 1 (k-ranges of steps_per_split steps): every workgroup writes its partial tile to
// P[split][M][N] and splitk_reduce_kernel, the next launch on the stream, sums them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernel_common.h"
#include "ternary_kernels.h"

namespace ternix_hip {
namespace {

struct DeepArgs {
    const int8_t* A;
    const uint8_t* B;
    int32_t* C;      // store target (splits == 1) or the partial slabs P (splits > 1)
    int M, K, N;
    int steps_per_split;
    int splits;
    int vec_store;   // C / os.Y is 16-byte aligned (always true for partial slabs)
    int n_out;       // splits == 1: C / os.Y has n_out <= N columns at pitch n_out (0: N)
    int tiled;       // W in the tile-64 layout (SW == 16 only): a step of the strip is one 1 KB block
    OutScale os;     // splits == 1: dequantised float output when os.Y is set
};

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 31] (the counter field must be an immediate).
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
    switch (n) {
#define TX_CASE(i) case i: TX_VMCNT(i); break;
        TX_CASE(0) TX_CASE(1) TX_CASE(2) TX_CASE(3) TX_CASE(4) TX_CASE(5) TX_CASE(6) TX_CASE(7)
        TX_CASE(8) TX_CASE(9) TX_CASE(10) TX_CASE(11) TX_CASE(12) TX_CASE(13) TX_CASE(14) TX_CASE(15)
        TX_CASE(16) TX_CASE(17) TX_CASE(18) TX_CASE(19) TX_CASE(20) TX_CASE(21) TX_CASE(22) TX_CASE(23)
        TX_CASE(24) TX_CASE(25) TX_CASE(26) TX_CASE(27) TX_CASE(28) TX_CASE(29) TX_CASE(30)
#undef TX_CASE
        default: TX_VMCNT(0); break;
    }
}

template <int NW, int NSW>
__global__ __launch_bounds__(64 * NW) void skinny_deep_kernel(DeepArgs args) {
    constexpr int SW = 16;                  // strip bytes per weight row
    constexpr int G = 1;                    // 16-byte column groups per strip
    constexpr int SLOT = 64 * SW;           // one k-step of the strip (1 KB)
    constexpr int VPS = 2;                  // vector memory instructions per step (DMA + activation)
    constexpr int RING = NW * NSW * SLOT;
    constexpr int RED = NW * G * 4 * 64 * 16;  // every wave's accumulators, 64 lanes
    static_assert((NSW - 1) * VPS <= 30, "vmcnt range");
    __shared__ __attribute__((aligned(16))) uint8_t lds[RING > RED ? RING : RED];

    const int M = args.M, K = args.K, NB = args.N >> 2;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane & 15, kb = lane >> 4;

    // Block -> (strip, split): consecutive numbers per XCD (the hardware deals block ids round-robin
    // to the 8 XCDs), so neighbouring strips, which share 128-byte lines of every weight row, are
    // fetched into one L2.
    const int n_strips = NB / SW;
    const int total = n_strips * args.splits;
    const int lin = xcd_linear(blockIdx.x, total);
    const int cx = lin % n_strips, sy = lin / n_strips;
    const int bc0 = cx * SW;
    const int m0 = blockIdx.z * 16;
    const int rows = min(16, M - m0);
    const int s_begin = sy * args.steps_per_split;
    const int nst = min(K >> 6, s_begin + args.steps_per_split) - s_begin;
    const int mine = wave < nst ? (nst - 1 - wave) / NW + 1 : 0;  // this wave's steps (wave-uniform)

    uint8_t* ring = lds + wave * NSW * SLOT;
    // DMA source of this lane: 16-byte position l of the slot holds row l ^ 8 ((l / 16) % 2).
    const uint32_t w_off = (uint32_t)(lane ^ (((lane >> 4) & 1) << 3)) * (uint32_t)NB + (uint32_t)bc0;
    const int8_t* a_row = args.A + (size_t)(m0 + min(q, rows - 1)) * (size_t)K + kb * 16;
    auto issue = [&](int it, int slot, v4i& a_dst) {
        const int s = s_begin + wave + NW * it;
        const uint8_t* src = args.tiled ? args.B + ((size_t)cx * (size_t)(K >> 6) + (size_t)s) * 1024 + lane * 16
                                        : args.B + (size_t)s * 64 * (size_t)NB + w_off;
        lds_dma16(src, ring + slot * SLOT);
        a_dst = *reinterpret_cast<const v4i*>(a_row + (size_t)s * 64);
    };
    // Transposing-read addresses: lane q reads byte-column q, rows 16 kb + q/2 (+ 8).
    uint32_t w_lo[G], w_hi[G];
    {
        const int r = kb * 16 + (q >> 1), r8 = r + 8;
        w_lo[0] = (uint32_t)((r ^ (((r >> 4) & 1) << 3)) * 16 + 8 * (q & 1));
        w_hi[0] = (uint32_t)((r8 ^ (((r8 >> 4) & 1) << 3)) * 16 + 8 * (q & 1));
    }

    v4i acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[g][j] = v4i{0, 0, 0, 0};

    v4i a_ring[NSW];
    int issued = 0;
#pragma unroll
    for (int p = 0; p < NSW; ++p)
        if (p < mine) {
            issue(p, p, a_ring[p]);
            ++issued;
        }
    for (int it0 = 0; it0 < mine; it0 += NSW) {
#pragma unroll
        for (int p = 0; p < NSW; ++p) {
            const int it = it0 + p;
            if (it < mine) {  // wave-uniform
                wait_vmcnt_dyn((issued - it - 1) * VPS);  // step `it` (DMAs and activation) has landed
                const uint32_t base = lds_u32(ring + p * SLOT);
                uint64_t lo[G], hi[G];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    lo[g] = lds_read_tr8_asm(base + w_lo[g]);
                    hi[g] = lds_read_tr8_asm(base + w_hi[g]);
                }
                TX_LGKMCNT0();  // the slot has been read: it may be refilled
#pragma unroll
                for (int g = 0; g < G; ++g) __asm__ volatile("" : "+v"(lo[g]), "+v"(hi[g]));
                const v4i a = a_ring[p];
                if (issued < mine) {
                    issue(issued, p, a_ring[p]);
                    ++issued;
                }
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

    // Sum the waves: every wave puts its accumulators (lanes holding valid rows only), then each
    // thread adds one (row, byte-column) over the waves and stores its four outputs.
    __syncthreads();  // all rings drained and read
    v4i* red = reinterpret_cast<v4i*>(lds);
    const bool low = rows <= 4;            // all rows in lanes 0-15 (rows 4 kb + i)
    const int nl = low ? 16 : 64;          // lanes stored per (wave, g, j)
    if (lane < nl) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) red[((wave * G + g) * 4 + j) * nl + lane] = acc[g][j];
    }
    __syncthreads();
    const int NO = (args.splits == 1 && args.n_out > 0) ? args.n_out : args.N;
    int32_t* out_base = args.C + (args.splits > 1 ? (size_t)sy * (size_t)M * (size_t)args.N : 0);
    const int32_t* redi = reinterpret_cast<const int32_t*>(lds);
    for (int idx = tid; idx < rows * SW; idx += 64 * NW) {
        const int row = idx / SW, bl = idx % SW;  // row of the m-group, byte-column of the strip
        const int g = bl >> 4, l = (bl & 15) + 16 * (row >> 2), i = row & 3;
        v4i v = {0, 0, 0, 0};
#pragma unroll 4
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] += redi[(((w * G + g) * 4 + j) * nl + l) * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] >>= 6;
        const int col = 4 * (bc0 + bl);
        if (col >= NO) continue;
        const int grow = m0 + row;
        if (args.splits == 1 && args.os.Y) {
            store_scaled(args.os, grow, NO, col, v, args.vec_store);
            continue;
        }
        const int pitch = args.splits > 1 ? args.N : NO;
        int32_t* out = out_base + (size_t)grow * (size_t)pitch + col;
        if (args.splits > 1 || args.vec_store) {
            *reinterpret_cast<v4i*>(out) = v;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) out[j] = v[j];
        }
    }
}

template <int NW, int NSW>
void launch_deep_t(const DeepArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((skinny_deep_kernel<NW, NSW>), grid, dim3(64 * NW), 0, st, a);
}

}  // namespace

bool skinny_deep_config_ok(int sw, int nw, int nsw) {
    return sw == 16 && (nw == 16 || nw == 8) && (nsw == 4 || nsw == 8);
}

bool skinny_deep_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int sw) {
    return M >= 1 && K >= 64 && K % 64 == 0 && (N / 4) % sw == 0 && N % 4 == 0 &&
           reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0 &&
           (size_t)K * (size_t)(N / 4) < ((size_t)1 << 32);
}

hipError_t launch_skinny_deep(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int sw, int nw,
                              int nsw, int splits, int steps_per_split, int32_t* partials, hipStream_t st,
                              const OutScale& os, int n_out, int tiled) {
    if (!skinny_deep_config_ok(sw, nw, nsw) || !skinny_deep_ok(A, B, M, K, N, sw) || splits < 1 ||
        steps_per_split < 1 || (long)steps_per_split * 64 > kMaxKPerAccumulator ||
        (long)(splits - 1) * steps_per_split >= K / 64 || (long)splits * steps_per_split < K / 64 ||
        (splits > 1 && (partials == nullptr || n_out > 0)))
        return hipErrorInvalidValue;
    DeepArgs a{};
    a.A = A;
    a.B = B;
    a.C = splits > 1 ? partials : C;
    a.M = M;
    a.K = K;
    a.N = N;
    a.steps_per_split = steps_per_split;
    a.splits = splits;
    a.n_out = n_out;
    a.tiled = tiled;
    if (splits == 1) a.os = os;
    const void* out = (splits == 1 && os.Y) ? static_cast<const void*>(os.Y) : static_cast<const void*>(a.C);
    a.vec_store = splits > 1 || reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const dim3 grid((unsigned)((N / 4 / sw) * splits), 1, (unsigned)((M + 15) / 16));
    if (nw == 16 && nsw == 4) launch_deep_t<16, 4>(a, grid, st);
    else if (nw == 16) launch_deep_t<16, 8>(a, grid, st);
    else if (nsw == 4) launch_deep_t<8, 4>(a, grid, st);
    else launch_deep_t<8, 8>(a, grid, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_splitk_reduce(partials, C, M, N, splits, os, st);
}

}  // namespace ternix_hip
