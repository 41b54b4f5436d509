// skinny_kernels.hip -- gfx950 GEMV / small-M kernels (M <= 32) for the ternary matmul: the
// wave-pipelined, DMA-staged and register-staged skinny kernels, their split-K reduce and launchers.
// Shared helpers, the weight layout and the decode forms are described in kernel_common.h.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "kernel_common.h"
#include "row_stats.h"
#include "ternary_kernels.h"

namespace ternix_hip {
namespace {

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
// inside one launch with device-scope release/acquire fences would write back and invalidate a whole
// L2 per workgroup on this multi-XCD part, and same-address device-scope atomics from several XCDs
// serialise at the memory side; the kernel boundary gives the ordering for free.  (SK_ATOMIC, used
// only when no workspace is available, accumulates into a pre-zeroed C instead; SK_LAST, below,
// exchanges through coherent stores and loads without fences, for the wave kernel's few splits.)
// LOW_M: at most 4 rows in this m-group, all held by lanes 0-15 (rows 4*kb + i of an MFMA tile), so
// only those lanes take part in the LDS exchange and the epilogue.
// ------------------------------------------------------------------------------------------------

constexpr int SK_WAVES = 4;
constexpr int kRowRegs = 32;  // fused activation quantisation: row elements per thread (K <= 8192)

// SK_LAST (skinny_wave_kernel only): every split stores its partial tile with agent-scope
// (L2 write-through) stores, waits for them, and counts itself on the tile's counter; the last
// split to arrive sums all partials of the tile (agent-scope loads) and writes C, then resets the
// counter.  No L2 writeback or invalidate is needed because only those coherent accesses touch the
// exchanged data, and no second launch is needed.
// SK_ATOMZ (skinny_wave_kernel only, one m-group): SK_ATOMIC without the fill launch.  Each strip
// has a 64-bit ticket counter and a 64-bit "zeroed" word that persist across calls.  Every split
// takes a ticket at its start (a returning add, issued after its first weight loads); each call
// uses one block of 64 ticket values per strip (the split holding the block's last ticket adds the
// rest of the block), so the first ticket of a call is a multiple of 64 and names the call.  The
// split that draws it zeroes the strip's outputs with coherent agent-scope stores, waits for them,
// and writes the call's number + 1 to the zeroed word; every other split checks that word before
// its atomics (it reads it with its last weight loads) and, if it is not there yet, waits:
// the split it waits for has already taken its ticket, so it is running and waits for nothing.
enum SkinnyMode { SK_STORE = 0, SK_ATOMIC = 1, SK_PARTIAL = 2, SK_LAST = 3, SK_ATOMZ = 4 };
// Bound of the SK_ATOMZ wait (each try is one memory round trip, so about a second): only a guard
// that every wave exits.
constexpr int kZeroSpinLimit = 1 << 20;

}  // namespace

// Device fault word of this library on each GPU: a wave whose bounded wait gives up ORs its bit in
// (kFaultZeroWait: the zeroed word of an SK_ATOMZ strip never arrived, so that split added into
// outputs that may not have been zeroed and the call's result is not trustworthy).  Read and cleared
// by take_faults (ternix_hip_take_faults); nothing else writes it.
__device__ unsigned int g_tx_fault_word;

namespace {

__device__ __forceinline__ void note_fault(unsigned bit) {
    __hip_atomic_fetch_or(&g_tx_fault_word, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The SK_ATOMZ wait of a non-zeroing split (one lane): re-read the strip's zeroed word until it holds
// this call's number, at most kZeroSpinLimit times; on giving up, record kFaultZeroWait.
__device__ __forceinline__ void wait_zeroed(unsigned long long* tk, unsigned long long zw, unsigned long long call1) {
    for (int n = 0; zw != call1 && n < kZeroSpinLimit; ++n) {
        __builtin_amdgcn_s_sleep(1);
        zw = __hip_atomic_load(tk + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (zw != call1) note_fault(kFaultZeroWait);
}

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
    int tiled;            // skinny_wave_kernel: W in the tile-64 layout (kernel_common.h)
    int* cnt;             // SK_LAST: arrival counters, one per (m-group, strip), zero between calls
    int order;            // SK_LAST: 1 = C++ release/acquire at agent scope, 0 = coherent accesses only
    unsigned long long* tick;  // SK_ATOMZ: per strip {ticket counter, zeroed word}, persistent
    int tk_stride;             // SK_ATOMZ: 64-bit words between consecutive strips' pairs (ticket_stride)
    int nt;               // DMA-staged / wave-pipelined kernels: non-temporal weight loads
    int defer_ticket;     // skinny_wave_kernel, SK_ATOMZ: wave 0 waits for its ticket with its first step
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
void skinny_dma_kernel(const uint8_t* Bp, const void* Ap, int32_t* Cp, unsigned long long* tkp, int Kp, int Np,
                                         int spsp, int tk_stride_p, unsigned flags_p, SkinnyArgs args) {
    // Leading scalars, preloaded into SGPRs by the command processor (SkinnyArgs holds the same
    // values): flags_p packs M (bits 0-7), splits (8-17), mode (18-20), nt (21), line_units (22),
    // defer_ticket (23), tiled (24) and order (25).
    const int f_M = (int)(flags_p & 0xFFu), f_splits = (int)((flags_p >> 8) & 0x3FFu);
    const int f_mode = (int)((flags_p >> 18) & 7u), f_nt = (int)((flags_p >> 21) & 1u);
    const int f_line = (int)((flags_p >> 22) & 1u), f_defer = (int)((flags_p >> 23) & 1u);
    const int f_tiled = (int)((flags_p >> 24) & 1u), f_order = (int)((flags_p >> 25) & 1u);
    (void)f_line; (void)f_defer; (void)f_tiled; (void)f_order; (void)f_nt;
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    __shared__ __attribute__((aligned(16))) uint8_t sW0[SD_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW1[SD_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sW2[NS > 2 ? SD_STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t sW3[NS > 3 ? SD_STAGE : 16];
    __shared__ __attribute__((aligned(16))) int8_t sA[NAD * 256 * 16];
    auto stage_w = [&](int i) -> uint8_t* { return i == 0 ? sW0 : (i == 1 ? sW1 : (i == 2 ? sW2 : sW3)); };

    const int8_t* __restrict__ A = reinterpret_cast<const int8_t*>(Ap);
    const uint8_t* __restrict__ B = Bp;
    const int M = f_M, K = Kp, NB = Np >> 2;
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
    const int s_begin = sy * spsp;
    const int nst = min(K >> 6, s_begin + spsp) - s_begin;  // >= 1 (planner)

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
    // SK_ATOMZ (as in skinny_wave_kernel): wave 0 takes the strip's ticket before any DMA; the
    // first loop wait of wave 0 (for a step issued after it) covers its return.
    const bool ticket = f_mode == SK_ATOMZ && wave == 0;
    unsigned long long* tk = tkp + (size_t)tk_stride_p * (size_t)cx;
    unsigned long long old = 0, call1 = 0, zw = 0;
    bool zeroer = false;
    if (ticket && lane == 0)
        __asm__ volatile("global_atomic_add_x2 %0, %1, %2, off sc0" : "=v"(old) : "v"(tk), "v"(1ull) : "memory");
    // After the first wait: learn the ticket; the strip's first split zeroes its 4 KB of C per row
    // (wave 0, coherent stores; they complete before the tail's full wait, which publishes them).
    auto take_ticket = [&]() {
        __asm__ volatile("" : "+v"(old));
        old = ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((int)(old >> 32)) << 32) |
              (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)old);
        const int rank = (int)(old & 63);
        call1 = (old >> 6) + 1;
        zeroer = rank == 0;
        if (rank == f_splits - 1 && f_splits < 64 && lane == 0)
            __hip_atomic_fetch_add(tk, (unsigned long long)(64 - f_splits), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (zeroer)
            for (int r = 0; r < a_rows; ++r) {
                unsigned long long* z =
                    reinterpret_cast<unsigned long long*>(Cp + (size_t)(m0 + r) * (size_t)Np + 4 * bc0);
                const int n8 = min(SD_BNB, NB - bc0) * 2;  // 8-byte units of this strip's outputs
                for (int u = lane; u < n8; u += 64)
                    __hip_atomic_store(z + u, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
    };
    // In the tail (after a full wait of every wave and a barrier): the zeroer publishes, the others
    // request the zeroed word.
    auto tail_ticket = [&]() {
        if (zeroer) {
            if (lane == 0) __hip_atomic_store(tk + 1, call1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (lane == 0) {
            zw = __hip_atomic_load(tk + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        if (f_nt) {
#pragma unroll
            for (int p = 0; p < SD_NL; ++p) lds_dma16_nt(wbase + w_off[p], wdst + (p * 4 + wave) * 1024);
        } else {
#pragma unroll
            for (int p = 0; p < SD_NL; ++p) lds_dma16(wbase + w_off[p], wdst + (p * 4 + wave) * 1024);
        }
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
        if (ticket && it == 0) take_ticket();
        issue(it + NS - 1, (it + NS - 1) % NS);
        step(it, it % NS);
        __builtin_amdgcn_sched_barrier(0);
    }
    const int tail0 = it;
    for (; it < nst; ++it) {
        TX_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (ticket) {
            if (it == 0) take_ticket();
            if (it == tail0) {
                if (it == 0) TX_VMCNT(0);  // a zeroer that took the ticket just now: its stores are complete
                tail_ticket();
            }
        }
        step(it, it % NS);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (f_mode == SK_ATOMZ) {
        // every wave's atomics wait until the strip is zeroed (wave 0 checks, the barrier spreads it)
        if (wave == 0 && !zeroer && lane == 0)
            wait_zeroed(tk, zw, call1);
        __syncthreads();
    }

    // Epilogue: lane (q, kb) holds rows 4kb+i of byte-columns bc0 + 16(4 wave + g) + q.
    if (LOW_M && f_mode == SK_ATOMZ) {
        // Few rows into C with atomics: each wave lays its row's 256 outputs out in column order in
        // its own 1 KB of the (now idle) stage buffer, then adds one column per lane per instruction
        // (64 consecutive int32 per atomic instruction, no per-element branch).  The barrier above
        // ended every wave's reads of the stage buffers.
        int32_t* row_lds = reinterpret_cast<int32_t*>(sW0) + wave * 256;
        const int rows = min(4, M - m0);
        const int col0 = bc0 + wave * 64;  // this wave's first byte-column
        for (int i = 0; i < rows; ++i) {
            if (kb == 0) {
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *reinterpret_cast<v4i*>(row_lds + (16 * g + q) * 4) =
                        v4i{acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            }
            __builtin_amdgcn_wave_barrier();
            int32_t vals[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) vals[u] = row_lds[64 * u + lane];
            int32_t* out = Cp + (size_t)(m0 + i) * (size_t)Np + 4 * col0;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (col0 + 16 * u + lane / 4 < NB) atomicAdd(out + 64 * u + lane, vals[u]);
            __builtin_amdgcn_wave_barrier();
            TX_LGKMCNT0();
        }
        return;
    }
    if (LOW_M && kb != 0) return;
    int32_t* out_base = f_mode == SK_PARTIAL ? args.P + (size_t)sy * (size_t)M * (size_t)Np : Cp;
    const bool vec = f_mode == SK_PARTIAL || args.vec_store;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 4 * kb + i;
        if (row >= M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int bcol = bc0 + (wave * 4 + g) * 16 + q;
            if (bcol >= NB) continue;
            const v4i v = {acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            if (f_mode == SK_STORE && args.os.Y) {
                store_scaled(args.os, row, Np, 4 * bcol, v, args.vec_store);
                continue;
            }
            int32_t* out = out_base + (size_t)row * (size_t)Np + 4 * bcol;
            if (f_mode == SK_ATOMIC || f_mode == SK_ATOMZ) {
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
// clamped, 16 bytes per lane) is loaded with the step's DMAs.  Narrow strips give many workgroups;
// the host splits K over a few more (blockIdx.x covers strip x split) and, for few splits, the
// splits are summed inside the launch (SK_LAST), so a decode GEMV is one launch.
//   * SW = 32: chunk c of row r at position c ^ ((r / 16) % 2) (the two 16-lane groups of a
//     transposing read use different banks); SW = 16: row r at position r ^ (8 ((r / 16) % 2)).
// Each wave issues its own steps only (the prologue's NSW-1 steps always, clamped past the range, no
// MFMAs for those); each wait names the number of steps issued after the one it waits for, one
// literal count per branch.
// ------------------------------------------------------------------------------------------------
template <int SW, int NSW, bool LOW_M, int AQ = 0, bool CW = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void skinny_wave_kernel(const uint8_t* Bp, const void* Ap, int32_t* Cp, unsigned long long* tkp, int Kp, int Np,
                                         int spsp, int tk_stride_p, unsigned flags_p, SkinnyArgs args) {
    // Leading scalars, preloaded into SGPRs by the command processor (SkinnyArgs holds the same
    // values): flags_p packs M (bits 0-7), splits (8-17), mode (18-20), nt (21), line_units (22),
    // defer_ticket (23), tiled (24) and order (25).
    const int f_M = (int)(flags_p & 0xFFu), f_splits = (int)((flags_p >> 8) & 0x3FFu);
    const int f_mode = (int)((flags_p >> 18) & 7u), f_nt = (int)((flags_p >> 21) & 1u);
    const int f_line = (int)((flags_p >> 22) & 1u), f_defer = (int)((flags_p >> 23) & 1u);
    const int f_tiled = (int)((flags_p >> 24) & 1u), f_order = (int)((flags_p >> 25) & 1u);
    (void)f_line; (void)f_defer; (void)f_tiled; (void)f_order; (void)f_nt;
    static_assert(SW == 16 || SW == 32, "16- or 32-byte strips");
    // CW (column waves, self-zeroing atomics at M <= 4 only): the workgroup owns a 4 * SW-byte strip
    // and wave w its w-th SW-byte part over every k-step of the range, so the four parts of each
    // weight line reach one CU together; each wave adds its own outputs (no cross-wave sum).
    static_assert(!CW || (AQ == 0 && LOW_M), "column waves: int32 atomics, M <= 4");
    constexpr int QK = 4096;                   // AQ: whole rows of K <= QK quantised into LDS
    constexpr int G = SW / 16;                 // 16-byte column groups per strip
    constexpr int SLOT = 64 * SW;              // bytes per ring slot (one k-step)
    constexpr int NL = SLOT / 1024;            // DMA instructions per step per wave
    constexpr int RED = 3 * 64 * 16 * G * 4;   // cross-wave reduction buffer (waves 1-3)
    constexpr int RING = 4 * NSW * SLOT;
    __shared__ __attribute__((aligned(16))) uint8_t lds[RING > RED ? RING : RED];
    __shared__ __attribute__((aligned(16))) int8_t qbuf[AQ ? 16 : 1][AQ ? QK : 16];
    __shared__ float rscale[16];

    const int8_t* __restrict__ A = reinterpret_cast<const int8_t*>(Ap);
    const uint8_t* __restrict__ B = Bp;
    const int M = f_M, K = Kp, NB = Np >> 2;
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
    const int n_cw = (NB + 4 * SW - 1) / (4 * SW);  // CW: 4*SW-byte strips (the last may be partial)
    int c4 = 0;
    bool part_ok = true;  // CW: this wave's part lies inside the matrix
    if (CW) {
        const int total = n_cw * f_splits;
        if ((int)blockIdx.x >= total) return;
        const int lin = xcd_linear(blockIdx.x, total);
        c4 = lin % n_cw;
        sy = lin / n_cw;
        part_ok = c4 * 4 + wave < n_strips;
        cx = min(c4 * 4 + wave, n_strips - 1);  // a part past the last column re-reads the last one
    } else if (f_line) {
        const int b = blockIdx.x, t = b >> 3;
        const int u = (b & 7) + 8 * (t / SPL);  // unit: (split, line group)
        sy = u / lines;
        cx = (u % lines) * SPL + t % SPL;
        if (sy >= f_splits || cx >= n_strips) return;  // whole workgroup: no barrier reached yet
    } else {
        // contiguous strip ranges per XCD (balanced; lines at range ends are fetched by two L2s)
        const int total = n_strips * f_splits;
        if ((int)blockIdx.x >= total) return;
        const int lin = xcd_linear(blockIdx.x, total);
        cx = lin % n_strips;
        sy = lin / n_strips;
    }
    const int bc0 = cx * SW;
    const int m0 = blockIdx.z * 16;
    const int s_begin = sy * spsp;
    const int nst = min(K >> 6, s_begin + spsp) - s_begin;  // >= 1
    const int nreal = CW ? nst : (nst > wave ? (nst - wave + 3) / 4 : 0);    // this wave's k-steps
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
        const int s = CW ? min(s_begin + it, s_last) : min(s_begin + wave + 4 * it, s_last);
        uint8_t* dst = ring + slot_c * SLOT;
        if (SW == 16 && f_tiled) {  // one contiguous 1 KB block, already in LDS order
            lds_dma16(B + ((size_t)cx * (size_t)(K >> 6) + (size_t)s) * 1024 + lane * 16, dst);
        } else {
            const uint8_t* wbase = B + (size_t)s * 64 * (size_t)NB;
            if (f_nt) {
#pragma unroll
                for (int p = 0; p < NL; ++p) lds_dma16_nt(wbase + w_off[p], dst + p * 1024);
            } else {
#pragma unroll
                for (int p = 0; p < NL; ++p) lds_dma16(wbase + w_off[p], dst + p * 1024);
            }
        }
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

    // SK_ATOMZ: ticket (wave 0; the other waves never touch C), requested before the first weight
    // loads and waited for after them (the vmcnt wait below counts them), so that waiting for it
    // does not wait for them.  Written as one instruction so that the compiler neither rewrites the
    // single-lane atomic nor places its own wait for the result right after it.
    unsigned long long call1 = 0;  // this call's number + 1, as the zeroer writes it
    bool zeroer = false;
    // Atomic modes: C has CN columns at pitch CN (a padded problem's real columns when n_out > 0)
    const int CN = args.n_out > 0 ? args.n_out : Np;
    // one ticket pair per (m-group, strip)
    unsigned long long* tk = CW ? tkp + (size_t)tk_stride_p * ((size_t)blockIdx.z * (size_t)n_cw + (size_t)c4)
                                : tkp + (size_t)tk_stride_p * ((size_t)blockIdx.z * (size_t)n_strips + (size_t)cx);
    unsigned long long old = 0;
    const bool ticket = AQ == 0 && f_mode == SK_ATOMZ && wave == 0;
    if (ticket && lane == 0)
        __asm__ volatile("global_atomic_add_x2 %0, %1, %2, off sc0" : "=v"(old) : "v"(tk), "v"(1ull) : "memory");
#pragma unroll
    for (int p = 0; p < NSW - 1; ++p) issue(p, p, a_ring[p]);
    // The ticket is learnt either right after the prologue (its own wait) or, with defer_ticket, in
    // the first loop step, whose wait covers it (it is older than step 0), so that wave 0 issues one
    // more weight step before it waits for the atomic's round trip.
    auto take_ticket = [&]() {
        __asm__ volatile("" : "+v"(old));
        old = ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((int)(old >> 32)) << 32) |
              (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)old);
        const int rank = (int)(old & 63);
        call1 = (old >> 6) + 1;
        zeroer = rank == 0;
        if (rank == f_splits - 1 && f_splits < 64 && lane == 0)
            __hip_atomic_fetch_add(tk, (unsigned long long)(64 - f_splits), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (zeroer) {
            // rows m0 .. m0 + a_rows - 1, the strip's columns (4 * SW, or 16 * SW with CW): 8 bytes a lane
            constexpr int ZB = CW ? 4 * SW : SW;  // strip bytes per row
            const int zb0 = CW ? c4 * 4 * SW : bc0;
            for (int r = 0; r < a_rows; ++r) {
                for (int u = lane; u < ZB * 2; u += 64) {
                    if (4 * zb0 + 2 * u < CN) {
                        unsigned long long* z =
                            reinterpret_cast<unsigned long long*>(Cp + (size_t)(m0 + r) * (size_t)CN + 4 * zb0) + u;
                        __hip_atomic_store(z, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(0);  // the zeroes are stored, coherent at agent scope
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (lane == 0) __hip_atomic_store(tk + 1, call1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    if (ticket && !f_defer) {
        TX_VMCNT((NSW - 1) * (NL + 1));  // the ticket has returned (the weight loads may not have)
        take_ticket();
    }
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
    // SK_ATOMZ: the zeroed word, read in wave 0's last step (wave 0 has the most steps); the full wait
    // after the loop covers it
    unsigned long long zw = 0;
    // Only the wave's own steps are issued (the prologue's NSW-1 always, clamped): each iteration
    // waits for its step with a count of the steps issued after it, a literal in each branch.
    for (int it0 = 0; it0 < nreal; it0 += NSW) {
#pragma unroll
        for (int p = 0; p < NSW; ++p) {
            const int it = it0 + p;
            if (it >= nreal) break;  // wave-uniform
            if (it + NSW - 1 < nreal) issue(it + NSW - 1, (p + NSW - 1) % NSW, a_ring[(p + NSW - 1) % NSW]);
            const int later = max(NSW - 1, min(nreal, it + NSW)) - it - 1;  // steps issued after `it`
            if (later >= NSW - 1) TX_VMCNT((NSW - 1) * VPS);  // step `it` (DMAs, activation load) has landed
            else if (later == 2) TX_VMCNT(2 * VPS);
            else if (later == 1) TX_VMCNT(VPS);
            else TX_VMCNT(0);
            if (ticket && f_defer && it == 0) take_ticket();  // the older ticket has too
            if (ticket && !zeroer && it == nreal - 1 && lane == 0)
                zw = __hip_atomic_load(tk + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            {
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
    TX_VMCNT(0);  // every DMA into the ring (and the zeroed word) has landed before the ring is reused

    if constexpr (CW) {
        // Column waves: wave 0 waits until the strip is zeroed, the barrier spreads it, then each wave
        // adds its own part's outputs (row by row, 64 consecutive int32 per atomic instruction) from
        // its own 512 bytes of LDS (the ring is idle: every wave's DMAs have landed).
        if (!zeroer && wave == 0 && lane == 0)
            wait_zeroed(tk, zw, call1);
        __syncthreads();
        if (!part_ok) return;
        int32_t* row_lds = reinterpret_cast<int32_t*>(lds) + wave * 4 * SW;
        const int rows = min(4, M - m0);
        for (int i = 0; i < rows; ++i) {
            if (kb == 0) {
#pragma unroll
                for (int g = 0; g < G; ++g)
                    *reinterpret_cast<v4i*>(row_lds + (16 * g + q) * 4) =
                        v4i{acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            }
            __builtin_amdgcn_wave_barrier();
            int32_t vals[G];
#pragma unroll
            for (int u = 0; u < G; ++u) vals[u] = row_lds[64 * u + lane];
            int32_t* out = Cp + (size_t)(m0 + i) * (size_t)CN + 4 * bc0;
#pragma unroll
            for (int u = 0; u < G; ++u)
                if (4 * bc0 + 64 * u + lane < CN) atomicAdd(out + 64 * u + lane, vals[u]);
            __builtin_amdgcn_wave_barrier();
            TX_LGKMCNT0();
        }
        return;
    }
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
    if (wave != 0 && f_mode != SK_LAST) return;
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < 3; ++w) {
            const v4i* r = reinterpret_cast<const v4i*>(lds) + w * 64 * 4 * G;
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[g][j] += r[(g * 4 + j) * 64 + lane];
        }
    }
    if (f_mode == SK_LAST) {
        __shared__ int s_last;
        const size_t MN = (size_t)M * (size_t)Np;
        int* counter = args.cnt + (size_t)blockIdx.z * (size_t)n_strips + cx;
        if (wave == 0) {
            int32_t* mine = args.P + (size_t)sy * MN;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + 4 * kb + i;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if ((LOW_M && kb != 0) || row >= M) continue;
                    int32_t* out = mine + (size_t)row * (size_t)Np + 4 * (bc0 + 16 * g + q);
                    if (f_order) {
                        *reinterpret_cast<v4i*>(out) =
                            v4i{acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
                        continue;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        __hip_atomic_store(out + j, acc[g][j][i] >> 6, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (!f_order) {
                __builtin_amdgcn_s_waitcnt(0);  // the partial stores are complete, coherent at agent scope
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                if (lane == 0)
                    s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                             f_splits - 1;
            }
        }
        if (f_order) {
            // Release/acquire form: the barrier orders every partial store of the workgroup before
            // thread 0's agent-scope release, and its acquire (with the barrier after it) orders the
            // last arriver's loads after every other split's release.
            __syncthreads();
            if (tid == 0)
                s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                         f_splits - 1;
        }
        __syncthreads();
        if (!s_last) return;  // workgroup-uniform
        // Last arrival: the whole workgroup sums the tile's partials (its own included) over all
        // splits, eight splits' loads in flight at a time (indices clamped: the loads are unconditional).
        const int rows = min(16, M - m0);
        for (int idx = tid; idx < rows * SW; idx += 256) {
            const int row = m0 + idx / SW, col = 4 * (bc0 + idx % SW);
            const size_t off = (size_t)row * (size_t)Np + col;
            v4i v = {0, 0, 0, 0};
            for (int c0 = 0; c0 < f_splits; c0 += 8) {
                uint64_t lo[8], hi[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint64_t* src =
                        reinterpret_cast<const uint64_t*>(args.P + (size_t)min(c0 + u, f_splits - 1) * MN + off);
                    lo[u] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    hi[u] = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (c0 + u >= f_splits) continue;
                    v[0] += (int)(uint32_t)lo[u];
                    v[1] += (int)(uint32_t)(lo[u] >> 32);
                    v[2] += (int)(uint32_t)hi[u];
                    v[3] += (int)(uint32_t)(hi[u] >> 32);
                }
            }
            if (args.os.Y) {
                store_scaled(args.os, row, Np, col, v, args.vec_store);
            } else if (args.vec_store) {
                *reinterpret_cast<v4i*>(Cp + off) = v;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) Cp[off + j] = v[j];
            }
        }
        if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (AQ == 0 && f_mode == SK_ATOMZ && !zeroer) {  // wave 0: wait until the strip is zeroed
        if (lane == 0)
            wait_zeroed(tk, zw, call1);
        __builtin_amdgcn_wave_barrier();
    }
    if (LOW_M && AQ == 0 && (f_mode == SK_ATOMIC || f_mode == SK_ATOMZ)) {
        // Few rows: wave 0 lays each row's 4 * SW outputs out in LDS in column order (lane q of
        // group g holds columns 4 (16 g + q) + j), then every lane adds one column per instruction:
        // 64 consecutive int32 per atomic instruction, no per-element branch.  The LDS area is the
        // reduction buffer this wave alone has just read.
        int32_t* row_lds = reinterpret_cast<int32_t*>(lds);
        const int rows = min(4, M - m0);
        for (int i = 0; i < rows; ++i) {
            if (kb == 0) {
#pragma unroll
                for (int g = 0; g < G; ++g)
                    *reinterpret_cast<v4i*>(row_lds + (16 * g + q) * 4) =
                        v4i{acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            }
            __builtin_amdgcn_wave_barrier();
            int32_t vals[G];
#pragma unroll
            for (int u = 0; u < G; ++u) vals[u] = row_lds[64 * u + lane];
            int32_t* out = Cp + (size_t)(m0 + i) * (size_t)CN + 4 * bc0;
#pragma unroll
            for (int u = 0; u < G; ++u)
                if (4 * bc0 + 64 * u + lane < CN) atomicAdd(out + 64 * u + lane, vals[u]);
            __builtin_amdgcn_wave_barrier();  // the reads are issued before the next row's writes
            TX_LGKMCNT0();
        }
        return;
    }
    if (!LOW_M && AQ == 0 && f_mode == SK_ATOMZ) {
        // Up to 16 rows: wave 0 lays every row's 4 * SW outputs out in LDS in column order (row r at
        // r * 4 * SW; lane (q, kb) holds rows 4 kb + i), then adds one column per lane per instruction,
        // row by row: 64 consecutive int32 per atomic instruction.  The LDS area is the reduction
        // buffer this wave alone has just read.
        int32_t* row_lds = reinterpret_cast<int32_t*>(lds);
        const int rows = min(16, M - m0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * kb + i;
            if (r < rows) {
#pragma unroll
                for (int g = 0; g < G; ++g)
                    *reinterpret_cast<v4i*>(row_lds + r * 4 * SW + (16 * g + q) * 4) =
                        v4i{acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            }
        }
        __builtin_amdgcn_wave_barrier();
        for (int r = 0; r < rows; ++r) {
            int32_t* out = Cp + (size_t)(m0 + r) * (size_t)CN + 4 * bc0;
#pragma unroll
            for (int u = 0; u < G; ++u)
                if (4 * bc0 + 64 * u + lane < CN) atomicAdd(out + 64 * u + lane, row_lds[r * 4 * SW + 64 * u + lane]);
        }
        return;
    }
    if (LOW_M && kb != 0) return;
    int32_t* out_base = f_mode == SK_PARTIAL ? args.P + (size_t)sy * (size_t)M * (size_t)Np : Cp;
    const bool vec = f_mode == SK_PARTIAL || args.vec_store;
    // Store mode writes n_out columns at pitch n_out (a padded problem's real columns).
    const int NO = (f_mode == SK_STORE && args.n_out > 0) ? args.n_out : Np;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 4 * kb + i;
        if (row >= M) continue;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int bcol = bc0 + 16 * g + q;
            if (4 * bcol >= NO) continue;
            const v4i v = {acc[g][0][i] >> 6, acc[g][1][i] >> 6, acc[g][2][i] >> 6, acc[g][3][i] >> 6};
            if (f_mode == SK_STORE && args.os.Y) {
                if constexpr (AQ != 0) store_scaled_f(args.os, rscale[row - m0] * args.os.ws, row, NO, 4 * bcol, v, args.vec_store);
                else store_scaled(args.os, row, NO, 4 * bcol, v, args.vec_store);
                continue;
            }
            int32_t* out = out_base + (size_t)row * (size_t)NO + 4 * bcol;
            if (f_mode == SK_ATOMIC || f_mode == SK_ATOMZ) {
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

// C[m][n] = sum over splits of P[s][m][n] (int32: exact in any order).  Thread t of workgroup b owns
// the kReduceU groups of four outputs b * 256 kReduceU + t + 256 u and adds every split's 16 bytes
// of each, eight splits' loads in flight at a time (read once: non-temporal loads).  The launcher
// takes the largest kReduceU in {4, 2, 1} that still gives every CU a workgroup (on MI355X, cold:
// 256x16384x4096 in 8 splits 29.2 -> 26.3 us against one group per thread and 64 per workgroup).
// P: [splits][M][n_in] int32 (slab stride slab4 16-byte units); C / os.Y: M x N (N <= n_in: the
// columns past N of a padded problem are dropped).
template <int kReduceU>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const int32_t* __restrict__ P, int32_t* __restrict__ C,
                                                            size_t n4, int splits, int vec_store, OutScale os,
                                                            int N, int n_in, size_t slab4) {
    const size_t base = (size_t)blockIdx.x * (256 * kReduceU) + threadIdx.x;
    const v4i* src = reinterpret_cast<const v4i*>(P);
    size_t si[kReduceU];
    v4i sum[kReduceU];
#pragma unroll
    for (int u = 0; u < kReduceU; ++u) {
        const size_t i = base + 256 * (size_t)u, ic = i < n4 ? i : n4 - 1;
        si[u] = n_in == N ? ic : (4 * ic / (size_t)N) * (size_t)(n_in / 4) + (4 * ic % (size_t)N) / 4;
        sum[u] = v4i{0, 0, 0, 0};
    }
    for (int s0 = 0; s0 < splits; s0 += 8) {
        v4i v[8][kReduceU];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int u = 0; u < kReduceU; ++u)
                v[j][u] = s0 + j < splits ? __builtin_nontemporal_load(src + (size_t)(s0 + j) * slab4 + si[u])
                                          : v4i{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int u = 0; u < kReduceU; ++u) sum[u] += v[j][u];
    }
#pragma unroll
    for (int u = 0; u < kReduceU; ++u) {
        const size_t i = base + 256 * (size_t)u;
        if (i >= n4) continue;
        if (os.Y) {
            const size_t e = 4 * i;  // N % 4 == 0: the four outputs share a row
            store_scaled(os, (int)(e / (size_t)N), N, (int)(e % (size_t)N), sum[u], vec_store);
        } else if (vec_store) {
            reinterpret_cast<v4i*>(C)[i] = sum[u];
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) C[4 * i + j] = sum[u][j];
        }
    }
}

void launch_reduce(const int32_t* P, int32_t* C, size_t n4, int splits, int vec_store, const OutScale& os, int N,
                   int n_in, size_t slab4, hipStream_t st) {
    const size_t cu = 256;  // workgroups wanted at least: one per CU of the chip
    const int u = n4 >= cu * 256 * 4 ? 4 : (n4 >= cu * 256 * 2 ? 2 : 1);
    const dim3 grid((unsigned)((n4 + 256 * (size_t)u - 1) / (256 * (size_t)u)));
    if (u == 4) hipLaunchKernelGGL(splitk_reduce_kernel<4>, grid, dim3(256), 0, st, P, C, n4, splits, vec_store, os, N, n_in, slab4);
    else if (u == 2) hipLaunchKernelGGL(splitk_reduce_kernel<2>, grid, dim3(256), 0, st, P, C, n4, splits, vec_store, os, N, n_in, slab4);
    else hipLaunchKernelGGL(splitk_reduce_kernel<1>, grid, dim3(256), 0, st, P, C, n4, splits, vec_store, os, N, n_in, slab4);
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

// The leading scalar arguments of skinny_dma_kernel / skinny_wave_kernel (see their flags_p).
unsigned sk_flags(const SkinnyArgs& a) {
    return (unsigned)a.M | ((unsigned)a.splits << 8) | ((unsigned)a.mode << 18) | ((a.nt ? 1u : 0u) << 21) |
           ((a.line_units ? 1u : 0u) << 22) | ((a.defer_ticket ? 1u : 0u) << 23) | ((a.tiled ? 1u : 0u) << 24) |
           ((a.order ? 1u : 0u) << 25);
}
#define TX_SK_ARGS(a) \
    (a).B, (const void*)(a).A, (a).C, (a).tick, (a).K, (a).N, (a).steps_per_split, (a).tk_stride, sk_flags(a), (a)

template <int NS, bool LOW_M, int AQ = 0>
void launch_dma_ns(const SkinnyArgs& a, dim3 grid, hipStream_t st) {
    const int sps = a.steps_per_split;
    if (sps <= 4) hipLaunchKernelGGL((skinny_dma_kernel<NS, 1, LOW_M, AQ>), grid, dim3(256), 0, st, TX_SK_ARGS(a));
    else if (sps <= 8) hipLaunchKernelGGL((skinny_dma_kernel<NS, 2, LOW_M, AQ>), grid, dim3(256), 0, st, TX_SK_ARGS(a));
    else hipLaunchKernelGGL((skinny_dma_kernel<NS, 4, LOW_M, AQ>), grid, dim3(256), 0, st, TX_SK_ARGS(a));
}

// Fused activation quantisation (aq 1 or 2) runs with 3 stages only.
hipError_t launch_dma(const SkinnyArgs& a, dim3 grid, int ns, int aq, hipStream_t st) {
    if (a.M > 255 || a.splits > 1023) return hipErrorInvalidValue;  // the packed leading scalars
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

}  // namespace

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
                         const ActQuant& aq, int dma_ns, int n_out, unsigned long long* tickets) {
    const int NB = N >> 2;
    int mode = splits <= 1 ? SK_STORE : (partials ? SK_PARTIAL : SK_ATOMIC);
    if (n_out > 0 && (mode != SK_PARTIAL || n_out > N || n_out % 4 != 0)) return hipErrorInvalidValue;
    if (mode == SK_ATOMIC && C == nullptr) return hipErrorInvalidValue;  // scaled call without int scratch
    if (aq.mode != 0 && !skinny_short_ok(B, M, K, N, steps_per_split, splits)) return hipErrorInvalidValue;
    // Self-zeroing atomics: DMA-staged kernel (also with fused activation quantisation), one m-group,
    // C rows 8-byte aligned, at most 64 splits.
    if (mode == SK_ATOMIC && tickets && dma_ns > 0 && M <= 16 && splits <= 64 &&
        (uintptr_t)C % 8 == 0 && N % 2 == 0)
        mode = SK_ATOMZ;
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
    a.tick = tickets;
    // Non-temporal weight loads for the DMA-staged kernel on matrices larger than the L2s together
    // (measured on MI355X, cold weights, cfg5 big 1x8192x28672: 13.35 -> 12.61 us; on the small
    // decode matrices, whose lines neighbouring strips share through L2, plain loads are faster).
    a.nt = debug_get(DBG_NT, 0) >= 0 ? debug_get(DBG_NT, 0) == 1 : (size_t)K * (size_t)NB >= (size_t(32) << 20);
    const int mt = M <= 16 ? 1 : 2;
    const int mgroups = (M + 16 * mt - 1) / (16 * mt);
    hipError_t e;
    const bool no_short = debug_get(DBG_SKINNY_SHORT) == 0;
    if (dma_ns != 0 && (!skinny_dma_aq_ok(aq.mode, K, splits) || dma_ns < 2 || dma_ns > 4 ||
                        !skinny_dma_ok(A, B, M, K, N, steps_per_split)))
        return hipErrorInvalidValue;
    if (dma_ns != 0) {
        const dim3 grid((NB + SD_BNB - 1) / SD_BNB, splits, mgroups);
        a.tk_stride = ticket_stride(grid.x);
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
        // One 16-row m-group per workgroup at every M (two row tiles per wave would need more than
        // the 256 VGPRs and spill).
        const dim3 grid((NB + 127) / 128, splits, (M + 15) / 16);
        if (M <= 4) e = launch_generic<1, true>(a, grid, st);
        else e = launch_generic<1, false>(a, grid, st);
    }
    if (e != hipSuccess) return e;
    if ((mode == SK_ATOMIC || mode == SK_ATOMZ) && scaled) return launch_dequant(C, os, M, N, st);  // C: alias of os.Y or scratch
    if (mode != SK_PARTIAL) return e;
    const size_t n4 = (size_t)M * (size_t)N / 4;
    const int n_c = n_out > 0 ? n_out : N;
    const size_t n4c = (size_t)M * (size_t)n_c / 4;
    const int vec_c = n_out > 0 ? ((uintptr_t)(scaled ? (const void*)os.Y : (const void*)C) % 16) == 0 : vec_store;
    launch_reduce(partials, C, n4c, splits, vec_c, os, n_c, N, n4, st);
    return hipGetLastError();
}

bool skinny_wave_ok(const int8_t* A, const uint8_t* B, int M, int K, int N, int sw) {
    const int NB = N >> 2;
    return M <= 64 && (sw == 16 || sw == 32) && K % 64 == 0 && NB % sw == 0 && (uintptr_t)B % 16 == 0 &&
           (uintptr_t)A % 16 == 0 && NB < (1 << 26);
}

hipError_t launch_skinny_wave(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int sw, int nsw,
                              int splits, int steps_per_split, int32_t* partials, hipStream_t st, const OutScale& os,
                              int n_out, const ActQuant& aq, int tiled, int* counters, unsigned long long* tickets, int column_waves) {
    if (tiled && (sw != 16 || n_out > 0)) return hipErrorInvalidValue;
    if (!skinny_wave_ok(A, B, M, K, N, sw) || nsw < 2 || nsw > 4 || steps_per_split < 1) return hipErrorInvalidValue;
    // Fused activation quantisation: one launch over whole rows (K <= 4096), 16-byte strips, 2 slots.
    if (aq.mode != 0 && (splits != 1 || K > 4096 || sw != 16 || nsw != 2 || n_out > 0 || aq.X == nullptr ||
                         aq.rs_out == nullptr || (aq.mode == 2 && aq.G == nullptr)))
        return hipErrorInvalidValue;
    const int NB = N >> 2;
    int mode = splits <= 1 ? SK_STORE : (partials ? SK_PARTIAL : SK_ATOMIC);
    if (mode == SK_PARTIAL && counters && n_out == 0 && aq.mode == 0) mode = SK_LAST;
    if (mode == SK_ATOMIC && C == nullptr) return hipErrorInvalidValue;
    // Self-zeroing atomics: up to four m-groups (tickets for m-groups x strips), C rows 8-byte aligned,
    // at most 64 splits; C may hold only the n_out real columns of a padded problem.
    if (mode == SK_ATOMIC && tickets && M <= 64 && aq.mode == 0 && splits <= 64 && (uintptr_t)C % 8 == 0 &&
        N % 2 == 0)
        mode = SK_ATOMZ;
    if (n_out > 0 && (mode == SK_ATOMIC || n_out > N || n_out % 4 != 0)) return hipErrorInvalidValue;
    if (mode == SK_ATOMIC) {
        const hipError_t e = launch_zero(C, (size_t)M * (size_t)N, st);
        if (e != hipSuccess) return e;
    }
    const bool scaled = os.Y != nullptr;
    const int vec_store = ((uintptr_t)(scaled ? (const void*)os.Y : (const void*)C) % 16) == 0;
    SkinnyArgs a{A, B, C, partials, M, K, N, steps_per_split, splits, mode, vec_store, 1, 1,
                 (mode == SK_STORE || mode == SK_LAST) ? os : OutScale{}};
    a.cnt = counters;
    a.tick = tickets;
    // Deferred ticket wait for k-ranges of 9 or more steps (measured on MI355X, cold weights, us:
    // cfg2 up 5.58 -> 5.42, down 5.75 -> 5.67, 4x11008x4096 8.70 -> 8.44, 16x11008x4096 9.55 -> 9.26);
    // with shorter ones the zeroing split's publish, which then also waits for the extra step, is
    // on the critical path (1x2560x2560, 7 steps: 3.93 -> 4.31).
    a.defer_ticket = debug_get(DBG_WAVE_TICKET) >= 0 ? debug_get(DBG_WAVE_TICKET) == 1 : steps_per_split >= 9;
    a.nt = debug_get(DBG_NT, 1) == 1;  // plain loads unless forced (slower here on every decode shape measured)
    a.order = debug_get(DBG_SK_ORDER) == 1;
    a.n_out = n_out;
    a.tiled = tiled;
    a.X = aq.X;
    a.G = aq.G;
    a.eps = aq.eps;
    a.rs_out = aq.rs_out;
    // Line units: 8 XCDs x (128 / sw) strips x enough rounds for every (split, line-group) unit.
    // Measured on MI355X (cold weights): line units help the one-launch shapes (cfg1 5.76 -> 5.24 us,
    // cfg2 up 6.75 -> 6.5, ragged 17x4093x1028 13.1 -> 11.5) and cost 2 % with a K split.
    a.line_units = (splits == 1);
    const int spl = 128 / sw, units = splits * ((NB / sw + spl - 1) / spl);
    const unsigned gx = a.line_units ? (unsigned)(8 * spl * ((units + 7) / 8)) : (unsigned)((NB / sw) * splits);
    const dim3 grid(gx, 1, (M + 15) / 16), block(256);
    const bool low = M <= 4;
    a.tk_stride = ticket_stride(column_waves ? (size_t)((NB + 127) / 128) : (size_t)(NB / sw) * (size_t)((M + 15) / 16));
    if (a.M > 255 || a.splits > 1023) return hipErrorInvalidValue;  // the packed leading scalars
    if (column_waves) {  // 128-byte strips, wave w on 32-byte part w (skinny_wave_kernel's CW form)
        if (!(mode == SK_ATOMZ && low && sw == 32 && nsw == 2 && aq.mode == 0 && !tiled)) return hipErrorInvalidValue;
        a.line_units = 0;
        const dim3 gcw((unsigned)(((NB + 127) / 128) * splits), 1, 1);
        hipLaunchKernelGGL((skinny_wave_kernel<32, 2, true, 0, true>), gcw, block, 0, st, TX_SK_ARGS(a));
        return hipGetLastError();
    }
#define TX_SW_LAUNCH(SW_, NSW_)                                                              \
    do {                                                                                      \
        if (low) hipLaunchKernelGGL((skinny_wave_kernel<SW_, NSW_, true>), grid, block, 0, st, TX_SK_ARGS(a));  \
        else hipLaunchKernelGGL((skinny_wave_kernel<SW_, NSW_, false>), grid, block, 0, st, TX_SK_ARGS(a));     \
    } while (0)
    if (aq.mode == 1) {
        if (low) hipLaunchKernelGGL((skinny_wave_kernel<16, 2, true, 1>), grid, block, 0, st, TX_SK_ARGS(a));
        else hipLaunchKernelGGL((skinny_wave_kernel<16, 2, false, 1>), grid, block, 0, st, TX_SK_ARGS(a));
    } else if (aq.mode == 2) {
        if (low) hipLaunchKernelGGL((skinny_wave_kernel<16, 2, true, 2>), grid, block, 0, st, TX_SK_ARGS(a));
        else hipLaunchKernelGGL((skinny_wave_kernel<16, 2, false, 2>), grid, block, 0, st, TX_SK_ARGS(a));
    } else if (sw == 32 && nsw == 4) TX_SW_LAUNCH(32, 4);
    else if (sw == 32) TX_SW_LAUNCH(32, 2);
    else if (nsw == 4) TX_SW_LAUNCH(16, 4);
    else if (nsw == 3) TX_SW_LAUNCH(16, 3);
    else TX_SW_LAUNCH(16, 2);
#undef TX_SW_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((mode == SK_ATOMIC || mode == SK_ATOMZ) && scaled) return launch_dequant(C, os, M, N, st);
    if (mode != SK_PARTIAL) return e;
    return n_out > 0 ? launch_splitk_reduce(partials, C, M, n_out, splits, os, st, N)
                     : launch_splitk_reduce(partials, C, M, N, splits, os, st);
}

hipError_t take_faults(unsigned* bits) {
    *bits = 0;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    unsigned v = 0;
    e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_tx_fault_word), sizeof(v), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    if (v != 0) {
        const unsigned zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_tx_fault_word), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
        if (e != hipSuccess) return e;
    }
    unsigned w = 0;
    e = take_line_faults(&w);
    *bits = v | w;
    return e;
}

hipError_t launch_splitk_reduce(const int32_t* P, int32_t* C, int M, int N, int splits, const OutScale& os,
                                hipStream_t st, int n_in) {
    if (n_in <= 0) n_in = N;
    const size_t n4 = (size_t)M * (size_t)N / 4;
    if (n4 == 0) return hipSuccess;
    const int vec = ((uintptr_t)(os.Y ? (const void*)os.Y : (const void*)C) % 16) == 0;
    launch_reduce(P, C, n4, splits, vec, os, N, n_in, (size_t)M * (size_t)n_in / 4, st);
    return hipGetLastError();
}

}  // namespace ternix_hip
