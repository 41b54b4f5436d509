// gemm_kernels.hip -- gfx950 LDS-tiled int8-MFMA GEMM kernels (M > 32, and 33..64 narrow tiles) for
// the ternary matmul, and their launcher.  Shared helpers, the weight layout and the decode forms are
// described in kernel_common.h.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

#include "kernel_common.h"
#include "ternary_kernels.h"

namespace ternix_hip {
namespace {

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

template <int BM, int WGN, int NS, int BK, bool TILED>
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
        w_off[p] = TILED ? tile64_offset((bc0 >> 4) + (pos ^ gf_swz_w(r)), r, K >> 6)
                         : (uint32_t)r * (uint32_t)NB + (uint32_t)(bc0 + (pos ^ gf_swz_w(r)) * 16);
    }
    auto issue = [&](int st, int buf) {
        const int sc = min(st, nst - 1);  // clamped: keeps the per-stage load count static
        const int8_t* abase = A + k_begin + (size_t)sc * BK;
        int8_t* adst = stage_a(buf);
#pragma unroll
        for (int p = 0; p < NA; ++p) lds_dma16(abase + a_off[p], adst + (p * 8 + wave) * 1024);
        const uint8_t* wbase = TILED ? B + (size_t)((k_begin + sc * BK) >> 6) * 1024
                                     : B + (size_t)(k_begin + sc * BK) * (size_t)NB;
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
                    *reinterpret_cast<v4i*>(out) = v;  // write-back stores (on MI355X, cold: 2048x4096x14336
                    // 103.9 -> 102.0 us, 4096x8192x28672 673 -> 665 against non-temporal ones; the pipelined
                    // kernel keeps non-temporal stores, 2048x4096x4096 27.0 against 28.4)
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
template <int MT, int GT>
struct PipeFrag {
    v4i a[MT];
    uint64_t lo[GT], hi[GT];
};

template <int BM, int WGN, int NS, int BK, int NWV, int BNB, bool TILED, int GM = 4>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_pipe_kernel(const int8_t* __restrict__ A, const uint8_t* __restrict__ B, int32_t* __restrict__ C, int M,
                      int K, int N, int tiles_n, int k_begin, int k_end, int accumulate, int vec_store,
                      int k_split, OutScale os, int group_m) {
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
        const int G_M = group_m > 0 ? group_m : GM;  // row tiles per group of the tile order
        const int first_m = (t / (G_M * tiles_n)) * G_M;
        const int gm = min(tiles_m - first_m, G_M);
        const int local = t % (G_M * tiles_n);
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
        w_off[p] = TILED ? tile64_offset((bc0 >> 4) + (pos ^ swz_w<BNB>(r)), r, K >> 6)
                         : (uint32_t)r * (uint32_t)NB + (uint32_t)(bc0 + (pos ^ swz_w<BNB>(r)) * 16);
    }
    auto issue = [&](int st, int buf) {
        const int sc = min(st, nst - 1);
        const int8_t* abase = A + k_begin + (size_t)sc * BK;
        int8_t* adst = stage_a(buf);
#pragma unroll
        for (int p = 0; p < NA; ++p) lds_dma16(abase + a_off[p], adst + (p * NWV + wave) * 1024);
        const uint8_t* wbase = TILED ? B + (size_t)((k_begin + sc * BK) >> 6) * 1024
                                     : B + (size_t)(k_begin + sc * BK) * (size_t)NB;
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

}  // namespace

// Narrow 64 x 64 tiles for M <= 64 when they alone fill at most one workgroup per CU (measured on
// MI355X: cfg3 M=64 up 18.0 -> 13.4 us with no K split, 4096^2 at M=64 16.2 -> 9.9 us; with more
// tiles than CUs, e.g. N = 28672, the 256-column tiles are faster).  The gemm_narrow debug switch (0 / 1) turns
// the choice off / on regardless (experiments).
bool gemm_narrow_wanted(int M, int K, int N, int tiled) {
    const int env = debug_get(DBG_GEMM_NARROW);
    const int NB = N >> 2;
    if (env == 0 || NB % 16 != 0 || K % 256 != 0) return false;
    if (env > 0) return true;
    // Row-major weights: not where K is split (K > 4096), where the 256-column tiles with more splits
    // win (on MI355X, cold, 64 / 256 columns: 64x11008x4096 14.4 / 13.1 us, 48x11008x4096 13.8 /
    // 11.9, 40x16384x4096 16.4 / 12.8, 64x16384x8192 30.1 / 21.4, 33x8192x4096 11.5 / 10.5).  The
    // tile-64 layout keeps them (its 1 KB blocks: 64x11008x4096 11.1 against 13.0 us).
    if (M > 64 || (K > 4096 && !tiled)) return false;
    return (long)((M + 63) / 64) * (NB / 16) <= device_cu_count();
}

bool gemm_narrow_ok(int M, int K, int N, int k_len, int splits, int k_split, int tiled) {
    return gemm_narrow_wanted(M, K, N, tiled) && k_len % 256 == 0 && (splits == 1 || k_split % 256 == 0);
}

// Tile height of a split-K launch: 64-row tiles of four waves or 128-row tiles of eight, each with
// the split count sized to one workgroup per CU (at most 16 splits of >= 256 k-rows).  The plan that
// keeps more CUs busy wins; on a tie the 64-row tiles win where they need no split at all on a full
// grid, the 128-row ones where each workgroup carries >= 80 M multiply-adds (their second wave per
// SIMD pays for the larger partials), else the 64-row ones.  On MI355X, cold weights, 64 / 128 rows:
// 128x11008x4096 15.4 / 19.3 us, 256x16384x4096 27.1 / 28.3, 256x8192x2048 14.4 / 19.3, 512x8192x2048
// 18.8 / 22.9 (ties, fewer multiply-adds); 512x11008x4096 33.2 / 32.1, 512x16384x4096 42.8 / 39.7,
// 768x16384x4096 64.1 / 55.1 (ties, more); 384x11008x4096 32.0 / 28.4 (192 against 240 workgroups);
// 1024x11008x4096 45.3 / 49.0 and 1024x16384x4096 65.1 / 62.4 (the 64-row tiles without a split).
int gemm_split_rows(int M, int K, int N) {
    const int bm_env = debug_get(DBG_GEMM_BM);
    if (bm_env == 64 || bm_env == 128) return bm_env;  // tests and measurements
    if (M % 128 != 0) return 64;  // no padding rows
    const long cus = device_cu_count();
    const long smax = std::min<long>(std::max(1, K / 256), 16);
    auto plan = [&](int rows, long* splits) {  // CUs busy in the plan's last wave of workgroups
        const long t = (long)((M + rows - 1) / rows) * (long)((N / 4 + 63) / 64);
        *splits = std::min<long>(t * 2 <= cus ? cus / t : 1, smax);
        const long wgs = t * *splits;
        return wgs % cus == 0 ? cus : wgs % cus;
    };
    long s64 = 1, s128 = 1;
    const long f64 = plan(64, &s64), f128 = plan(128, &s128);
    if (f128 != f64) return f128 > f64 ? 128 : 64;
    if (s64 == 1 && f64 == cus) return 64;
    const double macs = (double)M * (double)N * (double)K / (double)cus;
    return macs >= 80e6 ? 128 : 64;
}

// Which GEMM kernel a launch_gemm call runs (the single place the choice is made).
GemmChoice gemm_choice(const int8_t* A, const uint8_t* B, int M, int K, int N, int k_begin, int k_end, int splits,
                       int k_split, int tiled) {
    const int NB = N >> 2;
    const bool force_generic = debug_get(DBG_GEMM_GENERIC) == 1;  // tests
    if (splits < 1) splits = 1;
    const bool fast = (K % GF_BK == 0) && ((k_end - k_begin) % GF_BK == 0) && (k_begin % GF_BK == 0) &&
                      (splits == 1 || k_split % GF_BK == 0) &&
                      (NB % GF_BNB == 0) && ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0) &&
                      k_end > k_begin && (size_t)M * (size_t)K < ((size_t)1 << 32) &&
                      (size_t)GF_BK * (size_t)NB < ((size_t)1 << 32) &&
                      (tiled || !force_generic);
    // The tile-64 layout is read by the LDS-DMA GEMMs only (whole 128-row stages, at most 4 GiB of W).
    if (tiled && (!fast || (size_t)K * (size_t)NB >= ((size_t)1 << 32))) return GemmChoice::Invalid;
    if (!fast) return GemmChoice::Generic;
    const int tiles_n = NB / GF_BNB;
    const int bm_env = debug_get(DBG_GEMM_BM);
    // Measured on MI355X (cfg4 shapes): 256-row tiles only when they still give >= 1.5 tiles per
    // CU, else 128-row tiles; 8 waves as 2 (M) x 4 (N); 128-deep stages.
    const int cus = device_cu_count();
    int bm = (splits == 1 && (long)((M + 255) / 256) * tiles_n * 2 >= 3L * cus) ? 256 : 128;
    if (bm_env > 0) bm = bm_env == 128 ? 128 : (bm_env == 64 ? 64 : 256);  // tests and measurements
    constexpr int small_m_max = 64;
    // 64 x 64 output tiles (16 bytes of every weight row): enough workgroups without a K split where
    // the 256-column tiles would need one; one m-tile per wave, 256-deep stages.
    if ((M <= small_m_max || debug_get(DBG_GEMM_NARROW) > 0) && gemm_narrow_ok(M, K, N, k_end - k_begin, splits, k_split, tiled)) return GemmChoice::Narrow64;
    // Without a K split, 64-row tiles in workgroups of four waves (two co-resident per CU, whose
    // barriers and final stores overlap each other's work) instead of 128-row tiles of eight waves:
    // measured on MI355X, cold weights, 2048x4096x4096 29.1 -> 27.6 us, 1024x4096x4096 25.4 -> 20.3,
    // 512x4096x4096 25.1 -> 19.5, 768x4096x11008 52.2 -> 46.1, 1536x4096x11008 81.2 -> 71.7,
    // 2048x14336x4096 90.6 -> 90.4 (one round: equal).  With a K split: gemm_split_rows.  Small M (64
    // rows or fewer): the same four-wave workgroups, so no MFMA row or A byte is spent on padding
    // rows; the caller splits K to fill the chip.
    const bool split64 = splits > 1 && bm_env <= 0 && gemm_split_rows(M, K, N) == 64;
    if (M <= small_m_max || bm == 64 || split64 || (splits == 1 && bm == 128 && bm_env <= 0))
        return GemmChoice::Pipe64;
    return bm == 128 ? GemmChoice::Pipe128 : GemmChoice::Fast256;
}

const char* gemm_choice_name(GemmChoice c) {
    switch (c) {
        case GemmChoice::Narrow64: return "gemm_pipe_kernel<64 rows x 64 cols, 4 waves>";
        case GemmChoice::Pipe64: return "gemm_pipe_kernel<64 rows x 256 cols, 4 waves>";
        case GemmChoice::Pipe128: return "gemm_pipe_kernel<128 rows x 256 cols, 8 waves>";
        case GemmChoice::Fast256: return "gemm_fast_kernel<256 rows x 256 cols, 8 waves>";
        case GemmChoice::Generic: return "gemm_kernel<128 rows x 256 cols, register-staged>";
        default: return "invalid";
    }
}

hipError_t launch_gemm(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int k_begin, int k_end,
                       int accumulate, hipStream_t st, const OutScale& os, int splits, int k_split, int tiled) {
    const int NB = N >> 2;
    if (splits < 1) splits = 1;
    const GemmChoice choice = gemm_choice(A, B, M, K, N, k_begin, k_end, splits, k_split, tiled);
    if (choice == GemmChoice::Invalid) return hipErrorInvalidValue;
    if (choice == GemmChoice::Generic) {
        const bool aw = (NB % 4 == 0) && ((uintptr_t)B % 4 == 0);
        const bool aa = (K % 16 == 0) && ((uintptr_t)A % 16 == 0);
        return launch_gemm_t<128, 64>(A, B, C, M, K, N, aw, aa, k_begin, k_end, accumulate, st, os, splits, k_split);
    }
    const int vs = ((uintptr_t)(os.Y ? (const void*)os.Y : (const void*)C) % 16) == 0;
    const int tiles_n = NB / GF_BNB;
    const int gm_env = std::max(0, debug_get(DBG_GEMM_GM));  // tests and measurements: tile-order group
    if (choice == GemmChoice::Narrow64) {
        const dim3 gridn((unsigned)(((M + 63) / 64) * (NB / 16)), splits);
        if (tiled)
            hipLaunchKernelGGL((gemm_pipe_kernel<64, 1, 3, 256, 4, 16, true>), gridn, dim3(256), 0, st, A, B, C, M, K,
                               N, NB / 16, k_begin, k_end, accumulate, vs, k_split, os, gm_env);
        else
            hipLaunchKernelGGL((gemm_pipe_kernel<64, 1, 3, 256, 4, 16, false>), gridn, dim3(256), 0, st, A, B, C, M,
                               K, N, NB / 16, k_begin, k_end, accumulate, vs, k_split, os, gm_env);
    } else if (choice == GemmChoice::Pipe64) {
        // Tiles are visited in groups of 8 row tiles per column band (512 rows, as 4 groups of 128-row
        // tiles): measured on MI355X with cold weights, 2048x4096x4096 28.4 -> 27.0 us against groups of 4.
        const dim3 grid64((unsigned)(((M + 63) / 64) * tiles_n), splits);
        if (tiled)
            hipLaunchKernelGGL((gemm_pipe_kernel<64, 4, 3, 128, 4, 64, true, 8>), grid64, dim3(256), 0, st, A, B, C,
                               M, K, N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os, gm_env);
        else
            hipLaunchKernelGGL((gemm_pipe_kernel<64, 4, 3, 128, 4, 64, false, 8>), grid64, dim3(256), 0, st, A, B, C,
                               M, K, N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os, gm_env);
    } else if (choice == GemmChoice::Pipe128) {
        const dim3 grid(((M + 127) / 128) * tiles_n, splits);
        if (tiled)
            hipLaunchKernelGGL((gemm_pipe_kernel<128, 4, 3, 128, 8, GF_BNB, true>), grid, dim3(GF_THREADS), 0, st, A,
                               B, C, M, K, N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os, gm_env);
        else
            hipLaunchKernelGGL((gemm_pipe_kernel<128, 4, 3, 128, 8, GF_BNB, false>), grid, dim3(GF_THREADS), 0, st, A,
                               B, C, M, K, N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os, gm_env);
    } else {
        const dim3 grid(((M + 255) / 256) * tiles_n, splits);
        if (tiled)
            hipLaunchKernelGGL((gemm_fast_kernel<256, 4, 3, 128, true>), grid, dim3(GF_THREADS), 0, st, A, B, C, M, K,
                               N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os);
        else
            hipLaunchKernelGGL((gemm_fast_kernel<256, 4, 3, 128, false>), grid, dim3(GF_THREADS), 0, st, A, B, C, M,
                               K, N, tiles_n, k_begin, k_end, accumulate, vs, k_split, os);
    }
    return hipGetLastError();
}

}  // namespace ternix_hip
