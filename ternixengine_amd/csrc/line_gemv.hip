// line_gemv.hip -- gfx950 whole-line decode GEMV (M <= 4) for the ternary matmul, and its launcher.
// Shared helpers, the weight layout and the decode forms are described in kernel_common.h.
//
// Work unit: one 128-byte strip of the packed weight rows (one whole cache line per row, 512 output
// columns) over S consecutive 64-row k-steps.  Unit (strip s, split t) is workgroup t * strips + s,
// so every strip's split 0 is dispatched before any other split of it.
//
//   * Weights: the unit's S x 8 KB go global -> LDS with global_load_lds_dwordx4, all issued at
//     once (S instructions per wave for 8 data waves); one wave instruction moves 8 whole 128-byte
//     lines.  Stage row r keeps chunk c at 16-byte position c ^ swz(r), swz(r) = ((r/2) % 4) ^
//     4 * ((r/16) % 2): the 8 rows one 16-lane group of a transposing read touches cover 32 banks,
//     and the next 16-row group (read in the same instruction) the other 32.
//   * Data wave w owns the strip's w-th 16-byte column group (GW = 8 / NW groups per wave): per k-step
//     two ds_read_b64_tr_b8 give lane q byte-column q of 16 k-rows, the shift-form decode makes four
//     B operands, and v_mfma_i32_16x16x64_i8 against the activation fragment (row q < M, 16 bytes of
//     k-block kb, loaded straight from global memory) accumulates 64 output columns.
//   * K splits add into C with int32 atomics (exact, order-free).  C is zeroed inside the launch by
//     each strip's split 0, with no wait in any data wave: the workgroup's extra protocol wave takes
//     the call's ticket and, in split 0, zeroes the strip's outputs with agent-scope (write-through)
//     stores, waits for them and publishes the call's number in the strip's "zeroed" word; in the
//     other splits it waits for that word.  The data waves only meet it at the barrier before their
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

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernel_common.h"
#include "ternary_kernels.h"

namespace ternix_hip {

// This file's device fault word (its kernels cannot see the one in skinny_kernels.hip: every .hip
// file is its own device code object).  Read and cleared with the other by take_faults.
__device__ unsigned int g_line_fault_word;

namespace {

constexpr int kLineSpinLimit = 1 << 20;  // tries of the zeroed-word wait (about a second)

struct LineArgs {
    const int8_t* A;
    const uint8_t* B;
    int32_t* C;
    int M, K, N;
    int strips;                    // ceil(N/4 / 128)
    int splits;                    // workgroups per strip (<= 64)
    unsigned long long* tk;        // per strip {T, Z}
    int tk_stride;                 // 64-bit words between consecutive strips' {T, Z}
};


__device__ __forceinline__ int line_swz(int r) { return ((r >> 1) & 3) ^ (((r >> 4) & 1) << 2); }

template <int S, int NW>
__global__ __launch_bounds__(64 * (NW + 1)) void line_gemv_kernel(LineArgs args) {
    static_assert(NW == 4 || NW == 8, "4 or 8 data waves");
    constexpr int GW = 8 / NW;  // 16-byte column groups per data wave
    constexpr int STEP = 8192;  // bytes per k-step of the strip (64 rows x 128 bytes)
    __shared__ __attribute__((aligned(16))) uint8_t lds[S * STEP];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int strips = args.strips;
    const int split = (int)blockIdx.x / strips;
    const int s = (int)blockIdx.x - split * strips;
    const int M = args.M, K = args.K, N = args.N, NB = N >> 2;
    const int s0 = split * S;                 // first k-step
    const int nst = min(S, (K >> 6) - s0);    // k-steps of this unit (>= 1)
    const int bc0 = s * 128;                  // first byte-column of the strip
    const bool zeroer = split == 0;
    unsigned long long* tk = args.tk + (size_t)args.tk_stride * (size_t)s;

    if (wave == NW) {
        // Protocol wave.  Split 0 first issues the zeroing stores (they need no ticket).
        if (zeroer) {
            const int n8 = 2 * min(128, NB - bc0);  // 8-byte units of the strip's outputs in one row
            for (int r = 0; r < M; ++r) {
                unsigned long long* z = reinterpret_cast<unsigned long long*>(args.C + (size_t)r * (size_t)N + 4 * bc0);
                for (int u = lane; u < n8; u += 64) __hip_atomic_store(z + u, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (zeroer) {
            // Split 0: T += 64 - (splits - 1) (no return needed), barrier (1), wait until the zeroing
            // stores have completed, then Z += 1.  One statement, lane 0 alone enabled for the two
            // atomics, so that barrier (1) is reached at once and is one instruction of a uniform path.
            const unsigned long long inc = (unsigned long long)(64 - (args.splits - 1)), one = 1;
            unsigned long long saved_exec;
            __asm__ volatile(
                "s_mov_b64 %0, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add_x2 %1, %2, off\n\t"
                "s_mov_b64 exec, %0\n\t"
                "s_barrier\n\t"
                "s_waitcnt vmcnt(0)\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add_x2 %3, %4, off\n\t"
                "s_mov_b64 exec, %0"
                : "=&s"(saved_exec)
                : "v"(tk), "v"(inc), "v"(tk + 1), "v"(one)
                : "memory");
        } else {
            // Every other split: the returning T += 1 (its value / 64 + 1 names this call), barrier (1)
            // (this workgroup's weights have landed, so split 0 has long started its zeroing), then the
            // coherent (sc1) load of Z and the wait for both.  One statement, lane 0 alone enabled for
            // the memory operations: nothing reads `old` or `zw`, or reuses their registers, while they
            // are in flight.
            unsigned long long old, zw, saved_exec;
            __asm__ volatile(
                "s_mov_b64 %2, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add_x2 %0, %3, %4, off sc0\n\t"
                "s_mov_b64 exec, %2\n\t"
                "s_barrier\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_load_dwordx2 %1, %5, off sc1\n\t"
                "s_mov_b64 exec, %2\n\t"
                "s_waitcnt vmcnt(0)"
                : "=&v"(old), "=&v"(zw), "=&s"(saved_exec)
                : "v"(tk), "v"(1ull), "v"(tk + 1)
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

    // Data waves.  DMA instruction p (k-step p / 8, rows 8 (p % 8) .. +7) is issued by wave p % NW;
    // lane l fills 16-byte position l % 8 of row 8 (p % 8) + l / 8.
    {
        const int r_in = lane >> 3, pos = lane & 7;
#pragma unroll
        for (int i = 0; i < (S * 8 + NW - 1) / NW; ++i) {
            const int p = wave + NW * i;
            if (p < nst * 8) {
                const int step = p >> 3, r = (p & 7) * 8 + r_in;
                int c = pos ^ line_swz(r);
                if (bc0 + 16 * c >= NB) c = 0;  // past the last column (a partial last strip): a valid chunk, unused
                const uint8_t* src = args.B + ((size_t)(s0 + step) * 64 + (size_t)r) * (size_t)NB + (size_t)(bc0 + 16 * c);
                lds_dma16(src, lds + step * STEP + (p & 7) * 1024);
            }
        }
    }
    const int q = lane & 15, kb = lane >> 4;
    v4i a[S];
    {
        const int8_t* arow = args.A + (size_t)min(q, M - 1) * (size_t)K + (size_t)s0 * 64 + kb * 16;
#pragma unroll
        for (int st = 0; st < S; ++st) {
            a[st] = v4i{0, 0, 0, 0};
            if (st < nst && q < M) a[st] = *reinterpret_cast<const v4i*>(arow + st * 64);
        }
    }
    TX_VMCNT(0);
    __builtin_amdgcn_s_barrier();  // (1) every data wave's weights are in LDS
    __builtin_amdgcn_sched_barrier(0);

    v4i acc[GW][4];
#pragma unroll
    for (int gi = 0; gi < GW; ++gi)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[gi][j] = v4i{0, 0, 0, 0};
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
                for (int j = 0; j < 4; ++j) acc[gi][j] = mfma_i8(a[st], bfr[j], acc[gi][j]);
            }
        }
    }
    __builtin_amdgcn_s_barrier();  // (2) every wave is done with the stage buffers; C is zeroed
    __builtin_amdgcn_sched_barrier(0);

    // Epilogue: lane (q, kb = 0) holds rows i < 4 of columns 4 (bc0 + 16 g + q) + j.  Each wave lays a
    // row's 64 outputs of a group out in column order in its own 256 bytes of the idle stage buffer,
    // then adds one column per lane: 64 consecutive int32 per atomic instruction.
    int32_t* rb = reinterpret_cast<int32_t*>(lds) + wave * 64;
#pragma unroll
    for (int gi = 0; gi < GW; ++gi) {
        const int g = wave * GW + gi;
        if (bc0 + 16 * g >= NB) continue;  // wave-uniform
        int32_t* out = args.C + 4 * (bc0 + 16 * g) + lane;
        for (int i = 0; i < M; ++i) {
            if (kb == 0) {
                const v4i v = {acc[gi][0][i] >> 6, acc[gi][1][i] >> 6, acc[gi][2][i] >> 6, acc[gi][3][i] >> 6};
                *reinterpret_cast<v4i*>(rb + 4 * q) = v;
            }
            __builtin_amdgcn_wave_barrier();
            const int32_t v = rb[lane];
            __builtin_amdgcn_wave_barrier();
            __hip_atomic_fetch_add(out + (size_t)i * (size_t)N, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace

bool line_gemv_ok(const int8_t* A, const uint8_t* B, int M, int K, int N) {
    const int NB = N / 4;
    return M >= 1 && M <= 4 && K >= 64 && K % 64 == 0 && NB % 16 == 0 && (uintptr_t)A % 16 == 0 &&
           (uintptr_t)B % 16 == 0 && (size_t)K * (size_t)NB < ((size_t)1 << 40);
}

int line_gemv_splits(int K, int S) { return ((K / 64) + S - 1) / S; }

hipError_t launch_line_gemv(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, int S, int NW,
                            unsigned long long* tk, int tk_stride, hipStream_t st) {
    if (!line_gemv_ok(A, B, M, K, N) || tk == nullptr) return hipErrorInvalidValue;
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
    if (a.splits > 64 || (size_t)S * 64 > (size_t)kMaxKPerAccumulator) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(a.strips * a.splits));
#define TX_LINE(SS, WW)                                                                                    \
    if (S == SS && NW == WW) {                                                                             \
        hipLaunchKernelGGL((line_gemv_kernel<SS, WW>), grid, dim3(64 * (WW + 1)), 0, st, a);              \
        return hipGetLastError();                                                                          \
    }
    TX_LINE(1, 8)
    TX_LINE(2, 8)
    TX_LINE(3, 8)
    TX_LINE(4, 8)
    TX_LINE(6, 8)
    TX_LINE(8, 8)
    TX_LINE(2, 4)
    TX_LINE(4, 4)
#undef TX_LINE
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
