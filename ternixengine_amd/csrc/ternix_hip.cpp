// ternix_hip.cpp -- C-ABI launch layer of libternix_hip.so (declared in include/ternix/ternix_hip.h).
//
// Validates shapes before touching any pointer (reference contract: src/cuda_kernels.cu:127,135 and
// tests/test_cuda_matmul.cu:41-43), picks a kernel and its split, launches asynchronously on the
// caller's stream and returns the hipError_t of the launch.
#include "ternix/ternix_hip.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "ternary_kernels.h"

namespace {

constexpr int kSkinnyMaxM = 32;

int cu_count() { return ternix_hip::device_cu_count(); }

// ---- split-K workspace -------------------------------------------------------------------------
// The skinny kernel's split-K writes one partial C per split into a device workspace that the
// following reduce kernel sums.  One workspace per (device, stream), so concurrent streams never
// share one.  It is allocated the first time a shape needs more than the current size -- never
// while the stream is being captured into a graph (the call then takes the atomic path, which needs
// no workspace) -- and kept until the process ends.  A buffer outgrown by a larger shape is retired,
// not freed: work already queued and graphs captured earlier on the stream keep using it.
constexpr size_t kWorkspaceMax = size_t(256) << 20;

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    std::vector<void*> retired;
    int* counters = nullptr;  // arrival counters of the single-launch split-K GEMV (zero between calls)
};
std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

void* workspace(hipStream_t st, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& w = g_ws[{dev, st}];
    if (w.bytes >= bytes) return w.ptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    // Grow geometrically (at least 8 MiB, at least double), capped at kWorkspaceMax unless the
    // request itself is larger, rounded to 1 MiB.
    const size_t grown = std::min(std::max(size_t(8) << 20, 2 * w.bytes), kWorkspaceMax);
    size_t nb = std::max(bytes, grown);
    nb = (nb + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    void* p = nullptr;
    if (hipMalloc(&p, nb) != hipSuccess) return nullptr;
    if (w.ptr) w.retired.push_back(w.ptr);  // sizes at least double, so retired memory < the live buffer
    w.ptr = p;
    w.bytes = nb;
    return p;
}

// Largest split count for which the wave GEMV sums its K splits inside the launch (the last
// workgroup of each strip to arrive adds the partials) instead of in a reduce launch.  Measured on
// MI355X, cold weights, one box: with 2-5 splits the single launch wins (cfg2 up 7.7 -> 7.0 us,
// cfg3 M=4 up 11.1 -> 9.2, tile-64 cfg5 big 15.6 -> 15.0); from about 8 splits the serialised
// arrivals on each counter cost more than the launch (cfg3 M=16 down 12.1 -> 12.8 us).
// TERNIX_WAVE_LAST overrides it (experiments; 0 turns the scheme off).
int last_max_splits() {
    static const int v = [] {
        const char* e = std::getenv("TERNIX_WAVE_LAST");
        return e ? std::atoi(e) : 5;
    }();
    return v;
}

// Arrival counters of the wave GEMV's single-launch split-K (kCounterSlots ints per (device, stream),
// zeroed once when allocated; every call leaves them zero).  nullptr during graph capture before
// they exist, when `need` exceeds the slots or for more than last_max_splits() splits: the caller
// then uses the reduce launch.
constexpr size_t kCounterSlots = size_t(1) << 16;
int* arrival_counters(hipStream_t st, size_t need, int M, int splits, int sps) {
    // Up to 4 rows with long k-ranges per split (>= 8 steps) also sum up to 8 splits inside the
    // launch: their workgroups finish far apart, so the arrivals hardly queue (cold cfg3 M=4 down:
    // 8 splits 9.8 us against 11.5 for the DMA-staged kernel and its reduce launch; 12 splits of
    // cfg2 down 8.6 us against 7.8 with 8; 16 splits of tile-64 cfg3 M=4 down 12.2 against 9.3 us
    // with the reduce launch).
    const int lim = last_max_splits();
    if (lim <= 0 || (splits > lim && !(M <= 4 && sps >= 8 && splits <= 8)) || need > kCounterSlots)
        return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& w = g_ws[{dev, st}];
    if (w.counters) return w.counters;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, kCounterSlots * sizeof(int)) != hipSuccess) return nullptr;
    if (hipMemsetAsync(p, 0, kCounterSlots * sizeof(int), st) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    w.counters = static_cast<int*>(p);
    return w.counters;
}

// Shape / pointer validation shared by every device entry point.  Returns hipSuccess when the call
// is well formed; *trivial is set when there is nothing to launch (M == 0 or N == 0).
hipError_t validate(const void* dA, const void* dB, const void* dC, int64_t M, int64_t K, int64_t N, bool* trivial) {
    *trivial = false;
    if (M < 0 || K < 0 || N < 0) return hipErrorInvalidValue;
    if (N % 4 != 0) return hipErrorInvalidValue;
    if (M > INT_MAX || K > INT_MAX || N > INT_MAX) return hipErrorInvalidValue;
    if (M == 0 || N == 0) {
        *trivial = true;
        return hipSuccess;
    }
    if (dC == nullptr || reinterpret_cast<uintptr_t>(dC) % alignof(int32_t) != 0) return hipErrorInvalidValue;
    if (K > 0 && (dA == nullptr || dB == nullptr)) return hipErrorInvalidValue;
    return hipSuccess;
}

// Split-K plan of the skinny kernels: tb (64- or 128-byte column slab per wave), kw (waves per slab
// inside a workgroup of 4 waves), `splits` workgroups along K (splits > 1 adds the partial-sum
// reduce launch) with sps k-steps each.
// Experiment switches, read once per process (a lookup per call would cost host time on every launch).
const char* skinny_plan_env() {  // "tb,kw,splits": forces the skinny split plan
    static const char* const e = std::getenv("TERNIX_SKINNY_PLAN");
    return e;
}
const char* skinny_wave_env() {  // "sw,nsw,splits" forces a wave-kernel plan, "0" turns it off
    static const char* const e = std::getenv("TERNIX_SKINNY_WAVE");
    return e;
}

// Split count whose partial sums stay within 4 MiB: allowed whatever the weight size (small N).
long partials_floor(int M, int N) { return (4L << 20) / std::max(1L, 4L * M * N); }

struct SkinnyPlan {
    int tb, kw, splits, sps;
    int dma;  // > 0: skinny_dma_kernel with this many LDS stages
};

// Plan of the DMA-staged skinny kernel (one m-group of <= 16 rows, 256-byte column strips): the
// largest split count that keeps the grid within one workgroup per CU, capped, with several rows, so
// the partial sums stay below half the weight bytes.  Returns dma = 0 when the k-range per split
// would exceed the kernel's activation slice (16 k-steps).
SkinnyPlan plan_skinny_dma(int M, int K, int N, int ns) {
    const int nsteps = K / 64;
    const long col_wgs = (N / 4 + 255) / 256;
    const long cus = cu_count();
    long splits = std::max(1L, cus / col_wgs);
    splits = std::min(splits, std::max({1L, (long)K / (32L * M), partials_floor(M, N)}));
    splits = std::min<long>(splits, nsteps);
    int sps = (int)((nsteps + splits - 1) / splits);
    while (col_wgs * ((nsteps + sps - 1) / sps) > std::max(cus, col_wgs)) ++sps;  // no second wave
    SkinnyPlan p{1, 1, (nsteps + sps - 1) / sps, sps, ns};
    if (const char* env = skinny_plan_env()) {  // experiments: "tb,kw,splits"
        int etb = 0, ekw = 0, esp = 0;
        if (std::sscanf(env, "%d,%d,%d", &etb, &ekw, &esp) == 3 && esp >= 1) {
            p.sps = (nsteps + esp - 1) / esp;
            p.splits = (nsteps + p.sps - 1) / p.sps;
        }
    }
    if (p.sps > 16 || p.sps > ternix_hip::kMaxKPerAccumulator / 64) p.dma = 0;
    return p;
}

SkinnyPlan plan_skinny(int M, int K, int N, bool generic = false) {
    const int NB = N / 4;
    const int nsteps = (K + 63) / 64;
    const int mgroups = M <= 16 ? 1 : (M + 31) / 32;
    // Measured on MI355X (cfg1-3, cfg5 M=1 shapes): 64-byte slabs, four slabs per workgroup (256
    // contiguous bytes of every weight row per workgroup), and K split into as many ranges as keep
    // the grid within one workgroup per CU (a CU holding two of them finishes last).  With several
    // rows the partial sums ([splits][M][N] int32, written and read back once) are capped at about
    // the weight bytes (K*N/4): splits <= K / (32 M), or 4 MiB of partials when that allows more.
    // Above 4 rows two waves share each 64-byte slab (alternate k-steps, summed in LDS), which halves
    // the cross-workgroup splits -- and the partial sums, 4 bytes per row and column per split -- for
    // the same number of workgroups (measured on MI355X, cfg3 M=16: 13.9 vs 15.4 us up, 14.1 vs 15.4
    // us down).
    const int kw = M > 4 ? 2 : 1;
    SkinnyPlan p{1, kw, 1, nsteps, 0};
    const long col_wgs = (NB + 256 / kw - 1) / (256 / kw);
    const long wgs = col_wgs * mgroups;
    const long target = cu_count();
    if (wgs < target) {
        long splits = target / wgs;
        // The generic kernel (ragged or unaligned shapes) has a serial dword-load loop per k-step, so
        // it wants at least 32 splits whatever the partial-sum traffic (measured: M=17 K=4093 N=1028
        // 19.5 us with 32 splits vs 39 us with 7).
        const long traffic_cap = std::max({generic ? 32L : 1L, (long)K / (32L * M), partials_floor(M, N)});
        if (splits > traffic_cap) splits = traffic_cap;
        if (splits > nsteps) splits = nsteps;
        if (splits > 1) p.splits = (int)splits;
    }
    // Tuning override for experiments: TERNIX_SKINNY_PLAN="tb,kw,splits".
    if (const char* env = skinny_plan_env()) {
        int etb = 0, ekw = 0, esp = 0;
        if (std::sscanf(env, "%d,%d,%d", &etb, &ekw, &esp) == 3 && (etb == 1 || etb == 2) &&
            (ekw == 1 || ekw == 2 || ekw == 4) && esp >= 1) {
            p.tb = etb;
            p.kw = ekw;
            p.splits = esp;
        }
    }
    // Each split's k-range must stay within the accumulator bound and, for the fast kernel, its
    // activation slice within the LDS budget.
    int max_sps = ternix_hip::kMaxKPerAccumulator / 64;
    while (max_sps > 1 && ternix_hip::skinny_a_lds_bytes(M, max_sps) > ternix_hip::kSkinnyALdsMax) max_sps >>= 1;
    if (p.splits > 65535) p.splits = 65535;
    p.sps = (nsteps + p.splits - 1) / p.splits;
    if (p.sps > max_sps) p.sps = max_sps;
    if (p.sps < 1) p.sps = 1;
    p.splits = (nsteps + p.sps - 1) / p.sps;
    if (p.splits < 1) p.splits = 1;
    return p;
}

// TERNIX_SKINNY_WAVE=0 switches the wave-pipelined skinny kernel off (experiments).
bool wave_kernel_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("TERNIX_SKINNY_WAVE");
        return !(e && e[0] == '0' && e[1] == '\0');
    }();
    return on;
}

int wave_max_m() {
    static const int m = [] {
        const char* e = std::getenv("TERNIX_WAVE_MAX_M");  // experiments
        return e ? std::atoi(e) : 32;
    }();
    return m;
}

// K split of the wave-pipelined kernel (one workgroup per strip of sw bytes, m-group and split).
// 16-byte strips (tile-64 weights): enough workgroups for about 2.75 per CU, and for M <= 4 up to 7
// per CU, one per 8 KB of weights (more weight loads in flight on the large decode matrices, where
// the extra partial sums cost little).  32-byte strips (row-major weights): about one workgroup per
// CU.  At least two k-steps per split.  Measured on MI355X with cold weights (512 MiB pools, one
// box): 16-byte strips cfg2 up 9.35 -> 8.4 us against no split, tile-64 cfg5 big 17.8 -> 15.3 us;
// 32-byte strips against 16-byte ones, each with its split: cfg1 6.72 -> 6.14 us, cfg2 up 8.41 ->
// 7.56, cfg3 M=4 up 12.3 -> 10.9, M=16 up 13.8 -> 11.9, M=16 down 13.95 -> 11.8.
// TERNIX_WAVE_TARGET overrides the workgroup target (experiments).
int wave_splits(int M, int K, int N, int sw = 16) {
    static const long env = [] {
        const char* e = std::getenv("TERNIX_WAVE_TARGET");
        return e ? std::atol(e) : 0L;
    }();
    const long nsteps = K / 64, units = (long)(N / 4 / sw) * ((M + 15) / 16), cus = cu_count();
    long target = cus * 11 / 4;
    if (M <= 4) target = std::max(target, std::min(7 * cus, (long)K * (N / 4) / 8192));
    if (sw == 32) target = cus;
    if (env > 0) target = env;
    long sp = (target + units / 2) / std::max(1L, units);
    sp = std::max(1L, std::min(16L, std::min(sp, std::max(1L, nsteps / 2))));
    // 32-byte strips: at most one workgroup per CU (6 % slack); a CU given a second one finishes last
    // (cfg3 M=16 down: 8 splits, 256 workgroups 11.8 us; 10 splits, 320 workgroups 15.5 us), while a
    // few doubled CUs cost less than a smaller split (cfg2 up: 270 workgroups 6.9 us, 216 7.04 us).
    while (sw == 32 && sp > 1) {
        const long sps = (nsteps + sp - 1) / sp;
        if (units * ((nsteps + sps - 1) / sps) * 50 <= cus * 53) break;
        --sp;
    }
    // K <= 4096: few enough splits to sum them inside the launch (measured: cfg1 6.27 us with 10
    // splits and the reduce launch, 5.75 with 5 in one launch; tile-64 cfg2 up 6.88 -> 6.41).
    if (nsteps <= 64 && last_max_splits() > 0) sp = std::min<long>(sp, last_max_splits());
    return (int)sp;
}

hipError_t run_skinny(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, hipStream_t st,
                      const ternix_hip::OutScale& os = ternix_hip::OutScale{},
                      const ternix_hip::ActQuant& aq = ternix_hip::ActQuant{}) {
    const bool generic = !(K % 64 == 0 && (N / 4) % 64 == 0 && reinterpret_cast<uintptr_t>(dB) % 16 == 0 &&
                           (aq.mode != 0 || reinterpret_cast<uintptr_t>(dA) % 16 == 0));
    // Wave-pipelined kernel (32-byte strips, 16-byte with fused quantisation; 2 ring slots per wave),
    // measured on MI355X (16-byte strips) against the DMA-staged kernel: faster for K <= 4096 (cfg1
    // 6.26 -> 5.64 us, cfg2 up 6.94 -> 6.29, cfg3 M=4 up 11.62 -> 10.41, M=16 up 14.27 -> 11.45) and
    // for 4 < M <= 32 with longer K, whose partials are far fewer than the DMA kernel's (cfg3 M=16
    // down 14.59 -> 12.78 us); strip width and K split as in wave_splits.  M <= 4 with K > 4096 stays
    // on the DMA kernel (cold cfg2 down 7.8 us against 7.9-9.0 for the wave kernel).
    // TERNIX_SKINNY_WAVE="sw,nsw,splits" forces a plan, "0" turns the kernel off (experiments).
    // With fused activation quantisation (K <= 4096) it quantises whole rows itself and dequantises with
    // its own row scales: the FFN block's gate/up GEMV becomes one launch.
    if (!generic && M <= wave_max_m() && ternix_hip::skinny_wave_ok(dA, dB, M, K, N, 16) &&
        (aq.mode == 0 || (K <= 4096 && M <= 16))) {
        static const int sw_env = [] {
            const char* e = std::getenv("TERNIX_WAVE_SW");  // experiments: "16" for 16-byte strips
            return e && std::atoi(e) == 16 ? 16 : 32;
        }();
        const int nsteps = K / 64;
        int sw = aq.mode == 0 && ternix_hip::skinny_wave_ok(dA, dB, M, K, N, sw_env) ? sw_env : 16, nsw = 2, sp = 0;
        static const int long_small = [] {
            const char* e = std::getenv("TERNIX_WAVE_LONG");  // experiments: 0 keeps M <= 4, K > 4096 off it
            return e ? std::atoi(e) : 1;
        }();
        if (aq.mode != 0) sp = 1;
        else if (K <= 4096 || M > 4) sp = wave_splits(M, K, N, sw);
        else if (long_small && sw == 32 && last_max_splits() > 0) {
            // M <= 4 with long K: only when 32-byte strips split 4 to 8 ways within one round of
            // workgroups (cfg2 down 7.8 us, as the DMA-staged kernel; cfg3 M=4 down 11.5 -> 9.8 us),
            // summed inside the launch; wide matrices (cfg5 big: 224 strips) keep the DMA-staged kernel.
            const int s2 = std::min(8, wave_splits(M, K, N, sw));
            if (s2 >= 4) sp = s2;
        }
        // Wide matrices leave the wave kernel few splits and long k-ranges per workgroup; beyond 32
        // k-steps per workgroup (24 for M <= 2) the DMA-staged kernel is faster for M <= 16 (measured
        // on MI355X, cold: 8x8192x28672 31.2 -> 19.1 us, 6x4096x28672 16.9 -> 14.6, 12x6144x16384
        // 17.6 -> 16.6, 1x4096x14336 10.2 -> 9.2, 1x14336x4096 10.7 -> 9.6; at 28 steps and M >= 4 the
        // wave kernel still wins: 4x14336x4096 11.3 against 12.1).
        if (sp > 0 && aq.mode == 0 && M <= 16 && (nsteps + sp - 1) / sp > (M <= 2 ? 24 : 32) &&
            ternix_hip::skinny_dma_ok(dA, dB, M, K, N, 1))
            sp = 0;
        if (const char* env = skinny_wave_env()) {
            int esw = 0, ensw = 0, esp = 0;
            if (std::sscanf(env, "%d,%d,%d", &esw, &ensw, &esp) == 3 && esp >= 1 &&
                ternix_hip::skinny_wave_ok(dA, dB, M, K, N, esw)) {
                sw = esw;
                nsw = ensw;
                sp = esp;
            } else {
                sp = 0;
            }
        }
        if (sp > 0) {
            const int sps = (nsteps + sp - 1) / sp;
            const int splits = (nsteps + sps - 1) / sps;
            int32_t* partials = nullptr;
            if (splits > 1) {
                const size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(int32_t);
                if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(workspace(st, need));
            }
            if (sps * 64 <= ternix_hip::kMaxKPerAccumulator && (splits == 1 || partials || dC) &&
                (aq.mode == 0 || (splits == 1 && sw == 16 && nsw == 2))) {
                int* cnt = (partials && aq.mode == 0)
                               ? arrival_counters(st, (size_t)(N / 4 / sw) * (size_t)((M + 15) / 16), M, splits, sps)
                               : nullptr;
                return ternix_hip::launch_skinny_wave(dA, dB, dC, M, K, N, sw, nsw, splits, sps, partials, st, os, 0,
                                                      aq, 0, cnt);
            }
        }
    }
    // DMA-staged kernel: TERNIX_SKINNY_DMA=0 disables it, 2..4 sets its stage count (experiments).
    static const int dma_env = [] {
        const char* e = std::getenv("TERNIX_SKINNY_DMA");
        return e ? std::atoi(e) : -1;
    }();
    SkinnyPlan p{0, 0, 0, 0, 0};
    if (!generic && M <= 16 && dma_env != 0 && ternix_hip::skinny_dma_ok(dA, dB, M, K, N, 1)) {
        p = plan_skinny_dma(M, K, N, dma_env >= 2 && dma_env <= 4 ? dma_env : 3);
        if (p.splits <= 1) p.dma = 0;  // the kernel writes partials or atomics only through a split
        if (!ternix_hip::skinny_dma_aq_ok(aq.mode, K, p.splits)) p.dma = 0;
    }
    if (p.dma == 0) p = plan_skinny(M, K, N, generic);
    // Fused activation quantisation needs the DMA or the short kernel with a split; the caller falls
    // back to the standalone quantisation launch when this returns hipErrorInvalidValue.
    if (aq.mode != 0 && p.dma == 0 && !ternix_hip::skinny_short_ok(dB, M, K, N, p.sps, p.splits))
        return hipErrorInvalidValue;
    int32_t* partials = nullptr;
    if (p.splits > 1) {
        const size_t need = (size_t)p.splits * (size_t)M * (size_t)N * sizeof(int32_t);
        if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(workspace(st, need));
    }
    return ternix_hip::launch_skinny(dA, dB, dC, M, K, N, p.tb, p.kw, p.splits, p.sps, partials, st, os, aq, p.dma);
}

// Split-K for GEMMs with too few output tiles to fill the chip (mid-size M against a long K, e.g.
// cfg3 M=64, the worst case M=256): each split covers a contiguous k-range of whole 128-row stages,
// the partial tiles go through the same workspace and reduce launch as the skinny path.
int gemm_splits(int M, int K, int N) {
    static const int env = [] {
        const char* e = std::getenv("TERNIX_GEMM_SPLITS");  // experiments only
        return e ? std::atoi(e) : 0;
    }();
    const int bm = M <= 64 ? 64 : 128;  // the tile height launch_gemm picks
    const bool narrow = ternix_hip::gemm_narrow_wanted(M, K, N);  // 64-column tiles instead of 256
    const long tiles = (long)((M + bm - 1) / bm) * (long)((N / 4 + 63) / 64) * (narrow ? 4 : 1);
    const long cus = cu_count();
    // K <= 4096: the reduce launch and the partial sums cost more than the idle CUs (measured on
    // MI355X, cold weights: 40x1024x4096 7.6 -> 4.9 us without the split, 64x2560x6912 11.8 -> 8.8,
    // 256x1024x11008 31.1 -> 9.7, 256x4096x11008 35.2 -> 25.0; from K = 6144 the split wins:
    // 128x11008x4096 59.0 -> 22.4 us).
    if (env <= 0 && K <= 4096) return 1;
    long splits = env > 0 ? env : (tiles * 2 <= cus ? cus / tiles : 1);
    splits = std::min<long>(splits, std::max(1, K / 256));  // at least two 128-row stages per split
    return (int)std::max<long>(1, std::min<long>(splits, 16));
}

hipError_t run_gemm(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, hipStream_t st,
                    const ternix_hip::OutScale& os = ternix_hip::OutScale{}, int tiled = 0) {
    if (K <= ternix_hip::kMaxKPerAccumulator) {
        int splits = gemm_splits(M, K, N);
        if (splits > 1) {
            // whole stages per split: 256 rows for the narrow tiles, 128 for the others
            const int unit = ternix_hip::gemm_narrow_wanted(M, K, N) ? 256 : (K % 128 == 0 ? 128 : 64);
            const int k_split = ((K + splits - 1) / splits + unit - 1) / unit * unit;
            splits = (K + k_split - 1) / k_split;
            const size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(int32_t);
            int32_t* partials = (splits > 1 && need <= kWorkspaceMax) ? static_cast<int32_t*>(workspace(st, need))
                                                                       : nullptr;
            if (partials) {
                hipError_t e = ternix_hip::launch_gemm(dA, dB, partials, M, K, N, 0, K, 0, st, ternix_hip::OutScale{},
                                                       splits, k_split, tiled);
                if (e != hipSuccess) return e;
                return ternix_hip::launch_splitk_reduce(partials, dC, M, N, splits, os, st);
            }
        }
        return ternix_hip::launch_gemm(dA, dB, dC, M, K, N, 0, K, 0, st, os, 1, 0, tiled);
    }
    if (dC == nullptr) return hipErrorInvalidValue;  // scaled call without int scratch
    int acc = 0;
    for (long k0 = 0; k0 < K; k0 += ternix_hip::kMaxKPerAccumulator) {
        const long k1 = k0 + ternix_hip::kMaxKPerAccumulator < K ? k0 + ternix_hip::kMaxKPerAccumulator : K;
        const hipError_t e = ternix_hip::launch_gemm(dA, dB, dC, M, K, N, (int)k0, (int)k1, acc, st,
                                                     ternix_hip::OutScale{}, 1, 0, tiled);
        if (e != hipSuccess) return e;
        acc = 1;
    }
    // Several K chunks accumulate int32 in dC (which aliases os.Y when dequantising); convert last.
    return os.Y ? ternix_hip::launch_dequant(dC, os, M, N, st) : hipSuccess;
}

// Ragged shapes (K % 64 != 0 or N % 256 != 0) and misaligned operands on the automatic paths: one
// launch copies W into a padded K' x N'/4 layout (K' = K rounded up to 128, N'/4 to 64 bytes, zeros in
// the padding) and A into rows of K' bytes, inside the split-K workspace; the aligned kernels then run
// on the padded problem with split-K, and the reduce writes only the N real columns (zero weights
// and zero activations in the padding add nothing, so the sums are those of the original problem).
// Returns hipErrorNotSupported, before launching anything, when this does not apply (a skinny plan
// without a split, graph capture without a large enough workspace, sizes past the workspace cap);
// the caller then runs the generic kernels.
hipError_t run_padded(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, hipStream_t st,
                      const ternix_hip::OutScale& os, bool skinny) {
    const int NB = N / 4;
    const long Kp = ((long)K + 127) / 128 * 128;
    const long NBp = ((long)NB + 63) / 64 * 64;
    const long Np = 4 * NBp;
    if (K == 0 || Kp > INT_MAX || Np > INT_MAX || Kp * NBp >= (1L << 32)) return hipErrorNotSupported;
    SkinnyPlan p{0, 0, 0, 0, 0};
    int splits = 1, k_split = 0;
    // Short K at M <= 16: the wave-pipelined kernel in one launch, writing the N real columns itself.
    const bool wave = skinny && M <= wave_max_m() && Kp <= 4096 && wave_kernel_enabled();
    if (wave) {
        splits = 1;
    } else if (skinny) {
        if (M <= 16) p = plan_skinny_dma(M, (int)Kp, (int)Np, 3);
        if (p.dma == 0) p = plan_skinny(M, (int)Kp, (int)Np);
        splits = p.splits;
    } else {
        splits = gemm_splits(M, (int)Kp, (int)Np);
        if (splits > 1) {
            const long unit = ternix_hip::gemm_narrow_wanted(M, (int)Kp, (int)Np) ? 256 : 128;
            k_split = (int)(((Kp + splits - 1) / splits + unit - 1) / unit * unit);
            splits = (int)((Kp + k_split - 1) / k_split);
        }
    }
    // The skinny kernels write partials only through a split; the GEMM writes its one slab to the
    // workspace just the same, and the reduce launch keeps the N real columns.
    if (splits <= 1 && skinny && !wave) return hipErrorNotSupported;
    // Each split's k-range must fit one int32 accumulator (the skinny plans guarantee it).
    if (!skinny && k_split > ternix_hip::kMaxKPerAccumulator) return hipErrorNotSupported;
    auto up = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t w_bytes = up((size_t)Kp * (size_t)NBp);
    const size_t a_bytes = up((size_t)M * (size_t)Kp);
    const size_t p_bytes = wave ? 0 : (size_t)splits * (size_t)M * (size_t)Np * sizeof(int32_t);
    if (w_bytes + a_bytes + p_bytes > kWorkspaceMax) return hipErrorNotSupported;
    uint8_t* ws = static_cast<uint8_t*>(workspace(st, w_bytes + a_bytes + p_bytes));
    if (ws == nullptr) return hipErrorNotSupported;
    uint8_t* Wp = ws;
    int8_t* Ap = reinterpret_cast<int8_t*>(ws + w_bytes);
    int32_t* P = reinterpret_cast<int32_t*>(ws + w_bytes + a_bytes);
    hipError_t e = ternix_hip::launch_pad_rows(dB, Wp, K, (int)Kp, NB, NB, (int)NBp,
                                               reinterpret_cast<const uint8_t*>(dA), reinterpret_cast<uint8_t*>(Ap),
                                               M, M, K, K, (int)Kp, st);
    if (e != hipSuccess) return e;
    if (wave)
        return ternix_hip::launch_skinny_wave(Ap, Wp, dC, M, (int)Kp, (int)Np, 16, 2, 1, (int)(Kp / 64), nullptr, st,
                                              os, N);
    if (skinny)
        return ternix_hip::launch_skinny(Ap, Wp, dC, M, (int)Kp, (int)Np, p.tb, p.kw, p.splits, p.sps, P, st, os,
                                         ternix_hip::ActQuant{}, p.dma, N);
    e = ternix_hip::launch_gemm(Ap, Wp, P, M, (int)Kp, (int)Np, 0, (int)Kp, 0, st, ternix_hip::OutScale{}, splits,
                                k_split);
    if (e != hipSuccess) return e;
    return ternix_hip::launch_splitk_reduce(P, dC, M, N, splits, os, st, (int)Np);
}

// The aligned kernels need 16-byte aligned operands, N/4 % 64 == 0 and whole k-steps: 64 rows for
// the skinny kernels, 128 for the pipelined GEMM.
bool needs_padding(const int8_t* dA, const uint8_t* dB, int K, int N, bool skinny) {
    return !(K % (skinny ? 64 : 128) == 0 && (N / 4) % 64 == 0 && reinterpret_cast<uintptr_t>(dB) % 16 == 0 &&
             reinterpret_cast<uintptr_t>(dA) % 16 == 0);
}

// Automatic path for one call: the padded copy for ragged or misaligned shapes when it applies,
// else the skinny kernels up to kSkinnyMaxM rows and the GEMM above.
hipError_t run_auto(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, hipStream_t st,
                    const ternix_hip::OutScale& os, int skinny_max) {
    static const bool pad_off = [] {
        const char* e = std::getenv("TERNIX_RAGGED_PAD");  // experiments: 0 keeps the generic kernels
        return e && e[0] == '0';
    }();
    if (!pad_off && needs_padding(dA, dB, K, N, M <= skinny_max)) {
        const hipError_t e = run_padded(dA, dB, dC, M, K, N, st, os, M <= skinny_max);
        if (e != hipErrorNotSupported) return e;
    }
    return M <= skinny_max ? run_skinny(dA, dB, dC, M, K, N, st, os) : run_gemm(dA, dB, dC, M, K, N, st, os);
}

// Tile-64 weights (the opt-in pre-permuted layout): M <= 32 runs the wave-pipelined kernel, whose
// per-wave DMA of one 1 KB block is a single contiguous read, K split by wave_splits at every K
// (the contiguous reads make it faster than the DMA kernel for long K too: cold cfg2 down 6.7 us
// against 7.8 on the row-major layout; TERNIX_SKINNY_WAVE="16,2,splits" forces the split count,
// experiments).  Larger M runs the LDS-DMA GEMMs with the contract layout's split-K planning.
hipError_t run_tile64(const int8_t* dA, const uint8_t* dWt, int32_t* dC, int M, int K, int N, hipStream_t st,
                      const ternix_hip::OutScale& os = ternix_hip::OutScale{}) {
    if (M <= 32) {
        const int nsteps = K / 64;
        int sp = wave_splits(M, K, N);
        if (const char* env = skinny_wave_env()) {
            int esw = 0, ensw = 0, esp = 0;
            if (std::sscanf(env, "%d,%d,%d", &esw, &ensw, &esp) == 3 && esp >= 1) sp = esp;
        }
        const int sps = (nsteps + sp - 1) / sp;
        const int splits = (nsteps + sps - 1) / sps;
        if (sps * 64 > ternix_hip::kMaxKPerAccumulator) return hipErrorInvalidValue;
        int32_t* partials = nullptr;
        if (splits > 1) {
            const size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(int32_t);
            if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(workspace(st, need));
        }
        int* cnt = partials ? arrival_counters(st, (size_t)(N / 4 / 16) * (size_t)((M + 15) / 16), M, splits, sps)
                            : nullptr;
        return ternix_hip::launch_skinny_wave(dA, dWt, dC, M, K, N, 16, 2, splits, sps, partials, st, os, 0,
                                              ternix_hip::ActQuant{}, 1, cnt);
    }
    return run_gemm(dA, dWt, dC, M, K, N, st, os, 1);
}

enum class Path { Auto, Skinny, Gemm, Naive };

int dispatch(Path path, const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M64, int64_t K64, int64_t N64,
             void* stream) {
    bool trivial = false;
    hipError_t e = validate(dA, dB, dC, M64, K64, N64, &trivial);
    if (e != hipSuccess) return (int)e;
    if (path == Path::Skinny && M64 > kSkinnyMaxM) return (int)hipErrorInvalidValue;
    if (trivial) return (int)hipSuccess;
    const int M = (int)M64, K = (int)K64, N = (int)N64;
    hipStream_t st = static_cast<hipStream_t>(stream);
    static const int auto_skinny_max = [] {
        const char* e = std::getenv("TERNIX_SKINNY_MAX_M");  // experiments only
        return e ? std::atoi(e) : kSkinnyMaxM;
    }();
    if (path == Path::Auto) return (int)run_auto(dA, dB, dC, M, K, N, st, ternix_hip::OutScale{}, auto_skinny_max);
    switch (path) {
        case Path::Skinny: e = run_skinny(dA, dB, dC, M, K, N, st); break;
        case Path::Gemm: e = run_gemm(dA, dB, dC, M, K, N, st); break;
        default: e = ternix_hip::launch_naive(dA, dB, dC, M, K, N, st); break;
    }
    return (int)e;
}

}  // namespace

extern "C" {

int ternix_hip_mul_mat_ternary(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K, int64_t N,
                               void* stream) {
    return dispatch(Path::Auto, dA, dB, dC, M, K, N, stream);
}

int ternix_hip_mul_mat_ternary_gemv(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K,
                                    int64_t N, void* stream) {
    return dispatch(Path::Skinny, dA, dB, dC, M, K, N, stream);
}

int ternix_hip_mul_mat_ternary_gemm(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K,
                                    int64_t N, void* stream) {
    return dispatch(Path::Gemm, dA, dB, dC, M, K, N, stream);
}

int ternix_hip_mul_mat_ternary_tiled(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K,
                                     int64_t N, void* stream) {
    // Same precondition as the reference tiled kernel (src/cuda_kernels.cu:135), checked first.
    if (M % 64 != 0 || N % 64 != 0 || K % 64 != 0) return (int)hipErrorInvalidValue;
    return dispatch(Path::Gemm, dA, dB, dC, M, K, N, stream);
}

int ternix_hip_mul_mat_ternary_naive(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K,
                                     int64_t N, void* stream) {
    return dispatch(Path::Naive, dA, dB, dC, M, K, N, stream);
}

int ternix_hip_mul_mat_ternary_host(const int8_t* A, const uint8_t* B_packed, int32_t* C, int64_t M, int64_t K,
                                    int64_t N, int variant) {
    bool trivial = false;
    hipError_t e = validate(A, B_packed, C, M, K, N, &trivial);
    if (e != hipSuccess) return (int)e;
    if (variant < TERNIX_HIP_AUTO || variant > TERNIX_HIP_TILED) return (int)hipErrorInvalidValue;
    if (variant == TERNIX_HIP_GEMV && M > kSkinnyMaxM) return (int)hipErrorInvalidValue;
    if (variant == TERNIX_HIP_TILED && (M % 64 != 0 || N % 64 != 0 || K % 64 != 0)) return (int)hipErrorInvalidValue;
    if (trivial) return (int)hipSuccess;
    const size_t a_bytes = (size_t)M * (size_t)K, b_bytes = (size_t)K * (size_t)(N / 4),
                 c_bytes = (size_t)M * (size_t)N * sizeof(int32_t);
    int8_t* dA = nullptr;
    uint8_t* dB = nullptr;
    int32_t* dC = nullptr;
    // hipMalloc of 0 bytes returns a null pointer; keep the pointers non-null for validation.
    if ((e = hipMalloc(reinterpret_cast<void**>(&dA), a_bytes ? a_bytes : 16)) != hipSuccess) goto done;
    if ((e = hipMalloc(reinterpret_cast<void**>(&dB), b_bytes ? b_bytes : 16)) != hipSuccess) goto done;
    if ((e = hipMalloc(reinterpret_cast<void**>(&dC), c_bytes)) != hipSuccess) goto done;
    if (a_bytes && (e = hipMemcpy(dA, A, a_bytes, hipMemcpyHostToDevice)) != hipSuccess) goto done;
    if (b_bytes && (e = hipMemcpy(dB, B_packed, b_bytes, hipMemcpyHostToDevice)) != hipSuccess) goto done;
    {
        int s;
        switch (variant) {
            case TERNIX_HIP_NAIVE: s = ternix_hip_mul_mat_ternary_naive(dA, dB, dC, M, K, N, nullptr); break;
            case TERNIX_HIP_GEMV: s = ternix_hip_mul_mat_ternary_gemv(dA, dB, dC, M, K, N, nullptr); break;
            case TERNIX_HIP_GEMM: s = ternix_hip_mul_mat_ternary_gemm(dA, dB, dC, M, K, N, nullptr); break;
            case TERNIX_HIP_TILED: s = ternix_hip_mul_mat_ternary_tiled(dA, dB, dC, M, K, N, nullptr); break;
            default: s = ternix_hip_mul_mat_ternary(dA, dB, dC, M, K, N, nullptr); break;
        }
        e = static_cast<hipError_t>(s);
    }
    if (e != hipSuccess) goto done;
    if ((e = hipDeviceSynchronize()) != hipSuccess) goto done;
    e = hipMemcpy(C, dC, c_bytes, hipMemcpyDeviceToHost);
done:
    // Free on every path; a free failure never masks the first error.
    if (dA) (void)hipFree(dA);
    if (dB) (void)hipFree(dB);
    if (dC) (void)hipFree(dC);
    return (int)e;
}

int ternix_hip_mul_mat_ternary_dequant(const int8_t* dA, const uint8_t* dB, float* dY, int64_t M, int64_t K,
                                       int64_t N, const float* dRowScale, float w_scale, void* stream) {
    bool trivial = false;
    hipError_t e = validate(dA, dB, dY, M, K, N, &trivial);
    if (e != hipSuccess) return (int)e;
    if (trivial) return (int)hipSuccess;
    if (dRowScale == nullptr) return (int)hipErrorInvalidValue;
    const int m = (int)M, k = (int)K, n = (int)N;
    hipStream_t st = static_cast<hipStream_t>(stream);
    ternix_hip::OutScale os;
    os.Y = dY;
    os.rs = dRowScale;
    os.ws = w_scale;
    // The int32 C never exists in memory on the fused paths; where one is needed (atomic split-K, K
    // chunks) it is kept in dY itself (same size) and converted in place.
    int32_t* c_alias = reinterpret_cast<int32_t*>(dY);
    e = run_auto(dA, dB, c_alias, m, k, n, st, os, kSkinnyMaxM);
    return (int)e;
}

int ternix_hip_mul_mat_ternary_swiglu(const int8_t* dA, const uint8_t* dB, float* dH, int64_t M, int64_t K,
                                      int64_t N, const float* dRowScale, float w_scale, int32_t* dScratch,
                                      void* stream) {
    bool trivial = false;
    hipError_t e = validate(dA, dB, dH, M, K, N, &trivial);
    if (e != hipSuccess) return (int)e;
    if (trivial) return (int)hipSuccess;
    if (dRowScale == nullptr) return (int)hipErrorInvalidValue;
    if (dScratch != nullptr && reinterpret_cast<uintptr_t>(dScratch) % alignof(int32_t) != 0)
        return (int)hipErrorInvalidValue;
    const int m = (int)M, k = (int)K, n = (int)N;
    hipStream_t st = static_cast<hipStream_t>(stream);
    ternix_hip::OutScale os;
    os.Y = dH;
    os.rs = dRowScale;
    os.ws = w_scale;
    os.swiglu = 1;
    e = run_auto(dA, dB, dScratch, m, k, n, st, os, kSkinnyMaxM);
    return (int)e;
}

int ternix_hip_rms_norm(float* dOut, const float* dIn, const float* dWeight, int64_t rows, int64_t size, float eps,
                        void* stream) {
    if (rows < 0 || size < 0 || rows > INT_MAX || size > INT_MAX) return (int)hipErrorInvalidValue;
    if (rows == 0 || size == 0) return (int)hipSuccess;
    if (dOut == nullptr || dIn == nullptr || dWeight == nullptr) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_rmsnorm(dIn, dWeight, eps, dOut, nullptr, nullptr, (int)rows, (int)size,
                                           static_cast<hipStream_t>(stream));
}

int ternix_hip_rms_norm_quantize(int8_t* dQ, float* dRowScale, const float* dIn, const float* dWeight, int64_t rows,
                                 int64_t size, float eps, void* stream) {
    if (rows < 0 || size < 0 || rows > INT_MAX || size > INT_MAX) return (int)hipErrorInvalidValue;
    if (rows == 0) return (int)hipSuccess;
    if (dRowScale == nullptr || (size > 0 && (dQ == nullptr || dIn == nullptr || dWeight == nullptr)))
        return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_rmsnorm(dIn, dWeight, eps, nullptr, dQ, dRowScale, (int)rows, (int)size,
                                           static_cast<hipStream_t>(stream));
}

int ternix_hip_swiglu(float* dOut, const float* dIn, int64_t size, void* stream) {
    if (size < 0) return (int)hipErrorInvalidValue;
    if (size < 2) return (int)hipSuccess;
    if (dOut == nullptr || dIn == nullptr) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_swiglu(dIn, dOut, (size_t)size / 2, static_cast<hipStream_t>(stream));
}

namespace {

// Feed-forward workspace: q1 [M][H] int8 | rs1 [M] | h [M][F] f32 | q2 [M][F] int8 | rs2 [M] |
// scratch [M][2F] int32 (used only when a matmul cannot fuse its epilogue); 256-byte aligned regions.
struct FfnLayout {
    size_t q1, rs1, h, q2, rs2, scratch, total;
};
FfnLayout ffn_layout(int64_t M, int64_t H, int64_t F) {
    auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
    FfnLayout l{};
    size_t o = 0;
    l.q1 = o; o = up(o + (size_t)M * (size_t)H);
    l.rs1 = o; o = up(o + 4 * (size_t)M);
    l.h = o; o = up(o + 4 * (size_t)M * (size_t)F);
    l.q2 = o; o = up(o + (size_t)M * (size_t)F);
    l.rs2 = o; o = up(o + 4 * (size_t)M);
    l.scratch = o; o = up(o + 8 * (size_t)M * (size_t)F);
    l.total = o;
    return l;
}

}  // namespace

size_t ternix_hip_ffn_workspace_size(int64_t M, int64_t H, int64_t F) {
    if (M < 0 || H < 0 || F < 0) return 0;
    return ffn_layout(M, H, F).total;
}

int ternix_hip_ffn_forward(float* dY, const float* dX, const float* dNormWeight, float eps, const uint8_t* dWgu,
                           float ws_gu, const uint8_t* dWd, float ws_d, int64_t M, int64_t H, int64_t F,
                           void* dWorkspace, size_t workspace_bytes, void* stream) {
    if (M < 0 || H < 0 || F < 0 || M > INT_MAX || H > INT_MAX || 2 * F > INT_MAX) return (int)hipErrorInvalidValue;
    if (H % 4 != 0 || F % 2 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || H == 0) return (int)hipSuccess;
    const FfnLayout l = ffn_layout(M, H, F);
    if (dWorkspace == nullptr || workspace_bytes < l.total || reinterpret_cast<uintptr_t>(dWorkspace) % 256 != 0)
        return (int)hipErrorInvalidValue;
    if (dY == nullptr || dX == nullptr || dNormWeight == nullptr || (F > 0 && (dWgu == nullptr || dWd == nullptr)))
        return (int)hipErrorInvalidValue;
    char* ws = static_cast<char*>(dWorkspace);
    int8_t* q1 = reinterpret_cast<int8_t*>(ws + l.q1);
    float* rs1 = reinterpret_cast<float*>(ws + l.rs1);
    float* h = reinterpret_cast<float*>(ws + l.h);
    int8_t* q2 = reinterpret_cast<int8_t*>(ws + l.q2);
    float* rs2 = reinterpret_cast<float*>(ws + l.rs2);
    int32_t* scratch = reinterpret_cast<int32_t*>(ws + l.scratch);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, hd = (int)H, f = (int)F;
    // Decode shapes: the RMSNorm + quantisation of x and the requantisation of h run inside the two
    // skinny GEMVs (fused activation prologue, bit-identical to the standalone kernels), leaving
    // GEMV + reduce twice.  Otherwise: the four separate launches.
    if (m <= kSkinnyMaxM && F > 0) {
        ternix_hip::OutScale os1;
        os1.Y = h;
        os1.rs = rs1;
        os1.ws = ws_gu;
        os1.swiglu = 1;
        ternix_hip::ActQuant aq1;
        aq1.mode = 2;
        aq1.X = dX;
        aq1.G = dNormWeight;
        aq1.eps = eps;
        aq1.rs_out = rs1;
        ternix_hip::OutScale os2;
        os2.Y = dY;
        os2.rs = rs2;
        os2.ws = ws_d;
        ternix_hip::ActQuant aq2;
        aq2.mode = 1;
        aq2.X = h;
        aq2.rs_out = rs2;
        const SkinnyPlan p1 = plan_skinny(m, hd, 2 * f), p2 = plan_skinny(m, f, hd);
        if (ternix_hip::skinny_short_ok(dWgu, m, hd, 2 * f, p1.sps, p1.splits) &&
            ternix_hip::skinny_short_ok(dWd, m, f, hd, p2.sps, p2.splits)) {
            hipError_t e = run_skinny(nullptr, dWgu, scratch, m, hd, 2 * f, st, os1, aq1);
            if (e != hipSuccess) return (int)e;
            return (int)run_skinny(nullptr, dWd, reinterpret_cast<int32_t*>(dY), m, f, hd, st, os2, aq2);
        }
    }
    int s = ternix_hip_rms_norm_quantize(q1, rs1, dX, dNormWeight, M, H, eps, stream);
    if (s != 0) return s;
    s = ternix_hip_mul_mat_ternary_swiglu(q1, dWgu, h, M, H, 2 * F, rs1, ws_gu, scratch, stream);
    if (s != 0) return s;
    s = (int)ternix_hip::launch_quantize_rows(h, q2, rs2, (int)M, (int)F, st);
    if (s != 0) return s;
    return ternix_hip_mul_mat_ternary_dequant(q2, dWd, dY, M, F, H, rs2, ws_d, stream);
}

int ternix_hip_ffn_forward_tile64(float* dY, const float* dX, const float* dNormWeight, float eps,
                                  const uint8_t* dWguT, float ws_gu, const uint8_t* dWdT, float ws_d, int64_t M,
                                  int64_t H, int64_t F, void* dWorkspace, size_t workspace_bytes, void* stream) {
    if (M < 0 || H < 0 || F < 0 || M > INT_MAX || H > INT_MAX || 2 * F > INT_MAX) return (int)hipErrorInvalidValue;
    if (M == 0 || H == 0) return (int)hipSuccess;
    // The tile-64 matmul contract for both weight matrices: K % 128, N % 256 (H x 2F and F x H).
    if (H % 256 != 0 || F % 128 != 0 || (2 * F) % 256 != 0 || (size_t)H * (size_t)(2 * F / 4) >= ((size_t)1 << 32) ||
        (size_t)F * (size_t)(H / 4) >= ((size_t)1 << 32))
        return (int)hipErrorInvalidValue;
    const FfnLayout l = ffn_layout(M, H, F);
    if (dWorkspace == nullptr || workspace_bytes < l.total || reinterpret_cast<uintptr_t>(dWorkspace) % 256 != 0)
        return (int)hipErrorInvalidValue;
    if (dY == nullptr || dX == nullptr || dNormWeight == nullptr || dWguT == nullptr || dWdT == nullptr ||
        reinterpret_cast<uintptr_t>(dWguT) % 16 != 0 || reinterpret_cast<uintptr_t>(dWdT) % 16 != 0)
        return (int)hipErrorInvalidValue;
    char* ws = static_cast<char*>(dWorkspace);
    int8_t* q1 = reinterpret_cast<int8_t*>(ws + l.q1);
    float* rs1 = reinterpret_cast<float*>(ws + l.rs1);
    float* h = reinterpret_cast<float*>(ws + l.h);
    int8_t* q2 = reinterpret_cast<int8_t*>(ws + l.q2);
    float* rs2 = reinterpret_cast<float*>(ws + l.rs2);
    int32_t* scratch = reinterpret_cast<int32_t*>(ws + l.scratch);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, hd = (int)H, f = (int)F;
    ternix_hip::OutScale os1;
    os1.Y = h;
    os1.rs = rs1;
    os1.ws = ws_gu;
    os1.swiglu = 1;
    hipError_t e;
    if (m <= 16 && hd <= 4096) {
        // RMSNorm + quantisation of x inside the gate/up GEMV (one launch, whole rows per workgroup).
        ternix_hip::ActQuant aq1;
        aq1.mode = 2;
        aq1.X = dX;
        aq1.G = dNormWeight;
        aq1.eps = eps;
        aq1.rs_out = rs1;
        e = ternix_hip::launch_skinny_wave(nullptr, dWguT, scratch, m, hd, 2 * f, 16, 2, 1, hd / 64, nullptr, st, os1,
                                           0, aq1, 1);
    } else {
        const int s = ternix_hip_rms_norm_quantize(q1, rs1, dX, dNormWeight, M, H, eps, stream);
        if (s != 0) return s;
        e = run_tile64(q1, dWguT, scratch, m, hd, 2 * f, st, os1);
    }
    if (e != hipSuccess) return (int)e;
    e = ternix_hip::launch_quantize_rows(h, q2, rs2, m, f, st);
    if (e != hipSuccess) return (int)e;
    ternix_hip::OutScale os2;
    os2.Y = dY;
    os2.rs = rs2;
    os2.ws = ws_d;
    return (int)run_tile64(q2, dWdT, reinterpret_cast<int32_t*>(dY), m, f, hd, st, os2);
}

int ternix_hip_quantize_activations(const float* dX, int8_t* dQ, float* dRowScale, int64_t M, int64_t K,
                                    void* stream) {
    if (M < 0 || K < 0 || M > INT_MAX || K > INT_MAX) return (int)hipErrorInvalidValue;
    if (M == 0) return (int)hipSuccess;
    if (dRowScale == nullptr || (K > 0 && (dX == nullptr || dQ == nullptr))) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_quantize_rows(dX, dQ, dRowScale, (int)M, (int)K, static_cast<hipStream_t>(stream));
}

int ternix_hip_pack_ternary_weights(uint8_t* dPacked, const int8_t* dW, size_t size, void* stream) {
    if (size / 4 == 0) return (int)hipSuccess;
    if (dPacked == nullptr || dW == nullptr) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_pack(dPacked, dW, size, static_cast<hipStream_t>(stream));
}

int ternix_hip_unpack_ternary_weights(int8_t* dW, const uint8_t* dPacked, size_t size, void* stream) {
    if (size / 4 == 0) return (int)hipSuccess;
    if (dPacked == nullptr || dW == nullptr) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_unpack(dW, dPacked, size, static_cast<hipStream_t>(stream));
}

int ternix_hip_interleave_weights_offline(uint8_t* dOut, const uint8_t* dPacked, size_t size, void* stream) {
    const size_t nbytes = size / 4;
    if (nbytes == 0) return (int)hipSuccess;
    if (dOut == nullptr || dPacked == nullptr) return (int)hipErrorInvalidValue;
    if (dOut == dPacked) return (int)hipSuccess;
    return (int)hipMemcpyAsync(dOut, dPacked, nbytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream));
}

int ternix_hip_interleave_weights_tile64(uint8_t* dOut, const uint8_t* dPacked, int64_t K, int64_t N, void* stream) {
    if (K < 0 || N < 0 || N % 4 != 0 || K % 64 != 0 || (N / 4) % 16 != 0 || K > INT_MAX || N > INT_MAX)
        return (int)hipErrorInvalidValue;
    if (K == 0 || N == 0) return (int)hipSuccess;
    if (dOut == nullptr || dPacked == nullptr || dOut == dPacked) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_tile64(dPacked, dOut, (int)K, (int)N, static_cast<hipStream_t>(stream));
}

int ternix_hip_mul_mat_ternary_tile64(const int8_t* dA, const uint8_t* dWt, int32_t* dC, int64_t M, int64_t K,
                                      int64_t N, void* stream) {
    bool trivial = false;
    hipError_t e = validate(dA, dWt, dC, M, K, N, &trivial);
    if (e != hipSuccess) return (int)e;
    if (K % 128 != 0 || N % 256 != 0 || (size_t)K * (size_t)(N / 4) >= ((size_t)1 << 32) ||
        reinterpret_cast<uintptr_t>(dA) % 16 != 0 || reinterpret_cast<uintptr_t>(dWt) % 16 != 0)
        return (int)hipErrorInvalidValue;
    if (trivial) return (int)hipSuccess;
    return (int)run_tile64(dA, dWt, dC, (int)M, (int)K, (int)N, static_cast<hipStream_t>(stream));
}

int ternix_hip_mul_mat_ternary_tile64_dequant(const int8_t* dA, const uint8_t* dWt, float* dY, int64_t M, int64_t K,
                                              int64_t N, const float* dRowScale, float w_scale, void* stream) {
    bool trivial = false;
    hipError_t e = validate(dA, dWt, dY, M, K, N, &trivial);
    if (e != hipSuccess) return (int)e;
    if (K % 128 != 0 || N % 256 != 0 || (size_t)K * (size_t)(N / 4) >= ((size_t)1 << 32) ||
        reinterpret_cast<uintptr_t>(dA) % 16 != 0 || reinterpret_cast<uintptr_t>(dWt) % 16 != 0)
        return (int)hipErrorInvalidValue;
    if (trivial) return (int)hipSuccess;
    if (dRowScale == nullptr) return (int)hipErrorInvalidValue;
    ternix_hip::OutScale os;
    os.Y = dY;
    os.rs = dRowScale;
    os.ws = w_scale;
    // As in ternix_hip_mul_mat_ternary_dequant: an int32 C, where a path needs one, lives in dY.
    return (int)run_tile64(dA, dWt, reinterpret_cast<int32_t*>(dY), (int)M, (int)K, (int)N,
                           static_cast<hipStream_t>(stream), os);
}

const char* ternix_hip_error_string(int status) {
    const char* s = hipGetErrorString(static_cast<hipError_t>(status));
    return s ? s : "unknown error";
}

int ternix_hip_version(void) { return 100; }

}  // extern "C"
