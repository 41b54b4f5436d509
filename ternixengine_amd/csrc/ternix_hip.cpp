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
#include <cstdarg>
#include <map>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

#include "ternary_kernels.h"

namespace ternix_hip {
namespace {
// Switch values + 1 (0: not set), per key and index; relaxed atomics because a test may set a switch
// while another thread is inside a call (the call then sees the old or the new value).
std::atomic<int> g_debug[DBG_COUNT][4];
}  // namespace

int debug_get(DebugKey key, int idx) {
    if ((int)key < 0 || (int)key >= DBG_COUNT || idx < 0 || idx > 3) return -1;
    return g_debug[key][idx].load(std::memory_order_relaxed) - 1;
}
}  // namespace ternix_hip

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
// Key of a stream's buffers: (device, stream handle, thread).  hipStreamPerThread is one handle that
// names a different real stream in every host thread, so calls from two threads through it may run
// concurrently and must not share counters or tickets: for that handle the key also holds the
// calling thread.  Every other handle names one stream, whichever thread uses it (the null stream
// included: work on it runs in submission order), and the thread part is left empty.
struct WsKey {
    int dev;
    hipStream_t st;
    std::thread::id thread;
    bool operator<(const WsKey& o) const {
        if (dev != o.dev) return dev < o.dev;
        if (st != o.st) return std::less<hipStream_t>()(st, o.st);
        return thread < o.thread;
    }
};
WsKey ws_key(int dev, hipStream_t st) {
    return WsKey{dev, st, st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id()};
}
std::map<WsKey, Workspace> g_ws;
std::atomic<long long> g_alloc_count{0};  // device allocations made by the library (a test hook)

// Every device allocation of the library goes through here.  A failed hipMalloc leaves its error in
// the thread's last-error slot, which the launchers read back with hipGetLastError after their
// launch; the caller falls back to a path that needs no allocation, so the error is cleared here.
hipError_t lib_malloc(void** p, size_t bytes) {
    g_alloc_count.fetch_add(1, std::memory_order_relaxed);
    const hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
    }
    return e;
}

void* workspace(hipStream_t st, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& w = g_ws[ws_key(dev, st)];
    if (w.bytes >= bytes) return w.ptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    // Grow geometrically (at least 8 MiB, at least double), capped at kWorkspaceMax unless the
    // request itself is larger, rounded to 1 MiB.
    const size_t grown = std::min(std::max(size_t(8) << 20, 2 * w.bytes), kWorkspaceMax);
    size_t nb = std::max(bytes, grown);
    nb = (nb + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    void* p = nullptr;
    if (lib_malloc(&p, nb) != hipSuccess) return nullptr;
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
// The DBG_WAVE_LAST switch overrides it (tests; 0 turns the scheme off).
int last_max_splits() {
    const int v = ternix_hip::debug_get(ternix_hip::DBG_WAVE_LAST);
    return v >= 0 ? v : 5;
}

// Arrival counters of the wave GEMV's single-launch split-K (kCounterSlots ints per (device, stream),
// zeroed once when allocated; every call leaves them zero).  nullptr during graph capture before
// they exist, when `need` exceeds the slots or for more than last_max_splits() splits: the caller
// then uses the reduce launch.
constexpr size_t kCounterSlots = size_t(1) << 16;
// Up to 4 rows with long k-ranges per split (>= 8 steps) also sum up to 8 splits inside the
// launch: their workgroups finish far apart, so the arrivals hardly queue (cold cfg3 M=4 down:
// 8 splits 9.8 us against 11.5 for the DMA-staged kernel and its reduce launch; 12 splits of
// cfg2 down 8.6 us against 7.8 with 8; 16 splits of tile-64 cfg3 M=4 down 12.2 against 9.3 us
// with the reduce launch).
bool counters_wanted(size_t need, int M, int splits, int sps) {
    const int lim = last_max_splits();
    return !(lim <= 0 || (splits > lim && !(M <= 4 && sps >= 8 && splits <= 8)) || need > kCounterSlots);
}
// Self-zeroing atomic GEMV tickets (skinny_kernels.hip, SK_ATOMZ): two 64-bit words per strip after
// the arrival counters in the same zero-initialised buffer; they advance with every call and are
// never reset.
constexpr size_t kTicketStrips = size_t(1) << 14;
int* counter_buffer(hipStream_t st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& w = g_ws[ws_key(dev, st)];
    if (w.counters) return w.counters;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    void* p = nullptr;
    constexpr size_t words = kCounterSlots + 4 * kTicketStrips;
    if (lib_malloc(&p, words * sizeof(int)) != hipSuccess) return nullptr;
    // A fill kernel, not hipMemsetAsync (never inside capture here anyway: checked above).
    if (ternix_hip::launch_zero(static_cast<int32_t*>(p), words, st) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(p);
        return nullptr;
    }
    w.counters = static_cast<int*>(p);
    return w.counters;
}
int* arrival_counters(hipStream_t st, size_t need, int M, int splits, int sps) {
    return counters_wanted(need, M, splits, sps) ? counter_buffer(st) : nullptr;
}
unsigned long long* zero_tickets(hipStream_t st, size_t strips) {
    if (strips > kTicketStrips) return nullptr;
    int* b = counter_buffer(st);
    return b ? reinterpret_cast<unsigned long long*>(b + kCounterSlots) : nullptr;
}

// Execution context of one call: the stream, where split-K partials and padded copies live, and a
// dry-run mode for planning queries.
//   * library-owned workspace (default): the per-(device, stream) buffers above;
//   * caller-owned workspace (ternix_hip_mul_mat_ternary_ws, and the fixed device scratch of
//     ternix_hip_mul_mat_ternary_noalloc): a request larger than the buffer gets nullptr (the planners
//     then take a path that needs less), and the in-launch split sum is not used (its counters must be
//     zero between calls, which only library-owned memory guarantees);
//   * dry run: requests are recorded, nothing is launched, and the chosen kernels are described in
//     `desc`; under the caller-owned rules with an unbounded buffer for
//     ternix_hip_mul_mat_ternary_workspace_size, under the library-owned ones (counters granted when
//     they would be, nothing allocated) for ternix_hip_plan_describe.
struct Ctx {
    hipStream_t st = nullptr;
    char* caller = nullptr;
    size_t caller_bytes = 0;
    bool use_caller = false;
    bool dry = false;
    bool dry_library = false;  // dry run under the library-owned rules (plan description)
    size_t need = 0;
    char desc[192] = {0};

    void* get(size_t bytes) {
        if (bytes > kWorkspaceMax) return nullptr;
        if (dry) {
            need = std::max(need, bytes);
            return reinterpret_cast<void*>(uintptr_t(4096));  // never dereferenced: nothing launches
        }
        if (use_caller) return bytes <= caller_bytes ? caller : nullptr;
        return workspace(st, bytes);
    }
    int* counters(size_t slots, int M, int splits, int sps) {
        if (dry)  // never dereferenced: nothing launches
            return dry_library && counters_wanted(slots, M, splits, sps) ? reinterpret_cast<int*>(uintptr_t(4096))
                                                                        : nullptr;
        if (use_caller) return nullptr;
        return arrival_counters(st, slots, M, splits, sps);
    }
    // Tickets of the self-zeroing atomic GEMV, under the same ownership rules as the counters.
    unsigned long long* tickets(size_t strips) {
        if (dry)  // never dereferenced: nothing launches
            return dry_library && strips <= kTicketStrips ? reinterpret_cast<unsigned long long*>(uintptr_t(4096))
                                                          : nullptr;
        if (use_caller) return nullptr;
        return zero_tickets(st, strips);
    }
    void note(const char* fmt, ...) __attribute__((format(printf, 2, 3))) {
        if (!dry) return;
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(desc, sizeof(desc), fmt, ap);
        va_end(ap);
    }
};
// Library-owned-workspace context of a stream (a fresh temporary per call).
struct CtxOf {
    Ctx c;
    explicit CtxOf(hipStream_t st) { c.st = st; }
    operator Ctx&() { return c; }
};
inline Ctx& ctx_ref(CtxOf&& t) { return t.c; }
#define ctx_of(st) ctx_ref(CtxOf(st))
// Launch unless planning only.
#define TX_LAUNCH(c, expr) ((c).dry ? hipSuccess : (expr))

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
    const int forced = ternix_hip::debug_get(ternix_hip::DBG_SKINNY_DMA, 1);  // split count (tuning)
    if (forced > 0) sps = (nsteps + std::min(forced, nsteps) - 1) / std::min(forced, nsteps);
    SkinnyPlan p{1, 1, (nsteps + sps - 1) / sps, sps, ns};
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

// The DBG_SKINNY_WAVE switch set to 0 turns the wave-pipelined skinny kernel off (tests).
bool wave_kernel_enabled() { return ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE) != 0; }

constexpr int kWaveMaxM = 32;

// K split of the wave-pipelined kernel (one workgroup per strip of sw bytes, m-group and split).
// 16-byte strips (tile-64 weights): enough workgroups for about 2.75 per CU, and for M <= 4 up to 7
// per CU, one per 8 KB of weights (more weight loads in flight on the large decode matrices, where
// the extra partial sums cost little).  32-byte strips (row-major weights): about one workgroup per
// CU.  At least two k-steps per split.  Measured on MI355X with cold weights (512 MiB pools, one
// box): 16-byte strips cfg2 up 9.35 -> 8.4 us against no split, tile-64 cfg5 big 17.8 -> 15.3 us;
// 32-byte strips against 16-byte ones, each with its split: cfg1 6.72 -> 6.14 us, cfg2 up 8.41 ->
// 7.56, cfg3 M=4 up 12.3 -> 10.9, M=16 up 13.8 -> 11.9, M=16 down 13.95 -> 11.8.
int wave_splits(int M, int K, int N, int sw = 16) {
    const long nsteps = K / 64, units = (long)(N / 4 / sw) * ((M + 15) / 16), cus = cu_count();
    long target = cus * 11 / 4;
    if (M <= 4) target = std::max(target, std::min(7 * cus, (long)K * (N / 4) / 8192));
    if (sw == 32) target = cus;
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

// Plan of the whole-K deep GEMV (skinny_deep.hip); sw == 0 when it does not take the call.  Automatic
// only on tile-64 weights, for short K (<= 4096) and at most two workgroups per CU: measured on MI355X
// with cold weights against the split wave kernel, cfg1 5.31 -> 4.77 us, cfg2 up 6.25 -> 5.02, cfg3
// M=4 up 8.37 -> 6.45, M=16 up 10.68 -> 7.55; the long-K down projections and cfg5 big are slower
// whole (cfg2 down 6.80 -> 7.12, cfg5 big 14.9 -> 16.9).  On row-major weights only when forced.
struct DeepPlan {
    int sw, nw, nsw, splits, sps;
};
DeepPlan plan_deep(const int8_t* dA, const uint8_t* dB, int M, int K, int N, bool tiled) {
    DeepPlan p{0, 0, 0, 1, 0};
    const int nsteps = K / 64;
    if (ternix_hip::debug_get(ternix_hip::DBG_DEEP) > 0) {  // forced plan (tests and tuning)
        p.sw = ternix_hip::debug_get(ternix_hip::DBG_DEEP, 0);
        p.nw = ternix_hip::debug_get(ternix_hip::DBG_DEEP, 1);
        p.nsw = ternix_hip::debug_get(ternix_hip::DBG_DEEP, 2);
        const int sp = std::max(1, ternix_hip::debug_get(ternix_hip::DBG_DEEP, 3));
        if (M > 16 || !ternix_hip::skinny_deep_config_ok(p.sw, p.nw, p.nsw) ||
            !ternix_hip::skinny_deep_ok(dA, dB, M, K, N, p.sw))
            return DeepPlan{0, 0, 0, 1, 0};
        p.sps = (nsteps + sp - 1) / sp;
        p.splits = (nsteps + p.sps - 1) / p.sps;
        if (p.sps * 64 > ternix_hip::kMaxKPerAccumulator) return DeepPlan{0, 0, 0, 1, 0};
        return p;
    }
    if (!tiled || ternix_hip::debug_get(ternix_hip::DBG_DEEP) == 0 || M > 16 || K > 4096 ||
        !ternix_hip::skinny_deep_ok(dA, dB, M, K, N, 16) || (long)(N / 64) > 2L * cu_count())
        return p;
    return DeepPlan{16, 16, 4, 1, nsteps};
}

// The self-zeroing atomic split plan of the wave-pipelined GEMV (the measurements are with its call
// in run_skinny): true when it takes the call (*e then holds the launch status).  Int32 output, aligned
// operands (skinny_wave_ok), one ticket pair per (m-group, strip).
// n_out > 0: a padded problem (K, N the padded sizes) whose C holds its n_out real columns.
bool run_atomic_wave(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, Ctx& c, hipError_t* e,
                     int n_out = 0, const char* prefix = "") {
    const hipStream_t st = c.st;
    (void)st;
    const int atomic_max_m = ternix_hip::debug_get(ternix_hip::DBG_M1_ATOMIC, 1) > 0 ? ternix_hip::debug_get(ternix_hip::DBG_M1_ATOMIC, 1) : 64;
    if (!(M <= std::min(64, atomic_max_m) && dC != nullptr && wave_kernel_enabled() &&
          ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE) < 0 && ternix_hip::debug_get(ternix_hip::DBG_M1_ATOMIC) != 0))
        return false;
    const int NB = N / 4, nsteps = K / 64, cus = cu_count(), mgroups = (M + 15) / 16;
    int sw = 0, sp = 0;
    if (M == 1 && K <= 4096 && NB <= 1024 && NB % 16 == 0) {
        sw = 16;
        sp = std::max(1, std::min(6, cus / (NB / 16)));
    } else if (M == 1 && NB % 32 == 0 && (long)(NB / 32) * 4 * 50 <= (long)cus * 53) {
        sw = 32;
        sp = std::min(cus / (NB / 32), std::max(1, nsteps / 4));
    } else if (M > 1 && NB % 32 == 0) {
        // About one workgroup per CU for one m-group; about two, and at most 6 splits, for several
        // (measured on MI355X, cold, us, splits in brackets: 24x2560x6912 11.8 [1, another plan] ->
        // 7.26-7.64 [4-6], 24x4096x11008 13.4 -> 10.6 [3], 33x4096x4096 9.8 [2] -> 7.9-8.0 [4-6],
        // 64x6912x2560 10.3 [3] -> 9.4 [6]).
        sw = 32;
        const long per = mgroups > 1 ? 2L * cus * 53 / 50 : (long)cus * 53 / 50;
        sp = (int)std::min<long>(per / ((long)(NB / 32) * mgroups), std::max(1, nsteps / 4));
        if (mgroups > 1) sp = std::min(sp, 6);
    }
    const int fsw = ternix_hip::debug_get(ternix_hip::DBG_WAVE_SW, 0), fsp = ternix_hip::debug_get(ternix_hip::DBG_WAVE_SW, 1);
    if ((fsw == 16 || fsw == 32) && fsp > 1 && NB % fsw == 0) {  // forced split plan (tests and tuning)
        sw = fsw;
        sp = std::min(fsp, nsteps);
    }
    if (!(sw > 0 && sp > 1 && ternix_hip::skinny_wave_ok(dA, dB, M, K, N, sw))) return false;
    int sps = (nsteps + sp - 1) / sp, splits = (nsteps + sps - 1) / sps;
    if (!(splits > 1 && sps * 64 <= ternix_hip::kMaxKPerAccumulator)) return false;
    // 33..64 rows (several m-groups) only with short k-ranges per split: against the narrow-tile GEMM,
    // measured on MI355X (cold): 64x4096x4096 14.1 -> 10.6 us (32 steps per split), 64x6912x2560 11.1
    // -> 10.4 (36), but 64x11008x4096 15.6 -> 21.5 (86) and 64x14336x4096 17.9 -> 26.4 (112); with
    // the two-per-CU split count, 48x4096x11008 14.0 (32 steps) against 13.0 and 64x2560x6912 9.3
    // (20) against 9.6 for the GEMM, so at most 24 steps per split.  Up to
    // 32 rows it wins wherever it splits K (24 and 32 rows: 1.11-1.42x against the in-launch sums and
    // the reduce launch on five decode shapes).
    if (M > 32 && sps > 24 && fsp <= 1) return false;
    // ... and not where the narrow GEMM runs K whole on at least 96 of its 64-column tiles (on MI355X,
    // cold, wave / GEMM: 64x2560x6912 8.99 / 7.79 us, 48x2560x6912 8.08 / 7.61, 48x2048x8192 8.63 /
    // 6.91, 36x2048x8192 7.64 / 6.88; with fewer tiles the wave kernel stays faster, 48x4096x4096 7.67 /
    // 9.86, 64x6912x2560 8.70 / 10.41).
    if (M > 32 && fsp <= 1 && ternix_hip::gemm_narrow_wanted(M, K, N) && (N / 4) / 16 >= 96) return false;
    // Column waves (M <= 4, 32-byte parts): a workgroup owns a 128-byte strip and each wave one
    // 32-byte part over the workgroup's whole k-range, so the four parts of each weight line reach one
    // CU together.  More K splits for the same workgroups (more atomic adds per output), so only where
    // one round of workgroups (>= 3/4 of the CUs, none doubled) takes <= 32 splits.  Measured on
    // MI355X, cold weights (us, current plan -> column waves): 4x4096x11008 8.08 -> 7.47,
    // 4x11008x4096 8.4 -> 8.13, 4x4096x14336 9.85 -> 8.78, 1x14336x4096 9.0 -> 8.36, cfg2 up 5.35 ->
    // 5.27; cfg2 down (5 strips: 36 splits for 180 workgroups) 5.64 -> 5.93 stays.
    int cw = 0, cw_sps = 0;
    const int fcw = ternix_hip::debug_get(ternix_hip::DBG_WAVE_SW, 2);  // 1 / 0: force on / off (tests)
    if (M <= 4 && sw == 32 && n_out == 0 && fcw != 0 && fsp <= 1) {
        const long n_cw = (NB + 127) / 128;
        long best = 0;
        for (int q = 1; q * 64 <= ternix_hip::kMaxKPerAccumulator && q <= nsteps; ++q) {
            const long sc = (nsteps + q - 1) / q;
            if (sc >= 2 && sc <= 32 && n_cw * sc <= cus && n_cw * sc > best) {
                best = n_cw * sc;
                cw_sps = q;
            }
        }
        if (best > 0 && (best * 4 >= (long)cus * 3 || fcw == 1)) cw = 1;
    } else if (M <= 4 && sw == 32 && n_out == 0 && fcw == 1 && fsp > 1) {
        cw = 1;  // forced split count with column waves (tuning)
    }
    const int sps0 = sps, splits0 = splits;  // the plan without column waves
    if (cw && cw_sps > 0) {
        sps = cw_sps;
        splits = (nsteps + sps - 1) / sps;
    }
    // Up to 4 rows, more than 12 k-steps per workgroup (shapes the whole-line GEMV declines): the
    // DMA-staged kernel streams them faster (on MI355X, cold: 1x28672x8192 19.2 -> 12.5 us,
    // 4x28672x8192 22.5 -> 14.2, 1x14336x8192 11.0 -> 8.9, 1x32768x4096 12.4 -> 9.7, 4x11008x16384
    // 18.4 -> 12.1, 3x24576x6144 14.8 -> 11.0).
    if (M <= 4 && sps > 12 && fsp <= 1 && ternix_hip::skinny_dma_ok(dA, dB, M, K, N, 1)) return false;
    unsigned long long* tk = ternix_hip::debug_get(ternix_hip::DBG_SELF_ZERO) != 0 && splits <= 64
                                 ? c.tickets(ternix_hip::ticket_units(cw ? (size_t)((NB + 127) / 128) : (size_t)(NB / sw) * (size_t)mgroups))
                                 : nullptr;
    if (cw && !tk) {  // column waves need the tickets: the plan without them (zero fill at M = 1)
        cw = 0;
        sps = sps0;
        splits = splits0;
        if (ternix_hip::debug_get(ternix_hip::DBG_SELF_ZERO) != 0 && splits <= 64)
            tk = c.tickets(ternix_hip::ticket_units((size_t)(NB / sw) * (size_t)mgroups));
    }
    if (tk)
        c.note("%sskinny_wave_kernel sw=%d nsw=2 splits=%d%s (splits added with int32 atomics into C zeroed "
               "by each strip's first split)", prefix, sw, splits, cw ? " column waves" : "");
    else if (M == 1 && n_out == 0)
        c.note("zero_kernel + skinny_wave_kernel sw=%d nsw=2 splits=%d (splits added with int32 atomics)", sw, splits);
    if (!(tk || (M == 1 && n_out == 0))) return false;
    *e = TX_LAUNCH(c, ternix_hip::launch_skinny_wave(dA, dB, dC, M, K, N, sw, 2, splits, sps, nullptr, st,
                                                     ternix_hip::OutScale{}, n_out, ternix_hip::ActQuant{}, 0, nullptr, tk, cw));
    return true;
}

// The whole-line GEMV (line_gemv.hip): true when it takes the call (*e then holds the launch status).
// M <= 4, the library's tickets (one set per 128-byte strip, spread as ticket_stride says), and
// either an int32 output into a 16-byte aligned C, or a float output (os.Y, optionally SwiGLU) through
// the kernel's last-arriver epilogue with dC as the int32 buffer of the sums (dC == os.Y only without
// SwiGLU), with the activations given as int8 or quantised inside the kernel from fp32 rows (aq).
// Plan: the fewest k-steps per workgroup (2, 3, 4, 6 or 8) whose grid stays within about one
// workgroup per CU (<= 250 workgroups) with at most 64 splits per strip; none for wide matrices that
// would need more (the DMA-staged and wave kernels keep those).  The DBG_LINE switch turns it off (0)
// or forces the k-steps [0] and data waves [1]; [2] forces the unit order, [3] raises the row limit
// (up to 16).  Ragged operands (any K, N % 4 == 0, any A / W address) take the kernel's ragged form
// with an int32 output.
bool run_line_gemv(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, Ctx& c, hipError_t* e,
                   const ternix_hip::OutScale& os = ternix_hip::OutScale{},
                   const ternix_hip::ActQuant& aq = ternix_hip::ActQuant{}, int tiled = 0, bool pad_alt = false) {
    const int fs = ternix_hip::debug_get(ternix_hip::DBG_LINE, 0), fw = ternix_hip::debug_get(ternix_hip::DBG_LINE, 1);
    if (fs == 0) return false;
    const bool epi = os.Y != nullptr;
    // Ragged: the operands' sizes or addresses rule out the DMA form (not the row count: aligned
    // operands with 17-32 rows take the wave-pipelined kernel, 1.2-1.9x faster than the ragged form's
    // two row groups, e.g. 32x6912x2560 14.8 against 7.7 us on MI355X).
    const bool ragged = !ternix_hip::line_gemv_ok(dA, dB, std::min(M, 16), K, N);
    if (tiled && ragged) return false;  // (the tile-64 contract keeps its operands aligned)
    // Rows: up to 8 on aligned operands with int32 output, 4 with float output (9-16 rows measured
    // slower than the wave-pipelined kernel: 16x2560x6912 9.20 against 7.02 us, more splits of 16-row
    // atomics), more on ragged ones (no padded copy, below); the DBG_LINE switch [3] sets the limit.
    // Ragged rows: up to 8 at any K, up to 16 from K = 256 and up to 32 from K = 1024; on shorter K the
    // few workgroups serialise their 16-row atomics (on MI355X, cold, against the padded copy:
    // 8x130x2044 4.82 / 5.38 us, 16x130x2044 6.61 / 5.44, 16x500x2044 7.01 / 7.76, 12x600x4100 6.09 /
    // 8.08, 32x700x516 10.30 / 7.41, 24x1000x3076 8.90 / 8.40, 17x4093x1028 7.89 / 9.2).
    const int fm = ternix_hip::debug_get(ternix_hip::DBG_LINE, 3);
    const int ragged_rows = K >= 1024 ? 32 : (K >= 256 ? 16 : 8);
    // Aligned operands, int32 output: up to 8 rows (on MI355X, cold, against the wave-pipelined
    // kernel: 5x4096x11008 7.75 -> 6.30 us, 8x11008x4096 8.28 -> 7.51, 6x2560x6912 5.80 -> 5.05,
    // 8x4096x4096 5.5 either way; 12x4096x4096 6.8 against 5.9).
    const int aligned_rows = epi ? 4 : 8;
    // pad_alt: the caller's alternative is the padded copy (operands aligned for this kernel but not
    // for the wave-pipelined one, e.g. N/4 % 64 != 0): the ragged limits hold up to 16 rows (on MI355X,
    // cold, against the padded copy: 16x4864x896 6.71 / 8.15 us, 12x2432x896 5.51 / 7.35; above 16
    // rows the kernel's two-row-group form is slower, 32x4864x896 10.7 / 9.2).
    const bool rows_ragged = ragged || pad_alt;
    const int pad_rows = ragged ? ragged_rows : std::min(ragged_rows, 16);
    if (M > (fm > 0 ? std::min(fm, rows_ragged ? 32 : 16) : (rows_ragged ? pad_rows : aligned_rows))) return false;
    const bool rag_form = ragged || M > 16;
    if (!(dC != nullptr && reinterpret_cast<uintptr_t>(dC) % 16 == 0 &&
          (!rag_form || (!epi && aq.mode == 0 && ternix_hip::line_gemv_ragged_ok(M, K, N)))))
        return false;
    if (aq.mode != 0 && !(epi && M <= 4 && (aq.mode == 3 || (long)M * K <= 8192) && reinterpret_cast<uintptr_t>(aq.X) % 16 == 0 &&
                          (aq.mode != 2 || reinterpret_cast<uintptr_t>(aq.G) % 16 == 0)))
        return false;
    if (epi) {
        // the sums' buffer and the float output: the same buffer (same positions, no SwiGLU) or disjoint
        const uintptr_t c0 = reinterpret_cast<uintptr_t>(dC), c1 = c0 + (size_t)M * (size_t)N * 4;
        const uintptr_t y0 = reinterpret_cast<uintptr_t>(os.Y),
                        y1 = y0 + (size_t)M * (size_t)(os.swiglu ? N / 2 : N) * 4;
        const bool same = y0 == c0 && !os.swiglu, disjoint = y1 <= c0 || c1 <= y0;
        if (!(same || disjoint) || (os.swiglu && N % 8 != 0) || (aq.mode == 0 && os.rs == nullptr)) return false;
    }
    const int strips = (N / 4 + 127) / 128;
    if (epi && K > 65536) return false;  // the float output's 64-scaled sums stay inside int32
    int S = 0;
    if (fs > 0) {
        S = fs;
    } else {
        // About one workgroup per CU: first within 250 workgroups, else within the CU count (on MI355X,
        // cold: a full 256-workgroup grid of 2 k-steps is slower than 176 of 3 for 1x4096x4096, 4.29
        // against 4.19 us, but 1x8192x8192 runs 7.86 -> 6.91 us with 256 workgroups of 8 k-steps
        // against the wave-pipelined kernel).  The FFN's down launch, which quantises its slice of h
        // from the strip maxima first, starts at 4 k-steps (1x6912x2560: 27 splits instead of 36; the
        // block 12.31 -> 12.11 us).
        // Fewest k-steps per workgroup on aligned operands: more k-steps cut the splits' atomics and
        // each workgroup's fixed cost where the grid is narrow (on MI355X, cold, k-steps 2 / 3 / 4:
        // 1x8192x1024 4.52 / 3.81 / 3.57 us, 1x6144x1024 3.80 / 3.45 / 3.40, 1x4608x1024 3.46 / 3.29 /
        // 3.30, 1x5504x2048 3.78 / 3.63 / 3.88; with 5-8 rows 8x2560x6912 6.73 / 5.64 / 5.34 and 8x4096x4096
        // 6.21 / 5.56 / 5.29).  3 from 64 k-steps, 4 from 96, and 4 from 40 k-steps with 5-8 rows.
        const int ks = (K + 63) / 64;
        const int min_s = rag_form ? 2 : ((M >= 5 && ks >= 40) || ks >= 96 ? 4 : (ks >= 64 ? 3 : 2));
        for (const long cap : {std::max(1L, (long)cu_count() * 250 / 256), std::max(1L, (long)cu_count())}) {
            for (int cand : {2, 3, 4, 6, 8}) {
                if ((aq.mode == 3 && cand < 4) || cand < min_s) continue;
                const long sp = ternix_hip::line_gemv_splits(K, cand);
                if (sp <= 64 && (long)strips * sp <= cap) {
                    S = cand;
                    break;
                }
            }
            if (S != 0) break;
        }
        // int32 output: up to 6 k-steps within two workgroups per CU when nothing fits one (13x5120
        // K=13824: 7.94 -> 7.22 us with 360 workgroups of 6 k-steps against the wave-pipelined kernel;
        // 4x13824 K=5120 8.85 -> 7.71, 4x6144x16384 11.5 -> 8.96; with 8 k-steps the DMA-staged kernel
        // is faster, 1x4096x28672 9.1 against 11.8), and 4 k-steps on up to two per CU instead of 8 on
        // one (1x4096x14336 6.33 -> 6.02, 1x8192x8192 6.47 -> 6.28; measured on MI355X, cold).
        const long cap2 = 2L * (long)cu_count();
        const int S1 = S;  // the one-per-CU plan (0: none)
        if (S == 0 && !epi && aq.mode == 0) {
            for (int cand : {2, 3, 4, 6}) {
                if (cand < min_s) continue;
                const long sp = ternix_hip::line_gemv_splits(K, cand);
                if (sp <= 64 && (long)strips * sp <= cap2) {
                    S = cand;
                    break;
                }
            }
        }
        if (S == 8 && !epi && aq.mode == 0) {
            const long sp4 = ternix_hip::line_gemv_splits(K, 4);
            if (sp4 <= 64 && (long)strips * sp4 <= cap2) S = 4;
        }
        if (S == 0) return false;
        // 7-8 rows on operands the wave-pipelined kernel takes: no plan of two workgroups per CU
        // (on MI355X, cold, against that kernel: 8x8192x8192 10.48 / 9.79 us, 8x14336x4096 10.17 /
        // 8.99, 7x14336x4096 9.81 / 8.88; the one-per-CU plans stay, 8x11008x4096 7.47 / 8.33).
        if (M >= 7 && !rows_ragged && S != S1) return false;
        // One row: no 6-k-step plan of two workgroups per CU either; the DMA-staged kernel is level
        // or faster (1x5120x13824 7.41 / 7.14 us, 1x3584x18944 7.12 / 7.01, 1x2560x27648 7.36 / 7.39;
        // at 4 rows the whole-line GEMV stays well ahead, 4x5120x13824 7.84 / 8.67).
        if (M == 1 && !rows_ragged && S != S1 && S == 6) return false;
    }
    if (M > 16 && S > 6) return false;  // two 16-row groups: at most 6 k-steps per workgroup
    // Two 16-row groups need at least 64 workgroups (on MI355X, cold, against the padded copy:
    // 32x1500x516, 24 workgroups, 10.66 / 7.55 us; 17x4093x1028, 96, 7.60 / 9.55; 20x4093x2052, 160,
    // 10.0 / 11.0).
    if (M > 16 && (long)strips * ternix_hip::line_gemv_splits(K, S) < 64) return false;
    const int NW = fw == 4 && !epi && !rag_form ? 4 : 8;
    const int splits = ternix_hip::line_gemv_splits(K, S);
    if (splits > 64) return false;
    const int stride = ternix_hip::ticket_stride((size_t)strips);
    unsigned long long* tk = c.tickets(ternix_hip::ticket_units((size_t)strips));
    if (!tk) return false;
    c.note("line_gemv_kernel%s S=%d waves=%d+1 splits=%d%s%s (splits added with int32 atomics into C zeroed by each "
           "strip's split 0)", rag_form ? " ragged" : (tiled ? " (tile-64)" : ""), S, NW, splits, aq.mode == 2 ? " rmsnorm+quantise" : (aq.mode == 1 ? " quantise" : ""),
           epi ? (os.swiglu ? " dequant+swiglu" : " dequant") : "");
    // Rows whose length is not a multiple of 128 bytes share a cache line between neighbouring strips:
    // those launches take the XCD-chunked unit order (on MI355X, cold: 1x4096x11008 6.40 -> 5.70 us,
    // 4x4096x11008 7.15 -> 6.46, 1x2560x6912 4.35 -> 4.20; neutral to 3 % slower on aligned rows).
    // The DBG_LINE switch [2] forces it off (0) or on (1).
    // The chunked order does not dispatch every strip's split 0 ahead of the strip's other splits, so
    // it is only taken when the whole grid is resident at once (one workgroup per CU at most).
    const int fx = ternix_hip::debug_get(ternix_hip::DBG_LINE, 2);
    const bool resident = (long)strips * splits <= (long)cu_count();
    const int xcd = fx >= 0 ? fx : ((N / 4) % 128 != 0 && resident);
    *e = TX_LAUNCH(c, ternix_hip::launch_line_gemv(dA, dB, dC, M, K, N, S, NW, tk, stride, c.st, os, aq, xcd, tiled));
    return true;
}

hipError_t run_skinny(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, Ctx& c,
                      const ternix_hip::OutScale& os = ternix_hip::OutScale{},
                      const ternix_hip::ActQuant& aq = ternix_hip::ActQuant{}) {
    const hipStream_t st = c.st;
    (void)st;
    const bool generic = !(K % 64 == 0 && (N / 4) % 64 == 0 && reinterpret_cast<uintptr_t>(dB) % 16 == 0 &&
                           (aq.mode != 0 || reinterpret_cast<uintptr_t>(dA) % 16 == 0));
    if (!generic && aq.mode == 0) {
        const DeepPlan dp = plan_deep(dA, dB, M, K, N, false);
        if (dp.sw > 0) {
            int32_t* partials = nullptr;
            if (dp.splits > 1) {
                const size_t need = (size_t)dp.splits * (size_t)M * (size_t)N * sizeof(int32_t);
                if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(c.get(need));
            }
            c.note("skinny_deep_kernel sw=%d nw=%d nsw=%d splits=%d%s", dp.sw, dp.nw, dp.nsw, dp.splits,
                   dp.splits > 1 ? " + splitk_reduce_kernel" : "");
            if (dp.splits == 1 || partials)
                return TX_LAUNCH(c, ternix_hip::launch_skinny_deep(dA, dB, dC, M, K, N, dp.sw, dp.nw, dp.nsw, dp.splits, dp.sps,
                                                      partials, st, os));
        }
    }
    // M = 1 with an int32 output: the K splits add into C with int32 atomics after one fill kernel has
    // zeroed it (exact, order-free), instead of summing them inside the launch through a same-address
    // arrival counter or in a reduce launch.  Measured on MI355X with cold weights (graph timing): cfg1
    // 5.80 -> 5.08 us (16-byte strips, 6 splits), cfg2 up 6.70 -> 6.36 (32-byte, 4), cfg2 down 7.48 ->
    // 6.44 (32-byte, 10); at M = 4 and 16 the other plans stay faster (cfg3 M=4 up 9.3 vs 10.2), and
    // for wide matrices (cfg5 big, 224 32-byte strips) the DMA-staged kernel is (15.7 vs 24+ us).
    // With the library's tickets the fill launch goes too: each strip's first split zeroes its
    // outputs inside the launch (skinny_kernels.hip, SK_ATOMZ); measured on MI355X, cold weights,
    // graph timing of the cfg2 up + down pair: 6.75 -> 5.57 us per GEMV (5.25 with the coalesced
    // atomic epilogue).  With tickets the plan also serves 2..16 rows (32-byte strips, as many splits
    // as fit in one round of workgroups with 6 % slack): cfg3 M=4 up 9.45 -> 8.05 us (3 splits),
    // M=4 down 9.76 -> 8.47 (8 splits); without tickets those rows keep the plans below.
    // Up to 16 rows (one m-group) with tickets: 5..16 rows add their splits with the coalesced 16-row
    // atomic epilogue (skinny_kernels.hip), measured on MI355X with cold weights against the in-launch
    // sums / reduce launch they replaced (same strips and splits): 1.11-1.59x on 28 decode shapes
    // (M 5, 8, 12, 16 x K,N in {4096x11008, 11008x4096, 2560x6912, 6912x2560, 4096x4096, 4096x14336,
    // 14336x4096}); cfg3 M=16 up 12.39 -> 9.20 us, down 12.38 -> 9.51 us.  The DBG_M1_ATOMIC switch
    // [1] lowers the row limit (tests and measurements).
    {
        hipError_t e = hipSuccess;
        if (!generic && run_line_gemv(dA, dB, dC, M, K, N, c, &e, os, aq)) return e;
        if (!generic && aq.mode == 0 && os.Y == nullptr && run_atomic_wave(dA, dB, dC, M, K, N, c, &e)) return e;
    }
    // Wave-pipelined kernel (32-byte strips, 16-byte with fused quantisation; 2 ring slots per wave),
    // measured on MI355X (16-byte strips) against the DMA-staged kernel: faster for K <= 4096 (cfg1
    // 6.26 -> 5.64 us, cfg2 up 6.94 -> 6.29, cfg3 M=4 up 11.62 -> 10.41, M=16 up 14.27 -> 11.45) and
    // for 4 < M <= 32 with longer K, whose partials are far fewer than the DMA kernel's (cfg3 M=16
    // down 14.59 -> 12.78 us); strip width and K split as in wave_splits.  M <= 4 with K > 4096 stays
    // on the DMA kernel (cold cfg2 down 7.8 us against 7.9-9.0 for the wave kernel).
    // The DBG_SKINNY_WAVE switch forces a plan (sw, nsw, splits) or turns the kernel off (tests).
    // With fused activation quantisation (K <= 4096) it quantises whole rows itself and dequantises with
    // its own row scales: the FFN block's gate/up GEMV becomes one launch.
    if (!generic && M <= kWaveMaxM && wave_kernel_enabled() && ternix_hip::skinny_wave_ok(dA, dB, M, K, N, 16) &&
        (aq.mode == 0 || (K <= 4096 && M <= 16))) {
        const int sw_env = ternix_hip::debug_get(ternix_hip::DBG_WAVE_SW) == 16 ? 16 : 32;
        const int nsteps = K / 64;
        int sw = aq.mode == 0 && ternix_hip::skinny_wave_ok(dA, dB, M, K, N, sw_env) ? sw_env : 16, nsw = 2, sp = 0;
        if (aq.mode != 0) sp = 1;
        else if (K <= 4096 || M > 4) sp = wave_splits(M, K, N, sw);
        else if (sw == 32 && last_max_splits() > 0) {
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
        if (ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE) > 0) {
            const int esw = ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE, 0),
                      ensw = ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE, 1),
                      esp = ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE, 2);
            if (esp >= 1 && (ensw == 2 || ensw == 4) && ternix_hip::skinny_wave_ok(dA, dB, M, K, N, esw)) {
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
                if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(c.get(need));
            }
            if (sps * 64 <= ternix_hip::kMaxKPerAccumulator && (splits == 1 || partials || dC) &&
                (aq.mode == 0 || (splits == 1 && sw == 16 && nsw == 2))) {
                int* cnt = (partials && aq.mode == 0)
                               ? c.counters((size_t)(N / 4 / sw) * (size_t)((M + 15) / 16), M, splits, sps)
                               : nullptr;
                c.note("skinny_wave_kernel sw=%d nsw=%d splits=%d%s", sw, nsw, splits,
                       splits == 1 ? "" : (cnt ? " (splits summed in-launch)" : " + splitk_reduce_kernel"));
                return TX_LAUNCH(c, ternix_hip::launch_skinny_wave(dA, dB, dC, M, K, N, sw, nsw, splits, sps, partials, st, os, 0,
                                                      aq, 0, cnt));
            }
        }
    }
    // DMA-staged kernel: the DBG_SKINNY_DMA switch disables it (0) or sets its stage count (2..4).
    const int dma_env = ternix_hip::debug_get(ternix_hip::DBG_SKINNY_DMA);
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
    // DMA-staged kernel at M <= 4 into C: the splits add with int32 atomics into C zeroed by each
    // strip's first split instead of going through partial sums and the reduce launch (measured on
    // MI355X, cold weights, cfg5 big 1x8192x28672: 15.67 -> 13.5 us with the coalesced atomic
    // epilogue; 9 splits stay the best count, 11 to 18 splits 16.2-18.0 us).
    // Also with fused activation quantisation and a dequantised output (the int32 sums go into the output
    // buffer, which the dequantisation launch then converts in place), in place of the partial sums and
    // the reduce launch: the decode FFN block's down GEMV, 21.33 -> 20.96 us per block (bit-equal).
    if (p.dma && M <= 4 && p.splits > 1 && p.splits <= 64 && dC != nullptr &&
        ternix_hip::debug_get(ternix_hip::DBG_SELF_ZERO) != 0) {
        if (unsigned long long* tk = c.tickets(ternix_hip::ticket_units((size_t)((N / 4 + 255) / 256)))) {
            c.note("skinny_dma_kernel splits=%d (splits added with int32 atomics into C zeroed by each strip's first "
                   "split)%s", p.splits, os.Y ? " + dequant_kernel" : "");
            return TX_LAUNCH(c, ternix_hip::launch_skinny(dA, dB, dC, M, K, N, p.tb, p.kw, p.splits, p.sps, nullptr, st,
                                                          os, aq, p.dma, 0, tk));
        }
    }
    int32_t* partials = nullptr;
    if (p.splits > 1) {
        const size_t need = (size_t)p.splits * (size_t)M * (size_t)N * sizeof(int32_t);
        if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(c.get(need));
    }
    c.note("%s splits=%d%s", p.dma ? "skinny_dma_kernel" : (generic ? "skinny_generic_kernel" : "skinny_short/fast_kernel"),
           p.splits, p.splits > 1 ? " + splitk_reduce_kernel" : "");
    return TX_LAUNCH(c, ternix_hip::launch_skinny(dA, dB, dC, M, K, N, p.tb, p.kw, p.splits, p.sps, partials, st, os, aq, p.dma));
}

// Split-K for GEMMs with too few output tiles to fill the chip (mid-size M against a long K, e.g.
// cfg3 M=64, the worst case M=256): each split covers a contiguous k-range of whole 128-row stages,
// the partial tiles go through the same workspace and reduce launch as the skinny path.
int gemm_splits(int M, int K, int N, int tiled = 0) {
    const int env = ternix_hip::debug_get(ternix_hip::DBG_GEMM_SPLITS);  // tests
    // the tile height launch_gemm picks for a split launch; one workgroup per CU over the tiles and
    // splits
    const bool narrow = ternix_hip::gemm_narrow_wanted(M, K, N, tiled);  // 64-column tiles instead of 256
    const int bm = narrow ? 64 : ternix_hip::gemm_split_rows(M, K, N);
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

hipError_t run_gemm(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, Ctx& c,
                    const ternix_hip::OutScale& os = ternix_hip::OutScale{}, int tiled = 0) {
    const hipStream_t st = c.st;
    (void)st;
    if (K <= ternix_hip::kMaxKPerAccumulator) {
        int splits = gemm_splits(M, K, N, tiled);
        if (splits > 1) {
            // whole stages per split: 256 rows for the narrow tiles, 128 for the others
            const int unit = ternix_hip::gemm_narrow_wanted(M, K, N, tiled) ? 256 : (K % 128 == 0 ? 128 : 64);
            const int k_split = ((K + splits - 1) / splits + unit - 1) / unit * unit;
            splits = (K + k_split - 1) / k_split;
            const size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(int32_t);
            int32_t* partials = (splits > 1 && need <= kWorkspaceMax) ? static_cast<int32_t*>(c.get(need))
                                                                       : nullptr;
            if (partials) {
                c.note("%s splits=%d + splitk_reduce_kernel",
                       ternix_hip::gemm_choice_name(ternix_hip::gemm_choice(dA, dB, M, K, N, 0, K, splits, k_split, tiled)),
                       splits);
                hipError_t e = TX_LAUNCH(c, ternix_hip::launch_gemm(dA, dB, partials, M, K, N, 0, K, 0, st, ternix_hip::OutScale{},
                                                       splits, k_split, tiled));
                if (e != hipSuccess) return e;
                return TX_LAUNCH(c, ternix_hip::launch_splitk_reduce(partials, dC, M, N, splits, os, st));
            }
        }
        c.note("%s", ternix_hip::gemm_choice_name(ternix_hip::gemm_choice(dA, dB, M, K, N, 0, K, 1, 0, tiled)));
        return TX_LAUNCH(c, ternix_hip::launch_gemm(dA, dB, dC, M, K, N, 0, K, 0, st, os, 1, 0, tiled));
    }
    if (dC == nullptr) return hipErrorInvalidValue;  // scaled call without int scratch
    int acc = 0;
    for (long k0 = 0; k0 < K; k0 += ternix_hip::kMaxKPerAccumulator) {
        const long k1 = k0 + ternix_hip::kMaxKPerAccumulator < K ? k0 + ternix_hip::kMaxKPerAccumulator : K;
        const hipError_t e = TX_LAUNCH(c, ternix_hip::launch_gemm(dA, dB, dC, M, K, N, (int)k0, (int)k1, acc, st,
                                                     ternix_hip::OutScale{}, 1, 0, tiled));
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
hipError_t run_padded(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, Ctx& c,
                      const ternix_hip::OutScale& os, bool skinny) {
    const hipStream_t st = c.st;
    (void)st;
    const int NB = N / 4;
    const long Kp = ((long)K + 127) / 128 * 128;
    const long NBp = ((long)NB + 63) / 64 * 64;
    const long Np = 4 * NBp;
    if (K == 0 || Kp > INT_MAX || Np > INT_MAX || Kp * NBp >= (1L << 32)) return hipErrorNotSupported;
    SkinnyPlan p{0, 0, 0, 0, 0};
    int splits = 1, k_split = 0;
    // Short K at M <= 16: the wave-pipelined kernel in one launch, writing the N real columns itself.
    const bool wave = skinny && M <= kWaveMaxM && Kp <= 4096 && wave_kernel_enabled();
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
    uint8_t* ws = static_cast<uint8_t*>(c.get(w_bytes + a_bytes + p_bytes));
    if (ws == nullptr) return hipErrorNotSupported;
    c.note("pad_rows_kernel + %s", wave ? "skinny_wave_kernel" : (skinny ? (p.dma ? "skinny_dma_kernel" : "skinny_short/fast_kernel") : "gemm"));
    uint8_t* Wp = ws;
    int8_t* Ap = reinterpret_cast<int8_t*>(ws + w_bytes);
    int32_t* P = reinterpret_cast<int32_t*>(ws + w_bytes + a_bytes);
    hipError_t e = TX_LAUNCH(c, ternix_hip::launch_pad_rows(dB, Wp, K, (int)Kp, NB, NB, (int)NBp,
                                               reinterpret_cast<const uint8_t*>(dA), reinterpret_cast<uint8_t*>(Ap),
                                               M, M, K, K, (int)Kp, st));
    if (e != hipSuccess) return e;
    // int32 output up to 32 rows: the self-zeroing atomic split plan on the padded copies, writing the
    // N real columns (measured on MI355X, cold weights, us, against the whole-K store kernel:
    // 1x1000x3076 7.0 -> 6.6, 17x4093x1028 12.6 -> 10.1, both including the pad launch)
    if (skinny && os.Y == nullptr && dC != nullptr && N % 4 == 0 &&
        run_atomic_wave(Ap, Wp, dC, M, (int)Kp, (int)Np, c, &e, N, "pad_rows_kernel + "))
        return e;
    if (wave)
        return TX_LAUNCH(c, ternix_hip::launch_skinny_wave(Ap, Wp, dC, M, (int)Kp, (int)Np, 16, 2, 1, (int)(Kp / 64), nullptr, st,
                                              os, N));
    if (skinny)
        return TX_LAUNCH(c, ternix_hip::launch_skinny(Ap, Wp, dC, M, (int)Kp, (int)Np, p.tb, p.kw, p.splits, p.sps, P, st, os,
                                         ternix_hip::ActQuant{}, p.dma, N));
    e = TX_LAUNCH(c, ternix_hip::launch_gemm(Ap, Wp, P, M, (int)Kp, (int)Np, 0, (int)Kp, 0, st, ternix_hip::OutScale{}, splits,
                                k_split));
    if (e != hipSuccess) return e;
    return TX_LAUNCH(c, ternix_hip::launch_splitk_reduce(P, dC, M, N, splits, os, st, (int)Np));
}

// The aligned kernels need 16-byte aligned operands, N/4 % 64 == 0 and whole k-steps: 64 rows for
// the skinny kernels, 128 for the pipelined GEMM.
bool needs_padding(const int8_t* dA, const uint8_t* dB, int K, int N, bool skinny) {
    return !(K % (skinny ? 64 : 128) == 0 && (N / 4) % 64 == 0 && reinterpret_cast<uintptr_t>(dB) % 16 == 0 &&
             reinterpret_cast<uintptr_t>(dA) % 16 == 0);
}

// Automatic path for one call: the padded copy for ragged or misaligned shapes when it applies,
// else the skinny kernels up to kSkinnyMaxM rows and the GEMM above.
hipError_t run_auto(const int8_t* dA, const uint8_t* dB, int32_t* dC, int M, int K, int N, Ctx& c,
                    const ternix_hip::OutScale& os, int skinny_max) {
    const hipStream_t st = c.st;
    (void)st;
    const bool pad_off = ternix_hip::debug_get(ternix_hip::DBG_RAGGED_PAD) == 0;  // tests: generic kernels
    if (!pad_off && needs_padding(dA, dB, K, N, M <= skinny_max)) {
        // up to 32 rows, int32 output: the whole-line GEMV reads the ragged operands as they are, one launch
        hipError_t e = hipSuccess;
        if (M <= skinny_max && os.Y == nullptr &&
            run_line_gemv(dA, dB, dC, M, K, N, c, &e, ternix_hip::OutScale{}, ternix_hip::ActQuant{}, 0, true))
            return e;
        e = run_padded(dA, dB, dC, M, K, N, c, os, M <= skinny_max);
        if (e != hipErrorNotSupported) return e;
    }
    if (M > skinny_max && M <= 64 && os.Y == nullptr && K % 64 == 0) {  // 33..64 rows: the atomic wave plan if it applies
        hipError_t e = hipSuccess;
        if (run_atomic_wave(dA, dB, dC, M, K, N, c, &e)) return e;
    }
    return M <= skinny_max ? run_skinny(dA, dB, dC, M, K, N, c, os) : run_gemm(dA, dB, dC, M, K, N, c, os);
}

// Tile-64 weights (the opt-in pre-permuted layout): M <= 32 runs the wave-pipelined kernel, whose
// per-wave DMA of one 1 KB block is a single contiguous read, K split by wave_splits at every K
// (the contiguous reads make it faster than the DMA kernel for long K too: cold cfg2 down 6.7 us
// against 7.8 on the row-major layout; the DBG_SKINNY_WAVE switch forces the split count, tests).  Larger M runs the LDS-DMA GEMMs with the contract layout's split-K planning.
hipError_t run_tile64(const int8_t* dA, const uint8_t* dWt, int32_t* dC, int M, int K, int N, Ctx& c,
                      const ternix_hip::OutScale& os = ternix_hip::OutScale{}) {
    const hipStream_t st = c.st;
    (void)st;
    // One row: the whole-line GEMV, which reads the tile-64 blocks in the same 128-byte lines as
    // row-major rows (on MI355X, cold: 1x2560x6912 4.61 -> 4.23 us, 1x6912x2560 4.74 -> 4.50,
    // 1x4096x4096 4.94 -> 4.30; at 4 rows the wave-pipelined plans below are as fast or faster,
    // 4x11008x4096 6.62 against 6.81).
    if (M == 1) {
        hipError_t e = hipSuccess;
        if (run_line_gemv(dA, dWt, dC, M, K, N, c, &e, os, ternix_hip::ActQuant{}, 1)) return e;
    }
    // The self-zeroing atomic plan below applies to int32 output up to 16 rows; where it does, it is
    // faster than the whole-K kernel (cold, one box, us: cfg1 4.80 -> 3.64, cfg2 up 5.10 -> 4.49, 4x4096x11008
    // 6.46 -> 6.32, 16x4096x11008 7.69 -> 7.31), which keeps the dequantising calls.
    const int t64_atomic_max_m = ternix_hip::debug_get(ternix_hip::DBG_M1_ATOMIC, 2) > 0 ? ternix_hip::debug_get(ternix_hip::DBG_M1_ATOMIC, 2) : 16;
    const bool t64_atomic = M <= std::min(16, t64_atomic_max_m) && os.Y == nullptr && dC != nullptr &&
                            ternix_hip::debug_get(ternix_hip::DBG_SELF_ZERO) != 0 &&
                            ternix_hip::debug_get(ternix_hip::DBG_M1_ATOMIC) != 0;
    if (M <= 16 && !(t64_atomic && ternix_hip::debug_get(ternix_hip::DBG_DEEP) < 0)) {
        const DeepPlan dp = plan_deep(dA, dWt, M, K, N, true);
        if (dp.sw > 0) {
            int32_t* partials =
                dp.splits > 1 ? static_cast<int32_t*>(c.get((size_t)dp.splits * M * N * sizeof(int32_t))) : nullptr;
            c.note("skinny_deep_kernel (tile-64) nw=%d nsw=%d splits=%d%s", dp.nw, dp.nsw, dp.splits,
                   dp.splits > 1 ? " + splitk_reduce_kernel" : "");
            if (dp.splits == 1 || partials)
                return TX_LAUNCH(c, ternix_hip::launch_skinny_deep(dA, dWt, dC, M, K, N, 16, dp.nw, dp.nsw, dp.splits,
                                                                   dp.sps, partials, st, os, 0, 1));
        }
    }
    if (M <= 32) {
        const int nsteps = K / 64;
        int sp = wave_splits(M, K, N);
        // Atomic plan with few strips and long K: at least 12 k-steps per split (cold, one box, us:
        // cfg2 down 40 strips 16 -> 9 splits 5.75 -> 4.90; 4x11008x4096 64 strips 16 -> 14 splits).
        if (t64_atomic && N / 4 / 16 <= 64 && nsteps >= 96) sp = std::min(sp, std::max(1, nsteps / 12));
        if (ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE) > 0 && ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE, 2) >= 1)
            sp = ternix_hip::debug_get(ternix_hip::DBG_SKINNY_WAVE, 2);
        const int sps = (nsteps + sp - 1) / sp;
        const int splits = (nsteps + sps - 1) / sps;
        if (sps * 64 > ternix_hip::kMaxKPerAccumulator) return hipErrorInvalidValue;
        // Up to 16 rows into C: the splits add with int32 atomics into C zeroed by each strip's first
        // split (as on the row-major layout).  Measured on MI355X, cold weights, against the reduce
        // launch: cfg3 M=4 down 9.46 -> 6.72 us, M=16 down 10.70 -> 7.57 us.  The DBG_M1_ATOMIC switch
        // [2] lowers the row limit.
        if (t64_atomic && splits > 1 && splits <= 64) {
            if (unsigned long long* tk = c.tickets(ternix_hip::ticket_units((size_t)(N / 4 / 16)))) {
                c.note("skinny_wave_kernel (tile-64) sw=16 nsw=2 splits=%d (splits added with int32 atomics into C "
                       "zeroed by each strip's first split)", splits);
                return TX_LAUNCH(c, ternix_hip::launch_skinny_wave(dA, dWt, dC, M, K, N, 16, 2, splits, sps, nullptr, st,
                                                                   os, 0, ternix_hip::ActQuant{}, 1, nullptr, tk));
            }
        }
        int32_t* partials = nullptr;
        if (splits > 1) {
            const size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(int32_t);
            if (need <= kWorkspaceMax) partials = static_cast<int32_t*>(c.get(need));
        }
        int* cnt = partials ? c.counters((size_t)(N / 4 / 16) * (size_t)((M + 15) / 16), M, splits, sps)
                            : nullptr;
        return TX_LAUNCH(c, ternix_hip::launch_skinny_wave(dA, dWt, dC, M, K, N, 16, 2, splits, sps, partials, st, os, 0,
                                              ternix_hip::ActQuant{}, 1, cnt));
    }
    return run_gemm(dA, dWt, dC, M, K, N, c, os, 1);
}

enum class Path { Auto, Skinny, Gemm, Naive };

int dispatch_ctx(Path path, const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M64, int64_t K64,
                 int64_t N64, Ctx& c);

int dispatch(Path path, const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M64, int64_t K64, int64_t N64,
             void* stream) {
    Ctx c;
    c.st = static_cast<hipStream_t>(stream);
    return dispatch_ctx(path, dA, dB, dC, M64, K64, N64, c);
}

int dispatch_ctx(Path path, const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M64, int64_t K64,
                 int64_t N64, Ctx& c) {
    bool trivial = false;
    hipError_t e = validate(dA, dB, dC, M64, K64, N64, &trivial);
    if (e != hipSuccess) return (int)e;
    if (path == Path::Skinny && M64 > kSkinnyMaxM) return (int)hipErrorInvalidValue;
    if (trivial) return (int)hipSuccess;
    const int M = (int)M64, K = (int)K64, N = (int)N64;
    if (path == Path::Auto) return (int)run_auto(dA, dB, dC, M, K, N, c, ternix_hip::OutScale{}, kSkinnyMaxM);
    switch (path) {
        case Path::Skinny: e = run_skinny(dA, dB, dC, M, K, N, c); break;
        case Path::Gemm: e = run_gemm(dA, dB, dC, M, K, N, c); break;
        default:
            c.note("naive_kernel");
            e = TX_LAUNCH(c, ternix_hip::launch_naive(dA, dB, dC, M, K, N, c.st));
            break;
    }
    return (int)e;
}

// Dry run of the automatic path for operands at the given addresses (only their alignment matters;
// nothing is dereferenced or launched).
Ctx plan_auto(int64_t M, int64_t K, int64_t N, uintptr_t a_addr, uintptr_t b_addr, bool library = false) {
    Ctx c;
    c.dry = true;
    c.dry_library = library;
    std::snprintf(c.desc, sizeof(c.desc), "none");
    const int s = dispatch_ctx(Path::Auto, reinterpret_cast<const int8_t*>(a_addr),
                               reinterpret_cast<const uint8_t*>(b_addr), reinterpret_cast<int32_t*>(uintptr_t(1) << 20),
                               M, K, N, c);
    if (s != 0) std::snprintf(c.desc, sizeof(c.desc), "rejected");
    return c;
}

}  // namespace

extern "C" {

int ternix_hip_mul_mat_ternary(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K, int64_t N,
                               void* stream) {
    return dispatch(Path::Auto, dA, dB, dC, M, K, N, stream);
}

size_t ternix_hip_mul_mat_ternary_workspace_size(int64_t M, int64_t K, int64_t N) {
    // For 16-byte aligned A and W (what hipMalloc returns).
    return plan_auto(M, K, N, uintptr_t(1) << 20, uintptr_t(1) << 24).need;
}

size_t ternix_hip_mul_mat_ternary_workspace_size_for(const int8_t* dA, const uint8_t* dB, int64_t M, int64_t K,
                                                     int64_t N) {
    return plan_auto(M, K, N, reinterpret_cast<uintptr_t>(dA), reinterpret_cast<uintptr_t>(dB)).need;
}

int ternix_hip_mul_mat_ternary_ws(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K, int64_t N,
                                  void* dWorkspace, size_t workspace_bytes, void* stream) {
    if (workspace_bytes > 0 && (dWorkspace == nullptr || reinterpret_cast<uintptr_t>(dWorkspace) % 256 != 0))
        return (int)hipErrorInvalidValue;
    Ctx c;
    c.st = static_cast<hipStream_t>(stream);
    c.use_caller = true;
    c.caller = static_cast<char*>(dWorkspace);
    c.caller_bytes = dWorkspace ? workspace_bytes : 0;
    return dispatch_ctx(Path::Auto, dA, dB, dC, M, K, N, c);
}

int ternix_hip_plan_describe(const int8_t* dA, const uint8_t* dB, int64_t M, int64_t K, int64_t N, char* buf,
                             size_t len) {
    if (buf == nullptr || len == 0) return (int)hipErrorInvalidValue;
    const Ctx c = plan_auto(M, K, N, reinterpret_cast<uintptr_t>(dA), reinterpret_cast<uintptr_t>(dB), true);
    std::snprintf(buf, len, "%s", c.desc);
    return std::strcmp(c.desc, "rejected") == 0 ? (int)hipErrorInvalidValue : (int)hipSuccess;
}

int ternix_hip_release_stream(void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    Workspace w;
    {
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        auto it = g_ws.find(ws_key(dev, st));
        if (it == g_ws.end()) return (int)hipSuccess;
        w = std::move(it->second);
        g_ws.erase(it);
    }
    // Work already queued on the stream may still use the buffers.
    e = hipStreamSynchronize(st);
    if (w.ptr) (void)hipFree(w.ptr);
    for (void* p : w.retired) (void)hipFree(p);
    if (w.counters) (void)hipFree(w.counters);
    return (int)e;
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
    if ((e = lib_malloc(reinterpret_cast<void**>(&dA), a_bytes ? a_bytes : 16)) != hipSuccess) goto done;
    if ((e = lib_malloc(reinterpret_cast<void**>(&dB), b_bytes ? b_bytes : 16)) != hipSuccess) goto done;
    if ((e = lib_malloc(reinterpret_cast<void**>(&dC), c_bytes)) != hipSuccess) goto done;
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
    e = run_auto(dA, dB, c_alias, m, k, n, ctx_of(st), os, kSkinnyMaxM);
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
    e = run_auto(dA, dB, dScratch, m, k, n, ctx_of(st), os, kSkinnyMaxM);
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
    size_t q1, rs1, h, q2, rs2, scratch, amax, total;
};
// Per row, one float per 128-byte strip of the gate/up weights (2F/4 bytes a row), rounded up to 4.
int ffn_amax_stride(int64_t F) { return (int)(((2 * F / 4 + 127) / 128 + 3) / 4 * 4); }
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
    l.amax = o; o = up(o + 4 * (size_t)M * (size_t)ffn_amax_stride(F));
    l.total = o;
    return l;
}

// Both GEMVs of the decode FFN block on the whole-line GEMV, two launches: the gate/up launch applies
// RMSNorm + quantisation to x (aq1), dequantises with SwiGLU (os1) and leaves each strip's largest |h|
// per row in amax; the down launch quantises its slice of h from those maxima (the absmax is exact in
// any order), writing its row scales to rs2 (those os2 reads), and dequantises (os2) -- no workgroup
// reads whole rows of h.  Returns false, with nothing
// queued, when the gate/up plan does not apply; *down_done is false when only the gate/up launch ran
// (the caller then runs the down GEMV another way).  tiled: both weight matrices in the tile-64 layout.
bool ffn_line(const uint8_t* dWgu, const uint8_t* dWd, float* dY, int32_t* scratch, float* amax, int m, int hd, int f,
              const ternix_hip::OutScale& os1, const ternix_hip::ActQuant& aq1, const ternix_hip::OutScale& os2,
              float* rs2, Ctx c, int tiled, hipError_t* e, bool* down_done) {
    *down_done = false;
    if (ternix_hip::debug_get(ternix_hip::DBG_FFN_AMAX) == 0) return false;
    ternix_hip::ActQuant g1 = aq1;
    g1.amax_out = amax;
    g1.amax_stride = ffn_amax_stride(f);
    if (!run_line_gemv(nullptr, dWgu, scratch, m, hd, 2 * f, c, e, os1, g1, tiled)) return false;
    if (*e != hipSuccess) return true;
    ternix_hip::ActQuant g2;
    g2.mode = 3;
    g2.X = os1.Y;
    g2.rs_out = rs2;
    g2.amax_in = amax;
    g2.amax_stride = g1.amax_stride;
    g2.amax_n = (2 * f / 4 + 127) / 128;
    *down_done = run_line_gemv(nullptr, dWd, reinterpret_cast<int32_t*>(dY), m, f, hd, c, e, os2, g2, tiled);
    return true;
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
    float* amax = reinterpret_cast<float*>(ws + l.amax);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, hd = (int)H, f = (int)F;
    // Decode shapes: the RMSNorm + quantisation of x and the requantisation of h run inside the two
    // skinny GEMVs (fused activation prologue, bit-identical to the standalone kernels).  Up to 4 rows
    // with M x H <= 8192 that is two launches of the whole-line GEMV, each dequantising (and, for
    // gate/up, applying SwiGLU) in its last-arriving split, the down launch quantising h with the
    // gate/up launch's per-strip maxima (measured on MI355X, cold weights, 1 x 2560 x 6912: 20.2 ->
    // 13.2 us per block); otherwise the other skinny kernels with their reduce or dequantisation
    // launches.  Larger M: the four separate launches.
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
        // Both on the whole-line GEMV: the gate/up launch also leaves each strip's largest |h| per row,
        // so the down launch quantises h from its own slice and those maxima (the absmax is exact in
        // any order) instead of every workgroup reading whole rows of h.
        bool down_done = false;
        hipError_t e = hipSuccess;
        if (ffn_line(dWgu, dWd, dY, scratch, amax, m, hd, f, os1, aq1, os2, rs2, ctx_of(st), 0, &e, &down_done)) {
            if (e != hipSuccess || down_done) return (int)e;
            return (int)run_skinny(nullptr, dWd, reinterpret_cast<int32_t*>(dY), m, f, hd, ctx_of(st), os2, aq2);
        }
        const SkinnyPlan p1 = plan_skinny(m, hd, 2 * f), p2 = plan_skinny(m, f, hd);
        if (ternix_hip::skinny_short_ok(dWgu, m, hd, 2 * f, p1.sps, p1.splits) &&
            ternix_hip::skinny_short_ok(dWd, m, f, hd, p2.sps, p2.splits)) {
            hipError_t e = run_skinny(nullptr, dWgu, scratch, m, hd, 2 * f, ctx_of(st), os1, aq1);
            if (e != hipSuccess) return (int)e;
            return (int)run_skinny(nullptr, dWd, reinterpret_cast<int32_t*>(dY), m, f, hd, ctx_of(st), os2, aq2);
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
    hipError_t e = hipSuccess;
    {
        // Up to 4 rows: two launches of the whole-line GEMV on the tile-64 blocks, as on row-major
        // weights (on MI355X, cold, H 2560, F 6912, M = 1: 21.9 -> 12.8 us per block).
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
        bool down_done = false;
        float* amax = reinterpret_cast<float*>(ws + l.amax);
        if (ffn_line(dWguT, dWdT, dY, scratch, amax, m, hd, f, os1, aq1, os2, rs2, ctx_of(st), 1, &e, &down_done)) {
            if (e != hipSuccess || down_done) return (int)e;
            e = ternix_hip::launch_quantize_rows(h, q2, rs2, m, f, st);
            if (e != hipSuccess) return (int)e;
            return (int)run_tile64(q2, dWdT, reinterpret_cast<int32_t*>(dY), m, f, hd, ctx_of(st), os2);
        }
    }
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
        e = run_tile64(q1, dWguT, scratch, m, hd, 2 * f, ctx_of(st), os1);
    }
    if (e != hipSuccess) return (int)e;
    e = ternix_hip::launch_quantize_rows(h, q2, rs2, m, f, st);
    if (e != hipSuccess) return (int)e;
    ternix_hip::OutScale os2;
    os2.Y = dY;
    os2.rs = rs2;
    os2.ws = ws_d;
    return (int)run_tile64(q2, dWdT, reinterpret_cast<int32_t*>(dY), m, f, hd, ctx_of(st), os2);
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
    return (int)run_tile64(dA, dWt, dC, (int)M, (int)K, (int)N, ctx_of(static_cast<hipStream_t>(stream)));
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
                           ctx_of(static_cast<hipStream_t>(stream)), os);
}

int ternix_hip_debug_set(const char* key, int v0, int v1, int v2, int v3) {
    static const struct {
        const char* name;
        ternix_hip::DebugKey key;
    } names[] = {
        {"wave_last", ternix_hip::DBG_WAVE_LAST},     {"skinny_wave", ternix_hip::DBG_SKINNY_WAVE},
        {"wave_sw", ternix_hip::DBG_WAVE_SW},         {"skinny_dma", ternix_hip::DBG_SKINNY_DMA},
        {"skinny_short", ternix_hip::DBG_SKINNY_SHORT}, {"ragged_pad", ternix_hip::DBG_RAGGED_PAD},
        {"gemm_narrow", ternix_hip::DBG_GEMM_NARROW}, {"gemm_generic", ternix_hip::DBG_GEMM_GENERIC},
        {"gemm_splits", ternix_hip::DBG_GEMM_SPLITS}, {"gemm_bm", ternix_hip::DBG_GEMM_BM},
        {"deep", ternix_hip::DBG_DEEP},             {"sk_order", ternix_hip::DBG_SK_ORDER},
        {"m1_atomic", ternix_hip::DBG_M1_ATOMIC},     {"self_zero", ternix_hip::DBG_SELF_ZERO},
        {"gemm_gm", ternix_hip::DBG_GEMM_GM},         {"nt", ternix_hip::DBG_NT}, {"wave_ticket", ternix_hip::DBG_WAVE_TICKET},
        {"line", ternix_hip::DBG_LINE}, {"ffn_amax", ternix_hip::DBG_FFN_AMAX},
    };
    if (key == nullptr) return (int)hipErrorInvalidValue;
    for (const auto& n : names) {
        if (std::strcmp(n.name, key) != 0) continue;
        const int v[4] = {v0, v1, v2, v3};
        for (int i = 0; i < 4; ++i)
            ternix_hip::g_debug[n.key][i].store(v[i] < 0 ? 0 : v[i] + 1, std::memory_order_relaxed);
        return (int)hipSuccess;
    }
    return (int)hipErrorInvalidValue;
}

int ternix_hip_debug_stream_read(const void* dSrc, size_t bytes, int* dFlag, void* stream) {
    if (bytes / 16 == 0) return (int)hipSuccess;
    if (dSrc == nullptr || dFlag == nullptr || reinterpret_cast<uintptr_t>(dSrc) % 16 != 0)
        return (int)hipErrorInvalidValue;
    return (int)ternix_hip::launch_stream_read(dSrc, bytes, dFlag, static_cast<hipStream_t>(stream));
}

long long ternix_hip_debug_alloc_count(void) { return g_alloc_count.load(std::memory_order_relaxed); }

int ternix_hip_take_faults(unsigned int* bits) {
    if (bits == nullptr) return (int)hipErrorInvalidValue;
    return (int)ternix_hip::take_faults(bits);
}

void ternix_hip_debug_reset(void) {
    for (auto& k : ternix_hip::g_debug)
        for (auto& v : k) v.store(0, std::memory_order_relaxed);
}

const char* ternix_hip_error_string(int status) {
    const char* s = hipGetErrorString(static_cast<hipError_t>(status));
    return s ? s : "unknown error";
}

int ternix_hip_version(void) { return 200; }

int ternix_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

}  // extern "C"
