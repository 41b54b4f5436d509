// noalloc.hip -- ternix_hip_mul_mat_ternary_noalloc: the automatic matmul with its scratch in a fixed
// device array, for callers that cannot allocate device memory (code under hipGraph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// The scratch (split-K partial sums, padded copies of ragged operands) lives in `scratch`, a
// file-scope device array of kScratchBytes.  Host code never uses the array's name as an address:
// the device address is looked up once per device with hipGetSymbolAddress (each GPU holds its own
// copy at its own address) and passed to the kernels through the caller-workspace path of
// ternix_hip_mul_mat_ternary_ws.  Nothing here allocates.  No plan that runs with a caller-owned
// workspace reads scratch memory it has not written in the same call, so nothing has to be cleared
// between calls.  All calls on one GPU share its array: calls that overlap in time on one GPU race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ternix/ternix_hip.h"

namespace {

constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array (looked up on the first call on that device).
hipError_t scratch_for_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" {

size_t ternix_hip_noalloc_scratch_bytes(void) { return kScratchBytes; }

int ternix_hip_mul_mat_ternary_noalloc(const int8_t* dA, const uint8_t* dB, int32_t* dC, int64_t M, int64_t K,
                                       int64_t N, void* stream) {
    // Shape rejection first, like every other entry point (the size query returns 0 for it).
    if (M < 0 || K < 0 || N < 0 || N % 4 != 0) return (int)hipErrorInvalidValue;
    const size_t need = ternix_hip_mul_mat_ternary_workspace_size(M, K, N);
    if (need > kScratchBytes) return (int)hipErrorOutOfMemory;
    void* ws = nullptr;
    const hipError_t e = scratch_for_current_device(&ws);
    if (e != hipSuccess) return (int)e;
    return ternix_hip_mul_mat_ternary_ws(dA, dB, dC, M, K, N, ws, kScratchBytes, stream);
}

}  // extern "C"
