// test_hip_matmul.cpp -- C++ bit-exactness suite for libternix_hip.so through the C++ face a
// TernixEngine caller uses (include/ternix/hip_kernels.hpp, include/ternix/bitpack.hpp).
//
// It covers what the reference's GPU test checks (tests/test_cuda_matmul.cu:11-43: the naive and
// tiled host entry points against the scalar CPU kernel, and the tiled shape rejection) and the
// reference's CPU shape list (tests/test_ternary_matmul.cpp:44-69), plus the device-pointer automatic
// path on decode / ragged / misaligned shapes, the int8 extreme case, a hipGraph replay and the
// opt-in tile-64 weight layout (host conversion + its entry point).
// The checker is the CPU oracle (oracle/liboracle.so, a restatement of the reference's scalar
// kernel): test infrastructure only.  Dependency-free: no test framework, exit status 0 on success.
//
//   test_hip_matmul           run every case (needs a GPU)
//   test_hip_matmul --list    print the case names and exit without touching the GPU
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "ternix/bitpack.hpp"
#include "ternix/hip_kernels.hpp"
#include "ternix_oracle.h"

namespace {

int g_failures = 0;

#define EXPECT(cond, ...)                                            \
    do {                                                             \
        if (!(cond)) {                                               \
            std::printf("  FAILED %s:%d: %s -- ", __FILE__, __LINE__, #cond); \
            std::printf(__VA_ARGS__);                                \
            std::printf("\n");                                       \
            ++g_failures;                                            \
        }                                                            \
    } while (0)

#define HIP_OK(expr)                                                                          \
    do {                                                                                      \
        const hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess) {                                                               \
            std::printf("  FAILED %s:%d: %s = %s\n", __FILE__, __LINE__, #expr, hipGetErrorString(e_)); \
            ++g_failures;                                                                     \
            return;                                                                           \
        }                                                                                     \
    } while (0)

struct Problem {
    size_t M, K, N;
    std::vector<int8_t> A;
    std::vector<uint8_t> Wp;
};

// Uniform int8 activations, weights uniform over {-1, 0, +1}, packed with the library's host packer.
Problem make_problem(size_t M, size_t K, size_t N, uint32_t seed) {
    std::mt19937 rng(seed);
    std::uniform_int_distribution<int> act(-128, 127), wt(-1, 1);
    Problem p{M, K, N, std::vector<int8_t>(M * K), std::vector<uint8_t>(K * N / 4)};
    std::vector<int8_t> W(K * N);
    for (auto& a : p.A) a = static_cast<int8_t>(act(rng));
    for (auto& w : W) w = static_cast<int8_t>(wt(rng));
    ternix::pack_ternary_weights(p.Wp.data(), W.data(), W.size());
    return p;
}

std::vector<int32_t> expected(const Problem& p) {
    std::vector<int32_t> c(p.M * p.N, 0);
    oracle_mm_scalar(p.A.data(), p.Wp.data(), c.data(), p.M, p.K, p.N);
    return c;
}

size_t first_mismatch(const std::vector<int32_t>& a, const std::vector<int32_t>& b) {
    for (size_t i = 0; i < a.size(); ++i)
        if (a[i] != b[i]) return i;
    return a.size();
}

// Host entry point (reference mul_mat_ternary_cuda_host): allocates, copies, runs, frees.
void host_case(size_t M, size_t K, size_t N, bool tiled, uint32_t seed) {
    const Problem p = make_problem(M, K, N, seed);
    const std::vector<int32_t> ref = expected(p);
    std::vector<int32_t> got(ref.size(), -1);
    HIP_OK(ternix::mul_mat_ternary_hip_host(p.A.data(), p.Wp.data(), got.data(), (int)M, (int)K, (int)N, tiled));
    const size_t i = first_mismatch(ref, got);
    EXPECT(i == ref.size(), "%s M=%zu K=%zu N=%zu: C[%zu] = %d, expected %d", tiled ? "tiled" : "naive", M, K, N, i,
           got[i], ref[i]);
}

// Device-pointer automatic path on a stream; `offset` shifts A and W off 16-byte alignment.
void device_case(const Problem& p, size_t offset = 0) {
    const std::vector<int32_t> ref = expected(p);
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    int8_t* dA = nullptr;
    uint8_t* dW = nullptr;
    int32_t* dC = nullptr;
    HIP_OK(hipMalloc(&dA, p.A.size() + offset + 16));
    HIP_OK(hipMalloc(&dW, p.Wp.size() + offset + 16));
    HIP_OK(hipMalloc(&dC, ref.size() * sizeof(int32_t) + 16));
    HIP_OK(hipMemcpy(dA + offset, p.A.data(), p.A.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dW + offset, p.Wp.data(), p.Wp.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMemset(dC, 0xff, ref.size() * sizeof(int32_t)));
    HIP_OK(ternix::mul_mat_ternary_hip(dA + offset, dW + offset, dC, (int64_t)p.M, (int64_t)p.K, (int64_t)p.N, st));
    HIP_OK(hipStreamSynchronize(st));
    std::vector<int32_t> got(ref.size());
    HIP_OK(hipMemcpy(got.data(), dC, got.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
    const size_t i = first_mismatch(ref, got);
    EXPECT(i == ref.size(), "auto M=%zu K=%zu N=%zu offset=%zu: C[%zu] = %d, expected %d", p.M, p.K, p.N, offset, i,
           got[i], ref[i]);
    HIP_OK(hipFree(dA));
    HIP_OK(hipFree(dW));
    HIP_OK(hipFree(dC));
    HIP_OK(hipStreamDestroy(st));
}

void naive_matches_cpu() {
    host_case(64, 64, 64, false, 1);
    host_case(37, 100, 52, false, 2);
    host_case(128, 512, 256, false, 3);
}

void tiled_matches_cpu() {
    host_case(64, 64, 64, true, 4);
    host_case(128, 256, 192, true, 5);
    host_case(256, 1024, 512, true, 6);
    host_case(64, 4096, 64, true, 7);
}

void tiled_rejects_unsupported_shape() {
    // Rejected before any pointer is used (null pointers are never touched).
    EXPECT(ternix::mul_mat_ternary_hip_tiled(nullptr, nullptr, nullptr, 65, 64, 64) == hipErrorInvalidValue,
           "M=65 accepted");
    EXPECT(ternix::mul_mat_ternary_hip_tiled(nullptr, nullptr, nullptr, 64, 64, 66) == hipErrorInvalidValue,
           "N=66 accepted");
    EXPECT(ternix::mul_mat_ternary_hip(nullptr, nullptr, nullptr, 4, 64, 66) == hipErrorInvalidValue,
           "N not a multiple of 4 accepted");
}

void reference_cpu_shapes() {
    const size_t shapes[][3] = {{1, 8, 8}, {4, 16, 8}, {5, 33, 24}, {8, 64, 64}, {13, 100, 40}, {64, 256, 128}};
    uint32_t seed = 11;
    for (const auto& s : shapes) device_case(make_problem(s[0], s[1], s[2], seed++));
}

void decode_and_prefill_shapes() {
    device_case(make_problem(1, 2560, 2560, 21));     // decode GEMV
    device_case(make_problem(4, 4096, 2048, 22));     // small batch
    device_case(make_problem(16, 2048, 4096, 23));
    device_case(make_problem(64, 1024, 1024, 24));    // split-K GEMM tiles
    device_case(make_problem(256, 2048, 1024, 25));   // prefill GEMM
}

void ragged_and_misaligned_shapes() {
    device_case(make_problem(1, 1000, 3076, 31));
    device_case(make_problem(17, 4093, 1028, 32));
    device_case(make_problem(129, 1001, 516, 33));
    device_case(make_problem(3, 4096, 1024, 34), 3);  // aligned shape, misaligned operands
    device_case(make_problem(40, 512, 256, 35), 1);
}

void extreme_activations_do_not_overflow() {
    // A = -128 everywhere, W = -1 everywhere: every output is 128 * K.
    Problem p = make_problem(4, 4096, 256, 41);
    for (auto& a : p.A) a = -128;
    std::vector<int8_t> W(p.K * p.N, -1);
    ternix::pack_ternary_weights(p.Wp.data(), W.data(), W.size());
    const std::vector<int32_t> ref = expected(p);
    EXPECT(ref[0] == 128 * 4096, "oracle gives %d", ref[0]);
    device_case(p);
}

void graph_replay() {
    // One automatic call captured into a hipGraph and replayed; every replay must give C again.
    const Problem p = make_problem(1, 2560, 6912, 51);
    const std::vector<int32_t> ref = expected(p);
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    int8_t* dA = nullptr;
    uint8_t* dW = nullptr;
    int32_t* dC = nullptr;
    HIP_OK(hipMalloc(&dA, p.A.size()));
    HIP_OK(hipMalloc(&dW, p.Wp.size()));
    HIP_OK(hipMalloc(&dC, ref.size() * sizeof(int32_t)));
    HIP_OK(hipMemcpy(dA, p.A.data(), p.A.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dW, p.Wp.data(), p.Wp.size(), hipMemcpyHostToDevice));
    // One eager call first, so the split-K workspace exists before capture.
    HIP_OK(ternix::mul_mat_ternary_hip(dA, dW, dC, 1, 2560, 6912, st));
    HIP_OK(hipStreamSynchronize(st));
    hipGraph_t graph;
    hipGraphExec_t exec;
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    const hipError_t launch = ternix::mul_mat_ternary_hip(dA, dW, dC, 1, 2560, 6912, st);
    HIP_OK(hipStreamEndCapture(st, &graph));
    HIP_OK(launch);
    HIP_OK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    std::vector<int32_t> got(ref.size());
    for (int r = 0; r < 3; ++r) {
        HIP_OK(hipMemsetAsync(dC, 0, got.size() * sizeof(int32_t), st));
        HIP_OK(hipGraphLaunch(exec, st));
        HIP_OK(hipStreamSynchronize(st));
        HIP_OK(hipMemcpy(got.data(), dC, got.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
        const size_t i = first_mismatch(ref, got);
        EXPECT(i == ref.size(), "replay %d: C[%zu] = %d, expected %d", r, i, got[i], ref[i]);
    }
    HIP_OK(hipGraphExecDestroy(exec));
    HIP_OK(hipGraphDestroy(graph));
    HIP_OK(hipFree(dA));
    HIP_OK(hipFree(dW));
    HIP_OK(hipFree(dC));
    HIP_OK(hipStreamDestroy(st));
}

// The opt-in tile-64 layout: host conversion, then the tile-64 entry point on device memory.
void tile64_layout_matches_cpu() {
    const size_t shapes[][3] = {{1, 2560, 6912}, {4, 4096, 4096}, {24, 2048, 1024}, {64, 4096, 2048}};
    for (const auto& s : shapes) {
        const Problem p = make_problem(s[0], s[1], s[2], 31u + (uint32_t)s[0]);
        const std::vector<int32_t> ref = expected(p);
        std::vector<uint8_t> wt(p.Wp.size());
        EXPECT(ternix_interleave_weights_tile64(wt.data(), p.Wp.data(), p.K, p.N) == 0, "conversion");
        int8_t* dA = nullptr;
        uint8_t* dW = nullptr;
        int32_t* dC = nullptr;
        HIP_OK(hipMalloc(&dA, p.A.size()));
        HIP_OK(hipMalloc(&dW, wt.size()));
        HIP_OK(hipMalloc(&dC, ref.size() * sizeof(int32_t)));
        HIP_OK(hipMemcpy(dA, p.A.data(), p.A.size(), hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(dW, wt.data(), wt.size(), hipMemcpyHostToDevice));
        HIP_OK(ternix::mul_mat_ternary_hip_tile64(dA, dW, dC, (int64_t)p.M, (int64_t)p.K, (int64_t)p.N));
        HIP_OK(hipDeviceSynchronize());
        std::vector<int32_t> got(ref.size());
        HIP_OK(hipMemcpy(got.data(), dC, got.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
        const size_t i = first_mismatch(ref, got);
        EXPECT(i == ref.size(), "M=%zu K=%zu N=%zu: C[%zu] = %d, expected %d", p.M, p.K, p.N, i,
               i < got.size() ? got[i] : 0, i < ref.size() ? ref[i] : 0);
        HIP_OK(hipFree(dA));
        HIP_OK(hipFree(dW));
        HIP_OK(hipFree(dC));
    }
}

void pack_known_answer() {
    // {1,0,-1,1,-1,0,1,0}: byte 0 = 01 | 00<<2 | 11<<4 | 01<<6 = 0x71, byte 1 = 11 | 00<<2 | 01<<4 | 00<<6 = 0x13.
    const int8_t w[8] = {1, 0, -1, 1, -1, 0, 1, 0};
    uint8_t packed[2] = {0, 0};
    ternix::pack_ternary_weights(packed, w, 8);
    EXPECT(packed[0] == 0x71 && packed[1] == 0x13, "packed %02x %02x", packed[0], packed[1]);
    int8_t back[8];
    ternix::unpack_ternary_weights(back, packed, 8);
    EXPECT(std::memcmp(back, w, 8) == 0, "round trip");
}

}  // namespace

int main(int argc, char** argv) {
    const std::vector<std::pair<const char*, std::function<void()>>> cases = {
        {"PackKnownAnswer", pack_known_answer},
        {"NaiveMatchesCpu", naive_matches_cpu},
        {"TiledMatchesCpu", tiled_matches_cpu},
        {"TiledRejectsUnsupportedShape", tiled_rejects_unsupported_shape},
        {"ReferenceCpuShapes", reference_cpu_shapes},
        {"DecodeAndPrefillShapes", decode_and_prefill_shapes},
        {"RaggedAndMisalignedShapes", ragged_and_misaligned_shapes},
        {"ExtremeActivationsDoNotOverflow", extreme_activations_do_not_overflow},
        {"GraphReplay", graph_replay},
        {"Tile64LayoutMatchesCpu", tile64_layout_matches_cpu},
    };
    if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
        for (const auto& c : cases) std::printf("%s\n", c.first);
        return 0;
    }
    int failed_cases = 0;
    for (const auto& c : cases) {
        std::printf("[ RUN  ] %s\n", c.first);
        std::fflush(stdout);
        const int before = g_failures;
        c.second();
        const bool ok = g_failures == before;
        failed_cases += ok ? 0 : 1;
        std::printf("[ %s ] %s\n", ok ? " OK " : "FAIL", c.first);
        std::fflush(stdout);
    }
    std::printf("%zu cases, %d failed\n", cases.size(), failed_cases);
    return failed_cases == 0 ? 0 : 1;
}
