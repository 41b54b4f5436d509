// ternix_engine.cpp -- the `ternix_engine` Python module of TernixEngine (reference
// bindings/python/pybind11_wrapper.cpp:75-98) with the MI355X GPU path added.
//
// Same names, defaults and exception types as the reference module:
//   pack_ternary(w) / unpack_ternary(packed)                 (reference :21-39)
//   ternary_matmul(a, b_packed, impl="avx2_blocked")        (reference :41-71)
//   has_cuda (False here: no CUDA), Model                   (reference :86-97)
// plus impl strings "hip", "hip_gemv", "hip_gemm", "hip_tiled", "hip_naive" (libternix_hip.so through
// its C-ABI, GIL released during the device call, RuntimeError("HIP error: ...") on any device-side
// failure, including a shape the tiled kernel rejects, as the reference's cuda_tiled does) and has_hip.
// "cuda_naive" / "cuda_tiled" are not aliased: as in a reference build without CUDA they raise
// ValueError("unknown impl ...") and has_cuda is False; hip_naive / hip_tiled are their counterparts.
//
// The CPU impl strings ("naive", "scalar", "avx2", "avx2_blocked") run the reference's own CPU
// kernels, which the drop-in keeps unchanged in its ternix_core library (mul_mat_ternary.h:18-60).
// They are weak references here: a build that links ternix_core (the reference's CMake target)
// resolves them at link time, and a process that has loaded a library exporting them before
// importing this module resolves them at load time.  Without them the CPU impls raise
// RuntimeError; the HIP impls never use them.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "ternix/ternix_hip.h"

namespace ternix {
// The reference's CPU kernels (include/ternix/mul_mat_ternary.h:18-60), resolved from ternix_core.
__attribute__((weak)) void mul_mat_ternary_naive(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K,
                                                 size_t N);
__attribute__((weak)) void mul_mat_ternary_scalar(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K,
                                                  size_t N);
__attribute__((weak)) void mul_mat_ternary_avx2(const int8_t* A, const uint8_t* B, int32_t* C, size_t M, size_t K,
                                                size_t N);
__attribute__((weak)) void mul_mat_ternary_avx2_blocked(const int8_t* A, const uint8_t* B, int32_t* C, size_t M,
                                                        size_t K, size_t N);
}  // namespace ternix

namespace py = pybind11;

namespace {

using i8_array = py::array_t<int8_t, py::array::c_style | py::array::forcecast>;
using u8_array = py::array_t<uint8_t, py::array::c_style | py::array::forcecast>;

u8_array pack_ternary(i8_array w) {
    if (w.ndim() != 2) throw py::value_error("pack_ternary expects a 2-D (K, N) array");
    const py::ssize_t K = w.shape(0), N = w.shape(1);
    if (N % 4 != 0) throw py::value_error("N must be a multiple of 4");
    const int8_t* src = w.data();
    for (py::ssize_t i = 0; i < K * N; ++i)
        if (src[i] < -1 || src[i] > 1) throw py::value_error("weights must be in {-1, 0, +1}");
    u8_array out({K, N / 4});
    ternix_pack_ternary_weights(out.mutable_data(), src, static_cast<size_t>(K * N));
    return out;
}

i8_array unpack_ternary(u8_array packed) {
    if (packed.ndim() != 2) throw py::value_error("unpack_ternary expects a 2-D (K, N/4) array");
    const py::ssize_t K = packed.shape(0), N4 = packed.shape(1);
    i8_array out({K, N4 * 4});
    ternix_unpack_ternary_weights(out.mutable_data(), packed.data(), static_cast<size_t>(K * N4 * 4));
    return out;
}

using CpuKernel = void (*)(const int8_t*, const uint8_t*, int32_t*, size_t, size_t, size_t);

CpuKernel cpu_kernel(const std::string& impl) {
    if (impl == "naive") return &ternix::mul_mat_ternary_naive;
    if (impl == "scalar") return &ternix::mul_mat_ternary_scalar;
    if (impl == "avx2") return &ternix::mul_mat_ternary_avx2;
    if (impl == "avx2_blocked") return &ternix::mul_mat_ternary_avx2_blocked;
    return nullptr;
}

int hip_variant(const std::string& impl) {
    if (impl == "hip") return TERNIX_HIP_AUTO;
    if (impl == "hip_naive") return TERNIX_HIP_NAIVE;
    if (impl == "hip_gemv") return TERNIX_HIP_GEMV;
    if (impl == "hip_gemm") return TERNIX_HIP_GEMM;
    if (impl == "hip_tiled") return TERNIX_HIP_TILED;
    return -1;
}

bool is_cpu_impl(const std::string& impl) {
    return impl == "naive" || impl == "scalar" || impl == "avx2" || impl == "avx2_blocked";
}

py::array_t<int32_t> ternary_matmul(i8_array a, u8_array b_packed, const std::string& impl) {
    if (a.ndim() != 2 || b_packed.ndim() != 2) throw py::value_error("A must be (M, K) and B_packed (K, N/4)");
    const size_t M = a.shape(0), K = a.shape(1), N = static_cast<size_t>(b_packed.shape(1)) * 4;
    if (static_cast<size_t>(b_packed.shape(0)) != K) throw py::value_error("inner dimensions do not match");
    const int variant = hip_variant(impl);
    if (!is_cpu_impl(impl) && variant < 0) throw py::value_error("unknown impl '" + impl + "'");
    if ((impl == "avx2" || impl == "avx2_blocked") && N % 8 != 0)
        throw py::value_error("AVX2 kernels need N to be a multiple of 8");
    py::array_t<int32_t> c({static_cast<py::ssize_t>(M), static_cast<py::ssize_t>(N)});
    const int8_t* pa = a.data();
    const uint8_t* pb = b_packed.data();
    int32_t* pc = c.mutable_data();
    if (is_cpu_impl(impl)) {
        const CpuKernel k = cpu_kernel(impl);
        if (k == nullptr)
            throw std::runtime_error("impl '" + impl + "' needs the reference CPU kernels (ternix_core), "
                                     "which are not linked into this process");
        k(pa, pb, pc, M, K, N);
        return c;
    }
    int e;
    {
        py::gil_scoped_release release;
        e = ternix_hip_mul_mat_ternary_host(pa, pb, pc, static_cast<int64_t>(M), static_cast<int64_t>(K),
                                            static_cast<int64_t>(N), variant);
    }
    if (e != 0) throw std::runtime_error(std::string("HIP error: ") + ternix_hip_error_string(e));
    return c;
}

// The reference's Model (include/ternix/model.hpp, src/model.cpp): a configuration record whose
// load() creates the vocab_size x hidden_size fp32 embedding table.  Model loading is outside the
// matmul path; the class keeps the module's names and defaults.
struct Model {
    explicit Model(const std::string& path) : file_path(path) {}
    void load() { embedding.assign(vocab_size * hidden_size, 0.0f); }
    size_t vocab_size = 32000;
    size_t hidden_size = 4096;
    size_t num_layers = 32;
    std::string file_path;
    std::vector<float> embedding;
};

}  // namespace

PYBIND11_MODULE(ternix_engine, m) {
    m.doc() = "TernixEngine: 1.58-bit ternary GEMM kernels (reference CPU kernels, MI355X HIP kernels) and "
              "packing utilities";
    m.def("pack_ternary", &pack_ternary, py::arg("w"),
          "Pack a (K, N) int8 array in {-1,0,1} into a (K, N/4) uint8 array");
    m.def("unpack_ternary", &unpack_ternary, py::arg("packed"), "Inverse of pack_ternary");
    m.def("ternary_matmul", &ternary_matmul, py::arg("a"), py::arg("b_packed"), py::arg("impl") = "avx2_blocked",
          "C = A (M,K int8) @ W (K,N ternary packed) -> (M,N int32). impl: naive | scalar | avx2 | avx2_blocked "
          "| hip | hip_gemv | hip_gemm | hip_tiled | hip_naive");
    m.attr("has_cuda") = false;
    m.attr("has_hip") = ternix_hip_device_count() > 0;
    py::class_<Model>(m, "Model")
        .def(py::init<const std::string&>())
        .def("load", &Model::load)
        .def_readwrite("vocab_size", &Model::vocab_size)
        .def_readwrite("hidden_size", &Model::hidden_size)
        .def_readwrite("num_layers", &Model::num_layers);
}
