// layer_kernels.hip -- the gfx950 kernels around the ternary matmul: activation quantisation,
// dequantisation, the padded copy for ragged shapes, zero fill, the naive drop-in kernel, and the
// per-device CU count the launchers plan with.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include "kernel_common.h"
#include "row_stats.h"
#include "ternary_kernels.h"

namespace ternix_hip {
namespace {

// ------------------------------------------------------------------------------------------------
// Naive kernel: one work-item per output, weights decoded per k from global memory with
// w = (b & 1) - (b & 2) (the reference decode2, src/cuda_kernels.cu:40-54).
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void naive_kernel(const int8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                    int32_t* __restrict__ C, int M, int K, int N) {
    const int col = blockIdx.x * 64 + (threadIdx.x & 63);
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (row >= M || col >= N) return;
    const int NB = N >> 2;
    const int shift = (col & 3) * 2;
    int acc = 0;
    for (int k = 0; k < K; ++k) {
        const unsigned bits = (B[(size_t)k * NB + (col >> 2)] >> shift) & 3u;
        acc += (int)A[(size_t)row * K + k] * ((int)(bits & 1u) - (int)(bits & 2u));
    }
    C[(size_t)row * N + col] = acc;
}

// Bare streaming read of n16 16-byte chunks (the HBM floor the GEMVs are compared with): every
// thread keeps four non-temporal 16-byte loads in flight, block-contiguous chunks per iteration; the
// XOR of everything read is stored only if it equals a value it cannot reach in practice, so the
// loads are kept but nothing is written.  (Measured on MI355X, cold buffers: four workgroups per CU
// with non-temporal loads read 58.7 MB in 9.4 us, plain loads or more workgroups per CU 9.5-10.1.)
__global__ __launch_bounds__(256) void stream_read_kernel(const v4i* __restrict__ p, size_t n16, int* __restrict__ out) {
    size_t i = (size_t)blockIdx.x * 1024 + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * 1024;
    v4i acc = {0, 0, 0, 0};
    for (; i < n16; i += stride) {
        v4i v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = (i + 256 * u < n16) ? __builtin_nontemporal_load(p + i + 256 * u) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u];
    }
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x7e3a91c5) out[0] = 1;
}

__global__ __launch_bounds__(256) void zero_kernel(int32_t* __restrict__ C, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * 256;
    for (; i < n; i += stride) C[i] = 0;
}

// ------------------------------------------------------------------------------------------------
// Activation quantisation and dequantisation (the steps either side of the matmul in a BitNet b1.58
// layer; the reference leaves them as a stub, scripts/quantize.py:5, README.md:203).
//   quantize_rows_kernel: one workgroup per row; absmax by a max-reduction (exact, order-free),
//     s = 127 / max(absmax, 1e-5), q = clamp(rint(x * s), -128, 127) (round half to even),
//     row_scale = max(absmax, 1e-5) / 127 -- IEEE division and multiplication, no contraction, so the
//     CPU restatement reproduces every bit.
//   dequant_kernel: y = (float)c * (row_scale[m] * w_scale) for an int32 C (Y may alias C: each
//     element is read before the same element is written by the same thread).
// Both are HBM streams (quantise: 4 bytes read + 1 written per element, twice over the row if it
// does not stay in cache; dequantise: 4 + 4 bytes per output).
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_kernel(const int32_t* C, OutScale os, int N, size_t items, int vec) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= items) return;
    const size_t e = 4 * i;
    const int row = (int)(e / (size_t)N), col = (int)(e % (size_t)N);
    v4i c;
    if (vec) {
        c = reinterpret_cast<const v4i*>(C)[i];
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = C[e + j];
    }
    store_scaled(os, row, N, col, c, vec);
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ X, int8_t* __restrict__ Q,
                                                            float* __restrict__ row_scale, int K, int vec) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* x = X + (size_t)m * (size_t)K;
    int8_t* q = Q + (size_t)m * (size_t)K;
    float amax = 0.0f;
    if (vec) {
        for (int c = threadIdx.x; c < K / 4; c += 256) {
            const v4f v = reinterpret_cast<const v4f*>(x)[c];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
    } else {
        for (int c = threadIdx.x; c < K; c += 256) amax = fmaxf(amax, fabsf(x[c]));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float a = fmaxf(amax, 1e-5f);
    const float s = 127.0f / a;
    if (threadIdx.x == 0) row_scale[m] = a / 127.0f;
    auto qz = [&](float v) -> int {
        const float r = rintf(v * s);
        return (int)fminf(fmaxf(r, -128.0f), 127.0f);
    };
    if (vec) {
        for (int c = threadIdx.x; c < K / 16; c += 256) {
            const v4f* src = reinterpret_cast<const v4f*>(x) + 4 * c;
            v4i out;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const v4f v = src[u];
                out[u] = (int)((uint32_t)(qz(v[0]) & 0xFF) | ((uint32_t)(qz(v[1]) & 0xFF) << 8) |
                               ((uint32_t)(qz(v[2]) & 0xFF) << 16) | ((uint32_t)(qz(v[3]) & 0xFF) << 24));
            }
            reinterpret_cast<v4i*>(q)[c] = out;
        }
    } else {
        for (int c = threadIdx.x; c < K; c += 256) q[c] = (int8_t)qz(x[c]);
    }
}

// Tile-64 layout conversion (kernel_common.h): a permutation copy.  A workgroup of 8 waves takes one
// 64-row k-step of 8 adjacent strips; wave w writes block (strip, k-step) of its strip as one
// contiguous 1 KB store (lane = row), and the 8 waves together read 128 contiguous bytes of each row.
__global__ __launch_bounds__(512) void tile64_kernel(const uint8_t* __restrict__ W, uint8_t* __restrict__ Wt,
                                                     int nK, int strips) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int groups = (strips + 7) >> 3;
    const size_t NB = (size_t)strips * 16;
    for (size_t u = blockIdx.x; u < (size_t)groups * (size_t)nK; u += gridDim.x) {
        const int s = (int)(u % (size_t)nK), c = (int)(u / (size_t)nK) * 8 + wave;
        if (c >= strips) continue;
        const int r = s * 64 + tile64_pos(lane);  // the row stored at position `lane` of the block
        *reinterpret_cast<v4i*>(Wt + ((size_t)c * (size_t)nK + (size_t)s) * 1024 + (size_t)lane * 16) =
            *reinterpret_cast<const v4i*>(W + (size_t)r * NB + (size_t)c * 16);
    }
}

}  // namespace

hipError_t launch_zero(int32_t* C, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, C, n);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* p, size_t bytes, int* out, hipStream_t st) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    size_t blocks = (n16 + 1023) / 1024;
    const size_t cap = (size_t)device_cu_count() * 4;  // four 256-thread workgroups per CU at most
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<const v4i*>(p), n16,
                       out);
    return hipGetLastError();
}

// Compute units of the current device, read once per device (the attribute query is not free).
int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// ------------------------------------------------------------------------------------------------
// Padded copy for ragged shapes: rows of `len` bytes at pitch src_pitch (any alignment) into rows of
// dst_pitch bytes (16-byte aligned, dst_pitch % 16 == 0), zero-filled past len and for the rows
// rows..dst_rows-1.  Each thread writes one 16-byte chunk from the aligned dwords holding its bytes
// (one 16-byte load where the four lie inside the source's 4-byte aligned extent, dword by dword at
// its end) and v_alignbyte; an aligned dword holding at least one byte of the source buffer never
// crosses a page the buffer does not touch, so loads stay within the buffer's pages.
// ------------------------------------------------------------------------------------------------
struct PadJob {
    const uint8_t* src;
    uint8_t* dst;
    int rows, dst_rows, src_pitch, len, dst_pitch;
    size_t chunks;  // dst_rows * dst_pitch / 16
};

typedef uint32_t pad_u4 __attribute__((ext_vector_type(4), aligned(4)));
typedef __attribute__((address_space(1))) const uint32_t pad_g32;
typedef __attribute__((address_space(1))) const pad_u4 pad_g4;

template <typename I>
__device__ __forceinline__ void pad_chunk(const PadJob& j, I idx) {
    const I cpr = (I)(j.dst_pitch >> 4);
    const int r = (int)(idx / cpr), c = (int)(idx % cpr);
    v4i out = {0, 0, 0, 0};
    const int n = min(max(j.len - 16 * c, 0), 16);  // source bytes in this chunk
    if (r < j.rows && n > 0) {
        const uintptr_t p = reinterpret_cast<uintptr_t>(j.src) + (size_t)r * (size_t)j.src_pitch + 16 * c;
        const uintptr_t end = reinterpret_cast<uintptr_t>(j.src) + (size_t)(j.rows - 1) * (size_t)j.src_pitch + j.len;
        const uintptr_t pa = p & ~(uintptr_t)3;
        const uint32_t sh = (uint32_t)(p & 3);
        uint32_t d[5] = {0u, 0u, 0u, 0u, 0u};
        if (pa + 16 <= ((end + 3) & ~(uintptr_t)3)) {
            // the four dwords from the chunk's first one lie inside the source's aligned extent: one
            // 16-byte load, and the fifth dword when the chunk reaches into it
            const pad_u4 x = *(pad_g4*)pa;
#pragma unroll
            for (int k = 0; k < 4; ++k) d[k] = x[k];
            if (pa + 16 < end && sh + n > 16) d[4] = *((pad_g32*)pa + 4);
        } else {
#pragma unroll
            for (int k = 0; k < 5; ++k) d[k] = pa + 4 * k < end ? *((pad_g32*)pa + k) : 0u;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t v = __builtin_amdgcn_alignbyte(d[m + 1], d[m], sh);
            const int keep = min(max(n - 4 * m, 0), 4);  // bytes of this dword inside the row
            v = keep >= 4 ? v : (keep == 0 ? 0u : (v & ((1u << (8 * keep)) - 1u)));
            out[m] = (int)v;
        }
    }
    *reinterpret_cast<v4i*>(j.dst + (size_t)r * (size_t)j.dst_pitch + 16 * c) = out;
}

// I: the chunk index type (32-bit when both jobs' chunks fit, which keeps the row division short).
template <typename I>
__global__ __launch_bounds__(256) void pad_rows_kernel(PadJob j0, PadJob j1) {
    const I total = (I)(j0.chunks + j1.chunks), c0 = (I)j0.chunks;
    for (I i = (I)blockIdx.x * 256 + threadIdx.x; i < total; i += (I)gridDim.x * 256) {
        if (i < c0) pad_chunk<I>(j0, i);
        else pad_chunk<I>(j1, i - c0);
    }
}

hipError_t launch_pad_rows(const uint8_t* src0, uint8_t* dst0, int rows0, int dst_rows0, int src_pitch0, int len0,
                           int dst_pitch0, const uint8_t* src1, uint8_t* dst1, int rows1, int dst_rows1,
                           int src_pitch1, int len1, int dst_pitch1, hipStream_t st) {
    if (dst_pitch0 % 16 != 0 || (uintptr_t)dst0 % 16 != 0 || len0 > dst_pitch0 || rows0 > dst_rows0 ||
        (dst1 && (dst_pitch1 % 16 != 0 || (uintptr_t)dst1 % 16 != 0 || len1 > dst_pitch1 || rows1 > dst_rows1)))
        return hipErrorInvalidValue;
    const PadJob j0{src0, dst0, rows0, dst_rows0, src_pitch0, len0, dst_pitch0,
                    (size_t)dst_rows0 * (size_t)dst_pitch0 / 16};
    const PadJob j1{src1, dst1, rows1, dst_rows1, src_pitch1, len1, dst_pitch1,
                    dst1 ? (size_t)dst_rows1 * (size_t)dst_pitch1 / 16 : 0};
    const size_t total = j0.chunks + j1.chunks;
    if (total == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
    if (total < ((size_t)1 << 31))
        hipLaunchKernelGGL(pad_rows_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, j0, j1);
    else
        hipLaunchKernelGGL(pad_rows_kernel<size_t>, dim3(blocks), dim3(256), 0, st, j0, j1);
    return hipGetLastError();
}

hipError_t launch_dequant(const int32_t* C, const OutScale& os, int M, int N, hipStream_t st) {
    const size_t n = (size_t)M * (size_t)N;
    if (n == 0) return hipSuccess;
    const int vec = ((uintptr_t)C % 16 == 0) && ((uintptr_t)os.Y % 16 == 0);
    const size_t items = n / 4;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, C, os, N, items, vec);
    return hipGetLastError();
}

hipError_t launch_quantize_rows(const float* X, int8_t* Q, float* row_scale, int M, int K, hipStream_t st) {
    if (M == 0) return hipSuccess;
    const int vec = (K % 16 == 0) && ((uintptr_t)X % 16 == 0) && ((uintptr_t)Q % 16 == 0);
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)M), dim3(256), 0, st, X, Q, row_scale, K, vec);
    return hipGetLastError();
}

hipError_t launch_tile64(const uint8_t* W, uint8_t* Wt, int K, int N, hipStream_t st) {
    const int NB = N >> 2;
    if (K % 64 != 0 || NB % 16 != 0 || (uintptr_t)W % 16 != 0 || (uintptr_t)Wt % 16 != 0 ||
        (size_t)K * (size_t)NB >= ((size_t)1 << 32))
        return hipErrorInvalidValue;
    const size_t units = (size_t)K / 64 * (size_t)((NB / 16 + 7) / 8);
    if (units == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>(units, 65536);
    hipLaunchKernelGGL(tile64_kernel, dim3(blocks), dim3(512), 0, st, W, Wt, K / 64, NB / 16);
    return hipGetLastError();
}

hipError_t launch_naive(const int8_t* A, const uint8_t* B, int32_t* C, int M, int K, int N, hipStream_t st) {
    const dim3 grid((N + 63) / 64, (M + 3) / 4);
    hipLaunchKernelGGL(naive_kernel, grid, dim3(256), 0, st, A, B, C, M, K, N);
    return hipGetLastError();
}

}  // namespace ternix_hip
