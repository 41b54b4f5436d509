// bitpack_kernels.hip -- the 2-bit weight format on the GPU (gfx950).
//
// Same format and edge behaviour as the host routines of reference src/bitpack.cpp:
//   pack   (:5-15)  value at flat index 4i+j -> bits 2j..2j+1 of byte i; +1 -> 01, -1 -> 11, any other
//                   value -> 00; `size` elements give size/4 bytes (a trailing size%4 is ignored);
//   unpack (:17-27) 01 -> +1, 11 -> -1, 00 and 10 -> 0; writes 4*(size/4) elements;
//   interleave (:29-33) identity copy of size/4 bytes.
// Both kernels are byte streams bound by HBM bandwidth (5 bytes moved per 4 weights): each work-item
// turns 64 weights into 16 packed bytes (or back) with 16-byte loads and stores and SWAR bit
// arithmetic on 32-bit words (no per-weight branches, no tables).  Grids are sized to the data; the
// 16-byte path needs 16-byte aligned pointers, anything else takes the byte path.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ternary_kernels.h"

namespace ternix_hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// Per-byte equality mask: 0xFF in every byte of x equal to the same byte of pat, else 0x00.
__device__ __forceinline__ uint32_t byte_eq(uint32_t x, uint32_t pat) {
    const uint32_t y = x ^ pat;                                        // zero bytes where equal
    const uint32_t t = ((y & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | y;           // bit 7 set where byte != 0
    const uint32_t z = ~t & 0x80808080u;                                // bit 7 set where byte == 0
    return (z >> 7) * 0xFFu;
}

// Four int8 weights (one per byte of w) -> one packed byte.
__device__ __forceinline__ uint32_t pack4(uint32_t w) {
    const uint32_t code = (byte_eq(w, 0x01010101u) & 0x01010101u) | (byte_eq(w, 0xFFFFFFFFu) & 0x03030303u);
    return (code & 0x3u) | ((code >> 6) & 0xCu) | ((code >> 12) & 0x30u) | ((code >> 18) & 0xC0u);
}

// One packed byte (low 8 bits of b) -> four int8 weights, one per byte.
__device__ __forceinline__ uint32_t unpack4(uint32_t b) {
    const uint32_t d = (b & 0x3u) | ((b & 0xCu) << 6) | ((b & 0x30u) << 12) | ((b & 0xC0u) << 18);
    const uint32_t lo = d & 0x01010101u, hi = (d >> 1) & 0x01010101u;
    return (lo & ~hi) | ((lo & hi) * 0xFFu);
}

// 16 output bytes per work-item from 64 weights; items past the 16-byte body handle single bytes.
__global__ __launch_bounds__(256) void pack_kernel(uint8_t* __restrict__ packed, const int8_t* __restrict__ w,
                                                   size_t nbytes, int vec) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (vec) {
        const size_t nvec = nbytes / 16;
        if (i < nvec) {
            const v4i* src = reinterpret_cast<const v4i*>(w) + 4 * i;
            v4i out;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const v4i x = src[u];
                out[u] = (int)(pack4((uint32_t)x[0]) | (pack4((uint32_t)x[1]) << 8) |
                               (pack4((uint32_t)x[2]) << 16) | (pack4((uint32_t)x[3]) << 24));
            }
            reinterpret_cast<v4i*>(packed)[i] = out;
            return;
        }
        const size_t b = nvec * 16 + (i - nvec);  // tail bytes, one per item
        if (i >= nvec && b < nbytes) {
            const uint32_t x = (uint32_t)(uint8_t)w[4 * b] | ((uint32_t)(uint8_t)w[4 * b + 1] << 8) |
                               ((uint32_t)(uint8_t)w[4 * b + 2] << 16) | ((uint32_t)(uint8_t)w[4 * b + 3] << 24);
            packed[b] = (uint8_t)pack4(x);
        }
        return;
    }
    if (i < nbytes) {
        const uint32_t x = (uint32_t)(uint8_t)w[4 * i] | ((uint32_t)(uint8_t)w[4 * i + 1] << 8) |
                           ((uint32_t)(uint8_t)w[4 * i + 2] << 16) | ((uint32_t)(uint8_t)w[4 * i + 3] << 24);
        packed[i] = (uint8_t)pack4(x);
    }
}

// 16 packed bytes -> 64 weights per work-item; same tail handling.
__global__ __launch_bounds__(256) void unpack_kernel(int8_t* __restrict__ w, const uint8_t* __restrict__ packed,
                                                     size_t nbytes, int vec) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (vec) {
        const size_t nvec = nbytes / 16;
        if (i < nvec) {
            const v4i x = reinterpret_cast<const v4i*>(packed)[i];
            v4i* dst = reinterpret_cast<v4i*>(w) + 4 * i;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t p = (uint32_t)x[u];
                dst[u] = v4i{(int)unpack4(p & 0xFFu), (int)unpack4((p >> 8) & 0xFFu), (int)unpack4((p >> 16) & 0xFFu),
                             (int)unpack4(p >> 24)};
            }
            return;
        }
        const size_t b = nvec * 16 + (i - nvec);
        if (i >= nvec && b < nbytes) {
            const uint32_t v = unpack4(packed[b]);
#pragma unroll
            for (int j = 0; j < 4; ++j) w[4 * b + j] = (int8_t)(v >> (8 * j));
        }
        return;
    }
    if (i < nbytes) {
        const uint32_t v = unpack4(packed[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) w[4 * i + j] = (int8_t)(v >> (8 * j));
    }
}

unsigned grid_for(size_t nbytes, bool vec) {
    const size_t items = vec ? nbytes / 16 + nbytes % 16 : nbytes;
    return (unsigned)((items + 255) / 256);
}

}  // namespace

hipError_t launch_pack(uint8_t* packed, const int8_t* w, size_t size, hipStream_t st) {
    const size_t nbytes = size / 4;
    if (nbytes == 0) return hipSuccess;
    const bool vec = ((uintptr_t)packed % 16 == 0) && ((uintptr_t)w % 16 == 0);
    hipLaunchKernelGGL(pack_kernel, dim3(grid_for(nbytes, vec)), dim3(256), 0, st, packed, w, nbytes, (int)vec);
    return hipGetLastError();
}

hipError_t launch_unpack(int8_t* w, const uint8_t* packed, size_t size, hipStream_t st) {
    const size_t nbytes = size / 4;
    if (nbytes == 0) return hipSuccess;
    const bool vec = ((uintptr_t)packed % 16 == 0) && ((uintptr_t)w % 16 == 0);
    hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(nbytes, vec)), dim3(256), 0, st, w, packed, nbytes, (int)vec);
    return hipGetLastError();
}

}  // namespace ternix_hip
