// bitpack.cpp -- the 2-bit ternary weight format on the host: pack, unpack, offline interleave.
//
// Format (reference src/bitpack.cpp:5-27, README.md:46-53): element 4i+j of the flat int8 array
// occupies bits 2j..2j+1 of byte i; +1 -> 01, -1 -> 11, anything else -> 00.  Decoding maps
// 01 -> +1, 11 -> -1 and both 00 and the never-produced 10 -> 0.  A K x N matrix flattened
// row-major (N % 4 == 0) therefore packs to the K x (N/4) layout every kernel reads.
//
// Implementation: a 256-entry table per direction is built once at load time; packing combines four
// 2-bit codes per output byte, unpacking copies one 4-byte table entry per input byte.
#include <cmath>
#include <cstring>
#include <vector>

#include "ternix/bitpack.hpp"
#include "ternix/ternix_hip.h"

namespace {

struct Tables {
    uint8_t code_of[256];      // int8 value (as uint8 index) -> 2-bit code
    uint32_t unpacked_of[256]; // packed byte -> four int8 values, little-endian
    Tables() {
        for (int v = 0; v < 256; ++v) {
            const int8_t s = static_cast<int8_t>(v);
            code_of[v] = s == 1 ? 1 : (s == -1 ? 3 : 0);
        }
        for (int b = 0; b < 256; ++b) {
            uint32_t word = 0;
            for (int j = 0; j < 4; ++j) {
                const int code = (b >> (2 * j)) & 3;
                const uint8_t val = code == 1 ? 0x01 : (code == 3 ? 0xFF : 0x00);
                word |= static_cast<uint32_t>(val) << (8 * j);
            }
            unpacked_of[b] = word;
        }
    }
};

const Tables& tables() {
    static const Tables t;
    return t;
}

}  // namespace

namespace ternix {

void pack_ternary_weights(uint8_t* packed, const int8_t* unpacked, size_t size) {
    const Tables& t = tables();
    const uint8_t* u = reinterpret_cast<const uint8_t*>(unpacked);
    for (size_t i = 0; i < size / 4; ++i) {
        const uint8_t* e = u + 4 * i;
        packed[i] = static_cast<uint8_t>(t.code_of[e[0]] | (t.code_of[e[1]] << 2) | (t.code_of[e[2]] << 4) |
                                         (t.code_of[e[3]] << 6));
    }
}

void unpack_ternary_weights(int8_t* unpacked, const uint8_t* packed, size_t size) {
    const Tables& t = tables();
    for (size_t i = 0; i < size / 4; ++i) std::memcpy(unpacked + 4 * i, &t.unpacked_of[packed[i]], 4);
}

void interleave_weights_offline(uint8_t* interleaved, const uint8_t* packed, size_t size) {
    if (size / 4 && interleaved != packed) std::memmove(interleaved, packed, size / 4);
}

}  // namespace ternix

namespace {

// BitNet b1.58 absmean weight quantisation (the offline step the reference leaves as a stub,
// scripts/quantize.py:5): gamma = max(mean|W|, 1e-5) with the mean summed in double in index
// order, then w = clamp(rint(W / gamma), -1, 1) with an IEEE fp32 division (round half to even).
float absmean_quantize(int8_t* q, const float* w, size_t size) {
    double sum = 0.0;
    for (size_t i = 0; i < size; ++i) sum += std::fabs(static_cast<double>(w[i]));
    float gamma = size ? static_cast<float>(sum / static_cast<double>(size)) : 0.0f;
    if (!(gamma >= 1e-5f)) gamma = 1e-5f;
    for (size_t i = 0; i < size; ++i) {
        const float r = std::nearbyint(w[i] / gamma);
        q[i] = static_cast<int8_t>(r > 1.0f ? 1 : (r < -1.0f ? -1 : static_cast<int>(r)));
    }
    return gamma;
}

}  // namespace

extern "C" {

int ternix_quantize_weights_absmean(uint8_t* packed, float* w_scale, const float* W, size_t size) {
    if (size % 4 != 0 || w_scale == nullptr || (size && (packed == nullptr || W == nullptr))) return 1;
    std::vector<int8_t> q(size);
    *w_scale = absmean_quantize(q.data(), W, size);
    ternix::pack_ternary_weights(packed, q.data(), size);
    return 0;
}


void ternix_pack_ternary_weights(uint8_t* packed, const int8_t* unpacked, size_t size) {
    ternix::pack_ternary_weights(packed, unpacked, size);
}
void ternix_unpack_ternary_weights(int8_t* unpacked, const uint8_t* packed, size_t size) {
    ternix::unpack_ternary_weights(unpacked, packed, size);
}
void ternix_interleave_weights_offline(uint8_t* interleaved, const uint8_t* packed, size_t size) {
    ternix::interleave_weights_offline(interleaved, packed, size);
}

int ternix_interleave_weights_tile64(uint8_t* out, const uint8_t* packed, size_t K, size_t N) {
    const size_t NB = N / 4;
    if (N % 4 != 0 || K % 64 != 0 || NB % 16 != 0) return 1;  // hipErrorInvalidValue
    if (K * NB == 0) return 0;
    if (out == nullptr || packed == nullptr || out == packed) return 1;
    const size_t nK = K / 64, strips = NB / 16;
    for (size_t r = 0; r < K; ++r)
        for (size_t c = 0; c < strips; ++c) {
            // block (c, r / 64), row position r % 64 ^ (8 * ((r % 64 / 16) % 2)), 16 bytes per row
            const size_t rr = r % 64, pos = rr ^ (((rr >> 4) & 1) << 3);
            std::memcpy(out + ((c * nK + r / 64) * 64 + pos) * 16, packed + r * NB + c * 16, 16);
        }
    return 0;
}

}  // extern "C"
