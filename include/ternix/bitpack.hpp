// bitpack.hpp -- 2-bit ternary weight format (same API as the reference's include/ternix/bitpack.hpp:6-8).
// Implemented in libternix_hip.so (ternixengine_amd/csrc/bitpack.cpp); C-ABI twins are declared in
// ternix_hip.h as ternix_pack_ternary_weights / ternix_unpack_ternary_weights /
// ternix_interleave_weights_offline.
#pragma once
#include <cstddef>
#include <cstdint>

namespace ternix {
// `size` = number of weights (a multiple of 4); writes size/4 bytes.  +1 -> 01, -1 -> 11, else 00.
void pack_ternary_weights(uint8_t* packed, const int8_t* unpacked, size_t size);
// Inverse of pack_ternary_weights: 01 -> +1, 11 -> -1, 00 and 10 -> 0.
void unpack_ternary_weights(int8_t* unpacked, const uint8_t* packed, size_t size);
// Identity copy of size/4 bytes: the packed K x N/4 layout is what every kernel consumes.
void interleave_weights_offline(uint8_t* interleaved, const uint8_t* packed, size_t size);
}  // namespace ternix
