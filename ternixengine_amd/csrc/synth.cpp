// synth.cpp -- deterministic synthetic inputs (include/ternix/synth.h).  Host code; large arrays are
// filled by up to 16 threads over disjoint slices (each element depends only on its index).
#include "ternix/synth.h"

#include <algorithm>
#include <thread>
#include <vector>

namespace {

inline uint64_t mix(uint64_t seed, uint64_t stream, uint64_t i) {
    uint64_t z = (seed ^ (stream * 0xD1B54A32D192ED03ull)) + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <typename F>
void parallel_for(size_t n, F f) {
    const size_t kGrain = size_t(1) << 22;
    unsigned hw = std::thread::hardware_concurrency();
    if (hw == 0) hw = 1;
    const size_t nt = std::min<size_t>({(size_t)hw, (size_t)16, (n + kGrain - 1) / kGrain});
    if (nt <= 1) {
        f(size_t(0), n);
        return;
    }
    std::vector<std::thread> pool;
    for (size_t t = 0; t < nt; ++t) pool.emplace_back([=] { f(n * t / nt, n * (t + 1) / nt); });
    for (auto& th : pool) th.join();
}

inline int8_t ternary_of(uint64_t r, uint64_t p_neg, uint64_t p_pos) {
    const uint64_t u = r >> 32;
    return u < p_neg ? int8_t(-1) : (u < p_neg + p_pos ? int8_t(1) : int8_t(0));
}

}  // namespace

extern "C" {

uint64_t ternix_synth_u64(uint64_t seed, uint64_t stream, uint64_t index) { return mix(seed, stream, index); }

void ternix_synth_act_uniform(int8_t* a, size_t n, uint64_t seed, uint64_t stream) {
    parallel_for(n, [=](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) a[i] = static_cast<int8_t>(mix(seed, stream, i) & 0xFF);
    });
}

void ternix_synth_act_gauss(int8_t* a, size_t n, uint64_t seed, uint64_t stream, int sigma) {
    parallel_for(n, [=](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            int64_t s = 0;
            for (int d = 0; d < 3; ++d) {
                const uint64_t r = mix(seed, stream, 3 * i + d);
                s += (int64_t)(r & 0xFFFF) + (int64_t)((r >> 16) & 0xFFFF) + (int64_t)((r >> 32) & 0xFFFF) +
                     (int64_t)(r >> 48);
            }
            s -= 393210;
            int64_t v = (s * sigma + 32768) >> 16;  // arithmetic shift: floor
            v = std::max<int64_t>(-128, std::min<int64_t>(127, v));
            a[i] = static_cast<int8_t>(v);
        }
    });
}

void ternix_synth_ternary(int8_t* w, size_t n, uint64_t seed, uint64_t stream, uint64_t p_neg, uint64_t p_pos) {
    parallel_for(n, [=](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) w[i] = ternary_of(mix(seed, stream, i), p_neg, p_pos);
    });
}

void ternix_synth_ternary_packed(uint8_t* wp, size_t n, uint64_t seed, uint64_t stream, uint64_t p_neg,
                                 uint64_t p_pos) {
    parallel_for(n / 4, [=](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            unsigned byte = 0;
            for (unsigned j = 0; j < 4; ++j) {
                const int8_t v = ternary_of(mix(seed, stream, 4 * i + j), p_neg, p_pos);
                byte |= (v == 1 ? 1u : (v == -1 ? 3u : 0u)) << (2 * j);
            }
            wp[i] = static_cast<uint8_t>(byte);
        }
    });
}

}  // extern "C"
