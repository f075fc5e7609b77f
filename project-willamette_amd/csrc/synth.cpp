// Synthetic BitNet-shaped inputs (the role of src/synth.rs in the reference:
// seeded random ternary weights packed in the I2_S byte layout of
// src/synth.rs:239-265).  Host code only.
//
// Streams are counter-based SplitMix64: value i of stream (seed, tag) is
// mix(state0 + (i + 1) * golden) with state0 = wm_synth_stream_seed(seed,
// tag), i.e. the (i+1)-th output of a SplitMix64 generator started at
// state0.  Any element can be produced independently, so tensors are filled
// by several threads with results that do not depend on the thread count.
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "willamette_hip.h"

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t draw(uint64_t state0, uint64_t i) { return mix64(state0 + (i + 1) * kGolden); }

template <class F>
void parallel_for(size_t n, size_t min_per_thread, F f) {
    unsigned hw = std::thread::hardware_concurrency();
    size_t threads = hw ? hw : 1;
    if (threads > 16) threads = 16;
    if (n / min_per_thread < threads) threads = n / min_per_thread ? n / min_per_thread : 1;
    if (threads <= 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> pool;
    for (size_t t = 0; t < threads; t++)
        pool.emplace_back(f, n * t / threads, n * (t + 1) / threads);
    for (auto &th : pool) th.join();
}

// N(0,1) from draws 2i and 2i+1 (Box-Muller, double precision).
inline double std_normal(uint64_t state0, uint64_t i) {
    double u1 = (double)((draw(state0, 2 * i) >> 11) + 1) * 0x1p-53;  // (0, 1]
    double u2 = (double)(draw(state0, 2 * i + 1) >> 11) * 0x1p-53;    // [0, 1)
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

inline uint16_t f32_to_f16_rne(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

}  // namespace

extern "C" {

uint64_t wm_synth_stream_seed(uint64_t seed, uint64_t tag) {
    return mix64(seed ^ mix64(tag + 0x632BE59BD9B4E019ull));
}

void wm_synth_i2s(uint64_t seed, uint64_t tag, uint8_t *packed, size_t n_bytes) {
    const uint64_t s0 = wm_synth_stream_seed(seed, tag);
    parallel_for(n_bytes, 1 << 16, [&](size_t b, size_t e) {
        for (size_t j = b; j < e; j++) {
            uint32_t c0 = draw(s0, 4 * j) % 3, c1 = draw(s0, 4 * j + 1) % 3;
            uint32_t c2 = draw(s0, 4 * j + 2) % 3, c3 = draw(s0, 4 * j + 3) % 3;
            packed[j] = (uint8_t)((c0 << 6) | (c1 << 4) | (c2 << 2) | c3);
        }
    });
}

void wm_synth_normal(uint64_t seed, uint64_t tag, float *out, size_t n, double sigma) {
    const uint64_t s0 = wm_synth_stream_seed(seed, tag);
    parallel_for(n, 1 << 14, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; i++) out[i] = (float)(sigma * std_normal(s0, i));
    });
}

void wm_synth_uniform(uint64_t seed, uint64_t tag, float *out, size_t n, double lo, double hi) {
    const uint64_t s0 = wm_synth_stream_seed(seed, tag);
    parallel_for(n, 1 << 14, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; i++)
            out[i] = (float)(lo + (hi - lo) * ((double)(draw(s0, i) >> 40) * 0x1p-24));
    });
}

void wm_synth_q6k(uint64_t seed, uint64_t tag, uint8_t *blocks, size_t n_blocks, double d_sigma) {
    const uint64_t s0 = wm_synth_stream_seed(seed, tag);
    parallel_for(n_blocks, 1 << 10, [&](size_t b, size_t e) {
        for (size_t blk = b; blk < e; blk++) {
            uint8_t *p = blocks + blk * 210;
            const uint64_t base = blk * 256;
            for (int t = 0; t < 192; t++) p[t] = (uint8_t)(draw(s0, base + t) >> 56);
            for (int t = 0; t < 16; t++) p[192 + t] = (uint8_t)(int8_t)((int)(draw(s0, base + 192 + t) % 64) - 32);
            // |N(0, d_sigma)| from draws 208/209 of this block's range
            double u1 = (double)((draw(s0, base + 208) >> 11) + 1) * 0x1p-53;
            double u2 = (double)(draw(s0, base + 209) >> 11) * 0x1p-53;
            double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
            uint16_t d = f32_to_f16_rne((float)std::fabs(d_sigma * z));
            p[208] = (uint8_t)(d & 0xFF);
            p[209] = (uint8_t)(d >> 8);
        }
    });
}

}  // extern "C"
