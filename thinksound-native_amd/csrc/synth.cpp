// synth.cpp — the specified synthetic-data generator (weights and inputs of the workloads).
//
// Counter-based, so any element can be drawn independently and in parallel, bit-for-bit the same
// on every host:
//   mix64(z)         = SplitMix64 output function of z + 0x9E3779B97F4A7C15
//   key(seed, idx)   = mix64(mix64(seed) ^ (idx * 0xD1B54A32D192ED03))
//   uniform(key, i)  = ((mix64(key ^ mix64(i)) >> 11) + 0.5) * 2^-53            in (0, 1)
//   normal(key, i)   = Box-Muller on the pair p = i >> 1: u1 = uniform(key, 2p), u2 = uniform(key, 2p+1),
//                      r = sqrt(-2 ln u1), a = 2*pi*u2; even i -> r*cos(a), odd i -> r*sin(a)   (double)
//   value            = (float)(mean + std * normal), weights then rounded to bf16 (nearest-even)
// Tensor idx is the manifest index for weights; inputs use their own index space.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace tsn {

static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t synth_key(uint64_t seed, uint64_t idx) { return mix64(mix64(seed) ^ (idx * 0xD1B54A32D192ED03ull)); }
static inline double uniform01(uint64_t key, uint64_t i) {
    return ((double)(mix64(key ^ mix64(i)) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
static inline double normal01(uint64_t key, uint64_t i) {
    const uint64_t p = i >> 1;
    const double u1 = uniform01(key, 2 * p), u2 = uniform01(key, 2 * p + 1);
    const double r = sqrt(-2.0 * log(u1)), a = 6.283185307179586476925286766559 * u2;
    return (i & 1) ? r * sin(a) : r * cos(a);
}
uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <typename F>
static void parallel_for(size_t n, F &&fn) {
    const size_t nt = std::max<size_t>(1, std::min<size_t>(std::thread::hardware_concurrency(), 16));
    if (n < 65536 || nt == 1) { fn(0, n); return; }
    std::vector<std::thread> th;
    const size_t chunk = (n + nt - 1) / nt;
    for (size_t t = 0; t < nt; ++t) {
        const size_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        th.emplace_back([&fn, a, b] { fn(a, b); });
    }
    for (auto &x : th) x.join();
}

void synth_normal_f32(uint64_t seed, uint64_t idx, double mean, double std, size_t n, float *out) {
    const uint64_t key = synth_key(seed, idx);
    parallel_for(n, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i) out[i] = (float)(mean + std * normal01(key, i));
    });
}
void synth_normal_bf16(uint64_t seed, uint64_t idx, double mean, double std, size_t n, uint16_t *out) {
    const uint64_t key = synth_key(seed, idx);
    parallel_for(n, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i) out[i] = f32_to_bf16((float)(mean + std * normal01(key, i)));
    });
}
void synth_uniform_f32(uint64_t seed, uint64_t idx, double lo, double hi, size_t n, float *out) {
    const uint64_t key = synth_key(seed, idx);
    for (size_t i = 0; i < n; ++i) out[i] = (float)(lo + (hi - lo) * uniform01(key, i));
}

} // namespace tsn
