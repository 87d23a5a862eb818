// Synthetic inputs for benches and tests: random-init weights, caches,
// prompts.  Every element is a pure function of (seed, stream name, index):
//
//   key   = splitmix64(seed ^ fnv1a64(name))
//   u(c)  = splitmix64(key + (c + 1) * 0x9E3779B97F4A7C15)      (counter c)
//   normal pair p from u(2p), u(2p+1): Box-Muller in double,
//     r = sqrt(-2 ln U1), t = 2 pi U2, U = ((u >> 11) + 0.5) * 2^-53,
//     element 2p = r cos t, element 2p+1 = r sin t
//   value = bf16_rne((float)(mean + std * normal))
//
// so a slice can be produced anywhere (host threads here, or a tensor of any
// size) and reproduced exactly.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/ming_hip.h"

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t counter(uint64_t key, uint64_t c) { return mix64(key + (c + 1) * 0x9E3779B97F4A7C15ull); }

inline double unit53(uint64_t u) { return ((double)(u >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

inline uint16_t bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void normal_range(uint64_t key, double mean, double sd, uint16_t* out, size_t i0, size_t i1) {
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = i0;
    while (i < i1) {
        const size_t p = i / 2;
        const double r = std::sqrt(-2.0 * std::log(unit53(counter(key, 2 * p))));
        const double t = two_pi * unit53(counter(key, 2 * p + 1));
        const double z = (i % 2 == 0) ? r * std::cos(t) : r * std::sin(t);
        out[i] = bf16_rne((float)(mean + sd * z));
        i++;
    }
}

}  // namespace

extern "C" {

uint64_t ming_synth_stream(uint64_t seed, const char* name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (const unsigned char* p = reinterpret_cast<const unsigned char*>(name); p && *p; p++) {
        h ^= *p;
        h *= 0x100000001b3ull;
    }
    return mix64(seed ^ h);
}

void ming_synth_normal_bf16(uint64_t stream, float mean, float std, uint16_t* out, size_t n, int threads) {
    if (!out || n == 0) return;
    if (threads < 1) threads = 1;
    if ((size_t)threads > n / 65536 + 1) threads = (int)(n / 65536 + 1);
    if (threads == 1) {
        normal_range(stream, mean, std, out, 0, n);
        return;
    }
    std::vector<std::thread> pool;
    const size_t chunk = ((n + threads - 1) / threads + 1) & ~(size_t)1;
    for (int t = 0; t < threads; t++) {
        const size_t a = t * chunk, b = a + chunk < n ? a + chunk : n;
        if (a >= b) break;
        pool.emplace_back(normal_range, stream, (double)mean, (double)std, out, a, b);
    }
    for (auto& th : pool) th.join();
}

void ming_synth_uniform_i32(uint64_t stream, int32_t hi, int32_t* out, size_t n) {
    if (!out || hi <= 0) return;
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)((counter(stream, i) >> 32) % (uint64_t)hi);
}

}  // extern "C"
