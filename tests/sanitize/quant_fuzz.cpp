// Host-only AddressSanitizer driver for tmh_quantize_weights: exact-size
// heap buffers (so any overrun is reported), every kind, block counts 0..300
// and a few large ones, thread counts 0..17, values with NaN, infinities,
// subnormals and huge magnitudes.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>
#include "tensomite_hip.h"

int main() {
    std::mt19937 rng(7);
    std::uniform_real_distribution<float> u(-4.0f, 4.0f);
    const uint32_t bb[3] = {34, 18, 20};
    long calls = 0;
    std::vector<uint64_t> blocks;
    for (uint64_t b = 0; b <= 300; ++b) blocks.push_back(b);
    for (uint64_t b : {1023ull, 4096ull, 65537ull}) blocks.push_back(b);
    for (uint32_t kind = 0; kind < 3; ++kind) {
        for (uint64_t nb : blocks) {
            const uint64_t count = nb * 32;
            float* v = (float*)malloc(count * sizeof(float) + 1);
            uint8_t* out = (uint8_t*)malloc(nb * bb[kind] + 1);
            for (uint64_t i = 0; i < count; ++i) {
                const unsigned r = rng() % 50;
                v[i] = r == 0 ? NAN : r == 1 ? INFINITY : r == 2 ? -INFINITY : r == 3 ? 1e-42f : r == 4 ? 3e38f : u(rng);
            }
            const int32_t threads = (int32_t)(rng() % 18);
            const int e = tmh_quantize_weights(kind, v, count, out, threads);
            if (e != 0) { printf("kind %u blocks %llu: error %d\n", kind, (unsigned long long)nb, e); return 1; }
            ++calls;
            free(v);
            free(out);
        }
        // not a whole number of blocks: refused, nothing written
        float v[33] = {0};
        uint8_t out[64];
        if (tmh_quantize_weights(kind, v, 33, out, 1) == 0) { printf("33 values accepted\n"); return 1; }
    }
    printf("quantise calls %ld, no sanitizer report\n", calls);
    return 0;
}
