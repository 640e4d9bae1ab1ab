// Host-side weight quantisation: Quant.quantize (src/tensomite/quant.cr:77-90,
// 497-535), the step `Tensor#quantize` runs on the host whatever the device
// (src/tensomite/tensor/quantised.cr:11-19), over all host cores.
//
// Every block is independent, so blocks are split into contiguous ranges,
// one per thread; the bytes do not depend on the split. Each value goes
// through the reference's f32 operations in its order (the library is built
// with -ffp-contract=off: no fused multiply-add), and scales are rounded to
// F16 in integer arithmetic as F16.new does (f16.cr:29-41). Inputs are
// finite f32 values.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/tensomite_hip.h"
#include "tmh_internal.h"

namespace {

// F16.new(v).bits: round to nearest even; NaN -> 0x7e00 with its sign;
// 65520 and up overflow to infinity; subnormal halves from v · 2^24.
uint16_t half_bits(float v) {
    uint32_t word;
    std::memcpy(&word, &v, 4);
    const uint32_t sign = (word >> 16) & 0x8000u;
    const uint32_t mag = word & 0x7fffffffu;
    if (mag >= 0x7f800000u) return (uint16_t)(sign | (mag > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (mag >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (mag < 0x38800000u) {
        float m;
        std::memcpy(&m, &mag, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(m * 16777216.0f));
    }
    // Rebias the exponent, then round the 13 dropped bits to even.
    return (uint16_t)(sign | ((mag - 0x38000000u + 0xfffu + ((mag >> 13) & 1u)) >> 13));
}

void put_half(uint8_t* at, float v) {
    const uint16_t h = half_bits(v);
    at[0] = (uint8_t)(h & 0xffu);
    at[1] = (uint8_t)(h >> 8);
}

// The reference converts with Crystal's unchecked Float32#to_i8! (LLVM
// fptosi, which x86-64 carries out as cvttss2si): truncation toward zero,
// and for NaN or a value outside Int32's range the "integer indefinite"
// INT32_MIN, whose low byte -- what to_i8! keeps -- is 0. Written out, so
// that the C++ conversion is defined for those inputs too.
inline int32_t unchecked_i32(float v) {
    return v >= -2147483648.0f && v < 2147483648.0f ? (int32_t)v : INT32_MIN;
}

// A nibble: trunc(t) (t in [0, 16.5] for finite inputs), at most 15.
inline uint8_t nibble(float t) {
    const int32_t q = unchecked_i32(t);
    return (uint8_t)(q > 15 ? 15 : q);
}

// round(:ties_away) of a value within int8's range, as an int8 byte.
inline uint8_t round_away_byte(float v) { return (uint8_t)(int8_t)unchecked_i32(std::round(v)); }

void block_q8_0(const float* x, uint8_t* out) {
    // x.max_of(&.abs): the first value's magnitude, replaced by any larger
    // one (a NaN first stays; a NaN later is never larger)
    float amax = std::fabs(x[0]);
    for (int j = 1; j < 32; ++j)
        if (std::fabs(x[j]) > amax) amax = std::fabs(x[j]);
    const float d = amax / 127.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    put_half(out, d);
    for (int j = 0; j < 32; ++j) out[2 + j] = round_away_byte(x[j] * id);
}

void block_q4_0(const float* x, uint8_t* out) {
    // The first value of the largest magnitude, its sign kept, maps to -8.
    float top = x[0];
    for (int j = 1; j < 32; ++j)
        if (std::fabs(x[j]) > std::fabs(top)) top = x[j];
    const float d = top / -8.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    put_half(out, d);
    for (int j = 0; j < 16; ++j) {
        const float lo = x[j] * id + 8.5f;       // two roundings: no contraction
        const float hi = x[j + 16] * id + 8.5f;
        out[2 + j] = (uint8_t)(nibble(lo) | (nibble(hi) << 4));
    }
}

void block_q4_1(const float* x, uint8_t* out) {
    // Enumerable#min/#max: the first of equal values is kept (a signed zero).
    float lo_v = x[0], hi_v = x[0];
    for (int j = 1; j < 32; ++j) {
        if (x[j] < lo_v) lo_v = x[j];
        if (x[j] > hi_v) hi_v = x[j];
    }
    const float d = (hi_v - lo_v) / 15.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    put_half(out, d);
    put_half(out + 2, lo_v);
    for (int j = 0; j < 16; ++j) {
        const float lo = (x[j] - lo_v) * id + 0.5f;
        const float hi = (x[j + 16] - lo_v) * id + 0.5f;
        out[4 + j] = (uint8_t)(nibble(lo) | (nibble(hi) << 4));
    }
}

template <void (*BLOCK)(const float*, uint8_t*)>
void quantize_range(const float* x, uint8_t* out, size_t bb, uint64_t first, uint64_t last) {
    for (uint64_t b = first; b < last; ++b) BLOCK(x + 32 * b, out + bb * b);
}

}  // namespace

extern "C" int tmh_quantize_weights(uint32_t kind, const float* values, uint64_t count, uint8_t* out,
                                    int32_t threads) {
    if (kind > 2u) return TMH_ERROR_DTYPE;
    if (count % 32u != 0) return TMH_ERROR_SHAPE;
    if (count == 0) return TMH_SUCCESS;
    if (!values || !out) return TMH_ERROR_INVALID_VALUE;
    const uint64_t blocks = count / 32u;
    const size_t bb = tmh::block_bytes(kind);
    auto run = [&](uint64_t first, uint64_t last) {
        switch (kind) {
        case 0: quantize_range<block_q8_0>(values, out, bb, first, last); break;
        case 1: quantize_range<block_q4_0>(values, out, bb, first, last); break;
        default: quantize_range<block_q4_1>(values, out, bb, first, last); break;
        }
    };
    // At least 16K blocks (512K values) a thread: below that a thread's start
    // costs more than it saves.
    uint64_t t = threads > 0 ? (uint64_t)threads : std::max(1u, std::thread::hardware_concurrency());
    t = std::max<uint64_t>(1, std::min<uint64_t>(t, blocks / 16384u));
    if (t == 1) {
        run(0, blocks);
        return TMH_SUCCESS;
    }
    std::vector<std::thread> pool;
    pool.reserve(t - 1);
    for (uint64_t i = 1; i < t; ++i) pool.emplace_back(run, blocks * i / t, blocks * (i + 1) / t);
    run(0, blocks / t);
    for (std::thread& th : pool) th.join();
    return TMH_SUCCESS;
}
