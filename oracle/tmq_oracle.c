/*
 * tmq_oracle.c -- CPU restatement of tensomite's quantised-product path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP library is
 * compared against and the CPU baseline bench.py times beside it. Nothing in
 * the product (tensomite.cr_amd/) links, loads or calls it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function restates one function of the reference (paths relative to
 * the tensomite.cr repository) and cites the lines it follows. Arithmetic is
 * single-rounded IEEE f32 in the reference's expression order; the file must
 * be compiled with -ffp-contract=off and without -ffast-math (oracle/Makefile).
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   tmo_f16_bits / tmo_f16_value   exhaustive over all 65,536 halves, and f32->f16
 *                                  against numpy's IEEE conversion (every exponent)
 *   tmo_quantize / tmo_dequantize  spec/fixtures/quant/expected.json bytes and values,
 *                                  blocks.gguf, tiny_llama model-q8_0/q4_0.gguf
 *   tmo_quantize_activations       equals weight Q8_0 quantisation of the same
 *                                  values (expected.json); Q8_1 sum by closed form
 *   tmo_matmul_reference           float64 bound of block_matmul_spec.cr:11-31,
 *                                  special rows, expression-order cases
 *   tmo_matmul                     equal bits to tmo_matmul_reference on 1, 3, 8
 *                                  threads (quant_spec.cr:30-98)
 *   tmo_gather                     expected.json "table" values
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>
#if defined(__AVX512VNNI__) && defined(__AVX512VL__) && defined(__AVX512BW__)
#include <immintrin.h>
#define TMO_VNNI 1
#endif

/* Block kinds, numbered as the reference's GPU kernels number them
 * (src/tensomite/cuda.cr:774-781). */
enum { TMO_Q8_0 = 0, TMO_Q4_0 = 1, TMO_Q4_1 = 2 };

/* dtype.cr:237-244 */
int tmo_block_bytes(int kind) {
    switch (kind) {
    case TMO_Q8_0: return 34;
    case TMO_Q4_0: return 18;
    case TMO_Q4_1: return 20;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- F16 */

/* F16.new(Float32), f16.cr:29-41: RNE, subnormals as value * 2^24 rounded to
 * even, overflow from 65520 up, NaN -> 0x7e00 with the sign kept. */
uint16_t tmo_f16_bits(float value) {
    uint32_t word;
    memcpy(&word, &value, 4);
    uint16_t sign = (uint16_t)((word >> 16) & 0x8000u);
    uint32_t magnitude = word & 0x7fffffffu;
    if (magnitude >= 0x7f800000u) return sign | (magnitude > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (magnitude >= 0x477ff000u) return sign | 0x7c00u;
    if (magnitude < 0x38800000u) {
        float m;
        memcpy(&m, &magnitude, 4);
        return sign | (uint16_t)rintf(m * 16777216.0f); /* default mode: ties to even */
    }
    return sign | (uint16_t)((magnitude - 0x38000000u + 0xfffu + ((magnitude >> 13) & 1u)) >> 13);
}

/* F16#to_f32, f16.cr:44-57: exact. */
float tmo_f16_value(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
    uint32_t fraction = (uint32_t)bits & 0x3ffu;
    uint32_t word;
    float out;
    if (exponent == 0) {
        float magnitude = (float)fraction * 5.9604645e-8f;
        return sign == 0 ? magnitude : -magnitude;
    }
    if (exponent == 31) word = sign | 0x7f800000u | (fraction << 13);
    else word = sign | ((exponent + 112u) << 23) | (fraction << 13);
    memcpy(&out, &word, 4);
    return out;
}

/* Quant#read_half / #half, quant.cr:493-495, 564-566 */
static float read_half(const uint8_t* at) {
    return tmo_f16_value((uint16_t)(at[0] | (at[1] << 8)));
}

/* Quant#write_half, quant.cr:558-562 */
static void write_half(uint8_t* at, float value) {
    uint16_t bits = tmo_f16_bits(value);
    at[0] = (uint8_t)(bits & 0xff);
    at[1] = (uint8_t)(bits >> 8);
}

/* Crystal's unchecked Float32#to_i32! / #to_i8! (LLVM fptosi, which x86-64
 * carries out as cvttss2si): truncation toward zero, and for NaN or a value
 * outside Int32's range the "integer indefinite" INT32_MIN, whose low byte
 * (what to_i8! keeps) is 0. Written out so that C defines those cases. */
static inline int32_t unchecked_i32(float v) {
    return v >= -2147483648.0f && v < 2147483648.0f ? (int32_t)v : INT32_MIN;
}

/* ------------------------------------------------------ weight quantisers */

/* quantize_q8_0, quant.cr:499-505 */
static void quantize_q8_0(const float* x, uint8_t* target) {
    float amax = fabsf(x[0]);
    for (int j = 1; j < 32; j++)
        if (fabsf(x[j]) > amax) amax = fabsf(x[j]);
    float d = amax / 127.0f;
    float id = d == 0 ? 0.0f : 1.0f / d;
    write_half(target, d);
    for (int j = 0; j < 32; j++) target[2 + j] = (uint8_t)(int8_t)unchecked_i32(roundf(x[j] * id));
}

/* quantize_q4_0, quant.cr:509-520: the first value of largest magnitude,
 * sign kept, maps to -8. */
static void quantize_q4_0(const float* x, uint8_t* target) {
    float max = x[0];
    for (int j = 0; j < 32; j++)
        if (fabsf(x[j]) > fabsf(max)) max = x[j];
    float d = max / -8.0f;
    float id = d == 0 ? 0.0f : 1.0f / d;
    write_half(target, d);
    for (int j = 0; j < 16; j++) {
        float lo_v = x[j] * id;
        lo_v = lo_v + 8.5f;
        float hi_v = x[j + 16] * id;
        hi_v = hi_v + 8.5f;
        int8_t lo = (int8_t)unchecked_i32(lo_v), hi = (int8_t)unchecked_i32(hi_v);
        if (lo > 15) lo = 15;
        if (hi > 15) hi = 15;
        target[2 + j] = (uint8_t)((uint8_t)lo | (uint8_t)((uint8_t)hi << 4));
    }
}

/* quantize_q4_1, quant.cr:524-535: Enumerable#min/#max keep the first of
 * equal values. */
static void quantize_q4_1(const float* x, uint8_t* target) {
    float mn = x[0], mx = x[0];
    for (int j = 1; j < 32; j++) {
        if (x[j] < mn) mn = x[j];
        if (x[j] > mx) mx = x[j];
    }
    float d = (mx - mn) / 15.0f;
    float id = d == 0 ? 0.0f : 1.0f / d;
    write_half(target, d);
    write_half(target + 2, mn);
    for (int j = 0; j < 16; j++) {
        float lo_v = (x[j] - mn) * id;
        lo_v = lo_v + 0.5f;
        float hi_v = (x[j + 16] - mn) * id;
        hi_v = hi_v + 0.5f;
        int8_t lo = (int8_t)unchecked_i32(lo_v), hi = (int8_t)unchecked_i32(hi_v);
        if (lo > 15) lo = 15;
        if (hi > 15) hi = 15;
        target[4 + j] = (uint8_t)((uint8_t)lo | (uint8_t)((uint8_t)hi << 4));
    }
}

/* Quant.quantize, quant.cr:77-90. Returns 0, or -1 for a bad kind or count. */
int tmo_quantize(int kind, const float* values, int64_t count, uint8_t* out) {
    int bb = tmo_block_bytes(kind);
    if (bb < 0 || count % 32 != 0) return -1;
    for (int64_t b = 0; b < count / 32; b++) {
        const float* src = values + b * 32;
        uint8_t* dst = out + b * bb;
        if (kind == TMO_Q8_0) quantize_q8_0(src, dst);
        else if (kind == TMO_Q4_0) quantize_q4_0(src, dst);
        else quantize_q4_1(src, dst);
    }
    return 0;
}

/* dequantize_q8_0/q4_0/q4_1, quant.cr:537-556, driven as Quant.dequantize,
 * quant.cr:93-105. */
int tmo_dequantize(int kind, const uint8_t* bytes, int64_t count, float* values) {
    int bb = tmo_block_bytes(kind);
    if (bb < 0 || count % 32 != 0) return -1;
    for (int64_t b = 0; b < count / 32; b++) {
        const uint8_t* block = bytes + b * bb;
        float* x = values + b * 32;
        if (kind == TMO_Q8_0) {
            float d = read_half(block);
            for (int j = 0; j < 32; j++) x[j] = (float)(int8_t)block[2 + j] * d;
        } else if (kind == TMO_Q4_0) {
            float d = read_half(block);
            for (int j = 0; j < 16; j++) {
                x[j] = (float)((block[2 + j] & 0x0f) - 8) * d;
                x[j + 16] = (float)((block[2 + j] >> 4) - 8) * d;
            }
        } else {
            float d = read_half(block), m = read_half(block + 2);
            for (int j = 0; j < 16; j++) {
                float lo = d * (float)(block[4 + j] & 0x0f);
                float hi = d * (float)(block[4 + j] >> 4);
                x[j] = lo + m;
                x[j + 16] = hi + m;
            }
        }
    }
    return 0;
}

/* Quant.gather, quant.cr:417-422, with HostDevice#block_gather's id check
 * (devices/host.cr:648-658). Returns 0, or the index of the first id out of
 * range plus one. */
int64_t tmo_gather(int kind, const uint8_t* table, int32_t rows, int32_t width, const int32_t* ids,
                   int64_t count, float* dst) {
    int64_t row_bytes = (int64_t)width / 32 * tmo_block_bytes(kind);
    for (int64_t i = 0; i < count; i++) {
        if (ids[i] < 0 || ids[i] >= rows) return i + 1;
        tmo_dequantize(kind, table + ids[i] * row_bytes, width, dst + i * width);
    }
    return 0;
}

/* --------------------------------------------- activations and the oracle */

/* quantize_activations, quant.cr:424-442: per block of 32, d = amax/127,
 * values rounded halves away from zero (Float32#round(:ties_away) is roundf),
 * the scale kept in F16, and with sums, F16(Σq · d) with the unrounded d. */
void tmo_quantize_activations(const float* x, int32_t k, float* scales, float* sums, int8_t* qs, int with_sums) {
    for (int32_t block = 0; block < k / 32; block++) {
        const float* values = x + block * 32;
        float amax = fabsf(values[0]);
        for (int j = 1; j < 32; j++)
            if (fabsf(values[j]) > amax) amax = fabsf(values[j]);
        float d = amax / 127.0f;
        float id = d == 0 ? 0.0f : 1.0f / d;
        int32_t total = 0;
        for (int j = 0; j < 32; j++) {
            int8_t q = (int8_t)unchecked_i32(roundf(values[j] * id));
            qs[block * 32 + j] = q;
            total += q;
        }
        scales[block] = tmo_f16_value(tmo_f16_bits(d));
        if (with_sums) sums[block] = tmo_f16_value(tmo_f16_bits((float)total * d));
    }
}

/* dot_q8_0, quant.cr:446-457 */
static float dot_q8_0(const uint8_t* w, const float* scales, const int8_t* qs, int32_t blocks) {
    float sum = 0.0f;
    for (int32_t block = 0; block < blocks; block++) {
        const uint8_t* base = w + block * 34;
        const int8_t* qb = qs + block * 32;
        int32_t total = 0;
        for (int j = 0; j < 32; j++) total += (int32_t)(int8_t)base[2 + j] * qb[j];
        float scale = read_half(base) * scales[block];
        sum += (float)total * scale;
    }
    return sum;
}

/* dot_q4_0, quant.cr:459-474: ((float(t) * d) * sx) */
static float dot_q4_0(const uint8_t* w, const float* scales, const int8_t* qs, int32_t blocks) {
    float sum = 0.0f;
    for (int32_t block = 0; block < blocks; block++) {
        const uint8_t* base = w + block * 18;
        const int8_t* qb = qs + block * 32;
        int32_t low = 0, high = 0;
        for (int j = 0; j < 16; j++) {
            uint8_t packed = base[2 + j];
            low += ((int32_t)(packed & 0x0f) - 8) * qb[j];
            high += ((int32_t)(packed >> 4) - 8) * qb[j + 16];
        }
        float t = (float)(low + high) * read_half(base);
        t = t * scales[block];
        sum += t;
    }
    return sum;
}

/* dot_q4_1, quant.cr:476-491: (d * sx) * float(t) + m * (d·Σq) */
static float dot_q4_1(const uint8_t* w, const float* scales, const float* sums, const int8_t* qs, int32_t blocks) {
    float sum = 0.0f;
    for (int32_t block = 0; block < blocks; block++) {
        const uint8_t* base = w + block * 20;
        const int8_t* qb = qs + block * 32;
        int32_t low = 0, high = 0;
        for (int j = 0; j < 16; j++) {
            uint8_t packed = base[4 + j];
            low += (int32_t)(packed & 0x0f) * qb[j];
            high += (int32_t)(packed >> 4) * qb[j + 16];
        }
        float scaled = read_half(base) * scales[block];
        float first = scaled * (float)(low + high);
        float second = read_half(base + 2) * sums[block];
        sum += first + second;
    }
    return sum;
}

/* Quant.matmul_reference, quant.cr:122-142: dst[rows, n] = x[rows, k] · wᵀ.
 * Returns 0, or -1 for a bad kind or k. */
int tmo_matmul_reference(int kind, const float* x, const uint8_t* w, int32_t rows, int32_t n, int32_t k, float* dst) {
    int bb = tmo_block_bytes(kind);
    if (bb < 0 || k % 32 != 0) return -1;
    int32_t blocks = k / 32;
    int64_t row_bytes = (int64_t)blocks * bb;
    float* scales = malloc(sizeof(float) * (blocks + 1));
    float* sums = malloc(sizeof(float) * (blocks + 1));
    int8_t* qs = malloc((size_t)k + 1);
    for (int32_t row = 0; row < rows; row++) {
        tmo_quantize_activations(x + (int64_t)row * k, k, scales, sums, qs, kind == TMO_Q4_1);
        for (int32_t col = 0; col < n; col++) {
            const uint8_t* weight = w + col * row_bytes;
            float v;
            if (kind == TMO_Q8_0) v = dot_q8_0(weight, scales, qs, blocks);
            else if (kind == TMO_Q4_0) v = dot_q4_0(weight, scales, qs, blocks);
            else v = dot_q4_1(weight, scales, sums, qs, blocks);
            dst[(int64_t)row * n + col] = v;
        }
    }
    free(scales);
    free(sums);
    free(qs);
    return 0;
}

/* HostDevice#add_bias, devices/host.cr:725-734: a separate rounding. */
void tmo_add_bias(float* dst, const float* bias, int64_t rows, int32_t n) {
    for (int64_t r = 0; r < rows; r++)
        for (int32_t j = 0; j < n; j++) dst[r * n + j] = dst[r * n + j] + bias[j];
}

/* ------------------------------------------------------- the fast CPU path */

/* round_away, quant.cr:309-313 */
static inline int32_t round_away(float value) {
    int32_t whole = unchecked_i32(value);
    float fraction = value - (float)whole;
    return whole + (fraction >= 0.5f ? 1 : 0) - (fraction <= -0.5f ? 1 : 0);
}

/* fast_quantize, quant.cr:318-334 */
static void fast_quantize(const float* x, int32_t blocks, float* scales, float* sums, int32_t* totals, int8_t* qs,
                          int with_sums) {
    for (int32_t block = 0; block < blocks; block++) {
        const float* values = x + block * 32;
        float top = fabsf(values[0]);
        for (int j = 1; j < 32; j++)
            if (fabsf(values[j]) > top) top = fabsf(values[j]);
        float d = top / 127.0f;
        float id = d == 0 ? 0.0f : 1.0f / d;
        int8_t* qb = qs + block * 32;
        for (int j = 0; j < 32; j++) qb[j] = (int8_t)round_away(values[j] * id);
        int32_t total = 0;
        for (int j = 0; j < 32; j++) total += qb[j];
        totals[block] = total;
        scales[block] = tmo_f16_value(tmo_f16_bits(d));
        if (with_sums) sums[block] = tmo_f16_value(tmo_f16_bits((float)total * d));
    }
}

/* HALVES, quant.cr:339-344: every half's value by its bits. */
static float HALVES[65536];
static pthread_once_t halves_once = PTHREAD_ONCE_INIT;
static void build_halves(void) {
    for (int b = 0; b < 65536; b++) HALVES[b] = tmo_f16_value((uint16_t)b);
}
static inline float fast_half(const uint8_t* at) { return HALVES[at[0] | (at[1] << 8)]; }

#ifdef TMO_VNNI
/* The integer block dots of the fast path on AVX-512 VNNI (the vnni build):
 * vpdpbusd multiplies unsigned bytes by signed ones and sums them in 32-bit
 * lanes without saturation, so each dot is the exact integer the scalar
 * loops give (integer sums are exact in any order); the f32 arithmetic
 * around them is unchanged. */
static inline int32_t hsum8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}

/* Σ u·y over a block of 32 (u unsigned bytes, y signed). */
static inline int32_t udot32(__m256i u, __m256i y) {
    return hsum8(_mm256_dpbusd_epi32(_mm256_setzero_si256(), u, y));
}

/* A Q4 block's 16 bytes of nibbles as 32 unsigned bytes in value order:
 * values 0-15 the low nibbles, 16-31 the high ones (quant.cr:62-69). */
static inline __m256i nibbles32(const uint8_t* p) {
    const __m128i b = _mm_loadu_si128((const __m128i*)p);
    const __m128i m = _mm_set1_epi8(0x0f);
    return _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(b, 4), m), _mm_and_si128(b, m));
}

/* Eight blocks' 8-lane partial sums reduced together: lane b of the result
 * is the total of a[b] (three rounds of pairwise horizontal adds, then the
 * two 128-bit halves; integer sums, exact in any order). */
static inline __m256i hsum8x8(const __m256i a[8]) {
    const __m256i s01 = _mm256_hadd_epi32(a[0], a[1]), s23 = _mm256_hadd_epi32(a[2], a[3]);
    const __m256i s45 = _mm256_hadd_epi32(a[4], a[5]), s67 = _mm256_hadd_epi32(a[6], a[7]);
    const __m256i s0123 = _mm256_hadd_epi32(s01, s23), s4567 = _mm256_hadd_epi32(s45, s67);
    return _mm256_add_epi32(_mm256_permute2x128_si256(s0123, s4567, 0x20),
                            _mm256_permute2x128_si256(s0123, s4567, 0x31));
}

/* The halves at byte offset `at` of eight consecutive blocks `stride` bytes
 * apart, as floats (the F16 table, so every half converts as the host's
 * F16#to_f32 does). */
static inline __m256 halves8(const uint8_t* at, int stride) {
    float v[8];
    for (int b = 0; b < 8; b++) v[b] = fast_half(at + b * stride);
    return _mm256_loadu_ps(v);
}

/* Adds eight contributions to a running sum one by one, in block order. */
static inline float fold8(float sum, __m256 c) {
    float v[8];
    _mm256_storeu_ps(v, c);
    for (int b = 0; b < 8; b++) sum += v[b];
    return sum;
}
#endif

/* fast_q8_0, quant.cr:349-366: two weight rows share each activation pass. */
static void fast_q8_0(const uint8_t* w0, const uint8_t* w1, const float* sp, const int8_t* qp, int32_t blocks,
                      float* out0, float* out1) {
    float sum0 = 0.0f, sum1 = 0.0f;
    int32_t block = 0;
#ifdef TMO_VNNI
    /* eight blocks at a time: their totals as one vector, each block's
     * contribution (float(t) · (d · sx), each product rounded) as one
     * vector operation, then the eight added in block order */
    for (; block + 8 <= blocks; block += 8) {
        const __m256i flip = _mm256_set1_epi8((char)0x80), z = _mm256_setzero_si256();
        __m256i a0[8], a1[8], e[8];
        for (int b = 0; b < 8; b++) {
            const __m256i y = _mm256_loadu_si256((const __m256i*)(qp + (block + b) * 32));
            e[b] = _mm256_dpbusd_epi32(z, flip, y);
            a0[b] = _mm256_dpbusd_epi32(
                z, _mm256_xor_si256(_mm256_loadu_si256((const __m256i*)(w0 + (block + b) * 34 + 2)), flip), y);
            a1[b] = _mm256_dpbusd_epi32(
                z, _mm256_xor_si256(_mm256_loadu_si256((const __m256i*)(w1 + (block + b) * 34 + 2)), flip), y);
        }
        const __m256i bias = hsum8x8(e);
        const __m256 t0 = _mm256_cvtepi32_ps(_mm256_sub_epi32(hsum8x8(a0), bias));
        const __m256 t1 = _mm256_cvtepi32_ps(_mm256_sub_epi32(hsum8x8(a1), bias));
        const __m256 sx = _mm256_loadu_ps(sp + block);
        const __m256 s0 = _mm256_mul_ps(halves8(w0 + block * 34, 34), sx);
        const __m256 s1 = _mm256_mul_ps(halves8(w1 + block * 34, 34), sx);
        sum0 = fold8(sum0, _mm256_mul_ps(t0, s0));
        sum1 = fold8(sum1, _mm256_mul_ps(t1, s1));
    }
#endif
    for (; block < blocks; block++) {
        const uint8_t* base0 = w0 + block * 34;
        const uint8_t* base1 = w1 + block * 34;
        const int8_t* qb = qp + block * 32;
        int32_t total0 = 0, total1 = 0;
#ifdef TMO_VNNI
        {
            /* Σ v·y = Σ (v + 128)·y − 128·Σy, v + 128 as an unsigned byte */
            const __m256i y = _mm256_loadu_si256((const __m256i*)qb);
            const __m256i flip = _mm256_set1_epi8((char)0x80);
            const int32_t bias = udot32(flip, y);
            total0 = udot32(_mm256_xor_si256(_mm256_loadu_si256((const __m256i*)(base0 + 2)), flip), y) - bias;
            total1 = udot32(_mm256_xor_si256(_mm256_loadu_si256((const __m256i*)(base1 + 2)), flip), y) - bias;
        }
#else
        const int8_t* v0 = (const int8_t*)(base0 + 2);
        const int8_t* v1 = (const int8_t*)(base1 + 2);
        for (int j = 0; j < 32; j++) {
            int32_t y = qb[j];
            total0 += v0[j] * y;
            total1 += v1[j] * y;
        }
#endif
        float s0 = fast_half(base0) * sp[block];
        float s1 = fast_half(base1) * sp[block];
        sum0 += (float)total0 * s0;
        sum1 += (float)total1 * s1;
    }
    *out0 = sum0;
    *out1 = sum1;
}

/* nibble_dot, quant.cr:373-386: nibbles less 8 as signed bytes. */
static inline void nibble_dot(const uint8_t* p0, const uint8_t* p1, const int8_t* qb, int32_t* t0, int32_t* t1) {
#ifdef TMO_VNNI
    /* Σ (q − 8)·y = Σ q·y − 8·Σy */
    const __m256i y = _mm256_loadu_si256((const __m256i*)qb);
    const int32_t eight = udot32(_mm256_set1_epi8(8), y);
    *t0 = udot32(nibbles32(p0), y) - eight;
    *t1 = udot32(nibbles32(p1), y) - eight;
    return;
#endif
    int32_t total0 = 0, total1 = 0;
    for (int j = 0; j < 16; j++) {
        int32_t y = qb[j];
        total0 += (int32_t)(int8_t)((p0[j] & 0x0f) - 8) * y;
        total1 += (int32_t)(int8_t)((p1[j] & 0x0f) - 8) * y;
    }
    for (int j = 0; j < 16; j++) {
        int32_t y = qb[j + 16];
        total0 += (int32_t)(int8_t)((p0[j] >> 4) - 8) * y;
        total1 += (int32_t)(int8_t)((p1[j] >> 4) - 8) * y;
    }
    *t0 = total0;
    *t1 = total1;
}

/* fast_q4_0, quant.cr:388-399 */
static void fast_q4_0(const uint8_t* w0, const uint8_t* w1, const float* sp, const int8_t* qp, int32_t blocks,
                      float* out0, float* out1) {
    float sum0 = 0.0f, sum1 = 0.0f;
    int32_t block = 0;
#ifdef TMO_VNNI
    /* eight blocks at a time (as fast_q8_0): (float(t) · d) · sx */
    for (; block + 8 <= blocks; block += 8) {
        const __m256i eight = _mm256_set1_epi8(8), z = _mm256_setzero_si256();
        __m256i a0[8], a1[8], e[8];
        for (int b = 0; b < 8; b++) {
            const __m256i y = _mm256_loadu_si256((const __m256i*)(qp + (block + b) * 32));
            e[b] = _mm256_dpbusd_epi32(z, eight, y);
            a0[b] = _mm256_dpbusd_epi32(z, nibbles32(w0 + (block + b) * 18 + 2), y);
            a1[b] = _mm256_dpbusd_epi32(z, nibbles32(w1 + (block + b) * 18 + 2), y);
        }
        const __m256i e8 = hsum8x8(e);
        const __m256 t0 = _mm256_cvtepi32_ps(_mm256_sub_epi32(hsum8x8(a0), e8));
        const __m256 t1 = _mm256_cvtepi32_ps(_mm256_sub_epi32(hsum8x8(a1), e8));
        const __m256 sx = _mm256_loadu_ps(sp + block);
        sum0 = fold8(sum0, _mm256_mul_ps(_mm256_mul_ps(t0, halves8(w0 + block * 18, 18)), sx));
        sum1 = fold8(sum1, _mm256_mul_ps(_mm256_mul_ps(t1, halves8(w1 + block * 18, 18)), sx));
    }
#endif
    for (; block < blocks; block++) {
        const uint8_t* base0 = w0 + block * 18;
        const uint8_t* base1 = w1 + block * 18;
        int32_t total0, total1;
        nibble_dot(base0 + 2, base1 + 2, qp + block * 32, &total0, &total1);
        float a = (float)total0 * fast_half(base0);
        float b = (float)total1 * fast_half(base1);
        sum0 += a * sp[block];
        sum1 += b * sp[block];
    }
    *out0 = sum0;
    *out1 = sum1;
}

/* fast_q4_1, quant.cr:401-413: Σq·y = Σ(q-8)·y + 8·Σy. */
static void fast_q4_1(const uint8_t* w0, const uint8_t* w1, const float* sp, const float* mp, const int32_t* tp,
                      const int8_t* qp, int32_t blocks, float* out0, float* out1) {
    float sum0 = 0.0f, sum1 = 0.0f;
    int32_t block = 0;
#ifdef TMO_VNNI
    /* eight blocks at a time (as fast_q8_0): (d · sx) · float(dot + 8·Σq)
     * + m · mx */
    for (; block + 8 <= blocks; block += 8) {
        const __m256i eight = _mm256_set1_epi8(8), z = _mm256_setzero_si256();
        __m256i a0[8], a1[8], e[8];
        for (int b = 0; b < 8; b++) {
            const __m256i y = _mm256_loadu_si256((const __m256i*)(qp + (block + b) * 32));
            e[b] = _mm256_dpbusd_epi32(z, eight, y);
            a0[b] = _mm256_dpbusd_epi32(z, nibbles32(w0 + (block + b) * 20 + 4), y);
            a1[b] = _mm256_dpbusd_epi32(z, nibbles32(w1 + (block + b) * 20 + 4), y);
        }
        const __m256i e8 = hsum8x8(e);
        const __m256i shift = _mm256_slli_epi32(_mm256_loadu_si256((const __m256i*)(tp + block)), 3);
        const __m256 t0 = _mm256_cvtepi32_ps(_mm256_add_epi32(_mm256_sub_epi32(hsum8x8(a0), e8), shift));
        const __m256 t1 = _mm256_cvtepi32_ps(_mm256_add_epi32(_mm256_sub_epi32(hsum8x8(a1), e8), shift));
        const __m256 sx = _mm256_loadu_ps(sp + block), mx = _mm256_loadu_ps(mp + block);
        const __m256 c0 = _mm256_add_ps(_mm256_mul_ps(_mm256_mul_ps(halves8(w0 + block * 20, 20), sx), t0),
                                        _mm256_mul_ps(halves8(w0 + block * 20 + 2, 20), mx));
        const __m256 c1 = _mm256_add_ps(_mm256_mul_ps(_mm256_mul_ps(halves8(w1 + block * 20, 20), sx), t1),
                                        _mm256_mul_ps(halves8(w1 + block * 20 + 2, 20), mx));
        sum0 = fold8(sum0, c0);
        sum1 = fold8(sum1, c1);
    }
#endif
    for (; block < blocks; block++) {
        const uint8_t* base0 = w0 + block * 20;
        const uint8_t* base1 = w1 + block * 20;
        int32_t dot0, dot1;
        nibble_dot(base0 + 4, base1 + 4, qp + block * 32, &dot0, &dot1);
        int32_t shift = 8 * tp[block];
        float a0 = (fast_half(base0) * sp[block]) * (float)(dot0 + shift);
        float b0 = fast_half(base0 + 2) * mp[block];
        float a1 = (fast_half(base1) * sp[block]) * (float)(dot1 + shift);
        float b1 = fast_half(base1 + 2) * mp[block];
        sum0 += a0 + b0;
        sum1 += a1 + b1;
    }
    *out0 = sum0;
    *out1 = sum1;
}

/* ---- threads: Quant.threads, in_parallel and SpinPool, quant.cr:184-302 ---- */

typedef struct {
    int kind;
    const uint8_t* w;
    int64_t row_bytes;
    int32_t blocks;
    const float* scales;
    const float* sums;
    const int32_t* totals;
    const int8_t* qs;
    float* out;
    /* set for tmo_parallel_for's jobs instead of a product */
    void (*fn)(void* ctx, int32_t first, int32_t stop);
    void* ctx;
} tmo_job;

/* One span of a product: columns first...stop in pairs, quant.cr:167-180. */
static void run_span(const tmo_job* job, int32_t first, int32_t stop) {
    if (job->fn) {
        job->fn(job->ctx, first, stop);
        return;
    }
    for (int32_t col = first; col < stop; col += 2) {
        const uint8_t* w0 = job->w + col * job->row_bytes;
        const uint8_t* w1 = col + 1 < stop ? w0 + job->row_bytes : w0;
        float a, b;
        if (job->kind == TMO_Q8_0) fast_q8_0(w0, w1, job->scales, job->qs, job->blocks, &a, &b);
        else if (job->kind == TMO_Q4_0) fast_q4_0(w0, w1, job->scales, job->qs, job->blocks, &a, &b);
        else fast_q4_1(w0, w1, job->scales, job->sums, job->totals, job->qs, job->blocks, &a, &b);
        job->out[col] = a;
        if (col + 1 < stop) job->out[col + 1] = b;
    }
}

/* The spinning pool: one claim word holding the generation (high 32 bits),
 * the span count (next 16) and the next unclaimed span (low 16), claimed by
 * compare-and-set, as SpinPool does (quant.cr:219-302). */
typedef struct {
    _Atomic uint64_t claim;
    _Atomic int32_t done;
    _Atomic int32_t stop;
    int32_t count;
    const tmo_job* _Atomic job;
    int workers;
    pthread_t* threads;
} spin_pool;

static spin_pool* pool = NULL;
static int pool_threads = 0; /* Quant.threads */
static pthread_mutex_t pool_lock = PTHREAD_MUTEX_INITIALIZER;

static inline void cpu_pause(void) {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
}

static void pool_help(spin_pool* p, uint64_t generation) {
    for (;;) {
        uint64_t claim = atomic_load(&p->claim);
        if ((claim >> 32) != generation) return;
        int32_t spans = (int32_t)((claim >> 16) & 0xffff);
        int32_t span = (int32_t)(claim & 0xffff);
        if (span >= spans) return;
        if (!atomic_compare_exchange_strong(&p->claim, &claim, claim + 1)) continue;
        int32_t count = p->count;
        const tmo_job* job = atomic_load(&p->job);
        run_span(job, (int32_t)((int64_t)count * span / spans), (int32_t)((int64_t)count * (span + 1) / spans));
        atomic_fetch_add(&p->done, 1);
    }
}

static void* pool_work(void* arg) {
    spin_pool* p = arg;
    uint64_t seen = 0;
    for (;;) {
        long idle = 0;
        long nap_us = 100;
        uint64_t current;
        while ((current = atomic_load(&p->claim) >> 32) == seen) {
            if (atomic_load(&p->stop)) return NULL;
            if (idle < 1000000) {
                idle++;
                cpu_pause();
            } else {
                struct timespec ts = {0, nap_us * 1000};
                nanosleep(&ts, NULL);
                nap_us = nap_us * 2 < 10000 ? nap_us * 2 : 10000;
            }
        }
        seen = current;
        pool_help(p, current);
    }
}

static spin_pool* pool_new(int workers) {
    spin_pool* p = calloc(1, sizeof(spin_pool));
    p->workers = workers;
    p->threads = calloc((size_t)workers, sizeof(pthread_t));
    for (int i = 0; i < workers; i++) pthread_create(&p->threads[i], NULL, pool_work, p);
    return p;
}

static void pool_run(spin_pool* p, int32_t spans, int32_t count, const tmo_job* job) {
    p->count = count;
    atomic_store(&p->job, job);
    atomic_store(&p->done, 0);
    uint64_t generation = ((atomic_load(&p->claim) >> 32) + 1) & 0xffffffffu;
    atomic_store(&p->claim, generation << 32 | (uint64_t)spans << 16);
    pool_help(p, generation);
    while (atomic_load(&p->done) != spans) cpu_pause();
}

/* Quant.threads=, quant.cr:188 (clamped to 1...1024). The pool keeps the size
 * it was made with, as the reference's does. */
void tmo_set_threads(int threads) {
    pool_threads = threads < 1 ? 1 : threads > 1024 ? 1024 : threads;
}

int tmo_threads(void) {
    if (pool_threads == 0) {
        long cpus = sysconf(_SC_NPROCESSORS_ONLN);
        tmo_set_threads(cpus > 0 ? (int)cpus : 1);
    }
    return pool_threads;
}

/* Quant.in_parallel, quant.cr:204-211: spans = min(threads·4, min(count,
 * bytes / 64 KiB)). */
static void in_parallel(int32_t count, int64_t bytes, const tmo_job* job) {
    int threads = tmo_threads();
    int64_t by_bytes = bytes / (64 * 1024);
    int64_t spans = (int64_t)threads * 4;
    if (by_bytes < spans) spans = by_bytes;
    if (count < spans) spans = count;
    if (spans > 65535) spans = 65535;
    if (spans <= 1 || threads <= 1) {
        run_span(job, 0, count);
        return;
    }
    pthread_mutex_lock(&pool_lock);
    if (pool == NULL) pool = pool_new(threads - 1);
    pool_run(pool, (int32_t)spans, count, job);
    pthread_mutex_unlock(&pool_lock);
}

/* fn(ctx, first, stop) over spans of items 0 .. count - 1 on the spinning
 * pool (at most tmo_threads()·4 spans): for host ops whose items are
 * independent, each computed by one thread in its own order. */
void tmo_parallel_for(int32_t count, void (*fn)(void*, int32_t, int32_t), void* ctx) {
    int threads = tmo_threads();
    int64_t spans = (int64_t)threads * 4;
    if (count < spans) spans = count;
    if (spans > 65535) spans = 65535;
    if (spans <= 1 || threads <= 1) {
        if (count > 0) fn(ctx, 0, count);
        return;
    }
    tmo_job job;
    memset(&job, 0, sizeof job);
    job.fn = fn;
    job.ctx = ctx;
    pthread_mutex_lock(&pool_lock);
    if (pool == NULL) pool = pool_new(threads - 1);
    pool_run(pool, (int32_t)spans, count, &job);
    pthread_mutex_unlock(&pool_lock);
}

/* Quant.matmul, quant.cr:155-182: the oracle's bits, faster, on
 * tmo_threads() threads. */
int tmo_matmul(int kind, const float* x, const uint8_t* w, int32_t rows, int32_t n, int32_t k, float* dst) {
    int bb = tmo_block_bytes(kind);
    if (bb < 0 || k % 32 != 0) return -1;
    pthread_once(&halves_once, build_halves);
    int32_t blocks = k / 32;
    int64_t row_bytes = (int64_t)blocks * bb;
    float* scales = malloc(sizeof(float) * (blocks + 1));
    float* sums = malloc(sizeof(float) * (blocks + 1));
    int32_t* totals = malloc(sizeof(int32_t) * (blocks + 1));
    int8_t* qs = malloc((size_t)k + 1);
    for (int32_t row = 0; row < rows; row++) {
        fast_quantize(x + (int64_t)row * k, blocks, scales, sums, totals, qs, kind == TMO_Q4_1);
        tmo_job job = {kind, w, row_bytes, blocks, scales, sums, totals, qs, dst + (int64_t)row * n};
        in_parallel(n, (int64_t)n * row_bytes, &job);
    }
    free(scales);
    free(sums);
    free(totals);
    free(qs);
    return 0;
}

/* tmo_f16_bits over an array of f32 bit patterns, for the exhaustive tests. */
int64_t tmo_f16_bits_many(const uint32_t* words, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; i++) {
        float f;
        memcpy(&f, &words[i], 4);
        out[i] = tmo_f16_bits(f);
    }
    return count;
}

/* tmo_f16_value over an array of halves (no float passes through a double). */
int64_t tmo_f16_values_many(const uint16_t* bits, int64_t count, float* out) {
    for (int64_t i = 0; i < count; i++) out[i] = tmo_f16_value(bits[i]);
    return count;
}
