// Device helpers shared by the kernel sources of libtensomite_hip.so: F16
// conversions and the activation quantiser's arithmetic for one lane of an
// 8-lane block group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmh_internal.h"

namespace tmh {

// ------------------------------------------------------------------ halves

// Returns the half with bits `bits` (low 16 bits) as a float: exact for every
// half that is not a NaN (F16#to_f32, f16.cr:44-57).
__device__ __forceinline__ float half_value(uint32_t bits) {
    union {
        uint16_t u;
        _Float16 h;
    } v;
    v.u = (uint16_t)bits;
    return (float)v.h;
}

// Returns x rounded to the nearest half, ties to even, as a float: F16.new
// (f16.cr:29-41) -- NaN becomes 0x7e00, values from 65520 up overflow,
// subnormals are x * 2^24 rounded to even.
__device__ __forceinline__ uint32_t round_to_half_bits(float x) {
    uint32_t word = __float_as_uint(x);
    uint32_t sign = (word >> 16) & 0x8000u;
    uint32_t magnitude = word & 0x7fffffffu;
    uint32_t h;
    if (magnitude >= 0x7f800000u) h = sign | (magnitude > 0x7f800000u ? 0x7e00u : 0x7c00u);
    else if (magnitude >= 0x477ff000u) h = sign | 0x7c00u;
    else if (magnitude < 0x38800000u) h = sign | (uint32_t)__builtin_rintf(__uint_as_float(magnitude) * 16777216.0f);
    else h = sign | ((magnitude - 0x38000000u + 0xfffu + ((magnitude >> 13) & 1u)) >> 13);
    return h;
}

__device__ __forceinline__ float round_to_half(float x) { return half_value(round_to_half_bits(x)); }

// ------------------------------------------------------ activation quantise

// A value of another lane of this lane's 8-lane group, by DPP (no LDS
// round trip): XOR1 and XOR2 swap within quads, MIRROR takes lane 7 - i of
// the half row. Every lane of the group must be active.
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_MIRROR = 0x141 };

template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_float(float v) {
    return __int_as_float(dpp_int<CTRL>(__float_as_int(v)));
}

// The quantised form of 4 of a block's 32 activations, held by one lane of
// an 8-lane group (all 8 lanes active): the group's amax and Σq reduced over
// the 8 lanes, then quantize_activations' arithmetic (quant.cr:428-442).
struct Q8Quad {
    uint32_t packed;  // the 4 int8 values
    float scale;      // F16(d)
    float sum;        // F16(float(Σq) · d)
    int total;        // Σq over the block
};

__device__ __forceinline__ Q8Quad quantize_quad(float v0, float v1, float v2, float v3) {
    // The host's amax starts at the block's first value and skips every
    // later NaN (a comparison with NaN is false), so a lane other than the
    // block's first (the 8 lanes of a block are threadIdx.x / 8's group, the
    // quarter threadIdx.x % 8) skips a NaN in its own first value as well.
    float amax = fabsf(v0);
    if ((threadIdx.x & 7u) != 0 && amax != amax) amax = 0.0f;
    amax = fabsf(v1) > amax ? fabsf(v1) : amax;
    amax = fabsf(v2) > amax ? fabsf(v2) : amax;
    amax = fabsf(v3) > amax ? fabsf(v3) : amax;
    // The group's largest magnitude (max is exact in any order): the quad's
    // by two swaps, then the other quad's by the mirror.
    float other = dpp_float<DPP_XOR1>(amax);
    amax = other > amax ? other : amax;
    other = dpp_float<DPP_XOR2>(amax);
    amax = other > amax ? other : amax;
    other = dpp_float<DPP_MIRROR>(amax);
    amax = other > amax ? other : amax;
    const float d = amax / 127.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    const int q0 = (int8_t)(int)roundf(v0 * id);
    const int q1 = (int8_t)(int)roundf(v1 * id);
    const int q2 = (int8_t)(int)roundf(v2 * id);
    const int q3 = (int8_t)(int)roundf(v3 * id);
    Q8Quad out;
    out.packed = (uint32_t)(q0 & 0xff) | (uint32_t)(q1 & 0xff) << 8 | (uint32_t)(q2 & 0xff) << 16 |
                 (uint32_t)(q3 & 0xff) << 24;
    int total = q0 + q1 + q2 + q3;
    total += dpp_int<DPP_XOR1>(total);
    total += dpp_int<DPP_XOR2>(total);
    total += dpp_int<DPP_MIRROR>(total);
    out.total = total;
    out.scale = round_to_half(d);
    out.sum = round_to_half((float)total * d);
    return out;
}

// ---------------------------------------------------------- UNORDERED fold

// The fold of BlockMatMulMode::Unordered (quant.cr:14-17, a measurement
// mode): a row's contributions as four interleaved running sums, s[i % 4]
// += c[i], then (s0 + s1) + (s2 + s3) -- four independent chains of adds
// where the host's block order is one, so the last bits may differ. Each
// kernel's fold reads its contributions exactly as for the ordered fold and
// only adds them this way, so the mode prices the order alone.
struct Fold4 {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    __device__ __forceinline__ void add4(float a, float b, float c, float d) { s0 += a, s1 += b, s2 += c, s3 += d; }
    __device__ __forceinline__ void add2(float a, float b) { s0 += a, s1 += b; }
    __device__ __forceinline__ float total() const { return (s0 + s1) + (s2 + s3); }
};

// ---------------------------------------------------------------- Maths.exp

// Maths.exp (maths.cr:36-54): x = n·ln2 + r with n = round(x·log2 e) by the
// 1.5·2^23 rounder, r in two steps (ln2 split into a high and a low part),
// a degree-6 polynomial in r, then 2^n as two exponent halves; inf above
// 88.72, 0 below -87.34, NaN kept.
__device__ __forceinline__ float maths_exp(float x) {
    const float LOG2E = 1.44269504088896341f, LN2_HI = 0.693359375f, LN2_LO = -2.12194440e-4f;
    const float EXP_HI = 88.72283905f, EXP_LO = -87.3365447f, ROUNDER = 12582912.0f;
    const float clamped = (x > EXP_HI || x < EXP_LO) ? 0.0f : x;
    float n = clamped * LOG2E;
    n = n + ROUNDER;
    n = n - ROUNDER;
    float r = clamped - n * LN2_HI;
    r = r - n * LN2_LO;
    const float z = r * r;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * z + r;
    p = p + 1.0f;
    const int32_t whole = (int32_t)n;
    const int32_t half = whole >> 1;
    float result = p * __uint_as_float((uint32_t)(half + 127) << 23);
    result = result * __uint_as_float((uint32_t)(whole - half + 127) << 23);
    result = x > EXP_HI ? __builtin_inff() : result;
    result = x < EXP_LO ? 0.0f : result;
    return x != x ? x : result;
}

// SwiGLU of one element (kernels.cr:18): gate / (Maths.exp(-gate) + 1) · value.
__device__ __forceinline__ float swiglu_value(float gate, float value) {
    const float e = maths_exp(-gate);
    const float d = e + 1.0f;
    const float q = gate / d;
    return q * value;
}

// ------------------------------------------------------------ ordered sums

// Σ v[0..n) in index order from 0.0f (with SQ, Σ v[i]·v[i], each square
// rounded before its add), read by broadcast (every lane computes the same
// sum; from LDS, or global memory). The adds form one dependent chain, the
// only instructions on it; the reads of the next 32 values are issued
// before the adds of the current 32, from two register buffers used in turn.
template <int B = 8>
__device__ __forceinline__ void add32(float& s, const float4 (&b)[B]) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
        s += b[i].x;
        s += b[i].y;
        s += b[i].z;
        s += b[i].w;
    }
}

template <bool SQ = false, int B = 8>
__device__ __forceinline__ void read32(float4 (&b)[B], const float4* v4, uint32_t j) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
        b[i] = v4[j + i];
        if constexpr (SQ) b[i] = make_float4(b[i].x * b[i].x, b[i].y * b[i].y, b[i].z * b[i].z, b[i].w * b[i].w);
    }
}

// B: float4s per register buffer (8: 32 values; 4 where registers are short).
template <bool SQ = false, int B = 8>
__device__ __forceinline__ float ordered_sum(const float* v, uint32_t n) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    const uint32_t n4 = n >> 2;
    float s = 0.0f;
    uint32_t j = 0;
    if (n4 >= 2u * B) {
        float4 a[B], b[B];
        read32<SQ, B>(a, v4, 0);
        for (j = 0; j + 4u * B <= n4; j += 2u * B) {
            read32<SQ, B>(b, v4, j + B);
            add32<B>(s, a);
            read32<SQ, B>(a, v4, j + 2u * B);
            add32<B>(s, b);
        }
        // a holds [j, j + B); [j + B, n4) remain
        if (j + 2u * B <= n4) {
            read32<SQ, B>(b, v4, j + B);
            add32<B>(s, a);
            add32<B>(s, b);
            j += 2u * B;
        } else {
            add32<B>(s, a);
            j += B;
        }
    }
    for (; j < n4; ++j) {
        float4 c = v4[j];
        if constexpr (SQ) c = make_float4(c.x * c.x, c.y * c.y, c.z * c.z, c.w * c.w);
        s += c.x;
        s += c.y;
        s += c.z;
        s += c.w;
    }
    for (uint32_t i = n4 << 2; i < n; ++i) s += SQ ? v[i] * v[i] : v[i];
    return s;
}

// ------------------------------------------- ordered sums by speculation

// DPP moves across a wave64 (gfx9 controls): lane l receives lane l-1's value
// (wave_shr:1; lane 0 receives 0), and an inclusive prefix sum (row_shr 1, 2,
// 4, 8 within rows of 16, then row_bcast:15 and row_bcast:31 across rows).
__device__ __forceinline__ float wave_shift_up(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x138, 0xF, 0xF, true));
}

__device__ __forceinline__ float wave_prefix_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xF, 0xF, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xF, 0xF, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xF, 0xF, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xF, 0xF, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xA, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xC, 0xF, false));
    return x;
}

// Σ of 64·M values in index order from +0.0f -- the sequential fold's own
// bits -- by one whole wave, lane c holding values [c·M, c·M + M) in v.
// Each pass, every lane folds its M values in order from a start S_c (lane
// 0 from +0.0f) to an end E_c. If every S_c equals E_{c-1} bit for bit, the
// starts are the sequential fold's values at the chunk boundaries (by
// induction from lane 0), so E_63 is the sum. Otherwise each start is
// re-guessed as E_{c-1} plus the sum of the mismatches E_{j-1} - S_j of
// the lanes before it (within one binade of the running sum a start that
// is off by some ulps moves the end by the same amount), and the pass
// repeats. The first mismatching lane always receives its predecessor's
// exact end unchanged, so every pass fixes at least one more lane and 64
// passes bound the loop; typically 2-8 are needed (more when the running
// sum crosses many binades, or at exact ties).
template <int M>
__device__ __forceinline__ float ordered_sum_wave(const float (&v)[M]) {
    const uint32_t lane = threadIdx.x & 63u;
    float start = 0.0f, end = 0.0f;
    bool verified = false;
    for (int pass = 0; pass <= 64; ++pass) {
        end = start;
#pragma unroll
        for (int i = 0; i < M; ++i) end += v[i];
        const float prev = wave_shift_up(end);
        const bool ok = lane == 0 || __float_as_uint(prev) == __float_as_uint(start);
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) {
            verified = true;
            break;
        }
        const float miss = ok ? 0.0f : prev - start;
        const float before = wave_shift_up(wave_prefix_sum(miss));
        start = lane == 0 ? 0.0f : (before == 0.0f ? prev : prev + before);
    }
    if (!verified) {
        // not reached (the bound above suffices); the plain fold, lane by lane
        float sum = 0.0f;
        for (uint32_t c = 0; c < 64u; ++c)
            for (int i = 0; i < M; ++i) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), c));
        return sum;
    }
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(end), 63));
}

// ordered_sum_wave over v[0..n) (SQ: the squares v[i]·v[i], each rounded),
// lane c loading values [c·M, c·M + M); positions past n hold +0.0f, whose
// adds leave a running sum from +0.0f unchanged.
template <bool SQ, int M>
__device__ __forceinline__ float ordered_sum_wave_m(const float* v, uint32_t n) {
    float a[M];
    const uint32_t c0 = (threadIdx.x & 63u) * (uint32_t)M;
    if ((M % 4 == 0) && n % 4u == 0 && ((uintptr_t)v & 15u) == 0) {
        // 16-byte reads (a lane's chunk starts 16-byte aligned)
#pragma unroll
        for (int i = 0; i < M; i += 4) {
            const uint32_t j = c0 + (uint32_t)i;
            const float4 x = j < n ? *reinterpret_cast<const float4*>(v + j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            a[i] = SQ ? x.x * x.x : x.x;
            a[i + 1] = SQ ? x.y * x.y : x.y;
            a[i + 2] = SQ ? x.z * x.z : x.z;
            a[i + 3] = SQ ? x.w * x.w : x.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const uint32_t j = c0 + (uint32_t)i;
            const float x = j < n ? v[j] : 0.0f;
            a[i] = SQ ? x * x : x;
        }
    }
    return ordered_sum_wave<M>(a);
}

// Largest n the wave fold takes (64 lanes x 128 values).
constexpr uint32_t WAVE_SUM_MAX = 8192;

// Σ v[0..n) in index order from +0.0f (SQ: Σ v[i]·v[i]) by one whole wave:
// every lane of the wave calls it with the same v and n (n <= 64·MAXM, at
// most WAVE_SUM_MAX) and receives the sum. MAXM bounds the values a lane
// holds, and so the registers the caller's kernel is compiled for.
template <bool SQ = false, int MAXM = 128>
__device__ __forceinline__ float ordered_sum_by_wave(const float* v, uint32_t n) {
    if (n <= 64u * 8u) return ordered_sum_wave_m<SQ, 8>(v, n);
    if constexpr (MAXM >= 32) {
        if (n <= 64u * 32u) return ordered_sum_wave_m<SQ, 32>(v, n);
    }
    if constexpr (MAXM >= 128) return ordered_sum_wave_m<SQ, 128>(v, n);
    return 0.0f;
}

// The ordered sum of v[0..n) by wave 0 (ordered_sum_by_wave; beyond its
// limit, ordered_sum), shared through LDS. Every thread calls it.
__device__ __forceinline__ float shared_sum(const float* v, uint32_t n) {
    __shared__ float result;
    if (threadIdx.x < 64u) {
        const float sum = n <= WAVE_SUM_MAX ? ordered_sum_by_wave(v, n) : ordered_sum(v, n);
        if (threadIdx.x == 0) result = sum;
    }
    __syncthreads();
    return result;
}

// ------------------------------------------------------------------ RMSNorm

// Largest row the LDS kernels stage: 32 KB.
constexpr uint32_t RMSNORM_LDS_ROW = 8192;

// Stages row x (n values, at most RMSNORM_LDS_ROW) in LDS, then returns the
// root sqrt(Σx²/n + eps), the squares folded in index order by wave 0
// (ordered_sum_by_wave) and shared through LDS. Every thread calls it.
__device__ __forceinline__ float stage_root(const float* __restrict__ xr, uint32_t n, float eps, float* row) {
    // four loads in flight per thread before any store
    for (uint32_t j0 = threadIdx.x; j0 < n; j0 += 1024u) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t j = j0 + 256u * u;
            v[u] = j < n ? xr[j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t j = j0 + 256u * u;
            if (j < n) row[j] = v[u];
        }
    }
    __shared__ float root;
    __syncthreads();
    if (threadIdx.x < 64u) {
        const float squares = ordered_sum_by_wave<true>(row, n);
        if (threadIdx.x == 0) root = __builtin_sqrtf(squares / (float)n + eps);
    }
    __syncthreads();
    return root;
}

// RMSNorm of row xr (n values, a multiple of 32, at most RMSNORM_LDS_ROW)
// then the activation quantiser, by one workgroup: each 8-lane group
// normalises 4 values a lane of a block of 32 and quantises the block
// (quantize_activations, quant.cr:428-442, on the normalised row) into
// `act` row r, laid out as the quantise pass lays it out. row is LDS of n
// floats. Every thread calls it.
__device__ __forceinline__ void rmsnorm_quantise_row(const float* __restrict__ xr, uint32_t n,
                                                     const float* __restrict__ w, float eps, Activations act,
                                                     uint32_t r, float* row) {
    const uint32_t nb = n >> 5, sub = threadIdx.x & 7u;
    // this lane's weights, loaded before the fold (n ≤ 8192: at most 8 passes)
    float4 wv[RMSNORM_LDS_ROW / 1024];
#pragma unroll
    for (uint32_t pass = 0; pass < RMSNORM_LDS_ROW / 1024; ++pass) {
        const uint32_t blk = (threadIdx.x >> 3) + 32u * pass;
        wv[pass] = (w && blk < nb) ? *reinterpret_cast<const float4*>(w + blk * 32u + sub * 4u)
                                   : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
    const float root = stage_root(xr, n, eps, row);
#pragma unroll
    for (uint32_t pass = 0; pass < RMSNORM_LDS_ROW / 1024; ++pass) {
        const uint32_t blk = (threadIdx.x >> 3) + 32u * pass;
        if (blk >= nb) break;
        const uint32_t j = blk * 32u + sub * 4u;
        const float wj[4] = {wv[pass].x, wv[pass].y, wv[pass].z, wv[pass].w};
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q = row[j + i] / root;
            v[i] = w ? q * wj[i] : q;
        }
        const Q8Quad q = quantize_quad(v[0], v[1], v[2], v[3]);
        *(uint32_t*)((int8_t*)act.qs + (size_t)r * n + j) = q.packed;
        if (sub == 0) {
            const size_t g = (size_t)r * nb + blk;
            ((float*)act.scales)[g] = q.scale;
            ((float*)act.sums)[g] = q.sum;
            ((int32_t*)act.totals)[g] = q.total;
        }
    }
}

// ------------------------------------------------- LDS direct loads (gfx950)

typedef __attribute__((address_space(3))) uint8_t lds_byte;

// The LDS byte address of p (a pointer into shared memory), uniform.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_byte*)p);
}

// Direct loads from global memory into LDS: each lane's 16 (or 4) bytes at
// `from` land at LDS byte lds + 16·lane (4·lane). Written as inline asm so
// that the compiler does not see the LDS write: it would otherwise wait for
// every load in flight before any LDS access it cannot prove disjoint,
// which would end the streaming; the kernels order these writes themselves
// (counted waits and barriers). M0 carries the LDS address (an operand, so
// the compiler writes it); s_nop covers the wait state an M0 write needs
// before an LDS direct load.
__device__ __forceinline__ void lds_load16(const void* from, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(from), "{m0}"(lds) : "memory");
}

// lds_load16 marked non-temporal: weights stream through the caches once,
// so they should not displace what is read again (activations, tables).
__device__ __forceinline__ void lds_load16_nt(const void* from, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(from), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ void lds_load4(const void* from, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(from), "{m0}"(lds) : "memory");
}

// s_waitcnt: at most N vector memory operations of this wave outstanding,
// every LDS and scalar memory operation done.
template <uint32_t N>
__device__ __forceinline__ void wait_vm_lds() {
    static_assert(N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (7 << 4));
}

// wait_vm_lds<n> for a runtime n (at most 63; n past it waits for 63).
template <uint32_t N = 63>
__device__ __forceinline__ void wait_vm_lds_upto(uint32_t n) {
    if constexpr (N == 0) {
        wait_vm_lds<0>();
    } else {
        if (n >= N)
            wait_vm_lds<N>();
        else
            wait_vm_lds_upto<N - 1>(n);
    }
}

// wait_vm_lds<n> for a runtime n in [LO, HI] (n past HI waits for HI),
// chosen by halving the range: log2 of its width uniform branches rather
// than one compare per value above n (the stage loops of the matrix-core
// kernels wait once a stage).
template <uint32_t LO, uint32_t HI>
__device__ __forceinline__ void wait_vm_lds_in(uint32_t n) {
    if constexpr (LO == HI) {
        wait_vm_lds<LO>();
    } else {
        constexpr uint32_t MID = (LO + HI + 1u) / 2u;
        if (n >= MID)
            wait_vm_lds_in<MID, HI>(n);
        else
            wait_vm_lds_in<LO, MID - 1u>(n);
    }
}

// A workgroup barrier after this wave's LDS (and scalar memory) operations,
// leaving its direct loads in flight: __syncthreads() would wait for them.
// The empty asm statements keep the compiler from moving memory operations
// across it.
__device__ __forceinline__ void lds_sync() {
    asm volatile("" ::: "memory");
    wait_vm_lds<63>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

}  // namespace tmh
