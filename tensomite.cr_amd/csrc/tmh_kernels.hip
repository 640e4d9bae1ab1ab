// Kernels of libtensomite_hip.so for gfx950 (CDNA4, wave64).
//
// Every kernel computes what the reference's host path computes, operation
// for operation (src/tensomite/quant.cr; behaviour of the CUDA kernels in
// src/tensomite/cuda/kernels.cu:1114-1375), so results are bit-identical to
// tensomite's CPU quantised path:
//
//   - integer block dot products may be taken in any order (they are exact);
//   - each block's floating-point contribution uses the host's expression:
//       Q8_0  float(t) * (d * sx)             quant.cr:454
//       Q4_0  (float(t) * d) * sx             quant.cr:471
//       Q4_1  (d * sx) * float(t) + m * mx    quant.cr:488
//   - every output adds its contributions one by one in block order,
//     starting from 0.0f (quant.cr:447-455);
//   - the bias is a separate addition after the sum (host.cr:725-734).
//
// The library is compiled with -ffp-contract=off, so no multiply-add is
// fused, and with correctly rounded f32 division.
#include "tmh_device.h"
#include "tmh_internal.h"

#include <stdlib.h>
#include <string.h>

namespace tmh {

namespace {
thread_local bool t_tree_fold = false;
}  // namespace

bool tree_fold() { return t_tree_fold; }
TreeFold::TreeFold(bool on) : saved(t_tree_fold) { t_tree_fold = on; }
TreeFold::~TreeFold() { t_tree_fold = saved; }

// ------------------------------------------------------ activation quantise

// One group of 8 lanes per block of 32 activations, 4 values a lane: the
// block's largest magnitude and Σq are reduced over the 8 lanes by DPP (max
// and integer sums are exact in any order). Then, as quantize_activations
// (quant.cr:428-442): d = amax/127, id = 1/d (0 when d is 0),
// q = round-half-away(x·id) as int8, scale F16(d), sum F16(float(Σq)·d).
template <bool VEC>
__global__ __launch_bounds__(256) void k_quantize_rows_q8(const float* __restrict__ x, uint32_t ldx, uint32_t nb,
                                                          uint32_t k, uint32_t blocks, float* __restrict__ scales,
                                                          float* __restrict__ sums, int32_t* __restrict__ totals,
                                                          int8_t* __restrict__ qs) {
    const uint32_t g = (blockIdx.x * 256u + threadIdx.x) >> 3;
    const uint32_t sub = threadIdx.x & 7u;
    if (g >= blocks) return;  // all 8 lanes of a block leave together
    const uint32_t row = g / nb, blk = g - row * nb;
    const float* src = x + (size_t)row * ldx + blk * 32u + sub * 4u;
    float v0, v1, v2, v3;
    if constexpr (VEC) {
        float4 v = *(const float4*)src;
        v0 = v.x, v1 = v.y, v2 = v.z, v3 = v.w;
    } else {
        v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
    }
    float amax = fabsf(v0);
    if (sub != 0 && amax != amax) amax = 0.0f;  // a NaN not first in its block is skipped, as the host's loop does
    amax = fabsf(v1) > amax ? fabsf(v1) : amax;
    amax = fabsf(v2) > amax ? fabsf(v2) : amax;
    amax = fabsf(v3) > amax ? fabsf(v3) : amax;
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
    const uint32_t packed = (uint32_t)(q0 & 0xff) | (uint32_t)(q1 & 0xff) << 8 | (uint32_t)(q2 & 0xff) << 16 |
                            (uint32_t)(q3 & 0xff) << 24;
    *(uint32_t*)(qs + (size_t)row * k + blk * 32u + sub * 4u) = packed;
    int total = q0 + q1 + q2 + q3;
    total += dpp_int<DPP_XOR1>(total);
    total += dpp_int<DPP_XOR2>(total);
    total += dpp_int<DPP_MIRROR>(total);
    if (sub == 0) {
        scales[g] = round_to_half(d);
        sums[g] = round_to_half((float)total * d);
        totals[g] = total;
    }
}

// ------------------------------------------------------ block contributions

// Formats as the kernels see them: a pair of consecutive blocks is PW
// dwords, dword-aligned when the row is (two blocks of 18, 34 or 20 bytes are
// 36, 68 or 40 bytes).
template <int KIND>
struct Fmt;
template <>
struct Fmt<0> {
    static constexpr uint32_t BB = 34, PW = 17;
};
template <>
struct Fmt<1> {
    static constexpr uint32_t BB = 18, PW = 9;
};
template <>
struct Fmt<2> {
    static constexpr uint32_t BB = 20, PW = 10;
};

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, bytes);
}

// The contributions of the two blocks of one pair (dwords u) to one output,
// given the pair's quantised activations: a[0..7] and a[8..15] the int8
// values of the two blocks, sx the scales, ex the Q4_0 totals (as -8·Σq) or
// the Q4_1 F16(d·Σq).
template <int KIND>
struct Pair;

// Q8_0: block 0 = d at bytes 0-1, values at 2-33; block 1 = d at 34-35,
// values at 36-67 (dwords 9-16, aligned). t = Σ w·q; float(t) * (d * sx).
template <>
struct Pair<0> {
    __device__ __forceinline__ static void contribute(const uint32_t* u, const uint32_t* a, float sx0, float sx1,
                                                      int, int, float, float, float& c0, float& c1) {
        int t0 = 0, t1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) t0 = dot4(funnel(u[i + 1], u[i], 2), a[i], t0);
#pragma unroll
        for (int i = 0; i < 8; ++i) t1 = dot4(u[9 + i], a[8 + i], t1);
        const float s0 = half_value(u[0] & 0xffffu) * sx0;
        const float s1 = half_value(u[8] >> 16) * sx1;
        c0 = (float)t0 * s0;
        c1 = (float)t1 * s1;
    }
};

// Q4_0: block 0 = d at bytes 0-1, nibbles at 2-17; block 1 = d at 18-19,
// nibbles at 20-35 (dwords 5-8, aligned). Byte j holds element j (low) and
// j+16 (high). t = Σ(q-8)·y = Σq·y - 8·Σy; (float(t) * d) * sx.
template <>
struct Pair<1> {
    __device__ __forceinline__ static void contribute(const uint32_t* u, const uint32_t* a, float sx0, float sx1,
                                                      int neg8_0, int neg8_1, float, float, float& c0,
                                                      float& c1) {
        int t0 = neg8_0, t1 = neg8_1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = funnel(u[i + 1], u[i], 2);
            t0 = dot4(w & 0x0f0f0f0fu, a[i], t0);
            t0 = dot4((w >> 4) & 0x0f0f0f0fu, a[4 + i], t0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = u[5 + i];
            t1 = dot4(w & 0x0f0f0f0fu, a[8 + i], t1);
            t1 = dot4((w >> 4) & 0x0f0f0f0fu, a[12 + i], t1);
        }
        const float p0 = (float)t0 * half_value(u[0] & 0xffffu);
        const float p1 = (float)t1 * half_value(u[4] >> 16);
        c0 = p0 * sx0;
        c1 = p1 * sx1;
    }
};

// Q4_1: block 0 = d, m at bytes 0-3, nibbles at 4-19; block 1 = d, m at
// 20-23, nibbles at 24-39; all aligned. t = Σq·y;
// (d * sx) * float(t) + m * mx.
template <>
struct Pair<2> {
    __device__ __forceinline__ static void contribute(const uint32_t* u, const uint32_t* a, float sx0, float sx1,
                                                      int, int, float mx0, float mx1, float& c0, float& c1) {
        int t0 = 0, t1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            t0 = dot4(u[1 + i] & 0x0f0f0f0fu, a[i], t0);
            t0 = dot4((u[1 + i] >> 4) & 0x0f0f0f0fu, a[4 + i], t0);
            t1 = dot4(u[6 + i] & 0x0f0f0f0fu, a[8 + i], t1);
            t1 = dot4((u[6 + i] >> 4) & 0x0f0f0f0fu, a[12 + i], t1);
        }
        const float s0 = half_value(u[0] & 0xffffu) * sx0;
        const float s1 = half_value(u[5] & 0xffffu) * sx1;
        const float f0 = s0 * (float)t0;
        const float f1 = s1 * (float)t1;
        const float g0 = half_value(u[0] >> 16) * mx0;
        const float g1 = half_value(u[5] >> 16) * mx1;
        c0 = f0 + g0;
        c1 = f1 + g1;
    }
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Pointers known to be in global memory. Pointers read from a table are
// generic to the compiler, which then issues flat loads; those count
// against the LDS wait counter too, so every LDS wait would also drain the
// weight loads in flight. Casting to the global address space keeps them
// global loads.
template <typename T>
using gptr = const __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ gptr<T> global(const T* p) {
    return (gptr<T>)p;
}

// Four floats from global memory, one 16-byte load when `vec` (16-byte aligned).
__device__ __forceinline__ float4 load_f4(const float* p, bool vec) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    if (vec) {
        const f4 v = *(const __attribute__((address_space(1))) f4*)p;
        return make_float4(v.x, v.y, v.z, v.w);
    }
    const gptr<float> g = global(p);
    return make_float4(g[0], g[1], g[2], g[3]);
}

// Loads the PW dwords of a pair at p (dword-aligned).
template <int KIND>
__device__ __forceinline__ void load_pair(const uint32_t* __restrict__ pp, uint32_t* u) {
    constexpr uint32_t PW = Fmt<KIND>::PW;
    typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
    typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));
    const gptr<uint32_t> p = global(pp);
#pragma unroll
    for (uint32_t i = 0; i + 4 <= PW; i += 4) {
        const u32x4a v = *(const __attribute__((address_space(1))) u32x4a*)(p + i);
        u[i] = v.x, u[i + 1] = v.y, u[i + 2] = v.z, u[i + 3] = v.w;
    }
    if constexpr (PW % 4 == 1) {
        u[PW - 1] = p[PW - 1];
    } else if constexpr (PW % 4 == 2) {
        const u32x2a v = *(const __attribute__((address_space(1))) u32x2a*)(p + PW - 2);
        u[PW - 2] = v.x, u[PW - 1] = v.y;
    }
}

// The quantised activations of pair j of activation row b.
template <int KIND>
__device__ __forceinline__ void load_activations(const Activations& act, uint32_t k, uint32_t nb, uint32_t b,
                                                 uint32_t j, uint32_t* a, float& sx0, float& sx1, int& e0, int& e1,
                                                 float& mx0, float& mx1) {
    typedef uint32_t gu32x4 __attribute__((ext_vector_type(4)));
    const __attribute__((address_space(1))) gu32x4* q =
        (const __attribute__((address_space(1))) gu32x4*)(act.qs + (size_t)b * k + (size_t)j * 64u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const gu32x4 v = q[i];
        a[4 * i] = v.x, a[4 * i + 1] = v.y, a[4 * i + 2] = v.z, a[4 * i + 3] = v.w;
    }
    const size_t at = (size_t)b * nb + 2u * j;
    const gptr<float> sc = global(act.scales + at);
    sx0 = sc[0], sx1 = sc[1];
    if constexpr (KIND == 1) {
        const gptr<int32_t> tt = global(act.totals + at);
        e0 = -8 * tt[0], e1 = -8 * tt[1];
    }
    if constexpr (KIND == 2) {
        const gptr<float> m = global(act.sums + at);
        mx0 = m[0], mx1 = m[1];
    }
}

// --------------------------------------------------------- lanes: matvec

// x · wᵀ for NB activation rows and a tile of `tr` weight rows per
// workgroup of 256 threads, for rows of an even number of blocks nb ≤ 512
// starting dword-aligned.
//
// Work: each weight row is np = nb/2 pairs of blocks. Threads form row
// groups of np threads; thread t takes pair j = t % np of row t / np of each
// step of rpi = 256/np rows, so consecutive threads read consecutive bytes of
// one row and each thread keeps its pair's activations for the whole tile.
// A thread computes its pair's two contributions to each output it touches
// and writes them to LDS, part[output][block]. Then thread o < NB·tr adds
// the contributions of output o (and o + 256, ...) one by one in block order
// -- the host's order -- and writes it, plus the bias.
//
// GLU: w is a merged [gate | up] matrix of n = 2·H rows, and the tile's tr
// rows are gate rows tile·tr/2 .. + tr/2 then the up rows of the same
// indices (tr/2 a multiple of 32). The folded outputs stay in LDS; then
// each 8-lane group takes a block of 32 of them, SwiGLU
// (gate / (Maths.exp(-gate) + 1) · up) 4 a lane, and quantises the block
// into `glu` as the quantise pass lays out an [NB, H] activation.
template <int KIND, int NB, bool GLU = false, bool TREE = false>
__device__ __forceinline__ void matvec_tile(const uint8_t* __restrict__ w, Activations act, float* __restrict__ dst,
                                            const float* __restrict__ bias, uint32_t bias_ld, uint32_t n,
                                            uint32_t k, uint32_t tr, uint32_t stride, uint32_t tile, float* part,
                                            Activations glu = Activations{}) {
    constexpr bool tree = TREE;  // UNORDERED's fold (Fold4)
    constexpr uint32_t PW = Fmt<KIND>::PW;
    const uint32_t t = threadIdx.x;
    const uint32_t nb = k >> 5;
    const uint32_t np = nb >> 1;
    const uint32_t rpi = 256u / np;
    const uint32_t j = t % np, rsub = t / np;
    const uint32_t row0 = tile * tr;
    const uint32_t steps = tr / rpi;
    const size_t row_words = (size_t)np * PW;
    const uint32_t* wp = (const uint32_t*)w;
    // GLU: output r of the tile is gate row g0 + r, or up row H + g0 + r - h
    const uint32_t h = tr >> 1, H = n >> 1, g0 = tile * h;
    auto row_of = [&](uint32_t r) -> uint32_t { return GLU ? (r < h ? g0 + r : H + g0 + (r - h)) : row0 + r; };

    if (rsub < rpi) {
        // This thread's pair of every activation row, held in registers for
        // all steps (j is fixed per thread).
        uint32_t a[NB][16];
        float sx0[NB], sx1[NB], mx0[NB], mx1[NB];
        int e0[NB], e1[NB];
#pragma unroll
        for (uint32_t b = 0; b < (uint32_t)NB; ++b) {
            mx0[b] = mx1[b] = 0.0f;
            e0[b] = e1[b] = 0;
            load_activations<KIND>(act, k, nb, b, j, a[b], sx0[b], sx1[b], e0[b], e1[b], mx0[b], mx1[b]);
        }
#pragma unroll 2
        for (uint32_t s = 0; s < steps; ++s) {
            const uint32_t r = s * rpi + rsub;
            const uint32_t row = row_of(r);
            if (!GLU && row >= n) break;
            uint32_t u[PW];
            load_pair<KIND>(wp + (size_t)row * row_words + (size_t)j * PW, u);
#pragma unroll
            for (uint32_t b = 0; b < (uint32_t)NB; ++b) {
                float c0, c1;
                Pair<KIND>::contribute(u, a[b], sx0[b], sx1[b], e0[b], e1[b], mx0[b], mx1[b], c0, c1);
                *(float2*)(part + (size_t)(b * tr + r) * stride + 2u * j) = make_float2(c0, c1);
            }
        }
    }
    __syncthreads();
    float* outs = part + (size_t)NB * tr * stride;  // GLU: the tile's outputs, [NB][tr]
    for (uint32_t o = t; o < (uint32_t)NB * tr; o += 256u) {
        const uint32_t b = o / tr, r = o - b * tr;
        const uint32_t row = row_of(r);
        if (GLU || row < n) {
            const float* c = part + (size_t)o * stride;
            float sum = 0.0f;
            uint32_t i = 0;
            if (tree) {
                Fold4 u;
                for (; i + 4 <= nb; i += 4) {
                    const float4 v = *(const float4*)(c + i);
                    u.add4(v.x, v.y, v.z, v.w);
                }
                for (; i < nb; ++i) u.s0 += c[i];
                sum = u.total();
            } else {
                for (; i + 4 <= nb; i += 4) {
                    const float4 v = *(const float4*)(c + i);
                    sum += v.x;
                    sum += v.y;
                    sum += v.z;
                    sum += v.w;
                }
                for (; i < nb; ++i) sum += c[i];
            }
            if constexpr (GLU) {
                outs[o] = sum;
            } else {
                dst[(size_t)b * n + row] = bias ? sum + bias[(size_t)b * bias_ld + row] : sum;
            }
        }
    }
    if constexpr (GLU) {
        __syncthreads();
        // blocks of 32 outputs: NB rows x h / 32; every lane of a group takes
        // the same trip count (quantize_quad reduces across the 8 lanes)
        const uint32_t hb = h >> 5, sub = t & 7u, Hb = H >> 5;
        for (uint32_t g = t >> 3; g < (uint32_t)NB * hb; g += 32u) {
            const uint32_t b = g / hb, blk = g - b * hb;
            const float* gate = outs + (size_t)b * tr + blk * 32u + sub * 4u;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = swiglu_value(gate[i], gate[h + i]);
            const Q8Quad q = quantize_quad(v[0], v[1], v[2], v[3]);
            const uint32_t col = g0 + blk * 32u + sub * 4u;
            *(uint32_t*)((int8_t*)glu.qs + (size_t)b * H + col) = q.packed;
            if (sub == 0) {
                const size_t at = (size_t)b * Hb + (g0 >> 5) + blk;
                ((float*)glu.scales)[at] = q.scale;
                ((float*)glu.sums)[at] = q.sum;
                ((int32_t*)glu.totals)[at] = q.total;
            }
        }
    }
}

// bias_ld: the bias's elements per activation row (0: one bias row for
// every activation row; n: a row each, e.g. a residual).
template <int KIND, int NB, bool TREE>
__global__ __launch_bounds__(256) void k_matvec(const uint8_t* __restrict__ w, Activations act,
                                                float* __restrict__ dst, const float* __restrict__ bias,
                                                uint32_t bias_ld, uint32_t n, uint32_t k, uint32_t tr,
                                                uint32_t stride) {
    extern __shared__ float part[];
    matvec_tile<KIND, NB, false, TREE>(w, act, dst, bias, bias_ld, n, k, tr, stride, blockIdx.x, part);
}

// The lanes product over a merged [gate | up] matrix with SwiGLU and the
// activation quantiser in its epilogue (matvec_tile's GLU form): `glu`
// receives quantised SwiGLU(gate, up) rows of n / 2.
template <int KIND, int NB, bool TREE>
__global__ __launch_bounds__(256) void k_matvec_glu(const uint8_t* __restrict__ w, Activations act, uint32_t n,
                                                    uint32_t k, uint32_t tr, uint32_t stride, Activations glu) {
    extern __shared__ float part[];
    matvec_tile<KIND, NB, true, TREE>(w, act, nullptr, nullptr, 0, n, k, tr, stride, blockIdx.x, part, glu);
}


// ------------------------------------------------- one row, weights in LDS

// Threads of a k_matvec_one workgroup: 8 waves, two a SIMD, so one wave's
// waits overlap another's work.
constexpr uint32_t ONE_THREADS = 512;
constexpr uint32_t ONE_WAVES = ONE_THREADS / 64u;

// Direct loads of `bytes` contiguous bytes at src into LDS at `to` (a byte
// address), 1 KB a load, load i by the wave first + (i % waves); lanes past
// the end read the last 16 bytes again (the LDS region holds whole
// kilobytes). `bytes` a multiple of 16. Returns this wave's loads (0 for a
// wave outside [first, first + waves)).
// NT: the bytes are read once (weights), so they should not displace what
// other workgroups read again from the caches (the activation row).
template <bool NT>
__device__ __forceinline__ uint32_t stage_bytes(const uint8_t* src, uint32_t bytes, uint32_t to, uint32_t wave,
                                                uint32_t first, uint32_t waves) {
    if (wave < first || wave >= first + waves) return 0;
    const uint32_t lane = threadIdx.x & 63u;
    const uintptr_t base = (uintptr_t)src, last = base + bytes - 16u;
    const uint32_t loads = (bytes + 1023u) >> 10;
    uint32_t mine = 0;
    for (uint32_t i = wave - first; i < loads; i += waves, ++mine) {
        const uintptr_t at = base + (uintptr_t)i * 1024u + lane * 16u;
        if constexpr (NT) lds_load16_nt((const void*)(at < last ? at : last), to + i * 1024u);
        else lds_load16((const void*)(at < last ? at : last), to + i * 1024u);
    }
    return mine;
}

// Direct loads of `bytes` (a multiple of 16·G) at src into LDS at `to` (the
// region holds whole kilobytes) by wave `by` only, the 16-byte pieces of
// each group g of G rotated: piece i lands in slot G g + ((i + (g >> S)) %
// G), so that lanes reading piece i of consecutive groups together meet
// distinct bank groups (a group of G pieces spans G·4 banks of the 64). Lane
// l of load n fills slot 64 n + l with the piece that belongs there.
template <uint32_t G, uint32_t S>
__device__ __forceinline__ void stage_rotated(const uint8_t* src, uint32_t bytes, uint32_t to, uint32_t wave,
                                              uint32_t by) {
    static_assert((G & (G - 1u)) == 0, "whole groups of a power of two");
    if (wave != by) return;
    const uint32_t lane = threadIdx.x & 63u, pieces = bytes >> 4, loads = (pieces + 63u) >> 6;
    for (uint32_t n = 0; n < loads; ++n) {
        // a slot past the last piece takes a copy of the last slot's piece
        const uint32_t slot = min(n * 64u + lane, pieces - 1u), g = slot / G;
        const uint32_t i = ((slot & (G - 1u)) - (g >> S)) & (G - 1u);
        lds_load16(src + 16u * (G * g + i), to + n * 1024u);
    }
}

// Direct loads of `count` 4-byte values at src into LDS at `to`, 256 bytes
// a load, by wave `by` only; returns this wave's loads.
__device__ __forceinline__ uint32_t stage_words(const void* src, uint32_t count, uint32_t to, uint32_t wave,
                                                uint32_t by) {
    if (wave != by) return 0;
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t mine = 0;
    for (uint32_t c0 = 0; c0 < count; c0 += 64u, ++mine)
        lds_load4((const uint32_t*)src + min(c0 + lane, count - 1u), to + c0 * 4u);
    return mine;
}

// LDS layout of k_matvec_one, in bytes from the start of its dynamic LDS.
struct OneLds {
    uint32_t x, nw, qs, scales, sums, totals, arow, w, w2, part, outs, end;
};

__host__ __device__ inline OneLds one_lds(uint32_t k, uint32_t tr, uint32_t row_bytes, uint32_t stride, bool norm,
                                          bool glu, bool plain = false, uint32_t xr = 1u) {
    const uint32_t nb = k >> 5;
    auto kb = [](uint32_t b) { return (b + 1023u) & ~1023u; };
    OneLds l;
    l.x = 0;  // xr rows of kb(4k) bytes
    l.nw = norm ? xr * kb(4u * k) : 0u;
    l.qs = norm ? (plain ? xr : 2u) * kb(4u * k) : 0u;  // plain: no norm weights
    l.scales = l.qs + kb(k);
    l.sums = l.scales + ((4u * nb + 255u) & ~255u);
    l.totals = l.sums + ((4u * nb + 255u) & ~255u);
    l.arow = l.totals + kb(4u * nb) - l.qs;  // one quantised row and its tables; row b at + b·arow
    l.w = l.qs + xr * l.arow;
    const uint32_t wbytes = glu ? (tr / 2u) * row_bytes : tr * row_bytes;
    l.w2 = l.w + kb(wbytes);
    l.part = glu ? l.w2 + kb(wbytes) : l.w2;
    l.outs = l.part + 4u * xr * tr * stride;  // activation row b's contributions at part + b·tr rows
    l.end = l.outs + (glu ? 4u * (tr + tr / 2u) : 0u);
    return l;
}

// One activation row times a tile of `tr` weight rows per workgroup, the
// tile's weight bytes (contiguous rows; GLU: its gate rows and its up rows)
// brought into LDS by direct loads that waves 1..7 (NORM: 2..7) issue at
// the start, while wave 0 loads the activations alone (NORM: x, wave 1 the
// norm's weights), so its wait for them never waits for weights:
//   NORM: x is the f32 row, taken through Op::RMSNorm (host.cr:374-386;
//     weights nw, eps) and the activation quantiser -- the squares' sum in
//     index order by speculation across wave 0, root = sqrtf(Σ/k + eps),
//     v = x / root · nw, quantize_quad: the bits of k_rmsnorm_quantise_wave
//     -- while the weights are in flight;
//   NORM and PLAIN: x is the f32 row, quantised as it is (no norm; waves 0
//     and 1 stage it, half each when its bytes are whole kilobytes); XR = 2:
//     two rows (x and x + ldx, one a wave), each weight pair read once for
//     both, outputs dst[b·n + row];
//   else the row arrives quantised (act, as the quantise pass lays it out).
// Then matvec_tile's per-pair contributions and ordered fold, from LDS:
// dst[row] = Σ (+ bias[row], one rounding), or, GLU, SwiGLU and the
// quantiser on the tile's gate/up outputs into glu. k a multiple of 64 with
// ONE_THREADS % (k / 64) == 0 (whole rows of pairs per pass), rows whole
// 16-byte pieces starting 16-byte aligned.
template <int KIND, bool NORM, bool GLU, bool PLAIN = false, uint32_t XR = 1, bool TREE = false>
__global__ __launch_bounds__(ONE_THREADS) void k_matvec_one(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ nw, float eps, Activations act,
                                                            float* __restrict__ dst, const float* __restrict__ bias,
                                                            uint32_t n, uint32_t k, uint32_t tr, uint32_t stride,
                                                            Activations glu, uint32_t ldx) {
    constexpr bool tree = TREE;  // UNORDERED's fold (Fold4)
    extern __shared__ float4 lds4[];
    uint8_t* base = reinterpret_cast<uint8_t*>(lds4);
    __shared__ float root_slot;
    constexpr uint32_t PW = Fmt<KIND>::PW, BB = Fmt<KIND>::BB;
    const uint32_t t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nb = k >> 5, np = nb >> 1, row_bytes = nb * BB;
    const uint32_t tile = blockIdx.x, h = tr >> 1, H = n >> 1, g0 = tile * h;
    const uint32_t row0 = tile * tr, rows = GLU ? tr : min(tr, n - row0);
    static_assert(!PLAIN || (NORM && !GLU), "plain rows take the f32 path");
    static_assert(XR == 1 || (PLAIN && XR == 2), "two rows: plain f32 rows only");
    const OneLds L = one_lds(k, tr, row_bytes, stride, NORM, GLU, PLAIN, XR);
    const uint32_t xrow = (4u * k + 1023u) & ~1023u;
    const uint32_t lbase = lds_address(base);

    // Wave 0: the activations (NORM: x, while wave 1 brings the norm's
    // weights, so wave 0's wait before Σx² is for x alone), issued before
    // any weight load (the compute unit's loads queue in order, so the
    // weights would delay them). The other waves: the weights.
    constexpr uint32_t WFIRST = NORM ? 2u : 1u;  // the first wave of the weights
    // x in groups of 8 pieces (a lane's 32 values of Σx²) rotated by group / 2,
    // the quantised row in groups of 4 (a pair of blocks) rotated by group /
    // 4 (stage_rotated), so that the lanes' reads below meet distinct banks
    if constexpr (PLAIN && XR == 2) {
        stage_rotated<8, 1>(reinterpret_cast<const uint8_t*>(x), 4u * k, lbase + L.x, wave, 0u);
        stage_rotated<8, 1>(reinterpret_cast<const uint8_t*>(x + ldx), 4u * k, lbase + L.x + xrow, wave, 1u);
    } else if constexpr (PLAIN) {
        // halves only where each holds a multiple of 16 groups of 8 pieces
        // (k a multiple of 1024): stage_rotated rotates a group by its index
        // within the call, mod 16, and the readers below by its index within
        // the row, so the second half's first group must be one whose
        // row index is 0 mod 16
        const uint32_t half = (k % 1024u) == 0 ? 2u * k : 4u * k;
        stage_rotated<8, 1>(reinterpret_cast<const uint8_t*>(x), half, lbase + L.x, wave, 0u);
        if (half < 4u * k)
            stage_rotated<8, 1>(reinterpret_cast<const uint8_t*>(x) + half, half, lbase + L.x + half, wave, 1u);
    } else if constexpr (NORM) {
        stage_rotated<8, 1>(reinterpret_cast<const uint8_t*>(x), 4u * k, lbase + L.x, wave, 0u);
        stage_bytes<false>(reinterpret_cast<const uint8_t*>(nw), 4u * k, lbase + L.nw, wave, 1u, 1u);
    } else {
        stage_rotated<4, 2>(reinterpret_cast<const uint8_t*>(act.qs), k, lbase + L.qs, wave, 0u);
        stage_words(act.scales, nb, lbase + L.scales, wave, 0u);
        if constexpr (KIND == 2) stage_words(act.sums, nb, lbase + L.sums, wave, 0u);
        if constexpr (KIND == 1) stage_words(act.totals, nb, lbase + L.totals, wave, 0u);
    }
    lds_sync();
    if constexpr (GLU) {
        stage_bytes<true>(w + (size_t)g0 * row_bytes, h * row_bytes, lbase + L.w, wave, WFIRST, ONE_WAVES - WFIRST);
        stage_bytes<true>(w + (size_t)(H + g0) * row_bytes, h * row_bytes, lbase + L.w2, wave, WFIRST,
                          ONE_WAVES - WFIRST);
    } else {
        stage_bytes<true>(w + (size_t)row0 * row_bytes, rows * row_bytes, lbase + L.w, wave, WFIRST, ONE_WAVES - WFIRST);
    }

    int8_t* aq = reinterpret_cast<int8_t*>(base + L.qs);
    float* asc = reinterpret_cast<float*>(base + L.scales);
    float* asm_ = reinterpret_cast<float*>(base + L.sums);
    int32_t* atot = reinterpret_cast<int32_t*>(base + L.totals);
    if (wave == 0) {
        wait_vm_lds<0>();  // wave 0 issued only the activations
        if constexpr (NORM && !PLAIN) {
            const float4* xs4 = reinterpret_cast<const float4*>(base + L.x);
            float sq[32];
#pragma unroll
            for (uint32_t i = 0; i < 32u; i += 4u) {
                const uint32_t c = t * 32u + i;  // piece i / 4 of group t
                const float4 v = c < k ? xs4[8u * t + ((i / 4u + (t >> 1)) & 7u)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                sq[i] = v.x * v.x;
                sq[i + 1] = v.y * v.y;
                sq[i + 2] = v.z * v.z;
                sq[i + 3] = v.w * v.w;
            }
            const float total = ordered_sum_wave<32>(sq);
            if (t == 0) root_slot = __builtin_sqrtf(total / (float)k + eps);
        }
    }
    if (NORM && wave == 1) wait_vm_lds<0>();  // wave 1 issued only the norm's weights (PLAIN: x's second half)
    lds_sync();  // the activations (and the root) are in
    if constexpr (NORM) {
        const float4* xs4 = reinterpret_cast<const float4*>(base + L.x);
        const float* ws = reinterpret_cast<const float*>(base + L.nw);
        const float root = PLAIN ? 1.0f : root_slot;  // PLAIN: unused
#pragma unroll
        for (uint32_t b = 0; b < XR; ++b)
        for (uint32_t blk = t >> 3; blk < nb; blk += ONE_THREADS / 8u) {  // uniform across each 8-lane group
            const uint32_t c = blk * 32u + (t & 7u) * 4u;
            const float4 xq = xs4[b * (xrow / 16u) + 8u * blk + (((t & 7u) + (blk >> 1)) & 7u)];  // piece t % 8 of group blk
            float v[4] = {xq.x, xq.y, xq.z, xq.w};
            if constexpr (!PLAIN) {
                const float4 wq = *reinterpret_cast<const float4*>(ws + c);
                const float wj[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float q = v[i] / root;
                    v[i] = q * wj[i];
                }
            }
            const Q8Quad q = quantize_quad(v[0], v[1], v[2], v[3]);
            // byte o of pair blk / 2, in the rotated layout of the staged rows
            const uint32_t pj = blk >> 1, o = (blk & 1u) * 32u + (t & 7u) * 4u;
            const uint32_t ob = b * L.arow;  // row b's block of quantised values and tables
            *reinterpret_cast<uint32_t*>(aq + ob + 16u * (4u * pj + (((o >> 4) + (pj >> 2)) & 3u)) + (o & 15u)) =
                q.packed;
            if ((t & 7u) == 0) {
                reinterpret_cast<float*>(base + L.scales + ob)[blk] = q.scale;
                reinterpret_cast<float*>(base + L.sums + ob)[blk] = q.sum;
                reinterpret_cast<int32_t*>(base + L.totals + ob)[blk] = q.total;
            }
        }
    }
    wait_vm_lds<0>();  // this wave's weights
    lds_sync();

    // This thread's pair of the row (j = t % np: whole rows of pairs per pass).
    const uint32_t j = t % np, rpass = ONE_THREADS / np;
    uint32_t a[XR][16];
    float sx0[XR], sx1[XR], mx0[XR], mx1[XR];
    int e0[XR], e1[XR];
#pragma unroll
    for (uint32_t b = 0; b < XR; ++b) {
        const uint32_t ob = b * L.arow;
        const uint4* q4 = reinterpret_cast<const uint4*>(aq + ob) + 4u * j;  // the pair's pieces, rotated by j / 4
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint4 v = q4[(i + (j >> 2)) & 3u];
            a[b][4 * i] = v.x, a[b][4 * i + 1] = v.y, a[b][4 * i + 2] = v.z, a[b][4 * i + 3] = v.w;
        }
        const float* bsc = reinterpret_cast<const float*>(base + L.scales + ob);
        sx0[b] = bsc[2u * j], sx1[b] = bsc[2u * j + 1u];
        e0[b] = 0, e1[b] = 0, mx0[b] = 0.0f, mx1[b] = 0.0f;
        if constexpr (KIND == 1) {
            const int32_t* bt = reinterpret_cast<const int32_t*>(base + L.totals + ob);
            e0[b] = -8 * bt[2u * j], e1[b] = -8 * bt[2u * j + 1u];
        }
        if constexpr (KIND == 2) {
            const float* bs = reinterpret_cast<const float*>(base + L.sums + ob);
            mx0[b] = bs[2u * j], mx1[b] = bs[2u * j + 1u];
        }
    }
    float* part = reinterpret_cast<float*>(base + L.part);
    // up to UNITS rows' pairs read from LDS together, then their
    // contributions (one LDS latency a batch rather than a row)
    constexpr uint32_t UNITS = 4;
    for (uint32_t r0 = t / np; r0 < rows; r0 += UNITS * rpass) {
        uint32_t u[UNITS][PW];
#pragma unroll
        for (uint32_t q = 0; q < UNITS; ++q) {
            const uint32_t r = min(r0 + q * rpass, rows - 1u);
            const uint8_t* rp = GLU ? (r < h ? base + L.w + r * row_bytes : base + L.w2 + (r - h) * row_bytes)
                                    : base + L.w + r * row_bytes;
            const uint32_t* pw = reinterpret_cast<const uint32_t*>(rp + j * (PW * 4u));
#pragma unroll
            for (uint32_t i = 0; i < PW; ++i) u[q][i] = pw[i];
        }
#pragma unroll
        for (uint32_t q = 0; q < UNITS; ++q) {
            const uint32_t r = r0 + q * rpass;
            if (r < rows) {
#pragma unroll
                for (uint32_t b = 0; b < XR; ++b) {
                    float c0, c1;
                    Pair<KIND>::contribute(u[q], a[b], sx0[b], sx1[b], e0[b], e1[b], mx0[b], mx1[b], c0, c1);
                    *(float2*)(part + (size_t)(b * tr + r) * stride + 2u * j) = make_float2(c0, c1);
                }
            }
        }
    }
    lds_sync();
    float* outs = reinterpret_cast<float*>(base + L.outs);
    for (uint32_t ob = t; ob < XR * rows; ob += ONE_THREADS) {
        // output o of activation row b: its contributions in block order,
        // read 64 at a time into registers before they are added (an LDS
        // read's latency once a batch)
        const uint32_t b = XR == 2 && ob >= rows ? 1u : 0u, o = ob - b * rows;
        const float* c = part + (size_t)(b * tr + o) * stride;
        float sum = 0.0f;
        uint32_t i = 0;
        if (tree) {
            Fold4 u;
            for (; i + 64u <= nb; i += 64u) {
                float4 v[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) v[q] = *(const float4*)(c + i + 4u * q);
#pragma unroll
                for (int q = 0; q < 16; ++q) u.add4(v[q].x, v[q].y, v[q].z, v[q].w);
            }
            for (; i + 4 <= nb; i += 4) {
                const float4 v = *(const float4*)(c + i);
                u.add4(v.x, v.y, v.z, v.w);
            }
            for (; i < nb; ++i) u.s0 += c[i];
            sum = u.total();
        } else {
            for (; i + 64u <= nb; i += 64u) {
                float4 v[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) v[q] = *(const float4*)(c + i + 4u * q);
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    sum += v[q].x;
                    sum += v[q].y;
                    sum += v[q].z;
                    sum += v[q].w;
                }
            }
            for (; i + 4 <= nb; i += 4) {
                const float4 v = *(const float4*)(c + i);
                sum += v.x;
                sum += v.y;
                sum += v.z;
                sum += v.w;
            }
            for (; i < nb; ++i) sum += c[i];
        }
        if constexpr (GLU) {
            outs[o] = sum;
        } else {
            const uint32_t row = row0 + o;
            dst[(size_t)b * n + row] = bias ? sum + bias[row] : sum;
        }
    }
    if constexpr (GLU) {
        // SwiGLU one output a thread (the tile's h outputs), then the
        // quantiser, 8 lanes a block of 32
        lds_sync();
        float* act_out = outs + tr;
        for (uint32_t o = t; o < h; o += ONE_THREADS) act_out[o] = swiglu_value(outs[o], outs[h + o]);
        lds_sync();
        const uint32_t hb = h >> 5, sub = t & 7u;
        for (uint32_t g = t >> 3; g < hb; g += ONE_THREADS / 8u) {
            const float4 v4 = *reinterpret_cast<const float4*>(act_out + g * 32u + sub * 4u);
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
            const Q8Quad q = quantize_quad(v[0], v[1], v[2], v[3]);
            const uint32_t col = g0 + g * 32u + sub * 4u;
            *(uint32_t*)((int8_t*)glu.qs + col) = q.packed;
            if (sub == 0) {
                const size_t at = (g0 >> 5) + g;
                ((float*)glu.scales)[at] = q.scale;
                ((float*)glu.sums)[at] = q.sum;
                ((int32_t*)glu.totals)[at] = q.total;
            }
        }
    }
}

// ------------------------------------------- lanes, one row, fused quantise

// Steps of weight loads issued together per thread (a batch of D pairs),
// by kind: Q8_0 pairs are 17 dwords, Q4_0 9, Q4_1 10.
template <int KIND>
struct Depth {
    static constexpr uint32_t D = KIND == 0 ? 2 : 3;
};

// x · wᵀ for ONE activation row, quantised inside the workgroup: the
// activations are quantised once per workgroup into LDS (8 lanes a block),
// while the first steps of weight loads are already in flight; then the
// lanes scheme of k_matvec: thread t takes pair j = t % np of row t / np of
// each step of rpi = 256/np rows, its two contributions go to
// part[row][block], and thread r adds row r's contributions in block order.
// Weight loads are issued D steps at a time.
//
// LDS: k bytes of int8 values, nb scales, nb extras (Q4_0: -8·Σq; Q4_1:
// F16(d·Σq)), then tr × stride floats of contributions.
// Per-thread geometry of one tile of a one-row product. Thread t takes pair
// j = t % np of row group member rsub = t / np; threads past the last row
// group (rsub >= rpi) shadow the last member so that every load stays in
// bounds, and store nothing. Step s of the tile covers row group
// s * tiles + tile (rpi rows): at any moment all workgroups of a product
// read one compact window of rows.
struct TileGeo {
    uint32_t nb, np, rpi, j, rsub, load_rsub, steps, group_stride, row0;
    bool lane_on;
};

__device__ __forceinline__ TileGeo tile_geo(const RowProduct& p, uint32_t tile) {
    TileGeo g;
    const uint32_t t = threadIdx.x;
    g.nb = p.k >> 5;
    g.np = g.nb >> 1;
    g.rpi = 256u / g.np;
    g.j = t % g.np;
    g.rsub = t / g.np;
    g.lane_on = g.rsub < g.rpi;
    g.load_rsub = g.lane_on ? g.rsub : g.rpi - 1u;
    g.steps = p.tr / g.rpi;
    g.group_stride = p.tiles * g.rpi;
    g.row0 = tile * g.rpi;
    return g;
}

// Loads steps s0 ... s0 + D - 1 of a tile into u. Every thread loads -- a
// step past the tile's last, or a row past the product's last, reads the
// last one again -- so the loads are straight-line code and the compiler's
// wait counts stay exact (loads complete in issue order).
// With `idle` (a workgroup with no next tile: p and g are then this tile's),
// every load reads this tile's last step again, fetched just before and
// still in cache: the same loads are issued, none reaches HBM.
template <int KIND, uint32_t D>
__device__ __forceinline__ void load_steps(const RowProduct& p, const TileGeo& g, uint32_t s0,
                                           uint32_t (&u)[D][Fmt<KIND>::PW], bool idle = false) {
    constexpr uint32_t PW = Fmt<KIND>::PW;
    const uint32_t* wp = (const uint32_t*)p.w + (size_t)g.j * PW;
    const size_t row_words = (size_t)g.np * PW;
#pragma unroll
    for (uint32_t d = 0; d < D; ++d) {
        const uint32_t s = idle ? g.steps - 1u : min(s0 + d, g.steps - 1u);
        const uint32_t row = min(g.row0 + s * g.group_stride + g.load_rsub, p.n - 1u);
        load_pair<KIND>(wp + (size_t)row * row_words, u[d]);
    }
}

// The pair's activations, read from LDS.
struct PairActs {
    uint32_t a[16];
    float sx0, sx1, mx0, mx1;
    int e0, e1;
};

__device__ __forceinline__ void read_acts(const uint8_t* act, uint32_t k, uint32_t j, PairActs& v) {
    const uint32_t nb = k >> 5;
    const u32x4* q = (const u32x4*)(act + (size_t)j * 64u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 w = q[i];
        v.a[4 * i] = w.x, v.a[4 * i + 1] = w.y, v.a[4 * i + 2] = w.z, v.a[4 * i + 3] = w.w;
    }
    const float* lsc = (const float*)(act + k);
    const int32_t* lex = (const int32_t*)(lsc + nb);
    v.sx0 = lsc[2u * j], v.sx1 = lsc[2u * j + 1u];
    v.e0 = lex[2u * j], v.e1 = lex[2u * j + 1u];
    v.mx0 = __int_as_float(v.e0), v.mx1 = __int_as_float(v.e1);
}

// The contributions of steps s0 ... s0 + D - 1 (weights in u) to LDS
// part[row of the tile][block]. Every thread computes and stores, without a
// branch: a thread with no real row (an idle lane, or a step past the
// tile's last) stores into the spare row past the tile's, which is never
// folded; rows past the product's last are never folded either.
template <int KIND, uint32_t D>
__device__ __forceinline__ void compute_steps(const RowProduct& p, const TileGeo& g, uint32_t s0,
                                              const uint32_t (&u)[D][Fmt<KIND>::PW], const PairActs& v,
                                              float* part) {
#pragma unroll
    for (uint32_t d = 0; d < D; ++d) {
        const uint32_t s = s0 + d;
        float c0, c1;
        Pair<KIND>::contribute(u[d], v.a, v.sx0, v.sx1, v.e0, v.e1, v.mx0, v.mx1, c0, c1);
        const uint32_t slot = (g.lane_on && s < g.steps) ? s * g.rpi + g.rsub : p.tr;
        *(float2*)(part + (size_t)slot * p.stride + 2u * g.j) = make_float2(c0, c1);
    }
}

// Adds each row of a tile's contributions in block order -- the host's order
// -- and writes it plus its bias, already loaded (thread r takes row r).
template <bool tree>
__device__ __forceinline__ void fold_tile(const float* part, const RowProduct& p, const TileGeo& g, float bias) {
    const uint32_t r = threadIdx.x;
    if (r >= p.tr) return;
    const uint32_t row = g.row0 + (r / g.rpi) * g.group_stride + r % g.rpi;
    if (row >= p.n) return;
    const float* c = part + (size_t)r * p.stride;
    float sum = 0.0f;
    uint32_t i = 0;
    if (tree) {
        Fold4 u;
        for (; i + 4 <= g.nb; i += 4) {
            const float4 v = *(const float4*)(c + i);
            u.add4(v.x, v.y, v.z, v.w);
        }
        for (; i < g.nb; ++i) u.s0 += c[i];
        sum = u.total();
    } else {
        for (; i + 4 <= g.nb; i += 4) {
            const float4 v = *(const float4*)(c + i);
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
        }
        for (; i < g.nb; ++i) sum += c[i];
    }
    *(__attribute__((address_space(1))) float*)(p.dst + row) = p.bias ? sum + bias : sum;
}

// The bias of the row thread r folds (0 when there is none). Every thread
// loads -- with no bias, or no row, from a valid stand-in address -- so the
// load is straight-line code.
__device__ __forceinline__ float load_bias(const RowProduct& p, const TileGeo& g) {
    const uint32_t r = min((uint32_t)threadIdx.x, p.tr - 1u);
    const uint32_t row = min(g.row0 + (r / g.rpi) * g.group_stride + r % g.rpi, p.n - 1u);
    const float v = *global(p.bias ? p.bias + row : p.x);
    return p.bias ? v : 0.0f;
}

// The activations of the first XP quantise passes (32 blocks a pass, 8 lanes
// a block), loaded ahead of a product's weights.
constexpr uint32_t XP = 2;

__device__ __forceinline__ void load_x(const float* __restrict__ x, uint32_t k, float4 (&xv)[XP]) {
    const uint32_t t = threadIdx.x;
    const uint32_t nb = k >> 5;
    const bool vec = ((uintptr_t)x & 15u) == 0;
#pragma unroll
    for (uint32_t p = 0; p < XP; ++p) {
        const uint32_t g = min(p * 32u + (t >> 3), nb - 1u);
        xv[p] = load_f4(x + g * 32u + (t & 7u) * 4u, vec);
    }
}

// The RMSNorm of four values: x / root · w, the host's order.
__device__ __forceinline__ float4 normalise4(float4 v, float root, float4 w) {
    return make_float4(v.x / root * w.x, v.y / root * w.y, v.z / root * w.z, v.w / root * w.w);
}

// Quantises activation row x (k values) into LDS at act; the first XP
// passes come from xv. With norm, the row quantised is x / root · norm
// (an RMSNorm whose root the caller has). The caller synchronises before
// reading it.
template <int KIND>
__device__ __forceinline__ void quantise_into(uint8_t* act, const float* __restrict__ x, uint32_t k,
                                              const float4 (&xv)[XP], float root = 1.0f,
                                              const float* __restrict__ norm = nullptr) {
    const uint32_t t = threadIdx.x;
    const uint32_t nb = k >> 5;
    int8_t* lqs = (int8_t*)act;
    float* lsc = (float*)(act + k);
    int32_t* lex = (int32_t*)(lsc + nb);
    const bool vec = ((uintptr_t)x & 15u) == 0, wvec = ((uintptr_t)norm & 15u) == 0;
    for (uint32_t pass = 0; pass * 32u < nb; ++pass) {
        const uint32_t g = pass * 32u + (t >> 3), sub = t & 7u;
        if (g < nb) {
            float4 v;
            if (pass < XP) {
                v = pass == 0 ? xv[0] : xv[1];
            } else {
                v = load_f4(x + g * 32u + sub * 4u, vec);
            }
            if (norm) v = normalise4(v, root, load_f4(norm + g * 32u + sub * 4u, wvec));
            const Q8Quad q = quantize_quad(v.x, v.y, v.z, v.w);
            *(uint32_t*)(lqs + g * 32u + sub * 4u) = q.packed;
            if (sub == 0) {
                lsc[g] = q.scale;
                lex[g] = KIND == 1 ? -8 * q.total : __float_as_int(q.sum);
            }
        }
    }
}

// The product of a tile, read with scalar loads (the index is uniform).
__device__ __forceinline__ uint32_t owner_of(const uint32_t* __restrict__ owner, uint32_t tile) {
    return __builtin_amdgcn_readfirstlane(*global(owner + tile));
}

// One-row products, persistent: each workgroup walks tiles blockIdx.x,
// blockIdx.x + gridDim.x, ... of all `total` tiles (tile t belongs to
// product owner[t] of `table`; with no table, to `single`). A product's
// activations are quantised into LDS when its first tile on this workgroup
// comes up. Weights stream in batches of D steps, two batches in flight:
// batch B loads while batch A computes and the reverse; the last batch of a
// tile loads the next tile's first steps (and, for a new product, its
// activations and biases) ahead of this tile's fold. LDS: act_bytes for
// activations, then the contributions. Every workgroup leaves after its last
// tile; all loop bounds are uniform over the workgroup.
template <int KIND, uint32_t D, bool TREE>
__device__ __forceinline__ void matvec_rows(const RowProduct* __restrict__ table, const uint32_t* __restrict__ owner,
                                            const RowProduct& single, uint32_t total, uint32_t act_bytes) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr uint32_t PW = Fmt<KIND>::PW;
    uint8_t* act = smem;
    float* part = (float*)(smem + act_bytes);
    const uint32_t G = gridDim.x;
    uint32_t tile = blockIdx.x;
    if (tile >= total) return;

    uint32_t pi = table ? owner_of(owner, tile) : 0u;
    RowProduct p = table ? table[pi] : single;
    TileGeo g = tile_geo(p, tile - p.first);
    float4 xv[XP];
    load_x(p.x, p.k, xv);
    float bias = load_bias(p, g);
    uint32_t ua[D][PW], ub[D][PW];
    load_steps<KIND, D>(p, g, 0, ua);
    uint32_t have = 0xffffffffu;

    while (true) {
        if (pi != have) {
            quantise_into<KIND>(act, p.x, p.k, xv);
            __syncthreads();
            have = pi;
        }
        PairActs v;
        read_acts(act, p.k, g.j, v);

        // The next tile, found with scalar loads before any weight load:
        // with no next tile, the stand-in is this one (its loads are
        // issued again and unused), so every path issues the same loads.
        const uint32_t next = tile + G;
        const bool more = next < total;
        uint32_t npi = pi;
        if (table && more) npi = owner_of(owner, next);
        const RowProduct q = (table && npi != pi) ? table[npi] : p;
        const TileGeo h = more ? tile_geo(q, next - q.first) : g;

        // Whole rounds: batch B loads while A computes, then A while B.
        uint32_t s0 = 0;
        for (; s0 + 2u * D < g.steps; s0 += 2u * D) {
            load_steps<KIND, D>(p, g, s0 + D, ub);
            compute_steps<KIND, D>(p, g, s0, ua, v, part);
            load_steps<KIND, D>(p, g, s0 + 2u * D, ua);
            compute_steps<KIND, D>(p, g, s0 + D, ub, v, part);
        }
        // The last round: its second batch, then the next tile's first
        // loads (activations, biases, weights) go out before this tile's
        // fold.
        load_steps<KIND, D>(p, g, s0 + D, ub);
        compute_steps<KIND, D>(p, g, s0, ua, v, part);
        load_x(q.x, q.k, xv);
        const float nbias = load_bias(q, h);
        load_steps<KIND, D>(q, h, 0, ua, !more);
        compute_steps<KIND, D>(p, g, s0 + D, ub, v, part);

        __syncthreads();  // every contribution of this tile is in `part`
        fold_tile<TREE>(part, p, g, bias);
        if (!more) break;
        __syncthreads();  // the fold has read `part`; `act` may be replaced
        tile = next, pi = npi, p = q, g = h, bias = nbias;
    }
}

template <int KIND, uint32_t D, bool TREE>
__global__ __launch_bounds__(256) void k_matvec_rows(const RowProduct* __restrict__ table,
                                                     const uint32_t* __restrict__ owner, uint32_t total,
                                                     uint32_t act_bytes) {
    const RowProduct none{};
    matvec_rows<KIND, D, TREE>(table, owner, none, total, act_bytes);
}

template <int KIND, uint32_t D, bool TREE>
__global__ __launch_bounds__(256) void k_matvec_row(RowProduct p, uint32_t act_bytes) {
    matvec_rows<KIND, D, TREE>(nullptr, nullptr, p, p.tiles, act_bytes);
}

// ------------------------------------------- one row, streamed through LDS

// x · wᵀ for one activation row per product, for every product of a plan in
// one launch. The plan's weight rows form one sequence of steps (a step is
// the consecutive rows of one product that fit 8 KB, at most one pair of
// blocks per thread); workgroup b takes the steps from bound(b) to
// bound(b + 1), a share set by the planner whatever the products' sizes.
// Weights travel from HBM to LDS by the direct loads of gfx950
// (global_load_lds_dwordx4: 16 bytes a lane, 1 KB a wave; each wave brings
// 2 KB of a step) into a ring of R
// slots, R - 1 steps ahead of the step being computed: no VGPR holds weights
// in flight, and the ring runs on across product boundaries. One workgroup
// barrier per step; before it each wave waits for its own loads of the step
// (a counted s_waitcnt that leaves the later steps' loads in flight). After
// it, the step's slot is complete and is computed (thread t takes pair
// j = t % np of row t / np, as the lanes kernels do), and the previous
// step's contributions are complete and are folded by one thread per row in
// block order -- the host's order. A product's activations are quantised
// into one of two LDS buffers: the range's first two before the loop, from
// x brought in by direct loads ahead of every weight load; a later one when
// its turn comes. The loop keeps its scalar work small: the scalar unit is
// shared by every wave of a compute unit.

constexpr uint32_t STREAM_STEP = 8192;  // bytes of weights a step's loads bring

// The per-step workgroup barrier, after this wave's operations are done as
// wait_vm_lds<N> says. The empty asm statements keep the compiler from
// moving memory operations across it (s_barrier alone does not order memory
// for the compiler; __syncthreads() would wait for every load in flight).
template <uint32_t N>
__device__ __forceinline__ void step_barrier() {
    asm volatile("" ::: "memory");
    wait_vm_lds<N>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A workgroup barrier after this wave's LDS operations only; its direct
// loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() { step_barrier<63>(); }

// step_barrier<A·PS> for a runtime A in [0, AMAX]: the steps issued after the
// one about to be computed, PS operations each.
template <uint32_t PS, uint32_t AMAX>
__device__ __forceinline__ void step_barrier_ahead(uint32_t ahead) {
    if constexpr (AMAX == 0) {
        step_barrier<0>();
    } else {
        if (ahead >= AMAX)
            step_barrier<AMAX * PS>();
        else
            step_barrier_ahead<PS, AMAX - 1>(ahead);
    }
}

// Brings x (k floats) into LDS at `to` by direct loads, 1 KB per wave load
// (x 16-byte aligned and a whole number of 16-byte pieces) or 256 bytes
// (otherwise); lanes past the end read the last piece again and write it
// past the end (so a piece is never partial: it would come from the wrong
// place).
__device__ __forceinline__ void issue_x(const float* x, uint32_t k, uint32_t to, uint32_t wave) {
    const uint32_t lane = threadIdx.x & 63u;
    const uintptr_t base = (uintptr_t)x;
    if ((base & 15u) == 0 && k % 4u == 0) {
        const uintptr_t last = base + (uintptr_t)k * 4u - 16u;
        for (uint32_t q = wave; q * 1024u < k * 4u; q += 4u) {
            uintptr_t a = base + q * 1024u + lane * 16u;
            a = a < last ? a : last;
            lds_load16((const void*)a, to + q * 1024u);
        }
    } else {
        const uintptr_t last = base + (uintptr_t)k * 4u - 4u;
        for (uint32_t q = wave; q * 256u < k * 4u; q += 4u) {
            uintptr_t a = base + q * 256u + lane * 4u;
            a = a < last ? a : last;
            lds_load4((const void*)a, to + q * 256u);
        }
    }
}

// quantise_into with x read from LDS (xs, k floats); the norm's weights,
// if any, from global memory.
template <int KIND>
__device__ __forceinline__ void quantise_lds(uint8_t* act, const float* xs, uint32_t k, float root = 1.0f,
                                             const float* __restrict__ norm = nullptr) {
    const uint32_t t = threadIdx.x;
    const uint32_t nb = k >> 5;
    int8_t* lqs = (int8_t*)act;
    float* lsc = (float*)(act + k);
    int32_t* lex = (int32_t*)(lsc + nb);
    for (uint32_t pass = 0; pass * 32u < nb; ++pass) {
        const uint32_t g = pass * 32u + (t >> 3), sub = t & 7u;
        if (g < nb) {
            float4 v = *(const float4*)(xs + g * 32u + sub * 4u);
            if (norm) v = normalise4(v, root, load_f4(norm + g * 32u + sub * 4u, ((uintptr_t)norm & 15u) == 0));
            const Q8Quad q = quantize_quad(v.x, v.y, v.z, v.w);
            *(uint32_t*)(lqs + g * 32u + sub * 4u) = q.packed;
            if (sub == 0) {
                lsc[g] = q.scale;
                lex[g] = KIND == 1 ? -8 * q.total : __float_as_int(q.sum);
            }
        }
    }
}

// Bytes of a staged part of a quantised activation row: whole 1 KB direct loads.
__host__ __device__ constexpr uint32_t stage_part(uint32_t bytes) { return (bytes + 1023u) & ~1023u; }

// A product's activations quantised beforehand (int8 values, scales, block
// extras), staged at st as three parts of stage_part() bytes, into LDS at
// act in the layout quantise_into writes (for Q4_0, -8 · total).
template <int KIND>
__device__ __forceinline__ void unpack_lds(uint8_t* act, const uint8_t* st, uint32_t k) {
    const uint32_t t = threadIdx.x, nb = k >> 5;
    const uint32_t qb = stage_part(k), sb = stage_part(4u * nb);
    for (uint32_t i = t; i < k / 4u; i += 256u) ((uint32_t*)act)[i] = ((const uint32_t*)st)[i];
    float* lsc = (float*)(act + k);
    int32_t* lex = (int32_t*)(lsc + nb);
    const float* ssc = (const float*)(st + qb);
    const int32_t* sex = (const int32_t*)(st + qb + sb);
    for (uint32_t g = t; g < nb; g += 256u) {
        lsc[g] = ssc[g];
        lex[g] = KIND == 1 ? -8 * sex[g] : KIND == 2 ? sex[g] : 0;
    }
}

// A product's activations into LDS at act from global memory, whatever its
// input mode (for products not staged before the loop). free is LDS that
// nothing else uses (one float, for the RMSNorm's root). Every thread calls
// it; the caller synchronises before reading act.
template <int KIND>
__device__ __forceinline__ void prepare_global(uint8_t* act, const StreamProduct& q, float* free) {
    const uint32_t t = threadIdx.x, k = q.k, nb = k >> 5;
    if (q.mode == STREAM_X_QUANTISED) {
        const uint32_t* qs = (const uint32_t*)q.x;
        const float* sc = q.aux0;
        const int32_t* ex = (const int32_t*)q.aux1;
        for (uint32_t i = t; i < k / 4u; i += 256u) ((uint32_t*)act)[i] = qs[i];
        float* lsc = (float*)(act + k);
        int32_t* lex = (int32_t*)(lsc + nb);
        for (uint32_t g = t; g < nb; g += 256u) {
            lsc[g] = sc[g];
            lex[g] = KIND == 1 ? -8 * ex[g] : KIND == 2 ? ex[g] : 0;
        }
        return;
    }
    float root = 1.0f;
    const float* norm = nullptr;
    if (q.mode == STREAM_X_RMSNORM) {
        if (t == 0) {
            float squares = 0.0f;
            if (((uintptr_t)q.x & 15u) == 0) {
                squares = ordered_sum<true, 4>(q.x, k);
            } else {
                for (uint32_t i = 0; i < k; ++i) squares += q.x[i] * q.x[i];
            }
            free[0] = __builtin_sqrtf(squares / (float)k + q.eps);
        }
        step_barrier<0>();
        root = free[0];
        norm = q.aux0;
    }
    float4 xv[XP];
    load_x(q.x, k, xv);
    quantise_into<KIND>(act, q.x, k, xv, root, norm);
}

// The sum of a row's nb contributions c[0 ... nb-1] (nb even, the same in
// every lane) in block order, from 0. Each batch of 16 is read with all its
// LDS reads issued before the first add, so a batch costs one LDS round
// trip rather than one per four values (the fold is on every step's
// critical path); the last batch reads up to 14 floats past c[nb-1], other
// LDS data of the workgroup, and skips them.
__device__ __forceinline__ float fold_row_unordered(const float* c, uint32_t nb);

template <bool TREE>
__device__ __forceinline__ float fold_row(const float* c, uint32_t nb) {
    if constexpr (TREE) return fold_row_unordered(c, nb);
    float sum = 0.0f;
    for (uint32_t q = 0; q < nb; q += 16u) {
        float4 e[4];
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) e[u] = *(const float4*)(c + q + 4u * u);
        // Every read is needed here: the compiler may not sink them into the
        // branches below (one round trip each).
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) asm volatile("" : "+v"(e[u].x), "+v"(e[u].y), "+v"(e[u].z), "+v"(e[u].w));
        const uint32_t left = nb - q;
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) {
            if (4u * u >= left) break;
            sum += e[u].x;
            sum += e[u].y;
            if (4u * u + 2u >= left) break;
            sum += e[u].z;
            sum += e[u].w;
        }
    }
    return sum;
}

// fold_row's reads with UNORDERED's four running sums.
__device__ __forceinline__ float fold_row_unordered(const float* c, uint32_t nb) {
    Fold4 s;
    for (uint32_t q = 0; q < nb; q += 16u) {
        float4 e[4];
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) e[u] = *(const float4*)(c + q + 4u * u);
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) asm volatile("" : "+v"(e[u].x), "+v"(e[u].y), "+v"(e[u].z), "+v"(e[u].w));
        const uint32_t left = nb - q;
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) {
            if (4u * u >= left) break;
            s.add2(e[u].x, e[u].y);
            if (4u * u + 2u >= left) break;
            s.s2 += e[u].z, s.s3 += e[u].w;
        }
    }
    return s.total();
}

// Per-thread geometry of a product: the thread's row r of a step and pair j,
// its LDS byte offset within a step's weights, its offset (floats) within
// the contributions.
struct StreamLane {
    uint32_t r, j, wofs, pofs;
};

template <int KIND>
__device__ __forceinline__ StreamLane stream_lane(const StreamProduct& P) {
    StreamLane g;
    g.r = threadIdx.x / P.np;
    g.j = threadIdx.x - g.r * P.np;
    g.wofs = g.r * P.row_bytes + g.j * (Fmt<KIND>::PW * 4u);
    g.pofs = g.r * P.stride + 2u * g.j;
    return g;
}

// LDS layout of the streamed kernel: 16 bytes for an RMSNorm's root, biases
// (R + 1 slots of 256 floats, with HB), ring slots 0 ... R-1 of STREAM_STEP
// bytes, contributions (two buffers of part_floats), then from act_offset
// the activations (two buffers of act_bytes; one for a one-product plan). Before the loop, the x of the range's first two products
// (x_floats apart; none when x_floats is 0) is staged from ring slot R-1
// on, over memory first written in the loop.
template <int KIND, uint32_t R, bool HB, bool TREE>
__global__ __launch_bounds__(256) void k_matvec_stream(const StreamProduct* __restrict__ table,
                                                       const StreamStart* __restrict__ starts, uint32_t total,
                                                       uint32_t act_bytes, uint32_t part_floats, uint32_t x_floats,
                                                       uint32_t act_offset) {
    constexpr uint32_t PW = Fmt<KIND>::PW;
    constexpr uint32_t PS = HB ? 3u : 2u;  // vector memory operations a wave issues per step
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t b = blockIdx.x, t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const StreamStart st = starts[b];
    const uint32_t s_begin = st.s_begin, s_end = st.s_end;
    if (s_begin >= s_end) return;
    const uint32_t count = s_end - s_begin;
    float* root_slot = (float*)smem;  // an RMSNorm's root, shared
    float* biases = (float*)(smem + 16u);
    uint8_t* ring = smem + 16u + (HB ? (R + 1u) * 1024u : 0u);
    float* parts = (float*)(ring + R * STREAM_STEP);
    uint8_t* acts = smem + act_offset;
    float* xs = (float*)(ring + (R - 1u) * STREAM_STEP);
    const uint32_t ring_lds = lds_address(ring) + wave * 2048u, bias_lds = lds_address(biases) + wave * 256u;

    // The range's first product (and its second, when both take f32 x) is
    // prepared before the loop, from its activation row brought into LDS by
    // direct loads requested, with the first steps' weights, before the
    // product table is read: x (and the norm's weights in the second slot),
    // or the three parts of a quantised row.
    const uint32_t first_pi = st.first_pi, mode0 = st.mode0;
    const bool two = st.x1 != nullptr;
    const bool staged = x_floats != 0;
    if (staged) {
        const uint32_t to = lds_address(xs);
        if (mode0 == STREAM_X_QUANTISED) {
            const uint32_t qb = stage_part(st.k0);
            issue_x(st.x0, st.k0 / 4u, to, wave);
            issue_x(st.a0, st.k0 / 32u, to + qb, wave);
            if (st.a1) issue_x((const float*)st.a1, st.k0 / 32u, to + qb + stage_part(st.k0 / 8u), wave);
        } else {
            issue_x(st.x0, st.k0, to, wave);
            if (two) issue_x(st.x1, st.k1, to + x_floats * 4u, wave);
        }
    }

    // The issue cursor: the step's first weight byte, steps left in its
    // product, slots; with HB the step's first row and the product's bias
    // (or a stand-in, with ihas 0).
    uint32_t ipi = first_pi;
    uint64_t isrc = st.src, iwlast = st.wlast;
    uint32_t ileft = st.left, istep = st.step_bytes, irows = st.rows, irow = st.row, in = st.n;
    const float* ibias = st.bias;
    uint32_t ihas = st.has;
    uint32_t islot = 0, ibslot = 0, issued = 0;
    const uint32_t lane_bytes = wave * 2048u + lane * 16u;
    auto issue_next = [&]() {
        const uint64_t a0 = isrc & ~(uint64_t)15;
        uint64_t a = a0 + lane_bytes;
        lds_load16_nt((const void*)(a < iwlast ? a : iwlast), ring_lds + islot * STREAM_STEP);
        a += 1024u;
        lds_load16_nt((const void*)(a < iwlast ? a : iwlast), ring_lds + islot * STREAM_STEP + 1024u);
        if constexpr (HB) {
            const uint32_t row = min(irow + wave * 64u + lane, in - 1u);
            lds_load4(ibias + row * ihas, bias_lds + ibslot * 1024u);
            ibslot = ibslot == R ? 0u : ibslot + 1u;
            irow += irows;
        }
        ++issued;
        isrc += istep;
        islot = islot == R - 1u ? 0u : islot + 1u;
        if (--ileft == 0 && issued < count) {
            const StreamProduct& q = table[++ipi];
            isrc = (uint64_t)q.w, iwlast = q.wlast, ileft = q.steps, istep = q.step_bytes, irows = q.rows;
            irow = 0, in = q.n;
            ibias = q.bias ? q.bias : q.x;
            ihas = q.bias ? 1u : 0u;
        }
    };
    // The prologue issues R - 1 steps into slots 0 ... R-2 (the staged x
    // lies past them) and waits for the staged x only. Without staging (x
    // too long for the LDS), x is loaded directly, and the wait for it
    // waits for the prologue's weights too.
    const uint32_t prologue = min(R - 1u, count);
    for (uint32_t s = 0; s < prologue; ++s) issue_next();
    const StreamProduct p0 = table[first_pi];
    const StreamProduct p1 = two ? table[first_pi + 1u] : p0;
    if (staged) {
        step_barrier_ahead<PS, R - 1u>(prologue);  // the staged row is complete
        if (mode0 == STREAM_X_QUANTISED) {
            unpack_lds<KIND>(acts, (const uint8_t*)xs, p0.k);
        } else if (mode0 == STREAM_X_RMSNORM) {
            // The squares in parallel (in place), then Σx² in index order by
            // one lane -- adds only: a wave instruction a value -- while the
            // first weights arrive. x and the norm's weights are then read
            // from global memory, when the prologue's weight loads are in
            // (the compiler waits for every load there).
            for (uint32_t i = t; i < p0.k; i += 256u) xs[i] = xs[i] * xs[i];
            lds_barrier();
            if (t == 0) root_slot[0] = __builtin_sqrtf(ordered_sum<false, 4>(xs, p0.k) / (float)p0.k + p0.eps);
            lds_barrier();
            float4 xv[XP];
            load_x(p0.x, p0.k, xv);
            quantise_into<KIND>(acts, p0.x, p0.k, xv, root_slot[0], p0.aux0);
        } else {
            quantise_lds<KIND>(acts, xs, p0.k);
            if (two) quantise_lds<KIND>(acts + act_bytes, xs + x_floats, p1.k);
        }
    } else {
        prepare_global<KIND>(acts, p0, root_slot);
        if (two) prepare_global<KIND>(acts + act_bytes, p1, root_slot);
    }
    step_barrier_ahead<PS, R - 1u>(prologue);  // the staged x is read; the activations are complete

    // The compute cursor (product cpi, the nth of the range): the step's
    // first weight byte (its offset past 16 bytes is where the slot's data
    // starts), rows left in the product, slot. The fold cursor: the
    // previous step's outputs, rows, product geometry.
    uint32_t cpi = first_pi, nth = 0;
    uint64_t csrc = (uint64_t)p0.w + (uint64_t)(s_begin - p0.first) * p0.step_bytes;
    uint32_t cleft = p0.n - (s_begin - p0.first) * p0.rows, crows = p0.rows, cstep = p0.step_bytes;
    float* cdst = p0.dst + (s_begin - p0.first) * p0.rows;
    uint32_t cnb = 2u * p0.np, cstride = p0.stride, cslot = 0, cbslot = 0;
    bool cbias = p0.bias != nullptr;
    StreamLane g = stream_lane<KIND>(p0);
    PairActs v;
    read_acts(acts, p0.k, g.j, v);
    float* fdst = cdst;
    uint32_t frows = 0, fnb = cnb, fstride = cstride, fbslot = 0;
    bool fbias = cbias;
    const uint32_t prepared = two ? 2u : 1u;  // products prepared before the loop

    for (uint32_t i = 0; i < count; ++i) {
        step_barrier_ahead<PS, R - 2u>(issued - 1u - i);
        if (issued < count) issue_next();
        // The previous step's fold.
        if (t < frows) {
            float sum = fold_row<TREE>(parts + ((i - 1u) & 1u) * part_floats + t * fstride, fnb);
            if (HB && fbias) sum += biases[fbslot * 256u + t];
            *(__attribute__((address_space(1))) float*)(fdst + t) = sum;
        }
        // This step's contributions.
        const uint32_t rows = min(crows, cleft);
        if (g.r < rows) {
            const uint32_t* w = (const uint32_t*)(ring + cslot * STREAM_STEP + ((uint32_t)csrc & 15u) + g.wofs);
            uint32_t u[PW];
#pragma unroll
            for (uint32_t e = 0; e < PW; ++e) u[e] = w[e];
            float c0, c1;
            Pair<KIND>::contribute(u, v.a, v.sx0, v.sx1, v.e0, v.e1, v.mx0, v.mx1, c0, c1);
            *(float2*)(parts + (i & 1u) * part_floats + g.pofs) = make_float2(c0, c1);
        }
        fdst = cdst, frows = rows, fnb = cnb, fstride = cstride, fbias = cbias, fbslot = cbslot;
        cdst += rows, cleft -= rows, csrc += cstep;
        cslot = cslot == R - 1u ? 0u : cslot + 1u;
        if constexpr (HB) cbslot = cbslot == R ? 0u : cbslot + 1u;
        if (cleft == 0 && i + 1u < count) {
            const StreamProduct& q = table[++cpi];
            ++nth;
            csrc = (uint64_t)q.w, cleft = q.n, crows = q.rows, cstep = q.step_bytes, cdst = q.dst;
            cnb = 2u * q.np, cstride = q.stride, cbias = q.bias != nullptr;
            g = stream_lane<KIND>(q);
            if (nth >= prepared) {
                // Into the buffer of the product before last (read before the
                // barrier that began this step).
                prepare_global<KIND>(acts + (nth & 1u) * act_bytes, q, root_slot);
                step_barrier<0>();
            }
            read_acts(acts + (nth & 1u) * act_bytes, q.k, g.j, v);
        }
    }
    step_barrier<0>();
    if (t < frows) {
        float sum = fold_row<TREE>(parts + ((count - 1u) & 1u) * part_floats + t * fstride, fnb);
        if (HB && fbias) sum += biases[fbslot * 256u + t];
        *(__attribute__((address_space(1))) float*)(fdst + t) = sum;
    }
}

// ------------------------------------------------ matrix cores: many rows

// x · wᵀ for many activation rows on the int8 matrix cores. Workgroup tile
// 64 rows (M) x 64 outputs (N), 4 waves of 32 x 32 (2 x 2 MFMA tiles of
// 16 x 16). One v_mfma_i32_16x16x32_i8 spans exactly one block of 32, so
// each block's integer dot product comes out on its own, exact; then every
// output adds that block's contribution, in the host's expression, to its
// running f32 sum -- blocks in order, so the bits are the host's:
//   Q8_0  float(t) * (d * sx)             (t from the MFMA)
//   Q4_0  (float(t) * d) * sx             (t = MFMA(q, y) - 8·Σy: the MFMA
//                                          starts from C = -8·Σy)
//   Q4_1  (d * sx) * float(t) + m * mx
// Per stage (two blocks) the workgroup stages into LDS: the 64 weight rows'
// two blocks as aligned int8 (nibbles unpacked), their scales (and Q4_1
// minimums) as f32, and the 64 activation rows' scales and extras; stages
// are double-buffered so the next stage's loads fly while this one computes.
// MFMA operand layout (16x16x32 i8, checked on the device): lane l holds
// A[l % 16][8 (l / 16) ...] and B[8 (l / 16) ...][l % 16]; the result holds
// rows 4 (l / 16) + i, column l % 16.
constexpr uint32_t MM_TILE = 64;
constexpr uint32_t MM_BROW = 72;  // LDS bytes per weight row (64 values + pad): conflict-free 8-byte reads

typedef int v4i __attribute__((ext_vector_type(4)));

struct MmStage {
    int8_t wq[MM_TILE * MM_BROW];  // [n][2 blocks x 32 values + pad]
    float wd[2][MM_TILE];          // weight d by [block][n]
    float wm[2][MM_TILE];          // weight m (Q4_1) by [block][n]
    float sx[2][MM_TILE];          // activation scale by [block][row]
    float ex[2][MM_TILE];          // Q4_0: -8·Σq as int; Q4_1: F16(d·Σq)
};

// Issues the global loads of stage `pair` (blocks 2·pair, 2·pair + 1):
// threads 0-63 one weight row's pair, 64-191 one activation scale, 128-255
// one extra. Returns them in registers for stage_store.
template <int KIND>
struct MmLoad {
    uint32_t u[Fmt<KIND>::PW];
    float sx;
    int32_t ex;
};

template <int KIND>
__device__ __forceinline__ void stage_load(const uint8_t* __restrict__ w, const Activations& act, uint32_t n,
                                           uint32_t m, uint32_t nb, uint32_t n0, uint32_t m0, uint32_t pair,
                                           MmLoad<KIND>& L) {
    const uint32_t t = threadIdx.x;
    constexpr uint32_t PW = Fmt<KIND>::PW;
    if (t < MM_TILE) {
        const uint32_t row = min(n0 + t, n - 1u);
        const uint32_t* p = (const uint32_t*)w + ((size_t)row * (nb >> 1) + pair) * PW;
        load_pair<KIND>(p, L.u);
    }
    if (t >= 64u && t < 192u) {
        const uint32_t i = t - 64u, r = min(m0 + (i >> 1), m - 1u), b = 2u * pair + (i & 1u);
        L.sx = *global(act.scales + (size_t)r * nb + b);
    }
    if (t >= 128u) {
        const uint32_t i = t - 128u, r = min(m0 + (i >> 1), m - 1u), b = 2u * pair + (i & 1u);
        if constexpr (KIND == 1) L.ex = -8 * *global(act.totals + (size_t)r * nb + b);
        if constexpr (KIND == 2) L.ex = __float_as_int(*global(act.sums + (size_t)r * nb + b));
    }
}

template <int KIND>
__device__ __forceinline__ void stage_store(MmStage& S, const MmLoad<KIND>& L) {
    const uint32_t t = threadIdx.x;
    if (t < MM_TILE) {
        uint32_t* q = (uint32_t*)(S.wq + t * MM_BROW);
        const uint32_t* u = L.u;
        if constexpr (KIND == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = funnel(u[i + 1], u[i], 2);
#pragma unroll
            for (int i = 0; i < 8; ++i) q[8 + i] = u[9 + i];
            S.wd[0][t] = half_value(u[0] & 0xffffu);
            S.wd[1][t] = half_value(u[8] >> 16);
        } else if constexpr (KIND == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w0 = funnel(u[i + 1], u[i], 2), w1 = u[5 + i];
                q[i] = w0 & 0x0f0f0f0fu, q[4 + i] = (w0 >> 4) & 0x0f0f0f0fu;
                q[8 + i] = w1 & 0x0f0f0f0fu, q[12 + i] = (w1 >> 4) & 0x0f0f0f0fu;
            }
            S.wd[0][t] = half_value(u[0] & 0xffffu);
            S.wd[1][t] = half_value(u[4] >> 16);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q[i] = u[1 + i] & 0x0f0f0f0fu, q[4 + i] = (u[1 + i] >> 4) & 0x0f0f0f0fu;
                q[8 + i] = u[6 + i] & 0x0f0f0f0fu, q[12 + i] = (u[6 + i] >> 4) & 0x0f0f0f0fu;
            }
            S.wd[0][t] = half_value(u[0] & 0xffffu);
            S.wm[0][t] = half_value(u[0] >> 16);
            S.wd[1][t] = half_value(u[5] & 0xffffu);
            S.wm[1][t] = half_value(u[5] >> 16);
        }
    }
    if (t >= 64u && t < 192u) {
        const uint32_t i = t - 64u;
        S.sx[i & 1u][i >> 1] = L.sx;
    }
    if (t >= 128u) {
        const uint32_t i = t - 128u;
        ((int32_t*)S.ex[i & 1u])[i >> 1] = L.ex;
    }
}

template <int KIND>
__global__ __launch_bounds__(256) void k_matmul_mfma(const uint8_t* __restrict__ w, Activations act,
                                                     float* __restrict__ dst, const float* __restrict__ bias,
                                                     uint32_t m, uint32_t n, uint32_t k) {
    __shared__ MmStage stage[2];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t nb = k >> 5, pairs = nb >> 1;
    const uint32_t n0 = blockIdx.x * MM_TILE, m0 = blockIdx.y * MM_TILE;
    const uint32_t wm0 = (wave >> 1) * 32u, wn0 = (wave & 1u) * 32u;  // this wave's 32 x 32 within the tile
    const uint32_t lr = lane & 15u, lq = lane >> 4;                    // operand row/column, k quarter

    float acc[2][2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[a][b][i] = 0.0f;

    // A operand rows (activation rows), clamped in bounds.
    const int8_t* arow[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) arow[a] = act.qs + (size_t)min(m0 + wm0 + 16u * a + lr, m - 1u) * k + lq * 8u;

    MmLoad<KIND> L;
    stage_load<KIND>(w, act, n, m, nb, n0, m0, 0, L);
    stage_store<KIND>(stage[0], L);
    // This wave's activation operands of a pair of blocks ([block][a]), one
    // pair ahead of the MFMAs that take them (the last pair loads itself
    // again), so their latency hides behind a pair's work.
    long avc[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int a = 0; a < 2; ++a) avc[h][a] = *(const __attribute__((address_space(1))) long*)(arow[a] + h * 32u);
    __syncthreads();

    for (uint32_t pair = 0; pair < pairs; ++pair) {
        const MmStage& S = stage[pair & 1u];
        const bool more = pair + 1u < pairs;
        if (more) stage_load<KIND>(w, act, n, m, nb, n0, m0, pair + 1u, L);
        long avn[2][2];
        const uint32_t next = min(pair + 1u, pairs - 1u);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int a = 0; a < 2; ++a)
                avn[h][a] = *(const __attribute__((address_space(1))) long*)(arow[a] + (2u * next + h) * 32u);
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) {
            const long* av = avc[h];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const uint32_t col = wn0 + 16u * b + lr;
                const long bv = *(const long*)(S.wq + col * MM_BROW + h * 32u + lq * 8u);
                const float d = S.wd[h][wn0 + 16u * b + lr];
                float wmin = 0.0f;
                if constexpr (KIND == 2) wmin = S.wm[h][wn0 + 16u * b + lr];
#pragma unroll
                for (int a = 0; a < 2; ++a) {
                    const uint32_t r0 = wm0 + 16u * a + 4u * lq;  // this lane's 4 rows within the tile
                    v4i c = {0, 0, 0, 0};
                    if constexpr (KIND == 1) {
                        const int* e = (const int*)S.ex[h];
                        c = v4i{e[r0], e[r0 + 1], e[r0 + 2], e[r0 + 3]};
                    }
                    const v4i tv = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[a], bv, c, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float sx = S.sx[h][r0 + i];
                        float contribution;
                        if constexpr (KIND == 0) {
                            const float s = d * sx;
                            contribution = (float)tv[i] * s;
                        } else if constexpr (KIND == 1) {
                            const float p = (float)tv[i] * d;
                            contribution = p * sx;
                        } else {
                            const float s = d * sx;
                            const float f = s * (float)tv[i];
                            const float g = wmin * S.ex[h][r0 + i];
                            contribution = f + g;
                        }
                        acc[a][b][i] += contribution;
                    }
                }
            }
        }
        if (more) stage_store<KIND>(stage[(pair + 1u) & 1u], L);
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int a = 0; a < 2; ++a) avc[h][a] = avn[h][a];
    }

#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint32_t col = n0 + wn0 + 16u * b + lr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t row = m0 + wm0 + 16u * a + 4u * lq + i;
                if (row < m && col < n) dst[(size_t)row * n + col] = bias ? acc[a][b][i] + bias[col] : acc[a][b][i];
            }
        }
}

// ------------------------------------------ matrix cores: stages of 8 blocks

// x · wᵀ for many activation rows on the int8 matrix cores, for k a multiple
// of 256 and 16-byte aligned weights and activation parts. Workgroup tile 64
// activation rows x 64 outputs, 4 waves (one a SIMD), each a 32 x 32 tile:
// per block, one v_mfma_i32_32x32x32_i8 gives the tile's 1024 integer dot
// products of that block alone, exact (a lane holds 16 outputs: column
// lane % 32, rows 8 (i / 4) + 4 (lane / 32) + i % 4), and every output adds
// the block's contribution, in the host's expression, to its running f32 sum
// in block order (the expressions of k_matmul_mfma above). The factors
// those expressions take per output come from f16 MFMAs over operands whose
// k slots other than one hold zeros: d·sx and m·mx (products of two halves,
// exact in f32 -- the host's products) for Q8_0 and Q4_1, and d and sx
// themselves (times 1) for Q4_0. Each lane thus folds 16 outputs at three
// VALU operations each.
//
// The k axis goes in stages of 8 blocks, one workgroup barrier a stage, every
// byte brought by direct loads (global_load_lds_dwordx4: 16 bytes a lane, no
// VGPR holds data in flight, each wave waits for its own loads by count):
// the 64 weight rows' 8 blocks as they lie in memory, with the activation
// rows' scales (and Q4_1 sums), three stages ahead; the 64 activation rows'
// 256 int8 values (272 bytes apart in LDS), two stages ahead. While stage s
// is computed, the workgroup repacks the weights of stage s + 1: each
// block's 32 values 16-byte aligned (Q4 nibbles as bytes, Q4_0 less 8),
// rows 272 bytes apart, so that the 8 lanes the LDS serves together read 16
// bytes each from different banks; scales as f16 MFMA operands. A
// workgroup's tile comes from its id so that the 8 activation tiles of one
// weight tile run on one XCD (ids go round-robin over the 8 XCDs): the
// weight tile comes from HBM once, into that XCD's L2.
//
// FUSED (TMH_MODE_UNORDERED, measurement only) adds each contribution with
// one fused multiply-add instead of the host's separately rounded product
// and sum: the same work with one VALU operation fewer an output and block,
// which prices the exact fold; its results may differ in the last bits.
constexpr uint32_t MX_TILE = 64;
constexpr uint32_t MX_STAGE = 8;
constexpr uint32_t MX_THREADS = 512;  // 4 compute waves (one a SIMD) and 4 producer waves
constexpr uint32_t MX_COMPUTE = 4;
constexpr uint32_t MX_ROW = 272;   // LDS bytes per activation row and packed weight row (256 + a 16-byte pad)
constexpr uint32_t MX_TAB_ROW = MX_TILE + 1u;  // a table's entries per block: 64 rows and a zero

template <int KIND>
struct Mx {
    static constexpr uint32_t RB = MX_STAGE * Fmt<KIND>::BB;  // a weight row's bytes in a stage
    static constexpr uint32_t RC = RB / 16u;
    // Raw weight group (three buffers): weights [64][RB], scales [64][8]
    // f32, Q4_1 sums [64][8] f32.
    static constexpr uint32_t W_S = MX_TILE * RB;
    static constexpr uint32_t W_E = W_S + MX_TILE * MX_STAGE * 4u;
    static constexpr uint32_t W_BYTES = W_E + (KIND == 2 ? MX_TILE * MX_STAGE * 4u : 0u);
    static constexpr uint32_t W_LOADS = W_BYTES / 1024u;
    // Raw activations (three buffers): [64][MX_ROW].
    static constexpr uint32_t A_BYTES = MX_TILE * MX_ROW;
    static constexpr uint32_t A_LOADS = A_BYTES / 1024u;
    // Packed (two buffers): values [64][MX_ROW], then tables [8][65] of
    // 8-byte f16 MFMA operands (the half in the first k slot) by block, so
    // that 16 lanes' reads of one block fill the 32 banks: D (d of each
    // weight row), S (sx of each activation row), Q4_1 also M (m), E (mx);
    // entry 64 of each block is zero, for the lanes whose k slots must be.
    static constexpr uint32_t TAB = MX_STAGE * MX_TAB_ROW * 8u;
    static constexpr uint32_t TABLES = KIND == 2 ? 4u : 2u;
    static constexpr uint32_t P_D = MX_TILE * MX_ROW;
    static constexpr uint32_t P_S = P_D + TAB;
    static constexpr uint32_t P_M = P_S + TAB;
    static constexpr uint32_t P_E = P_M + (KIND == 2 ? TAB : 0u);
    static constexpr uint32_t P_BYTES = P_E + (KIND == 2 ? TAB : 0u);
    static constexpr uint32_t RW = 0, RA = 3u * W_BYTES, PK = RA + 3u * A_BYTES;
    static constexpr uint32_t LDS = PK + 2u * P_BYTES;
    static_assert(W_BYTES % 1024u == 0 && A_BYTES % 1024u == 0, "whole wave loads");
    static_assert(LDS <= 160u * 1024u, "one workgroup's LDS");
};

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef long v2l __attribute__((ext_vector_type(2)));

__device__ __forceinline__ long mx_half_op(float x) { return (long)__builtin_bit_cast(uint16_t, (_Float16)x); }

__device__ __forceinline__ v4h mx_op(long v) { return __builtin_bit_cast(v4h, v); }

// The nibbles of one dword of a Q4 block (values 4 i .. as low nibbles,
// 16 + 4 i .. as high) as bytes, dwords i and 4 + i of the block's values;
// Q4_0 less 8 (for v in 0..15, ((v ^ 8) + 0x78) ^ 0x78 is v - 8 as a byte,
// with no carry between bytes).
template <int KIND>
__device__ __forceinline__ void mx_unpack(uint32_t v, uint32_t& lo, uint32_t& hi) {
    lo = v & 0x0f0f0f0fu;
    hi = (v >> 4) & 0x0f0f0f0fu;
    if constexpr (KIND == 1) {
        lo = ((lo ^ 0x08080808u) + 0x78787878u) ^ 0x78787878u;
        hi = ((hi ^ 0x08080808u) + 0x78787878u) ^ 0x78787878u;
    }
}

// Repacks a raw weight group into a packed buffer: thread t takes pair
// t % 4 of weight row t / 4, and blocks 2 (t % 4) + 0, 1 of activation row
// t / 4's scales.
template <int KIND>
__device__ __forceinline__ void mx_repack(const uint8_t* raw, uint8_t* pk, uint32_t t) {
    using M = Mx<KIND>;
    constexpr uint32_t PB = 2u * Fmt<KIND>::BB;  // bytes of a raw pair
    const uint32_t c = t >> 2, p = t & 3u;
    const uint32_t* r = (const uint32_t*)(raw + c * M::RB + PB * p);
    uint32_t v[16];
    long d0, d1;
    if constexpr (KIND == 0) {
        uint32_t e[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) e[i] = r[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = funnel(e[i + 1], e[i], 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[8 + i] = e[9 + i];
        d0 = (long)(e[0] & 0xffffu), d1 = (long)(e[8] >> 16);
    } else if constexpr (KIND == 1) {
        uint32_t e[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) e[i] = r[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mx_unpack<KIND>(funnel(e[i + 1], e[i], 2), v[i], v[4 + i]);
            mx_unpack<KIND>(e[5 + i], v[8 + i], v[12 + i]);
        }
        d0 = (long)(e[0] & 0xffffu), d1 = (long)(e[4] >> 16);
    } else {
        uint32_t e[10];
#pragma unroll
        for (int i = 0; i < 10; ++i) e[i] = r[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mx_unpack<KIND>(e[1 + i], v[i], v[4 + i]);
            mx_unpack<KIND>(e[6 + i], v[8 + i], v[12 + i]);
        }
        d0 = (long)(e[0] & 0xffffu), d1 = (long)(e[5] & 0xffffu);
            long* mt = (long*)(pk + M::P_M) + 2u * p * MX_TAB_ROW + c;
        mt[0] = (long)(e[0] >> 16), mt[MX_TAB_ROW] = (long)(e[5] >> 16);
    }
    uint8_t* dst = pk + c * MX_ROW + 64u * p;
#pragma unroll
    for (int i = 0; i < 4; ++i) *(uint4*)(dst + 16u * i) = make_uint4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    const uint32_t at = 2u * p * MX_TAB_ROW + c;  // entry of block 2p, row c
    long* dt = (long*)(pk + M::P_D) + at;
    dt[0] = d0, dt[MX_TAB_ROW] = d1;
    const float2 sx = *(const float2*)(raw + M::W_S + (c * 8u + 2u * p) * 4u);
    long* st = (long*)(pk + M::P_S) + at;
    st[0] = mx_half_op(sx.x), st[MX_TAB_ROW] = mx_half_op(sx.y);
    if constexpr (KIND == 2) {
        const float2 mx = *(const float2*)(raw + M::W_E + (c * 8u + 2u * p) * 4u);
        long* et = (long*)(pk + M::P_E) + at;
        et[0] = mx_half_op(mx.x), et[MX_TAB_ROW] = mx_half_op(mx.y);
    }
}

// One block's MFMA results: the dot products and the factors of the
// contributions ([0]: d·sx, or Q4_0 d; [1]: Q4_1 m·mx, Q4_0 sx).
struct MxBlock {
    v16i t;
    v16f f[2];
};

// Operand bases of a lane within a stage (the tables' for lanes 0-31;
// zeros for the others, whose k slots must be zero).
struct MxBase {
    const uint8_t* a;     // activation row + 16 (lane / 32)
    const uint8_t* w;     // packed weight row + 16 (lane / 32)
    const uint8_t* d;     // D row (Q4_1: M at + P_M - P_D)
    const uint8_t* s;     // S row (Q4_1: E at + P_E - P_S)
    const uint8_t* m;     // Q4_1: M row
    const uint8_t* e;     // Q4_1: E row
};

// One block's operands, read from LDS a stage at a time.
struct MxOps {
    v4i a, w;
    long d, s, m, e;
};

template <int KIND>
__device__ __forceinline__ void mx_operands(MxOps& o, const MxBase& B, uint32_t b) {
    o.a = *(const v4i*)(B.a + 32u * b);
    o.w = *(const v4i*)(B.w + 32u * b);
    o.d = *(const long*)(B.d + 8u * MX_TAB_ROW * b);
    o.s = *(const long*)(B.s + 8u * MX_TAB_ROW * b);
    if constexpr (KIND == 2) {
        o.m = *(const long*)(B.m + 8u * MX_TAB_ROW * b);
        o.e = *(const long*)(B.e + 8u * MX_TAB_ROW * b);
    }
}

template <int KIND>
__device__ __forceinline__ void mx_block(MxBlock& o, const MxOps& p, long one) {
    const v16i zi = {};
    const v16f zf = {};
    o.t = __builtin_amdgcn_mfma_i32_32x32x32_i8(p.a, p.w, zi, 0, 0, 0);
    if constexpr (KIND == 1) {
        o.f[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(mx_op(one), mx_op(p.d), zf, 0, 0, 0);
        o.f[1] = __builtin_amdgcn_mfma_f32_32x32x8f16(mx_op(p.s), mx_op(one), zf, 0, 0, 0);
    } else {
        o.f[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(mx_op(p.s), mx_op(p.d), zf, 0, 0, 0);
        if constexpr (KIND == 2) o.f[1] = __builtin_amdgcn_mfma_f32_32x32x8f16(mx_op(p.e), mx_op(p.m), zf, 0, 0, 0);
    }
}

// Adds one block's contributions to the lane's 16 sums.
template <int KIND, bool FUSED>
__device__ __forceinline__ void mx_add(float (&acc)[16], const MxBlock& o) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ft = (float)o.t[i];
        if constexpr (KIND == 0) {
            if constexpr (FUSED) acc[i] = __builtin_fmaf(ft, o.f[0][i], acc[i]);
            else acc[i] += ft * o.f[0][i];
        } else if constexpr (KIND == 1) {
            const float p = ft * o.f[0][i];
            if constexpr (FUSED) acc[i] = __builtin_fmaf(p, o.f[1][i], acc[i]);
            else acc[i] += p * o.f[1][i];
        } else {
            if constexpr (FUSED) {
                acc[i] = __builtin_fmaf(o.f[0][i], ft, acc[i] + o.f[1][i]);
            } else {
                const float f = o.f[0][i] * ft;
                acc[i] += f + o.f[1][i];
            }
        }
    }
}

template <int KIND, bool FUSED>
__global__ __launch_bounds__(MX_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_matmul_mx(
    const uint8_t* __restrict__ w, Activations act, float* __restrict__ dst, const float* __restrict__ bias,
    uint32_t m, uint32_t n, uint32_t k, uint32_t tiles_m, uint32_t tiles) {
    using M = Mx<KIND>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[M::LDS];
    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const bool producer = wave >= MX_COMPUTE;
    const uint32_t pw = wave - MX_COMPUTE, pt = t - 64u * MX_COMPUTE;  // producer wave, thread
    const uint32_t l32 = lane & 31u, half = lane >> 5;
    const uint32_t nb = k >> 5, stages = nb / MX_STAGE;
    uint32_t g = blockIdx.x;
    if (tiles % 8u == 0) g = (g & 7u) * (tiles >> 3) + (g >> 3);
    const uint32_t n0 = (g / tiles_m) * MX_TILE, m0 = (g % tiles_m) * MX_TILE;
    const uint32_t mw = (wave & 1u) * 32u, nw = ((wave >> 1) & 1u) * 32u;
    const size_t row_bytes = (size_t)nb * Fmt<KIND>::BB;
    // The tables' zero entries (the repack never writes them).
    if (t < 2u * M::TABLES * MX_STAGE) {
        const uint32_t buffer = t / (M::TABLES * MX_STAGE), table = (t / MX_STAGE) % M::TABLES, b = t % MX_STAGE;
        ((long*)(lds + M::PK + buffer * M::P_BYTES + M::P_D + table * M::TAB))[b * MX_TAB_ROW + MX_TILE] = 0;
    }

    // A producer wave's direct loads: weight-group instructions iw = pw + 4 j
    // (below W_LOADS) and activation instructions ia with (ia + W_LOADS) % 4
    // = pw; lane l fills bytes 1024 i + 16 l of the group's buffer, from
    // src + stage · step. (A pad chunk of an activation row brings the row's
    // last chunk again.)
    constexpr uint32_t PW = MX_THREADS / 64u - MX_COMPUTE;
    constexpr uint32_t WJ = (M::W_LOADS + PW - 1u) / PW, AJ = (M::A_LOADS + PW - 1u) / PW;
    const uint8_t* wsrc[WJ];
    uint32_t wstep[WJ], wcount = 0;
#pragma unroll
    for (uint32_t j = 0; j < WJ; ++j) {
        const uint32_t i = pw + PW * j, at = 1024u * i + 16u * lane;
        wsrc[j] = w, wstep[j] = 0;
        if (!producer || i >= M::W_LOADS) continue;
        ++wcount;
        if (at < M::W_S) {
            const uint32_t p = at / 16u, row = p / M::RC, chunk = p % M::RC;
            wsrc[j] = w + (size_t)min(n0 + row, n - 1u) * row_bytes + 16u * chunk;
            wstep[j] = M::RB;
        } else {
            const bool ex = at >= M::W_E;
            const uint32_t e = (at - (ex ? M::W_E : M::W_S)) / 16u, row = e >> 1;
            const float* from = ex ? act.sums : act.scales;
            wsrc[j] = (const uint8_t*)(from + (size_t)min(m0 + row, m - 1u) * nb + 4u * (e & 1u));
            wstep[j] = MX_STAGE * 4u;
        }
    }
    const uint8_t* asrc[AJ];
    const uint32_t afirst = (pw + PW - M::W_LOADS % PW) % PW;
    uint32_t acount = 0;
#pragma unroll
    for (uint32_t j = 0; j < AJ; ++j) {
        const uint32_t i = afirst + PW * j;
        asrc[j] = (const uint8_t*)act.qs;
        if (!producer || i >= M::A_LOADS) continue;
        ++acount;
        const uint32_t p = 64u * i + lane, row = p / 17u, chunk = min(p % 17u, 15u);
        asrc[j] = (const uint8_t*)act.qs + (size_t)min(m0 + row, m - 1u) * k + 16u * chunk;
    }
    auto issue_w = [&](uint32_t s) {
        const uint32_t to = lds_address(lds + M::RW + (s % 3u) * M::W_BYTES) + pw * 1024u;
#pragma unroll
        for (uint32_t j = 0; j < WJ; ++j)
            if (pw + PW * j < M::W_LOADS) lds_load16(wsrc[j] + (size_t)s * wstep[j], to + j * (PW * 1024u));
    };
    auto issue_a = [&](uint32_t s) {
        const uint32_t to = lds_address(lds + M::RA + (s % 3u) * M::A_BYTES) + afirst * 1024u;
#pragma unroll
        for (uint32_t j = 0; j < AJ; ++j)
            if (afirst + PW * j < M::A_LOADS) lds_load16(asrc[j] + (size_t)s * 256u, to + j * (PW * 1024u));
    };
    auto barrier = [&](uint32_t outstanding) {
        asm volatile("" ::: "memory");
        wait_vm_lds_in<0u, 16u>(outstanding);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

    // Weights of stages 0-2 and activations of 0-1 in flight; stage 0
    // repacked.
    if (producer) {
        issue_w(0);
        issue_a(0);
        if (stages > 1u) issue_w(1), issue_a(1);
        if (stages > 2u) issue_w(2);
    }
    barrier((stages > 1u ? acount : 0u) + (stages > 2u ? wcount : 0u));
    if (producer) mx_repack<KIND>(lds + M::RW, lds + M::PK, pt);
    barrier(63);

    const long one = half == 0 ? 0x3c00l : 0l;  // the f16 operand (1, 0, 0, 0) for lanes 0-31
    for (uint32_t s = 0; s < stages; ++s) {
        if (producer) {
            // The loads of stage s + 3 (weights) and s + 2 (activations),
            // and the repack of stage s + 1.
            if (s + 3u < stages) issue_w(s + 3u);
            if (s + 2u < stages) issue_a(s + 2u);
            if (s + 1u < stages)
                mx_repack<KIND>(lds + M::RW + ((s + 1u) % 3u) * M::W_BYTES,
                                lds + M::PK + ((s + 1u) & 1u) * M::P_BYTES, pt);
        } else {
            const uint8_t* pk = lds + M::PK + (s & 1u) * M::P_BYTES;
            MxBase B;
            B.a = lds + M::RA + (s % 3u) * M::A_BYTES + (mw + l32) * MX_ROW + 16u * half;
            B.w = pk + (nw + l32) * MX_ROW + 16u * half;
            const uint32_t wcol = half == 0 ? (nw + l32) * 8u : MX_TILE * 8u;  // the zero entry for lanes 32-63
            const uint32_t arow = half == 0 ? (mw + l32) * 8u : MX_TILE * 8u;
            B.d = pk + M::P_D + wcol;
            B.s = pk + M::P_S + arow;
            B.m = pk + M::P_M + wcol;
            B.e = pk + M::P_E + arow;
            // The stage's operand reads go out together, then the blocks:
            // the MFMAs of block b + 1 before the additions of block b.
            MxOps ops[MX_STAGE];
#pragma unroll
            for (uint32_t b = 0; b < MX_STAGE; ++b) mx_operands<KIND>(ops[b], B, b);
            MxBlock cur, nxt;
            mx_block<KIND>(cur, ops[0], one);
#pragma unroll
            for (uint32_t b = 0; b < MX_STAGE; ++b) {
                if (b + 1u < MX_STAGE) mx_block<KIND>(nxt, ops[b + 1u], one);
                mx_add<KIND, FUSED>(acc, cur);
                cur = nxt;
            }
            // The stage's sums are complete before the barrier: the
            // compiler would otherwise move the additions after it.
#pragma unroll
            for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(acc[i]));
        }
        // Weights of stage s + 2 and activations of s + 1 have landed (the
        // loads issued above stay in flight); every wave is done with this
        // stage's buffers.
        if (s + 1u < stages) barrier((s + 3u < stages ? wcount : 0u) + (s + 2u < stages ? acount : 0u));
    }

    if (producer) return;
    const uint32_t col = n0 + nw + l32;
    const float b = (bias && col < n) ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t row = m0 + mw + 8u * (i / 4) + 4u * half + (i % 4);
        if (row < m && col < n) dst[(size_t)row * n + col] = bias ? acc[i] + b : acc[i];
    }
}

// ------------------------------------ matrix cores: a few activation rows

// x · wᵀ for up to 16 activation rows (batched decode) on the int8 matrix
// cores, k a multiple of 512, weights and activation parts 16-byte aligned.
// Workgroup: 16 outputs (weight rows) for all rows over the whole of k, 8
// waves; the weights are read from HBM once whatever the row count (the
// lanes kernels read them once per group of 8 rows and take ~13 VALU
// operations a row and block for the dot products).
//
// The k axis goes in stages of 16 blocks through a ring of DEPTH LDS
// buffers, the loads of stages s + 1 .. s + DEPTH - 1 in flight while stage
// s is computed, one workgroup barrier a stage; all of it by direct loads
// (raw weight rows, the activation rows 528 bytes apart, their scales and
// extras). In a stage, wave v issues the v_mfma_i32_16x16x32_i8 of blocks
// 2v and 2v + 1 (the 16 x 16 tile of rows x outputs of one block; operands
// read where the blocks lie: Q8_0 values
// funnel-shifted in even blocks, Q4 nibbles unpacked a dword at a time with
// the activations taken in the same order; Q4_0's -8·Σq as the MFMA's C),
// forms each output's contribution of the block in the host's expression
// (Q8_0 float(t)·(d·sx); Q4_0 (float(t)·d)·sx; Q4_1 (d·sx)·float(t) + m·mx,
// each operation rounded as the host rounds it) and writes it to LDS by
// block, row and output. In the next stage each of the first 256 threads
// adds one output's contributions (row t / 16, output t % 16) in block
// order: the ordered fold is spread one output a lane over the workgroup.

// The B operand (8 int8 values) of a lane for block b of a stage, from the
// stage's raw weight row at `row` (LDS); q is the lane's k quarter.
//   Q8_0  the lane's 8 bytes 2 + 8 q .. of the block's 34: dword-aligned in
//         odd blocks, two bytes off in even ones (funnel shifts);
//   Q4_x  one dword of nibbles, bytes 4 q .. 4 q + 3 of the 16: its low
//         nibbles are values 4 q .., its high ones 16 + 4 q .. (few_acts
//         takes the activations in the same order).
template <int KIND>
__device__ __forceinline__ long few_weights(const uint8_t* row, uint32_t b, uint32_t q);

template <int KIND>
__device__ __forceinline__ long few_weights(const uint8_t* row, uint32_t b, uint32_t q) {
    if constexpr (KIND == 0) {
        if (b % 2u == 0) {
            const uint32_t* p = (const uint32_t*)(row + 34u * b + 8u * q);
            const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
            return (long)funnel(d1, d0, 2) | ((long)funnel(d2, d1, 2) << 32);
        }
        const uint32_t* p = (const uint32_t*)(row + 34u * b + 2u + 8u * q);
        return (long)p[0] | ((long)p[1] << 32);
    } else {
        uint32_t v;
        if constexpr (KIND == 1) {
            if (b % 2u == 0) {
                const uint32_t* p = (const uint32_t*)(row + 18u * b + 4u * q);
                v = funnel(p[1], p[0], 2);
            } else {
                v = *(const uint32_t*)(row + 18u * b + 2u + 4u * q);
            }
        } else {
            v = *(const uint32_t*)(row + 20u * b + 4u + 4u * q);
        }
        return (long)(v & 0x0f0f0f0fu) | ((long)((v >> 4) & 0x0f0f0f0fu) << 32);
    }
}

// The A operand of block b from the stage's activation row at `row` (LDS):
// the 8 values few_weights pairs with.
template <int KIND>
__device__ __forceinline__ long few_acts(const uint8_t* row, uint32_t b, uint32_t q) {
    if constexpr (KIND == 0) {
        return *(const long*)(row + 32u * b + 8u * q);
    } else {
        const uint32_t* p = (const uint32_t*)(row + 32u * b);
        return (long)p[q] | ((long)p[4u + q] << 32);
    }
}

constexpr uint32_t FEW_ROWS = 16;
constexpr uint32_t FEW_COLS = 16;
constexpr uint32_t FEW_STAGE = 16;  // blocks a stage at least (k a multiple of 512)
constexpr uint32_t FEW_THREADS = 512;
constexpr uint32_t FEW_WAVES = FEW_THREADS / 64u;

// Stages of SB blocks through a ring of DEPTH buffers.
template <int KIND, uint32_t DEPTH, uint32_t SB>
struct Few {
    static constexpr uint32_t PER = SB / FEW_WAVES;      // blocks of a stage a wave takes
    static constexpr uint32_t AROW = SB * 32u + 16u;     // LDS bytes per activation row: values + a 16-byte pad
    static constexpr uint32_t ACH = AROW / 16u;          // its 16-byte pieces
    static constexpr uint32_t BB = Fmt<KIND>::BB;
    static constexpr uint32_t RB = SB * BB;  // a weight row's bytes in a stage
    static constexpr uint32_t RC = RB / 16u;
    static constexpr uint32_t KB1 = 1024u;
    static constexpr uint32_t W_BYTES = (FEW_COLS * RB + KB1 - 1u) / KB1 * KB1;  // whole 1 KB wave loads
    static constexpr uint32_t A_CHUNKS = FEW_ROWS * ACH;
    static constexpr uint32_t A_BYTES = (FEW_ROWS * AROW + KB1 - 1u) / KB1 * KB1;
    static constexpr uint32_t S_BYTES = FEW_ROWS * SB * 4u;  // scales [row][SB]
    static constexpr uint32_t E_BYTES = KIND == 0 ? 0u : S_BYTES;  // Q4_0 Σq, Q4_1 sums
    // a raw stage: weights, activations, scales, extras
    static constexpr uint32_t R_A = W_BYTES, R_S = R_A + A_BYTES, R_E = R_S + S_BYTES, R_BYTES = R_E + E_BYTES;
    static constexpr uint32_t LOADS = R_BYTES / KB1;
    // a stage's contributions [block][row][output], f32
    static constexpr uint32_t P_BYTES = SB * FEW_ROWS * FEW_COLS * 4u;
    static constexpr uint32_t NBUF = DEPTH;
    static constexpr uint32_t RAW = 0, PK = NBUF * R_BYTES, LDS = PK + 2u * P_BYTES;
    static_assert(NBUF >= 3u, "a ring of three stages at least");
    static_assert(R_BYTES % KB1 == 0, "whole wave loads");
    static_assert(LDS <= 160u * 1024u, "one workgroup's LDS");
};

template <int KIND, uint32_t DEPTH, uint32_t SB, bool TREE>
__global__ __launch_bounds__(FEW_THREADS) void k_matmul_few(const uint8_t* __restrict__ w, Activations act,
                                                            float* __restrict__ dst, const float* __restrict__ bias,
                                                            uint32_t bias_ld, uint32_t rows, uint32_t n, uint32_t k) {
    constexpr bool tree = TREE;  // UNORDERED's fold (four running sums a stage)
    using F = Few<KIND, DEPTH, SB>;
    constexpr uint32_t PER = F::PER;
    __shared__ __attribute__((aligned(16))) uint8_t lds[F::LDS];
    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t lr = lane & 15u, lq = lane >> 4;
    const uint32_t nb = k >> 5, stages = nb / SB;
    const uint32_t n0 = blockIdx.x * FEW_COLS;
    const size_t row_bytes = (size_t)nb * F::BB;

    // This wave's direct loads of a stage: instructions i = wave + 4 j below
    // LOADS; lane l fills bytes 1024 i + 16 l of the stage's buffer, from
    // src + stage · step. (Lanes past a part's data bring a piece of it
    // again, into the part's padding.)
    constexpr uint32_t J = (F::LOADS + FEW_WAVES - 1u) / FEW_WAVES;
    const uint8_t* src[J];
    uint32_t step[J], mine = 0;
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) {
        const uint32_t i = wave + FEW_WAVES * j, at = 1024u * i + 16u * lane;
        src[j] = w, step[j] = 0;
        if (i >= F::LOADS) continue;
        ++mine;
        if (at < F::R_A) {
            const uint32_t p = min(at / 16u, FEW_COLS * F::RC - 1u), col = p / F::RC, chunk = p % F::RC;
            src[j] = w + (size_t)min(n0 + col, n - 1u) * row_bytes + 16u * chunk;
            step[j] = F::RB;
        } else if (at < F::R_S) {
            const uint32_t p = min((at - F::R_A) / 16u, F::A_CHUNKS - 1u), row = p / F::ACH;
            const uint32_t chunk = min(p % F::ACH, F::ACH - 2u);
            src[j] = (const uint8_t*)act.qs + (size_t)min(row, rows - 1u) * k + 16u * chunk;
            step[j] = SB * 32u;
        } else {
            const bool ex = at >= F::R_E;
            const uint32_t p = (at - (ex ? F::R_E : F::R_S)) / 16u, row = p / (SB / 4u);
            const void* from = !ex ? (const void*)act.scales
                                   : (KIND == 1 ? (const void*)act.totals : (const void*)act.sums);
            src[j] = (const uint8_t*)from + ((size_t)min(row, rows - 1u) * nb + 4u * (p % (SB / 4u))) * 4u;
            step[j] = SB * 4u;
        }
    }
    auto issue = [&](uint32_t s) {
        const uint32_t to = lds_address(lds + F::RAW + (s % F::NBUF) * F::R_BYTES) + wave * 1024u;
#pragma unroll
        for (uint32_t j = 0; j < J; ++j)
            if (wave + FEW_WAVES * j < F::LOADS) lds_load16(src[j] + (size_t)s * step[j], to + j * (FEW_WAVES * 1024u));
    };
    auto barrier = [&](uint32_t outstanding) {
        asm volatile("" ::: "memory");
        wait_vm_lds_in<0u, 32u>(outstanding);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Stages 0 .. NBUF - 2 in flight; wait for stage 0.
    const uint32_t ahead = min(stages, F::NBUF - 1u);
    for (uint32_t s = 0; s < ahead; ++s) issue(s);
    barrier((ahead - 1u) * mine);

    const uint32_t fr = t >> 4, fc = t & 15u;  // the output this thread adds up
    float acc = 0.0f;
    for (uint32_t s = 0; s <= stages; ++s) {
        if (s + F::NBUF - 1u < stages) issue(s + F::NBUF - 1u);
        if (s < stages) {
            // This wave's blocks of stage s (2v, 2v + 1): their
            // contributions, written as the MFMA result lies (block, lane,
            // the lane's 4 rows), one 16-byte write a block.
            const uint8_t* raw = lds + F::RAW + (s % F::NBUF) * F::R_BYTES;
            uint8_t* pk = lds + F::PK + (s & 1u) * F::P_BYTES;
            const uint8_t* wrow = raw + lr * F::RB;
            const uint8_t* arow = raw + F::R_A + lr * F::AROW;
            // the lane's 4 rows' scales (and extras) of the wave's blocks
            float sxv[4][PER], exv[4][PER];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (uint32_t u = 0; u < PER; u += 2u) {
                    const uint32_t at = ((4u * lq + i) * SB + PER * wave + u) * 4u;
                    const float2 x = *(const float2*)(raw + F::R_S + at);
                    sxv[i][u] = x.x, sxv[i][u + 1u] = x.y;
                    if constexpr (KIND != 0) {
                        const float2 e = *(const float2*)(raw + F::R_E + at);
                        exv[i][u] = e.x, exv[i][u + 1u] = e.y;
                    }
                }
            // Every read of the wave's blocks first (the LDS writes below would
            // otherwise hold each block's reads behind the previous block's
            // write), then the MFMAs, then the contributions and writes.
            long av[PER], bv[PER];
            uint32_t dm[PER];
#pragma unroll
            for (uint32_t u = 0; u < PER; ++u) {
                const uint32_t b = PER * wave + u;
                av[u] = few_acts<KIND>(arow, b, lq);
                bv[u] = few_weights<KIND>(wrow, b, lq);
                if constexpr (KIND == 2) dm[u] = *(const uint32_t*)(wrow + 20u * b);
                else dm[u] = *(const uint16_t*)(wrow + F::BB * b);
            }
            v4i tv[PER];
#pragma unroll
            for (uint32_t u = 0; u < PER; ++u) {
                v4i c = {0, 0, 0, 0};
                if constexpr (KIND == 1) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) c[i] = -8 * __float_as_int(exv[i][u]);
                }
                tv[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u], bv[u], c, 0, 0, 0);
            }
#pragma unroll
            for (uint32_t u = 0; u < PER; ++u) {
                const uint32_t b = PER * wave + u;
                const float d = half_value(dm[u] & 0xffffu);
                const float m = KIND == 2 ? half_value(dm[u] >> 16) : 0.0f;
                float cv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = sxv[i][u], ft = (float)tv[u][i];
                    if constexpr (KIND == 0) {
                        const float sc = d * x;
                        cv[i] = ft * sc;
                    } else if constexpr (KIND == 1) {
                        const float p = ft * d;
                        cv[i] = p * x;
                    } else {
                        const float sc = d * x;
                        const float f = sc * ft;
                        const float g = m * exv[i][u];
                        cv[i] = f + g;
                    }
                }
                *(float4*)(pk + (b * 64u + lane) * 16u) = make_float4(cv[0], cv[1], cv[2], cv[3]);
            }
        }
        if (s > 0 && t < FEW_ROWS * FEW_COLS) {
            // Stage s - 1's contributions to this thread's output, in block
            // order: output (row r, column c) is element r % 4 of lane
            // c + 16 (r / 4).
            const float* ct = (const float*)(lds + F::PK + ((s - 1u) & 1u) * F::P_BYTES) +
                              (fc + 16u * (fr >> 2)) * 4u + (fr & 3u);
            if (tree) {
                // UNORDERED: the stage's contributions as four running sums
                float u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (uint32_t b = 0; b < SB; ++b) u[b & 3u] += ct[b * 256u];
                acc += (u[0] + u[1]) + (u[2] + u[3]);
            } else {
#pragma unroll
                for (uint32_t b = 0; b < SB; ++b) acc += ct[b * 256u];
            }
        }
        // Stage s + 1 has landed (the loads of later stages stay in
        // flight); the contributions written above are complete, and the
        // ones read are done.
        if (s < stages) barrier(min(stages - 1u - min(s + 1u, stages - 1u), F::NBUF - 2u) * mine);
    }
    const uint32_t col = n0 + fc;
    if (t < FEW_ROWS * FEW_COLS && fr < rows && col < n) {
        float v = acc;
        if (bias) v = v + bias[(size_t)fr * bias_ld + col];
        dst[(size_t)fr * n + col] = v;
    }
}

// ------------------------------------------- a few rows, weights in LDS

// Threads of a k_matvec_nb workgroup: 8 waves, two a SIMD.
constexpr uint32_t NB_THREADS = 512;
// Blocks of a fold chunk: the contributions of NB_CHUNK blocks are held in
// LDS at a time, a run of consecutive blocks a wave.
constexpr uint32_t NB_CHUNK = 64;
// One or two rows: 16 waves a workgroup, four a SIMD, each with 4 blocks
// (2 pairs) of a chunk, so that a SIMD has more waves to hide each one's LDS
// reads and MFMA results (measured, config 3 8192x2048: B = 1 and 2 0.25 us
// faster a call, B = 4 the same, B = 8 0.15 us slower); else 8 waves of 8
// blocks (4 pairs).
template <int NB>
struct NbShape {
    static constexpr uint32_t THREADS = NB <= 2 ? 1024u : NB_THREADS;
    static constexpr uint32_t WAVES = THREADS / 64u;
    static constexpr uint32_t PER = NB_CHUNK / WAVES;  // blocks of a chunk a wave
    static_assert(PER % 2u == 0 && PER <= 8u, "whole pairs, at most 4 a wave");
};

// LDS of k_matvec_nb in bytes from the start of its dynamic LDS:
//   [0, w)   F32/NORM: the f32 rows [NB][xrow] and the norm's weights while
//            the prologue reads them; then (and for QUANT from the start)
//            the quantised rows qs [NB][k] and their tables [NB][nb]
//            (scales; Q4_1 sums; Q4_0 totals), the contributions part
//            [bufs][tpp][NB][prow] ([rt][pstride] and a skew) of the tpp
//            tiles of 16 weight rows of a phase and one chunk of blocks (two
//            buffers: a phase's fold runs while the next one's contributions
//            are formed), the GLU outputs, a zero piece and a dummy slot
//            per lane (below);
//   [w, end) the weight tile, direct-loaded (GLU: its gate rows at w, its
//            up rows at w2).
struct NbLds {
    uint32_t x, xrow, nw, qs, arow, scales, sums, totals, trow, part, pstride, rt, prow, region, bufs, outs, zeros,
        dummy, w, w2, wrow, end;
};

// The LDS stride of rows of `bytes` bytes (a multiple of 16) read 16 rows at
// a time by the matrix-core operands: bytes plus whole 16-byte pieces, so
// that 16 rows start on 16 different 4-bank groups (stride / 4 an odd
// multiple of 4, modulo the 64 banks).
__host__ __device__ inline uint32_t nb_row_stride(uint32_t bytes) {
    uint32_t s = bytes + 16u;
    while ((((s >> 2) & 63u) >> 2 & 1u) == 0) s += 16u;
    return s;
}

__host__ __device__ inline NbLds nb_lds(uint32_t nbatch, uint32_t kind, uint32_t k, uint32_t tr, uint32_t row_bytes,
                                        uint32_t mode, bool glu, uint32_t tpp = 1u, uint32_t bufs = 1u) {
    const uint32_t nb = k >> 5;
    auto kb = [](uint32_t b) { return (b + 1023u) & ~1023u; };
    NbLds l;
    l.qs = 0;
    l.arow = nb_row_stride(k);
    l.trow = nb_row_stride(4u * nb);
    const uint32_t tab = kb(nbatch * l.trow);
    l.scales = kb(nbatch * l.arow);
    l.sums = l.scales + tab;
    l.totals = l.sums + (kind == 2 ? tab : 0u);
    const uint32_t act_end = l.totals + (kind == 1 ? tab : 0u);
    l.pstride = ((nb < NB_CHUNK ? nb : NB_CHUNK) + 3u) / 4u * 4u + 4u;  // 16-byte rows, apart by 4 banks
    // An activation row's contribution rows (16; 8 for a tile of at most 8
    // weight rows), then a skew: 16·pstride is a multiple of the 64 banks,
    // so without it the pair MFMAs' writes of 8 activation rows (a lane's
    // row b, weight row 4 g + i, block j: bank 16 g + j + b·(prow mod 64))
    // would meet on 8 banks; 2 floats spread them over all 64 (8 rows:
    // b·34 + 16 g + j, 32 lanes on distinct banks).
    l.rt = tr <= 8u ? 8u : 16u;
    l.prow = l.rt * l.pstride + 2u;
    l.part = act_end;
    l.region = tpp * nbatch * l.prow;  // floats of one phase's contributions
    l.bufs = bufs;
    l.outs = l.part + 4u * bufs * l.region;
    const uint32_t outs_end = l.outs + (glu ? 4u * nbatch * (tr + tr / 2u) : 0u);
    l.x = 0;
    l.xrow = kb(4u * k);  // whole kilobytes: a row's last direct load may write past its end
    l.nw = nbatch * l.xrow;
    const uint32_t x_end = mode == NB_QUANT ? 0u : l.nw + (mode == NB_NORM ? kb(4u * k) : 0u);
    // the weight tile's direct loads fill whole kilobytes from its start,
    // which needs 16-byte alignment only (x_end is whole kilobytes)
    // 512 bytes of zeros, read as the B operand by the lanes whose values
    // must be zero, and 512 bytes the lanes with no contribution slot write
    l.zeros = (outs_end + 15u) & ~15u;
    l.dummy = l.zeros + 512u;
    const uint32_t extra_end = l.dummy + 512u;
    l.w = ((x_end > extra_end ? x_end : extra_end) + 255u) & ~255u;
    l.wrow = nb_row_stride(row_bytes);
    const uint32_t half = kb((tr / 2u) * l.wrow);
    l.w2 = glu ? l.w + half : l.w;
    l.end = glu ? l.w2 + half : l.w + kb(tr * l.wrow);
    return l;
}

// Direct loads of one f32 row of nb blocks of 32 values at src into LDS at
// `to` (the region holds whole kilobytes), by wave `by` only, swizzled for
// reading a block a lane: the 16-byte piece i of block c lands in slot
// 8 c + ((i + c) & 7), so that lanes c reading their piece i together fall
// on 16 different 4-bank groups. Returns this wave's loads.
__device__ __forceinline__ uint32_t stage_blocks_swizzled(const float* src, uint32_t nb, uint32_t to, uint32_t wave,
                                                          uint32_t by) {
    if (wave != by) return 0;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t slots = 8u * nb, loads = (slots + 63u) >> 6;
    for (uint32_t n = 0; n < loads; ++n) {
        const uint32_t slot = min(n * 64u + lane, slots - 1u), c = slot >> 3, i = (slot - c) & 7u;
        lds_load16(src + 32u * c + 4u * i, to + n * 1024u);
    }
    return loads;
}

// Direct loads of `rows` rows of `bytes` bytes (a multiple of 16) at src,
// src_stride apart, into LDS rows `dst_stride` bytes apart from `to` (a
// byte address; the region holds whole kilobytes), 1 KB a load, load i by
// wave first + (i % waves): lane l of load i fills LDS piece 64 i + l of the
// region with the row piece that lies there (a padding piece, or a piece
// past the last row, takes a copy of a piece of the row). Returns this
// wave's loads (0 for a wave outside [first, first + waves)).
template <bool NT>
__device__ __forceinline__ uint32_t stage_rows(const uint8_t* src, uint32_t bytes, size_t src_stride, uint32_t rows,
                                               uint32_t to, uint32_t dst_stride, uint32_t wave, uint32_t first,
                                               uint32_t waves) {
    if (wave < first || wave >= first + waves) return 0;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t pp = dst_stride >> 4, per = bytes >> 4;
    const uint32_t loads = (rows * pp + 63u) >> 6;
    // piece q of the region is piece q % pp of row q / pp: the quotient by
    // a float reciprocal, exact here (q + 1/2 never lies within 2^-11 of a
    // multiple of pp, which is below 2^10, for q below 2^16)
    const float inv = 1.0f / (float)pp;
    uint32_t mine = 0;
    for (uint32_t i = wave - first; i < loads; i += waves, ++mine) {
        const uint32_t q = i * 64u + lane;
        uint32_t r = (uint32_t)(((float)q + 0.5f) * inv);
        uint32_t e = q - r * pp;
        if (r >= rows) r = rows - 1u, e = per - 1u;
        if (e >= per) e = per - 1u;
        const uint8_t* at = src + (size_t)r * src_stride + 16u * e;
        if constexpr (NT) lds_load16_nt(at, to + i * 1024u);
        else lds_load16(at, to + i * 1024u);
    }
    return mine;
}

// One block of 32 activations (v) quantised by one lane, as
// quantize_activations does it (quant.cr:428-442): d = amax/127, id = 1/d
// (0 when d is 0), q = round-half-away(v·id) as int8; scale F16(d), sum
// F16(float(Σq)·d). amax is the host's largest |v| taken in index order,
// which skips a NaN unless it is v[0]: here a tree of the same comparison
// that takes the right operand when the left is NaN (any order gives the
// largest of the non-NaN values), then v[0]'s NaN if it is one.
__device__ __forceinline__ void quantize_block32(const float (&v)[32], uint32_t (&packed)[8], float& scale,
                                                 float& sum, int& total) {
    float m[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) m[i] = fabsf(v[i]);
#pragma unroll
    for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) {
            const float a = m[i], b = m[i + w];
            m[i] = (b > a || a != a) ? b : a;
        }
    const float first = fabsf(v[0]);
    const float amax = first != first ? first : m[0];
    const float d = amax / 127.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    int tot = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q0 = (int8_t)(int)roundf(v[4 * i] * id);
        const int q1 = (int8_t)(int)roundf(v[4 * i + 1] * id);
        const int q2 = (int8_t)(int)roundf(v[4 * i + 2] * id);
        const int q3 = (int8_t)(int)roundf(v[4 * i + 3] * id);
        packed[i] = (uint32_t)(q0 & 0xff) | (uint32_t)(q1 & 0xff) << 8 | (uint32_t)(q2 & 0xff) << 16 |
                    (uint32_t)(q3 & 0xff) << 24;
        tot += q0 + q1 + q2 + q3;
    }
    total = tot;
    scale = round_to_half(d);
    sum = round_to_half((float)tot * d);
}

// 8 bytes at byte address p in LDS, p any alignment (three dword reads
// and two byte funnels; the dword after them must lie in LDS).
__device__ __forceinline__ void lds_read8(const uint8_t* p, uint32_t& lo, uint32_t& hi) {
    const uint32_t s = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - s);
    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
    lo = funnel(d1, d0, s), hi = funnel(d2, d1, s);
}

// The 16 values of half h of block b of a weight row (LDS) as one lane's
// v_mfma_i32_16x16x64_i8 operand: values 8h .. 8h + 7 and 16 + 8h .. 16 +
// 8h + 7 (Q4: bytes 8h .. 8h + 7 of the nibbles, low then high; Q8_0 the
// two runs of bytes), in that order; pair_acts takes the activations alike.
template <int KIND>
__device__ __forceinline__ v4i pair_weights(const uint8_t* row, uint32_t b, uint32_t h) {
    uint32_t x0, x1;
    if constexpr (KIND == 0) {
        const uint8_t* q = row + 34u * b + 2u + 8u * h;
        uint32_t y0, y1;
        lds_read8(q, x0, x1);
        lds_read8(q + 16, y0, y1);
        return v4i{(int)x0, (int)x1, (int)y0, (int)y1};
    } else {
        if constexpr (KIND == 1) {
            lds_read8(row + 18u * b + 2u + 8u * h, x0, x1);
        } else {
            const uint32_t* q = reinterpret_cast<const uint32_t*>(row + 20u * b + 4u + 8u * h);
            x0 = q[0], x1 = q[1];
        }
        return v4i{(int)(x0 & 0x0f0f0f0fu), (int)(x1 & 0x0f0f0f0fu), (int)((x0 >> 4) & 0x0f0f0f0fu),
                   (int)((x1 >> 4) & 0x0f0f0f0fu)};
    }
}

// pair_weights with q at half h of block b already: row + BB·b + (Q4_1: 4,
// else 2) + 8h; pair_acts with q at row + 32·b + 8h.
template <int KIND>
__device__ __forceinline__ v4i pair_weights_at(const uint8_t* q) {
    uint32_t x0, x1;
    if constexpr (KIND == 0) {
        uint32_t y0, y1;
        lds_read8(q, x0, x1);
        lds_read8(q + 16, y0, y1);
        return v4i{(int)x0, (int)x1, (int)y0, (int)y1};
    } else {
        if constexpr (KIND == 1) {
            lds_read8(q, x0, x1);
        } else {
            const uint32_t* d = reinterpret_cast<const uint32_t*>(q);
            x0 = d[0], x1 = d[1];
        }
        return v4i{(int)(x0 & 0x0f0f0f0fu), (int)(x1 & 0x0f0f0f0fu), (int)((x0 >> 4) & 0x0f0f0f0fu),
                   (int)((x1 >> 4) & 0x0f0f0f0fu)};
    }
}

__device__ __forceinline__ v4i pair_acts_at(const uint8_t* q) {
    const uint2 lo = *reinterpret_cast<const uint2*>(q);
    const uint2 hi = *reinterpret_cast<const uint2*>(q + 16);
    return v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
}

__device__ __forceinline__ v4i pair_acts(const uint8_t* row, uint32_t b, uint32_t h) {
    const uint2 lo = *reinterpret_cast<const uint2*>(row + 32u * b + 8u * h);
    const uint2 hi = *reinterpret_cast<const uint2*>(row + 32u * b + 16u + 8u * h);
    return v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
}

// NB (at most 8) activation rows times a tile of `tr` weight rows per
// workgroup, the tile's weights direct-loaded into LDS at the start (as
// k_matvec_one does for one row). Every wave issues its share of the
// activations first, then of the weights, so that its wait for the
// activations never waits for weights.
//   F32/NORM (k <= 2048, NB <= 8): wave b takes row b into registers, lane
//     c its block c (32 values; stage_blocks_swizzled; one f32 row is
//     quantised by the whole workgroup, 8 lanes a block); NORM first takes
//     the row through Op::RMSNorm (host.cr:374-386): Σx² in index order by
//     speculation across the wave (ordered_sum_wave), root = sqrtf(Σ/k +
//     eps), v = x / root · nw; then the lane quantises its block
//     (quantize_block32) into LDS, while the weights are in flight;
//   QUANT: the rows arrive quantised.
// Products on the int8 matrix cores: per tile of 16 weight rows and pair of
// blocks, one v_mfma_i32_16x16x64_i8 of the weight rows (A) against columns
// (activation row, block of the pair) (B), operands taken where the blocks
// lie (Q4_0's -8·Σq as C; below); each (row, output, block)
// contribution is formed in the host's expression (Q8_0 float(t)·(d·sx);
// Q4_0 (float(t)·d)·sx; Q4_1 (d·sx)·float(t) + m·mx) and written to LDS, a
// chunk of NB_CHUNK blocks at a time, each wave a run of consecutive blocks
// of the chunk; then one thread an output adds the output's contributions of
// the chunk in block order to its running sum (quant.cr:447-455).
// dst[b][row] = Σ (+ bias[b · bias_ld + row], one rounding); GLU: SwiGLU and
// the quantiser on the tile's gate/up outputs into glu, as k_matvec_one. Each
// output depends on its own activation row only, so the bits are those of one
// row at a time.
template <int KIND, uint32_t MODE, bool GLU, int NB, bool TREE>
__global__ __launch_bounds__(NbShape<NB>::THREADS) void k_matvec_nb(
    const uint8_t* __restrict__ w, const float* __restrict__ x, uint32_t ldx, const float* __restrict__ nw, float eps,
    Activations act, float* __restrict__ dst, const float* __restrict__ bias, uint32_t bias_ld, uint32_t n, uint32_t k,
    uint32_t tr, uint32_t tpp, uint32_t bufs, Activations glu) {
    constexpr bool tree = TREE;  // UNORDERED's fold (Fold4)
    static_assert(NB >= 1 && NB <= 8, "activation rows of a launch");
    constexpr uint32_t WAVES = NbShape<NB>::WAVES, THREADS = NbShape<NB>::THREADS, PER = NbShape<NB>::PER;
    constexpr uint32_t PP = PER / 2u;  // pairs of a chunk a wave (up to 8 rows)
    extern __shared__ float4 lds4[];
    uint8_t* base = reinterpret_cast<uint8_t*>(lds4);
    constexpr uint32_t BB = Fmt<KIND>::BB;
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nb = k >> 5, row_bytes = nb * BB;
    const uint32_t tile = blockIdx.x, h = tr >> 1, H = n >> 1, g0 = tile * h;
    const uint32_t row0 = tile * tr, rows = GLU ? tr : min(tr, n - row0);
    const NbLds L = nb_lds(NB, KIND, k, tr, row_bytes, MODE, GLU, tpp, bufs);
    const uint32_t lbase = lds_address(base);

    // Activations first, every wave its share, then the weights.
    if constexpr (MODE == NB_QUANT) {
        // rows and tables contiguous (the quantise pass's layout); NB·nb a
        // multiple of 4 and the tables 16-byte aligned
        stage_rows<false>(reinterpret_cast<const uint8_t*>(act.qs), k, k, NB, lbase + L.qs, L.arow, wave, 0u,
                          WAVES);
        stage_rows<false>(reinterpret_cast<const uint8_t*>(act.scales), 4u * nb, 4u * nb, NB, lbase + L.scales, L.trow,
                          wave, 0u, WAVES);
        if constexpr (KIND == 2)
            stage_rows<false>(reinterpret_cast<const uint8_t*>(act.sums), 4u * nb, 4u * nb, NB, lbase + L.sums, L.trow,
                              wave, 0u, WAVES);
        if constexpr (KIND == 1)
            stage_rows<false>(reinterpret_cast<const uint8_t*>(act.totals), 4u * nb, 4u * nb, NB, lbase + L.totals,
                              L.trow, wave, 0u, WAVES);
    } else {
        if constexpr (MODE == NB_F32 && NB == 1) {
            stage_bytes<false>(reinterpret_cast<const uint8_t*>(x), 4u * k, lbase + L.x, wave, 0u, 1u);
        } else {
#pragma unroll
            for (uint32_t b = 0; b < (uint32_t)NB; ++b)
                stage_blocks_swizzled(x + (size_t)b * ldx, nb, lbase + L.x + b * L.xrow, wave, b % WAVES);
            if constexpr (MODE == NB_NORM) stage_blocks_swizzled(nw, nb, lbase + L.nw, wave, NB % WAVES);
        }
    }
    uint32_t mine;
    if constexpr (GLU) {
        mine = stage_rows<true>(w + (size_t)g0 * row_bytes, row_bytes, row_bytes, h, lbase + L.w, L.wrow, wave, 0u,
                                WAVES);
        mine += stage_rows<true>(w + (size_t)(H + g0) * row_bytes, row_bytes, row_bytes, h, lbase + L.w2, L.wrow, wave,
                                 0u, WAVES);
    } else {
        mine = stage_rows<true>(w + (size_t)row0 * row_bytes, row_bytes, row_bytes, rows, lbase + L.w, L.wrow, wave,
                                0u, WAVES);
    }
    wait_vm_lds_upto(mine);  // this wave's activation loads (issued before its weights) have landed
    lds_sync();

    int8_t* aq = reinterpret_cast<int8_t*>(base + L.qs);
    float* asc = reinterpret_cast<float*>(base + L.scales);
    float* asm_ = reinterpret_cast<float*>(base + L.sums);
    int32_t* atot = reinterpret_cast<int32_t*>(base + L.totals);
    if constexpr (MODE == NB_F32 && NB == 1) {
        // One row: the quantiser spread over the workgroup, 8 lanes a block
        // (one wave a row would take every block's arithmetic alone), the
        // quarters read before the quantised row overwrites them.
        const uint32_t jobs = nb * 8u;
        float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t < jobs) xv = *reinterpret_cast<const float4*>(base + L.x + 16u * t);
        lds_sync();
        if (t < jobs) {  // the same for the 8 lanes of a block (jobs a multiple of 8)
            const Q8Quad q = quantize_quad(xv.x, xv.y, xv.z, xv.w);
            *reinterpret_cast<uint32_t*>(aq + 4u * t) = q.packed;
            if ((t & 7u) == 0) {
                asc[t >> 3] = q.scale;
                if constexpr (KIND == 2) asm_[t >> 3] = q.sum;
                if constexpr (KIND == 1) atot[t >> 3] = q.total;
            }
        }
    } else if constexpr (MODE != NB_QUANT) {
        // wave b: row b, lane c its block c (lanes past the row hold zeros),
        // its pieces read where the swizzled staging put them
        const bool live = lane < nb;
        float v[32], nv[32];
        if (wave < (uint32_t)NB) {
            const float4* xs = reinterpret_cast<const float4*>(base + L.x + wave * L.xrow) + 8u * lane;
            const float4* ws = reinterpret_cast<const float4*>(base + L.nw) + 8u * lane;
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) {
                const uint32_t slot = (i + lane) & 7u;
                const float4 q = live ? xs[slot] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                v[4 * i] = q.x, v[4 * i + 1] = q.y, v[4 * i + 2] = q.z, v[4 * i + 3] = q.w;
                if constexpr (MODE == NB_NORM) {
                    const float4 g = live ? ws[slot] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    nv[4 * i] = g.x, nv[4 * i + 1] = g.y, nv[4 * i + 2] = g.z, nv[4 * i + 3] = g.w;
                }
            }
        }
        lds_sync();  // every row is in registers: the quantised rows may overwrite them
        if (wave < (uint32_t)NB) {
            if constexpr (MODE == NB_NORM) {
                float sq[32];
#pragma unroll
                for (int i = 0; i < 32; ++i) sq[i] = v[i] * v[i];
                const float total = ordered_sum_wave<32>(sq);
                const float root = __builtin_sqrtf(total / (float)k + eps);
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const float q = v[i] / root;
                    v[i] = q * nv[i];
                }
            }
            if (live) {
                uint32_t packed[8];
                float scale, sum;
                int total;
                quantize_block32(v, packed, scale, sum, total);
                uint4* to = reinterpret_cast<uint4*>(aq + (size_t)wave * L.arow + lane * 32u);
                to[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
                to[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
                const uint32_t at = wave * (L.trow >> 2) + lane;
                asc[at] = scale;
                if constexpr (KIND == 2) asm_[at] = sum;
                if constexpr (KIND == 1) atot[at] = total;
            }
        }
    }
    // the zero piece (below the weights; any staged f32 rows are in
    // registers or quantised by now)
    for (uint32_t z = t; z < 128u; z += THREADS) reinterpret_cast<float*>(base + L.zeros)[z] = 0.0f;
    wait_vm_lds<0>();  // this wave's weights
    lds_sync();

    // The lane's place in the MFMA operands: lr = lane % 16 (a weight row of
    // A, a (row, block) column of B), lq = lane / 16 (its k group).
    const uint32_t lr = lane & 15u, lq = lane >> 4;
    const uint32_t chunk = min(nb, NB_CHUNK), pstride = L.pstride;
    float* parts = reinterpret_cast<float*>(base + L.part);
    float* outs = reinterpret_cast<float*>(base + L.outs);
    const uint32_t tstride = L.trow >> 2, wstride = L.wrow;
    // A phase takes tpp tiles of 16 weight rows (2 only up to 8 rows): the
    // output this thread adds up is row fb, weight row 16·(c + ft) + fr.
    const uint32_t ft = tpp > 1u ? t >> 7 : 0u;
    const uint32_t fb = tpp > 1u ? (t >> 4) & 7u : t >> 4, fr = t & 15u;
    const uint32_t prow = L.prow, tile_floats = (uint32_t)NB * prow;
    // The fold of one phase: this thread adds its output's contributions of
    // the chunk (cl blocks, in `from`) in block order to its running sum,
    // and after a tile's last chunk stores the output (tile oc).
    float acc = 0.0f;
    auto fold = [&](const float* from, uint32_t cl, bool live, uint32_t oc, bool last) {
        if (!live) return;
        // read 32 at a time into registers before they are added
        const float* cp = from + ft * tile_floats + fb * prow + fr * pstride;
        uint32_t i = 0;
        if (tree) {
            Fold4 u;
            for (; i + 32u <= cl; i += 32u) {
                float2 vv[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) vv[e] = *reinterpret_cast<const float2*>(cp + i + 2u * e);
#pragma unroll
                for (int e = 0; e < 16; e += 2) u.add4(vv[e].x, vv[e].y, vv[e + 1].x, vv[e + 1].y);
            }
            for (; i < cl; ++i) u.s0 += cp[i];
            acc += u.total();
        } else {
            for (; i + 32u <= cl; i += 32u) {
                float2 vv[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) vv[e] = *reinterpret_cast<const float2*>(cp + i + 2u * e);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    acc += vv[e].x;
                    acc += vv[e].y;
                }
            }
            for (; i < cl; ++i) acc += cp[i];
        }
        if (last) {
            const uint32_t r = 16u * oc + fr;
            if constexpr (GLU) {
                outs[fb * tr + r] = acc;
            } else {
                const uint32_t row = row0 + r;
                dst[(size_t)fb * n + row] = bias ? acc + bias[(size_t)fb * bias_ld + row] : acc;
            }
            acc = 0.0f;
        }
    };
    // Two buffers: the previous phase's fold, held here, runs after this
    // phase's contributions are written (one barrier a phase).
    uint32_t buf = 0, held_cl = 0, held_oc = 0;
    bool held = false, held_live = false, held_last = false;
    for (uint32_t c = 0; c * 16u < rows; c += tpp) {
        const uint32_t fc = c + ft;  // the tile of this thread's output
        const bool folds = ft < tpp && fb < (uint32_t)NB && 16u * fc + fr < rows;
        for (uint32_t q0 = 0; q0 < nb; q0 += chunk) {
            const uint32_t cl = min(chunk, nb - q0);  // blocks of this chunk, a multiple of 8
            const uint32_t u0 = PER * wave;           // this wave's first block of the chunk
            float* part = parts + buf * L.region;     // this phase's contributions
            if (u0 < cl) {
                // Pairs of blocks on v_mfma_i32_16x16x64_i8: A is the tile's 16
                // weight rows (lane (m, g): row m, half g % 2 of block g / 2 of
                // the pair), B's 16 columns n = b + 8 j are activation row b in
                // block j of the pair (lane (n, g): zero unless g / 2 == j), so
                // D[m][n] is weight row m's dot product with row b over block j
                // alone. A lane's outputs: weight rows 4 g + i of column n.
                // Every pair's operands at constant offsets from one base a
                // phase (pairs 2·BB bytes apart in a weight row, 64 in an
                // activation row, 2 entries in a table).
                const uint32_t jj = lq >> 1, hh = lq & 1u, ab = lr & 7u, aj = lr >> 3;
                const bool breal = ab < (uint32_t)NB && aj == jj;
                const uint32_t b0 = q0 + u0;  // the wave's first block of the chunk (even)
                // B: row ab's half hh of block b0 + 2p + aj, or the zero piece
                // for a lane whose values must be zero
                const uint8_t* bq =
                    breal ? reinterpret_cast<const uint8_t*>(aq) + (size_t)ab * L.arow + 32u * (b0 + aj) + 8u * hh
                          : base + L.zeros + 8u * hh;
                const uint32_t sat = min(ab, (uint32_t)NB - 1u) * tstride + b0 + aj;
                v4i bv[PP];
                float sx[PP], ex[PP];
#pragma unroll
                for (uint32_t p = 0; p < PP; ++p) {
                    bv[p] = pair_acts_at(bq + 64u * p);
                    sx[p] = asc[sat + 2u * p];
                    ex[p] = 0.0f;
                    if constexpr (KIND == 2) ex[p] = asm_[sat + 2u * p];
                    if constexpr (KIND == 1) ex[p] = __int_as_float(-8 * atot[sat + 2u * p]);
                }
                // the lane's output i goes to its slot (weight row 4 lq + i of
                // row ab), or to the lane's own dummy slot when the region has
                // no such slot (ab past NB; a row past 8 in a tile of 8 rows);
                // a slot of a weight row past the tile's rows is never folded
                float* dummy = reinterpret_cast<float*>(base + L.dummy) + lane;
#pragma unroll
                for (uint32_t tt = 0; tt < 2u; ++tt) {
                const uint32_t ct = c + tt;
                if (tt >= tpp || ct * 16u >= rows) break;
                const uint32_t wrt = min(16u * ct + lr, rows - 1u);
                const uint8_t* trow = GLU ? (wrt < h ? base + L.w + wrt * wstride : base + L.w2 + (wrt - h) * wstride)
                                          : base + L.w + wrt * wstride;
                const uint8_t* wq = trow + BB * (b0 + jj) + (KIND == 2 ? 4u : 2u) + 8u * hh;
                const uint8_t* dq[4];
                float* wp[4];
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    const uint32_t r = min(16u * ct + 4u * lq + i, rows - 1u);
                    const uint8_t* rp = GLU ? (r < h ? base + L.w + r * wstride : base + L.w2 + (r - h) * wstride)
                                            : base + L.w + r * wstride;
                    dq[i] = rp + BB * (b0 + aj);
                    const bool slot = ab < (uint32_t)NB && 4u * lq + i < L.rt;
                    wp[i] = slot ? part + tt * tile_floats + ab * prow + (4u * lq + i) * pstride + u0 + aj : dummy;
                }
                v4i av[PP];
                uint32_t dm[PP][4];
#pragma unroll
                for (uint32_t p = 0; p < PP; ++p) {
                    av[p] = pair_weights_at<KIND>(wq + 2u * BB * p);
#pragma unroll
                    for (uint32_t i = 0; i < 4; ++i) {
                        if constexpr (KIND == 2) dm[p][i] = *reinterpret_cast<const uint32_t*>(dq[i] + 2u * BB * p);
                        else dm[p][i] = *reinterpret_cast<const uint16_t*>(dq[i] + 2u * BB * p);
                    }
                }
                v4i tv[PP];
#pragma unroll
                for (uint32_t p = 0; p < PP; ++p) {
                    v4i cin = {0, 0, 0, 0};
                    if constexpr (KIND == 1) {
                        const int neg8 = __float_as_int(ex[p]);
                        cin = v4i{neg8, neg8, neg8, neg8};
                    }
                    tv[p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[p], bv[p], cin, 0, 0, 0);
                }
#pragma unroll
                for (uint32_t p = 0; p < PP; ++p) {
#pragma unroll
                    for (uint32_t i = 0; i < 4; ++i) {
                        const float ft = (float)tv[p][i], d = half_value(dm[p][i] & 0xffffu);
                        float cv;
                        if constexpr (KIND == 0) {
                            const float sc = d * sx[p];
                            cv = ft * sc;
                        } else if constexpr (KIND == 1) {
                            const float pr = ft * d;
                            cv = pr * sx[p];
                        } else {
                            const float sc = d * sx[p];
                            const float f = sc * ft;
                            const float g = half_value(dm[p][i] >> 16) * ex[p];
                            cv = f + g;
                        }
                        wp[i][2u * p] = cv;
                    }
                }
                }
            }
            const bool last = q0 + chunk >= nb;
            if (bufs > 1u) {
                if (held) fold(parts + (buf ^ 1u) * L.region, held_cl, held_live, held_oc, held_last);
                lds_sync();  // this phase's contributions written; the held fold done with the other buffer
                held = true, held_cl = cl, held_live = folds, held_oc = fc, held_last = last;
                buf ^= 1u;
            } else {
                lds_sync();
                fold(part, cl, folds, fc, last);
                lds_sync();
            }
        }
    }
    if (held) fold(parts + (buf ^ 1u) * L.region, held_cl, held_live, held_oc, held_last);
    if constexpr (GLU) {
        // SwiGLU one output a thread, then the quantiser, 8 lanes a block
        lds_sync();
        float* act_out = outs + NB * tr;
        for (uint32_t o = t; o < (uint32_t)NB * h; o += THREADS) {
            const uint32_t b = o / h, i = o - b * h;
            act_out[o] = swiglu_value(outs[b * tr + i], outs[b * tr + h + i]);
        }
        lds_sync();
        const uint32_t hb = h >> 5, Hb = H >> 5, sub = t & 7u;
        for (uint32_t g = t >> 3; g < (uint32_t)NB * hb; g += THREADS / 8u) {  // uniform across each 8-lane group
            const uint32_t b = g / hb, blk = g - b * hb;
            const float4 v4 = *reinterpret_cast<const float4*>(act_out + b * h + blk * 32u + sub * 4u);
            const Q8Quad q = quantize_quad(v4.x, v4.y, v4.z, v4.w);
            const uint32_t col = g0 + blk * 32u + sub * 4u;
            *(uint32_t*)((int8_t*)glu.qs + (size_t)b * H + col) = q.packed;
            if (sub == 0) {
                const size_t at = (size_t)b * Hb + (g0 >> 5) + blk;
                ((float*)glu.scales)[at] = q.scale;
                ((float*)glu.sums)[at] = q.sum;
                ((int32_t*)glu.totals)[at] = q.total;
            }
        }
    }
}

// ------------------------------------------------- thread per output

// One thread per output, adding its blocks in order from byte loads: any
// alignment, any k (block_matmul_f32's division of work, cuda/kernels.cu:1230-1246).
template <int KIND>
__global__ __launch_bounds__(256) void k_block_matmul_thread(const uint8_t* __restrict__ w, Activations act,
                                                             float* __restrict__ dst,
                                                             const float* __restrict__ bias, uint32_t n,
                                                             uint32_t k, uint32_t count) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= count) return;
    const uint32_t row = i / n, col = i - row * n;
    const uint32_t nb = k >> 5;
    constexpr uint32_t BB = Fmt<KIND>::BB;
    const uint8_t* wr = w + (size_t)col * nb * BB;
    const int8_t* qr = act.qs + (size_t)row * k;
    float sum = 0.0f;
    for (uint32_t blk = 0; blk < nb; ++blk) {
        const uint8_t* p = wr + blk * BB;
        const int8_t* q = qr + blk * 32u;
        const float d = half_value((uint32_t)p[0] | (uint32_t)p[1] << 8);
        const float sx = act.scales[(size_t)row * nb + blk];
        if constexpr (KIND == 0) {
            int t = 0;
            for (int e = 0; e < 32; ++e) t += (int)(int8_t)p[2 + e] * (int)q[e];
            const float s = d * sx;
            sum += (float)t * s;
        } else if constexpr (KIND == 1) {
            int t = 0;
            for (int e = 0; e < 16; ++e) {
                t += ((int)(p[2 + e] & 0x0f) - 8) * (int)q[e];
                t += ((int)(p[2 + e] >> 4) - 8) * (int)q[e + 16];
            }
            const float c = (float)t * d;
            sum += c * sx;
        } else {
            int t = 0;
            for (int e = 0; e < 16; ++e) {
                t += (int)(p[4 + e] & 0x0f) * (int)q[e];
                t += (int)(p[4 + e] >> 4) * (int)q[e + 16];
            }
            const float m = half_value((uint32_t)p[2] | (uint32_t)p[3] << 8);
            const float s = d * sx;
            const float f = s * (float)t;
            const float g = m * act.sums[(size_t)row * nb + blk];
            sum += f + g;
        }
    }
    dst[i] = bias ? sum + bias[col] : sum;
}

// ---------------------------------------------------------------- gather

// One thread per output element: element i is value i % width of table row
// ids[i / width], dequantised as dequantize_* (quant.cr:537-556). An id out of
// range writes 0 and is reported: errors[0] counts reports, and the first
// reporter writes the id and the row count (cuda/kernels.cu:176-184).
template <int KIND>
__global__ __launch_bounds__(256) void k_gather_blocks(const uint8_t* __restrict__ table,
                                                       const int32_t* __restrict__ ids, float* __restrict__ dst,
                                                       int32_t* __restrict__ errors, int32_t rows, uint32_t width,
                                                       uint32_t total) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t r = i / width, e = i - r * width;
    const int32_t id = ids[r];
    if (id < 0 || id >= rows) {
        if (atomicAdd(&errors[0], 1) == 0) {
            errors[1] = id;
            errors[2] = rows;
        }
        dst[i] = 0.0f;
        return;
    }
    constexpr uint32_t BB = Fmt<KIND>::BB;
    const uint8_t* p = table + (size_t)id * (width >> 5) * BB + (e >> 5) * BB;
    const uint32_t at = e & 31u;
    const float d = half_value((uint32_t)p[0] | (uint32_t)p[1] << 8);
    float v;
    if constexpr (KIND == 0) {
        v = (float)(int8_t)p[2 + at] * d;
    } else {
        const uint32_t packed = p[(KIND == 1 ? 2u : 4u) + (at & 15u)];
        const uint32_t q = at < 16u ? (packed & 0x0fu) : (packed >> 4);
        if constexpr (KIND == 1) {
            v = (float)((int)q - 8) * d;
        } else {
            const float m = half_value((uint32_t)p[2] | (uint32_t)p[3] << 8);
            const float s = d * (float)q;
            v = s + m;
        }
    }
    dst[i] = v;
}

// dst[i] = F16 bits of the float whose word is first + i (the test hook
// tmh_debug_f16_words): the device's own f32 -> f16 rounding, swept.
__global__ __launch_bounds__(256) void k_f16_words(uint32_t first, uint32_t count, uint16_t* __restrict__ dst) {
    for (uint64_t i = blockIdx.x * 256u + threadIdx.x; i < count; i += (uint64_t)gridDim.x * 256u)
        dst[i] = (uint16_t)round_to_half_bits(__uint_as_float(first + (uint32_t)i));
}

// The read-rate hook (tmh_debug_read): workgroup b of G reads 16-byte
// pieces b·256 + t, then G·256 further on, four pieces in flight a lane, and
// writes the XOR of what it read to out[b] (so no load can be dropped).
// Pieces = bytes / 16.
typedef uint32_t piece16 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_read_pieces(const piece16* __restrict__ src, uint64_t pieces,
                                                     uint32_t* __restrict__ out) {
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    piece16 acc = {0u, 0u, 0u, 0u};
    for (; i + 3u * stride < pieces; i += 4u * stride) {
        const piece16 a = __builtin_nontemporal_load(src + i);
        const piece16 b = __builtin_nontemporal_load(src + i + stride);
        const piece16 c = __builtin_nontemporal_load(src + i + 2u * stride);
        const piece16 d = __builtin_nontemporal_load(src + i + 3u * stride);
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < pieces; i += stride) acc ^= __builtin_nontemporal_load(src + i);
    uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) v ^= __shfl_xor(v, o);
    __shared__ uint32_t waves[4];
    if ((threadIdx.x & 63u) == 0) waves[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = waves[0] ^ waves[1] ^ waves[2] ^ waves[3];
}

// ---------------------------------------------------------------- launchers

hipError_t launch_read(const void* src, uint64_t bytes, uint32_t workgroups, uint32_t* out, hipStream_t stream) {
    if (bytes < 16u || workgroups == 0) return hipSuccess;
    TMH_LAUNCH(k_read_pieces, dim3(workgroups), dim3(256), 0, stream, (const piece16*)src, bytes / 16u, out);
    return hipGetLastError();
}

hipError_t launch_f16_words(uint32_t first, uint32_t count, uint16_t* dst, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    const uint32_t grid = std::min<uint32_t>((count + 255u) / 256u, 65536u);
    TMH_LAUNCH(k_f16_words, dim3(grid), dim3(256), 0, stream, first, count, dst);
    return hipGetLastError();
}

hipError_t launch_quantize(const float* x, uint32_t ldx, uint32_t rows, uint32_t k, float* scales, float* sums,
                           int32_t* totals, int8_t* qs, hipStream_t stream) {
    const uint32_t nb = k >> 5;
    const uint32_t blocks = rows * nb;
    if (blocks == 0) return hipSuccess;
    const uint32_t grid = (blocks * 8u + 255u) / 256u;
    const bool vec = ((uintptr_t)x % 16u == 0) && (ldx % 4u == 0);
    if (vec)
        TMH_LAUNCH(k_quantize_rows_q8<true>, dim3(grid), dim3(256), 0, stream, x, ldx, nb, k, blocks, scales,
                           sums, totals, qs);
    else
        TMH_LAUNCH(k_quantize_rows_q8<false>, dim3(grid), dim3(256), 0, stream, x, ldx, nb, k, blocks,
                           scales, sums, totals, qs);
    return hipGetLastError();
}

// Padded LDS row stride, in floats, for a row of nb contributions: a
// multiple of 4 (16-byte reads) whose quarter is odd, so 8 consecutive
// output rows start in 8 different 16-byte bank groups.
static uint32_t lanes_stride(uint32_t nb) {
    uint32_t s = (nb + 3u) & ~3u;
    if (((s >> 2) & 1u) == 0) s += 4u;
    return s;
}

static constexpr size_t LANES_LDS_LIMIT = 56u * 1024u;

// Chooses the rows per workgroup: a multiple of the rows one step covers,
// with every output's fold on its own thread and the contributions within
// the LDS limit, as large as still leaves about two workgroups per compute
// unit, else the smallest. From 8 activation rows, whose reads of each
// pair's activations the rows of a workgroup share: the tile with the
// fewest rows on the busiest compute unit (rounds of workgroups × rows),
// the larger on a tie.
static uint32_t lanes_tile(uint32_t nb, uint32_t nbatch, uint32_t n, int compute_units) {
    const uint32_t np = nb / 2u;
    const uint32_t rpi = 256u / np;
    const uint32_t stride = lanes_stride(nb);
    const uint32_t cus = (uint32_t)(compute_units > 0 ? compute_units : 256);
    auto fits = [&](uint32_t tr) { return nbatch * tr <= 256u && (size_t)nbatch * tr * stride * 4u <= LANES_LDS_LIMIT; };
    uint32_t best = rpi;
    if (nbatch >= 8u) {
        uint64_t best_cost = ~0ull;
        for (uint32_t tr = rpi; fits(tr); tr += rpi) {
            const uint64_t groups = (n + tr - 1u) / tr;
            const uint64_t cost = (groups + cus - 1u) / cus * tr;
            if (cost <= best_cost) best_cost = cost, best = tr;
        }
        return best;
    }
    const uint64_t want = (uint64_t)2u * cus;
    for (uint32_t m = 2;; ++m) {
        const uint32_t tr = rpi * m;
        if (!fits(tr)) break;
        if ((n + tr - 1u) / tr < want) break;
        best = tr;
    }
    return best;
}

template <int KIND, int NB>
static hipError_t launch_lanes_nb(const uint8_t* w, Activations act, float* dst, const float* bias, uint32_t bias_ld,
                                  uint32_t n, uint32_t k, int compute_units, hipStream_t stream) {
    const uint32_t nb = k >> 5;
    const uint32_t tr = lanes_tile(nb, NB, n, compute_units);
    const uint32_t stride = lanes_stride(nb);
    const size_t lds = (size_t)NB * tr * stride * sizeof(float);
    const uint32_t grid = (n + tr - 1u) / tr;
    if (tree_fold())
        TMH_LAUNCH((k_matvec<KIND, NB, true>), dim3(grid), dim3(256), lds, stream, w, act, dst, bias, bias_ld, n, k,
                   tr, stride);
    else
        TMH_LAUNCH((k_matvec<KIND, NB, false>), dim3(grid), dim3(256), lds, stream, w, act, dst, bias, bias_ld, n, k,
                   tr, stride);
    return hipGetLastError();
}

template <int KIND>
static hipError_t launch_lanes(const uint8_t* w, Activations act, float* dst, const float* bias, uint32_t rows,
                               uint32_t n, uint32_t k, int compute_units, hipStream_t stream, uint32_t bias_ld = 0) {
    // Activation rows in groups of 8, 4, 2 and 1 (a thread holds its pair
    // of every row of a group in registers; measured, one group of 8 beats
    // two of 4, which read the weights twice): each output depends on
    // its own row only, so the grouping changes no bits.
    const uint32_t nb = k >> 5;
    const uint32_t rpi = 256u / (nb / 2u);
    const size_t smallest = (size_t)rpi * lanes_stride(nb) * sizeof(float);  // LDS of one row group
    uint32_t done = 0;
    while (done < rows) {
        const uint32_t left = rows - done;
        Activations a = act;
        a.scales += (size_t)done * nb;
        a.sums += (size_t)done * nb;
        a.totals += (size_t)done * nb;
        a.qs += (size_t)done * k;
        float* d = dst + (size_t)done * n;
        const float* bi = bias ? bias + (size_t)done * bias_ld : nullptr;
        hipError_t err;
        uint32_t take;
        if (left >= 8 && 8u * smallest <= LANES_LDS_LIMIT)
            err = launch_lanes_nb<KIND, 8>(w, a, d, bi, bias_ld, n, k, compute_units, stream), take = 8;
        else if (left >= 4 && 4u * smallest <= LANES_LDS_LIMIT)
            err = launch_lanes_nb<KIND, 4>(w, a, d, bi, bias_ld, n, k, compute_units, stream), take = 4;
        else if (left >= 2 && 2u * smallest <= LANES_LDS_LIMIT)
            err = launch_lanes_nb<KIND, 2>(w, a, d, bi, bias_ld, n, k, compute_units, stream), take = 2;
        else err = launch_lanes_nb<KIND, 1>(w, a, d, bi, bias_ld, n, k, compute_units, stream), take = 1;
        if (err != hipSuccess) return err;
        done += take;
    }
    return hipSuccess;
}

template <int KIND>
static hipError_t launch_thread(const uint8_t* w, Activations act, float* dst, const float* bias, uint32_t rows,
                                uint32_t n, uint32_t k, hipStream_t stream) {
    const uint32_t count = rows * n;
    const uint32_t grid = (count + 255u) / 256u;
    TMH_LAUNCH(k_block_matmul_thread<KIND>, dim3(grid), dim3(256), 0, stream, w, act, dst, bias, n, k, count);
    return hipGetLastError();
}

// Whether the lanes kernel can take a weight: rows of an even number of
// blocks, at most 512, starting dword-aligned.
static bool lanes_fit(const uint8_t* w, uint32_t k) {
    const uint32_t nb = k >> 5;
    return nb >= 2 && nb % 2 == 0 && nb <= 512 && (uintptr_t)w % 4u == 0;
}

// LDS of the one-row kernel before its contributions: values, scales, extras.
static size_t row_act_lds(uint32_t k) { return (size_t)k + 8u * (k >> 5); }

// Weight bytes a workgroup of the one-row kernel aims to stream: enough
// steps to keep loads in flight and to amortise the workgroup's own
// quantise pass and fold (TMH_ROW_TILE_BYTES overrides, for tuning).
static size_t row_tile_bytes() {
    static const size_t bytes = [] {
        const char* env = getenv("TMH_ROW_TILE_BYTES");
        long v = env ? atol(env) : 0;
        return v > 0 ? (size_t)v : (size_t)48 * 1024;
    }();
    return bytes;
}

// Rows per tile of the one-row kernel: a multiple of the rows one step
// covers, about row_tile_bytes() of weights, within the LDS limit and 256
// folds, and small enough to leave at least `min_tiles` tiles when the
// product has the rows for them.
static uint32_t row_tile(uint32_t nb, uint32_t n, size_t row_bytes_, uint32_t min_tiles) {
    const uint32_t np = nb / 2u;
    const uint32_t rpi = 256u / np;
    const uint32_t stride = lanes_stride(nb);
    const size_t base = row_act_lds(nb * 32u);
    uint32_t m = (uint32_t)(row_tile_bytes() / (row_bytes_ * rpi));
    if (m < 1) m = 1;
    const uint32_t fill = n / (rpi * (min_tiles > 0 ? min_tiles : 1u));
    if (m > fill) m = fill > 0 ? fill : 1;
    while (m > 1 && (rpi * m > 256u || base + (size_t)(rpi * m + 1u) * stride * 4u > LANES_LDS_LIMIT)) --m;
    return rpi * m;
}

bool row_kernel_fits(uint32_t mode, const uint8_t* w, uint32_t k) {
    if (mode == 1u /* THREAD */ || !lanes_fit(w, k)) return false;
    const uint32_t nb = k >> 5;
    const uint32_t rpi = 256u / (nb / 2u);
    return row_act_lds(k) + (size_t)(rpi + 1u) * lanes_stride(nb) * 4u <= LANES_LDS_LIMIT;
}

// Workgroups per compute unit of the persistent one-row kernel
// (TMH_ROW_WGS_PER_CU overrides, for tuning).
static uint32_t row_wgs_per_cu() {
    static const uint32_t v = [] {
        const char* env = getenv("TMH_ROW_WGS_PER_CU");
        long x = env ? atol(env) : 0;
        return x > 0 ? (uint32_t)x : 4u;
    }();
    return v;
}

static size_t align16(size_t v) { return (v + 15u) & ~(size_t)15u; }

// Workgroups for `tiles` tiles: at most row_wgs_per_cu() per compute unit
// (measured: evening out the tiles per workgroup did not pay).
static uint32_t balanced_grid(uint32_t tiles, int compute_units) {
    const uint32_t cus = (uint32_t)(compute_units > 0 ? compute_units : 256);
    return std::min<uint32_t>(tiles, cus * row_wgs_per_cu());
}

void plan_row(uint32_t kind, RowProduct& p, int compute_units) {
    (void)compute_units;
    const uint32_t nb = p.k >> 5;
    p.tr = row_tile(nb, p.n, (size_t)nb * block_bytes(kind), 1u);
    p.stride = lanes_stride(nb);
    p.tiles = (p.n + p.tr - 1u) / p.tr;
}

size_t row_act_bytes(const RowProduct& p) { return align16(row_act_lds(p.k)); }

size_t row_part_bytes(const RowProduct& p) { return (size_t)(p.tr + 1u) * p.stride * sizeof(float); }

hipError_t launch_rows(uint32_t kind, const RowProduct* table, const uint32_t* owner, uint32_t tiles,
                       size_t act_bytes, size_t part_bytes, int compute_units, hipStream_t stream) {
    if (tiles == 0) return hipSuccess;
    const uint32_t grid = balanced_grid(tiles, compute_units);
    const uint32_t ab = (uint32_t)align16(act_bytes);
    const size_t lds = ab + part_bytes;
    const bool tree = tree_fold();
    if (kind == 0) {
        if (tree)
            TMH_LAUNCH((k_matvec_rows<0, Depth<0>::D, true>), dim3(grid), dim3(256), lds, stream, table,
                       owner, tiles, ab);
        else
            TMH_LAUNCH((k_matvec_rows<0, Depth<0>::D, false>), dim3(grid), dim3(256), lds, stream, table,
                       owner, tiles, ab);
    } else if (kind == 1) {
        if (tree)
            TMH_LAUNCH((k_matvec_rows<1, Depth<1>::D, true>), dim3(grid), dim3(256), lds, stream, table,
                       owner, tiles, ab);
        else
            TMH_LAUNCH((k_matvec_rows<1, Depth<1>::D, false>), dim3(grid), dim3(256), lds, stream, table,
                       owner, tiles, ab);
    } else {
        if (tree)
            TMH_LAUNCH((k_matvec_rows<2, Depth<2>::D, true>), dim3(grid), dim3(256), lds, stream, table,
                       owner, tiles, ab);
        else
            TMH_LAUNCH((k_matvec_rows<2, Depth<2>::D, false>), dim3(grid), dim3(256), lds, stream, table,
                       owner, tiles, ab);
    }
    return hipGetLastError();
}

hipError_t launch_row(uint32_t kind, const uint8_t* w, const float* x, float* dst, const float* bias, uint32_t n,
                      uint32_t k, int compute_units, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const uint32_t cus = (uint32_t)(compute_units > 0 ? compute_units : 256);
    RowProduct p{};
    p.w = w, p.x = x, p.dst = dst, p.bias = bias, p.n = n, p.k = k;
    const uint32_t nb = k >> 5;
    p.tr = row_tile(nb, n, (size_t)nb * block_bytes(kind), cus * row_wgs_per_cu());
    p.stride = lanes_stride(nb);
    p.tiles = (n + p.tr - 1u) / p.tr;
    p.first = 0;
    const uint32_t grid = balanced_grid(p.tiles, compute_units);
    const uint32_t ab = (uint32_t)row_act_bytes(p);
    const size_t lds = ab + row_part_bytes(p);
    const bool tree = tree_fold();
    if (kind == 0) {
        if (tree)
            TMH_LAUNCH((k_matvec_row<0, Depth<0>::D, true>), dim3(grid), dim3(256), lds, stream, p, ab);
        else
            TMH_LAUNCH((k_matvec_row<0, Depth<0>::D, false>), dim3(grid), dim3(256), lds, stream, p, ab);
    } else if (kind == 1) {
        if (tree)
            TMH_LAUNCH((k_matvec_row<1, Depth<1>::D, true>), dim3(grid), dim3(256), lds, stream, p, ab);
        else
            TMH_LAUNCH((k_matvec_row<1, Depth<1>::D, false>), dim3(grid), dim3(256), lds, stream, p, ab);
    } else {
        if (tree)
            TMH_LAUNCH((k_matvec_row<2, Depth<2>::D, true>), dim3(grid), dim3(256), lds, stream, p, ab);
        else
            TMH_LAUNCH((k_matvec_row<2, Depth<2>::D, false>), dim3(grid), dim3(256), lds, stream, p, ab);
    }
    return hipGetLastError();
}

// Ring slots and workgroups per compute unit of the streamed kernel
// (TMH_STREAM_RING, TMH_STREAM_WGS override, for tuning).
static uint32_t env_u32(const char* name, uint32_t fallback) {
    const char* env = getenv(name);
    const long v = env ? atol(env) : 0;
    return v > 0 ? (uint32_t)v : fallback;
}

static constexpr uint32_t STREAM_RING_MIN = 2, STREAM_RING_MAX = 8, STREAM_WGS = 6, STREAM_RAMP_PERCENT = 20;
static constexpr size_t STREAM_LDS_LIMIT = 64u * 1024u, CU_LDS = 160u * 1024u;

bool plan_stream(uint32_t kind, std::vector<StreamProduct>& products, int compute_units, StreamLaunch& l,
                 std::vector<StreamStart>& starts, uint32_t wgs_per_cu) {
    const uint32_t bb = block_bytes(kind);
    uint64_t total = 0;
    uint32_t max_k = 0, part = 0, stage = 0;
    bool bias = false;
    for (StreamProduct& p : products) {
        const uint32_t nb = p.k >> 5;
        if (p.n == 0 || nb < 2 || nb % 2 != 0 || nb > 512 || (uintptr_t)p.w % 4u != 0) return false;
        if (p.mode > STREAM_X_QUANTISED) return false;
        if (p.mode == STREAM_X_RMSNORM && p.aux0 == nullptr) return false;
        if (p.mode == STREAM_X_QUANTISED &&
            ((uintptr_t)p.x % 4u != 0 || p.aux0 == nullptr || (kind != 0 && p.aux1 == nullptr)))
            return false;
        // Floats one staging slot must hold: x (the norm's weights take the
        // second slot), or a quantised row's three parts.
        stage = std::max(stage, p.mode == STREAM_X_QUANTISED
                                    ? (stage_part(p.k) + 2u * stage_part(p.k / 8u)) / 4u
                                    : p.k);
        p.np = nb / 2u;
        p.row_bytes = nb * bb;
        // Rows per step: a pair per thread, within the step's 8 KB after the
        // first row's offset past 16 bytes (at most 12).
        p.rows = std::min(256u / p.np, (STREAM_STEP - 12u) / p.row_bytes);
        if (p.rows == 0) return false;
        p.step_bytes = p.rows * p.row_bytes;
        p.stride = lanes_stride(nb);
        p.steps = (p.n + p.rows - 1u) / p.rows;
        p.first = (uint32_t)total;
        p.wlast = ((uint64_t)(uintptr_t)p.w + (uint64_t)p.n * p.row_bytes - 1u) & ~(uint64_t)15;
        total += p.steps;
        max_k = std::max(max_k, p.k);
        part = std::max(part, p.rows * p.stride);
        bias = bias || p.bias != nullptr;
    }
    if (total == 0 || total > 0x7fffffffull) return false;
    l.total = (uint32_t)total;
    l.act_bytes = (uint32_t)align16((size_t)max_k + 8u * (max_k >> 5));
    l.part_floats = (part + 3u) & ~3u;
    l.has_bias = bias ? 1u : 0u;
    const uint32_t x_floats = (stage + 255u) & ~255u;  // whole 1 KB direct loads
    l.x_floats = x_floats;
    const size_t bias_slots = bias ? 1024u : 0u;
    // One product needs one staging slot and one activation buffer; more
    // need two of each (a workgroup's first two products).
    const size_t buffers = products.size() == 1 ? 1u : 2u;
    // LDS with `ring` slots: the root's slot, biases, ring, contributions,
    // then the activations, no earlier than the end of the x staged from
    // slot R-1.
    auto lds_for = [&](uint32_t ring, size_t& act_offset) {
        const size_t head = 16u + (ring + 1u) * bias_slots;
        act_offset = head + (size_t)ring * STREAM_STEP + 2u * (size_t)l.part_floats * 4u;
        act_offset = std::max(act_offset, head + (size_t)(ring - 1u) * STREAM_STEP + buffers * l.x_floats * 4u);
        return act_offset + buffers * (size_t)l.act_bytes;
    };
    // Measured on the config-2 matvec set: more workgroups per compute unit
    // beat a deeper ring (6 with two slots: 15.9 us; 4 with three: 18.0 us;
    // 3 with four: 21 us), so the ring gets what `wgs` workgroups leave.
    const uint32_t wgs = wgs_per_cu ? wgs_per_cu : env_u32("TMH_STREAM_WGS", STREAM_WGS);
    uint32_t ring = env_u32("TMH_STREAM_RING", 0u);
    size_t act_offset = 0;
    if (ring == 0) {
        const size_t budget = std::min(CU_LDS / wgs, STREAM_LDS_LIMIT);
        ring = STREAM_RING_MIN;
        while (ring < STREAM_RING_MAX && lds_for(ring + 1u, act_offset) <= budget) ++ring;
    }
    ring = std::min(std::max(ring, STREAM_RING_MIN), STREAM_RING_MAX);
    l.ring = ring;
    l.lds = lds_for(ring, act_offset);
    if (l.lds > STREAM_LDS_LIMIT) {
        l.x_floats = 0;  // no staging: x too long
        l.lds = lds_for(ring, act_offset);
    }
    l.act_offset = (uint32_t)act_offset;
    if (l.lds > STREAM_LDS_LIMIT) return false;
    // Workgroups resident at once (LDS allocated in 1 KB pieces), so that no
    // workgroup waits for another to finish.
    const uint32_t fit = (uint32_t)std::max<size_t>(1u, CU_LDS / ((l.lds + 1023u) & ~(size_t)1023u));
    const uint32_t cus = (uint32_t)(compute_units > 0 ? compute_units : 256);
    l.grid = (uint32_t)std::min<uint64_t>(total, (uint64_t)cus * std::min(wgs, fit));
    // Workgroup b's steps start at bound(b): shares that shrink linearly
    // from the first workgroup to the last, by `ramp` at either end. Later
    // workgroups are dispatched later and their first activations arrive
    // later, behind the earlier ones' weight loads (measured: the loop
    // starts ≈1.6 us after launch for the first workgroups, ≈4.3 us for the
    // last, and then runs at the same rate), so equal shares end unevenly.

    const char* ramp_env = getenv("TMH_STREAM_RAMP");  // percent, for tuning
    const double ramp = ramp_env ? atof(ramp_env) : (double)STREAM_RAMP_PERCENT;
    const double a = ramp / 100.0, G = (double)l.grid;
    auto bound = [&](uint32_t b) -> uint64_t {
        if (b >= l.grid) return total;
        const double w = b * (1.0 + a * (1.0 - b / G)) / G;  // cumulative share, 0 ... 1
        return std::min<uint64_t>(total, (uint64_t)(w * (double)total));
    };
    starts.assign(l.grid, StreamStart{});
    uint32_t pi = 0;
    for (uint32_t b = 0; b < l.grid; ++b) {
        const uint64_t s = bound(b), e = bound(b + 1u);
        while (pi + 1u < products.size() && products[pi].first + products[pi].steps <= s) ++pi;
        StreamStart& st = starts[b];
        const StreamProduct& p = products[pi];
        const uint32_t sp = (uint32_t)s - p.first;
        st.s_begin = (uint32_t)s, st.s_end = (uint32_t)e, st.first_pi = pi;
        st.src = (uint64_t)(uintptr_t)p.w + (uint64_t)sp * p.step_bytes, st.wlast = p.wlast;
        st.bias = p.bias ? p.bias : p.x, st.has = p.bias ? 1u : 0u;
        st.x0 = p.x, st.k0 = p.k, st.mode0 = p.mode, st.a0 = p.aux0, st.a1 = kind != 0 ? p.aux1 : nullptr;
        // A second product is staged with the first when both take f32 x.
        const bool two = e > s && (uint64_t)p.first + p.steps < e && p.mode == STREAM_X_F32 &&
                         products[pi + 1u].mode == STREAM_X_F32;
        st.x1 = two ? products[pi + 1u].x : nullptr, st.k1 = two ? products[pi + 1u].k : 0u;
        st.left = p.steps - sp, st.step_bytes = p.step_bytes, st.rows = p.rows, st.row = sp * p.rows, st.n = p.n;
    }
    return true;
}

template <int KIND, bool HB>
static hipError_t launch_stream_kind(const StreamLaunch& l, hipStream_t stream) {
#define TMH_STREAM(RING)                                                                                     \
    case RING:                                                                                               \
        if (l.tree)                                                                                          \
            TMH_LAUNCH((k_matvec_stream<KIND, RING, HB, true>), dim3(l.grid), dim3(256), l.lds, stream,      \
                       l.table, l.starts, l.total, l.act_bytes, l.part_floats, l.x_floats, l.act_offset);    \
        else                                                                                                 \
            TMH_LAUNCH((k_matvec_stream<KIND, RING, HB, false>), dim3(l.grid), dim3(256), l.lds, stream,     \
                       l.table, l.starts, l.total, l.act_bytes, l.part_floats, l.x_floats, l.act_offset);    \
        break;
    switch (l.ring) {
        TMH_STREAM(2) TMH_STREAM(3) TMH_STREAM(4) TMH_STREAM(5) TMH_STREAM(6) TMH_STREAM(7) TMH_STREAM(8)
    default:
        return hipErrorInvalidValue;
    }
#undef TMH_STREAM
    return hipGetLastError();
}

hipError_t launch_stream(uint32_t kind, const StreamLaunch& given, hipStream_t stream) {
    StreamLaunch l = given;
    l.tree = tree_fold() ? 1u : 0u;
    if (l.grid == 0) return hipSuccess;
    switch (kind * 2u + l.has_bias) {
    case 0: return launch_stream_kind<0, false>(l, stream);
    case 1: return launch_stream_kind<0, true>(l, stream);
    case 2: return launch_stream_kind<1, false>(l, stream);
    case 3: return launch_stream_kind<1, true>(l, stream);
    case 4: return launch_stream_kind<2, false>(l, stream);
    default: return launch_stream_kind<2, true>(l, stream);
    }
}

template <int KIND>
static hipError_t launch_mfma(const uint8_t* w, Activations act, float* dst, const float* bias, uint32_t rows,
                              uint32_t n, uint32_t k, hipStream_t stream) {
    const dim3 grid((n + MM_TILE - 1u) / MM_TILE, (rows + MM_TILE - 1u) / MM_TILE);
    TMH_LAUNCH(k_matmul_mfma<KIND>, grid, dim3(256), 0, stream, w, act, dst, bias, rows, n, k);
    return hipGetLastError();
}

// The staged matrix-core kernel takes k a multiple of 256 (whole stages of
// 8 blocks) over 16-byte aligned weights and activation parts (its direct
// loads bring 16 bytes a lane).
static bool mx_fits(const uint8_t* w, const Activations& act, uint32_t kind, uint32_t k) {
    const uint32_t nb = k >> 5;
    const uintptr_t extra = kind == 2 ? (uintptr_t)act.sums : 0;
    return k % 32u == 0 && nb >= MX_STAGE && nb % MX_STAGE == 0 &&
           (((uintptr_t)w | (uintptr_t)act.qs | (uintptr_t)act.scales | extra) % 16u) == 0;
}

template <int KIND>
static hipError_t launch_mx(bool fused, const uint8_t* w, Activations act, float* dst, const float* bias,
                            uint32_t rows, uint32_t n, uint32_t k, hipStream_t stream) {
    const uint32_t tiles_m = (rows + MX_TILE - 1u) / MX_TILE, tiles = tiles_m * ((n + MX_TILE - 1u) / MX_TILE);
    if (fused)
        TMH_LAUNCH((k_matmul_mx<KIND, true>), dim3(tiles), dim3(MX_THREADS), 0, stream, w, act, dst, bias,
                           rows, n, k, tiles_m, tiles);
    else
        TMH_LAUNCH((k_matmul_mx<KIND, false>), dim3(tiles), dim3(MX_THREADS), 0, stream, w, act, dst, bias,
                           rows, n, k, tiles_m, tiles);
    return hipGetLastError();
}

// Activation rows from which AUTO takes the matrix cores rather than lanes.
static constexpr uint32_t MATRIX_ROWS = 32;

// AUTO takes the few-rows kernel from 9 rows to 16, where the lanes kernels
// would read the weights twice (measured on config 3's shapes: at 8 rows the
// lanes kernel is as fast or faster, at 16 the few-rows one is 1.2-1.8x).
static constexpr uint32_t FEW_MIN_ROWS = 9;

// The few-rows kernel: up to 16 rows, whole stages of 16 blocks, 16-byte
// aligned weights and activation parts (its direct loads).
static bool few_fits(const uint8_t* w, const Activations& act, uint32_t kind, uint32_t rows, uint32_t k) {
    const uint32_t nb = k >> 5;
    const uintptr_t extra = kind == 1 ? (uintptr_t)act.totals : kind == 2 ? (uintptr_t)act.sums : 0;
    return rows >= FEW_MIN_ROWS && rows <= FEW_ROWS && k % 32u == 0 && nb >= FEW_STAGE && nb % FEW_STAGE == 0 &&
           (((uintptr_t)w | (uintptr_t)act.qs | (uintptr_t)act.scales | extra) % 16u) == 0;
}

// A ring of 3 stage buffers leaves LDS for two workgroups a compute unit
// (wide products: more than 256 workgroups); narrow ones take a ring of 6.
template <int KIND>
static hipError_t launch_few(const uint8_t* w, Activations act, float* dst, const float* bias, uint32_t bias_ld,
                             uint32_t rows, uint32_t n, uint32_t k, hipStream_t stream) {
    const uint32_t grid = (n + FEW_COLS - 1u) / FEW_COLS;
    const bool tree = tree_fold();
    if (grid > 256u && tree)
        TMH_LAUNCH((k_matmul_few<KIND, 3, 16, true>), dim3(grid), dim3(FEW_THREADS), 0, stream, w, act, dst, bias,
                   bias_ld, rows, n, k);
    else if (grid > 256u)
        TMH_LAUNCH((k_matmul_few<KIND, 3, 16, false>), dim3(grid), dim3(FEW_THREADS), 0, stream, w, act, dst, bias,
                   bias_ld, rows, n, k);
    else if (tree)
        TMH_LAUNCH((k_matmul_few<KIND, 6, 16, true>), dim3(grid), dim3(FEW_THREADS), 0, stream, w, act, dst, bias,
                   bias_ld, rows, n, k);
    else
        TMH_LAUNCH((k_matmul_few<KIND, 6, 16, false>), dim3(grid), dim3(FEW_THREADS), 0, stream, w, act, dst, bias,
                   bias_ld, rows, n, k);
    return hipGetLastError();
}

static hipError_t launch_few_kind(uint32_t kind, const uint8_t* w, Activations act, float* dst, const float* bias,
                                  uint32_t bias_ld, uint32_t rows, uint32_t n, uint32_t k, hipStream_t stream) {
    switch (kind) {
    case 0: return launch_few<0>(w, act, dst, bias, bias_ld, rows, n, k, stream);
    case 1: return launch_few<1>(w, act, dst, bias, bias_ld, rows, n, k, stream);
    default: return launch_few<2>(w, act, dst, bias, bias_ld, rows, n, k, stream);
    }
}

// Whether AUTO products of up to 8 rows take the kernel with weights in
// LDS (TMH_FEW_ROWS_KERNEL=lanes keeps the lanes kernels, for comparisons).
static bool few_rows_kernel() {
    static const bool lanes = [] {
        const char* env = getenv("TMH_FEW_ROWS_KERNEL");
        return env && strcmp(env, "lanes") == 0;
    }();
    return !lanes;
}

hipError_t launch_block_matmul(uint32_t kind, uint32_t mode, const uint8_t* w, Activations act, float* dst,
                               const float* bias, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                               hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    const bool fits = lanes_fit(w, k);
    const bool matrix = fits && (mode == 7u /* MATRIX */ || (mode == 0u /* AUTO */ && rows >= MATRIX_ROWS));
    const bool fused = mode == 3u /* UNORDERED */ && rows >= MATRIX_ROWS;
    // Below MATRIX_ROWS, UNORDERED takes AUTO's kernels, each folding in its
    // own order (tree_fold, set by the entry point)
    const bool autoish = mode == 0u /* AUTO */ || mode == 3u /* UNORDERED */;
    if ((matrix || fused) && mx_fits(w, act, kind, k)) {
        switch (kind) {
        case 0: return launch_mx<0>(fused, w, act, dst, bias, rows, n, k, stream);
        case 1: return launch_mx<1>(fused, w, act, dst, bias, rows, n, k, stream);
        default: return launch_mx<2>(fused, w, act, dst, bias, rows, n, k, stream);
        }
    }
    if (autoish && (rows == 1u || rows == 8u) && few_rows_kernel()) {
        // one or 8 rows: the weights of each workgroup's tile staged into LDS
        // at once, the products on the matrix cores (measured, Q4_1: 8 rows
        // 9.8 / 13.4 us against 12.2 / 14.9 for the lanes kernel at 8192x2048
        // / 2048x8192, one row 9.1 against 10.4 at 2048x8192; from 2 to 4 rows
        // the lanes kernel is as fast or faster, 10.7 against 11.9 at 2 rows
        // of 2048x8192)
        const hipError_t e = launch_rows_product(kind, NB_QUANT, w, nullptr, 0, nullptr, 0.0f, act, dst, bias, 0, rows,
                                                 n, k, compute_units, stream);
        if (e != hipErrorInvalidValue) return e;
    }
    if (autoish && few_fits(w, act, kind, rows, k))
        return launch_few_kind(kind, w, act, dst, bias, 0, rows, n, k, stream);
    if (matrix) {
        switch (kind) {
        case 0: return launch_mfma<0>(w, act, dst, bias, rows, n, k, stream);
        case 1: return launch_mfma<1>(w, act, dst, bias, rows, n, k, stream);
        default: return launch_mfma<2>(w, act, dst, bias, rows, n, k, stream);
        }
    }
    const bool thread = mode == 1u /* THREAD */ || !fits;
    switch (kind) {
    case 0:
        return thread ? launch_thread<0>(w, act, dst, bias, rows, n, k, stream)
                      : launch_lanes<0>(w, act, dst, bias, rows, n, k, compute_units, stream);
    case 1:
        return thread ? launch_thread<1>(w, act, dst, bias, rows, n, k, stream)
                      : launch_lanes<1>(w, act, dst, bias, rows, n, k, compute_units, stream);
    default:
        return thread ? launch_thread<2>(w, act, dst, bias, rows, n, k, stream)
                      : launch_lanes<2>(w, act, dst, bias, rows, n, k, compute_units, stream);
    }
}

hipError_t launch_product_residual(uint32_t kind, const uint8_t* w, Activations act, float* dst, const float* residual,
                                  uint32_t rows, uint32_t n, uint32_t k, int compute_units, hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (!lanes_fit(w, k) || rows >= MATRIX_ROWS) return hipErrorInvalidValue;
    if (few_fits(w, act, kind, rows, k)) return launch_few_kind(kind, w, act, dst, residual, n, rows, n, k, stream);
    switch (kind) {
    case 0: return launch_lanes<0>(w, act, dst, residual, rows, n, k, compute_units, stream, n);
    case 1: return launch_lanes<1>(w, act, dst, residual, rows, n, k, compute_units, stream, n);
    default: return launch_lanes<2>(w, act, dst, residual, rows, n, k, compute_units, stream, n);
    }
}

// The GLU tile: h gate rows and the h up rows of the same indices, h a
// multiple of 32 (whole quantisation blocks) and 2h a multiple of the rows
// one step of the lanes kernel covers (256 / pairs per row, a power of two).
static uint32_t glu_half(uint32_t nb) { return std::max(32u, (256u / (nb / 2u)) / 2u); }

static size_t glu_lds(uint32_t nbatch, uint32_t nb) {
    const size_t tr = 2u * glu_half(nb);
    return ((size_t)nbatch * tr * lanes_stride(nb) + (size_t)nbatch * tr) * sizeof(float);
}

template <int KIND, int NB>
static hipError_t launch_glu_nb(const uint8_t* w, Activations act, uint32_t H, uint32_t k, Activations glu,
                                hipStream_t stream) {
    const uint32_t nb = k >> 5, h = glu_half(nb);
    if (tree_fold())
        TMH_LAUNCH((k_matvec_glu<KIND, NB, true>), dim3(H / h), dim3(256), glu_lds(NB, nb), stream, w, act, 2u * H, k,
                   2u * h, lanes_stride(nb), glu);
    else
        TMH_LAUNCH((k_matvec_glu<KIND, NB, false>), dim3(H / h), dim3(256), glu_lds(NB, nb), stream, w, act, 2u * H,
                   k, 2u * h, lanes_stride(nb), glu);
    return hipGetLastError();
}

template <int KIND>
static hipError_t launch_glu(const uint8_t* w, Activations act, uint32_t rows, uint32_t H, uint32_t k,
                             Activations glu, hipStream_t stream) {
    const uint32_t nb = k >> 5, hb = H >> 5;
    uint32_t done = 0;
    while (done < rows) {
        const uint32_t left = rows - done;
        Activations a = act, g = glu;
        a.scales += (size_t)done * nb;
        a.sums += (size_t)done * nb;
        a.totals += (size_t)done * nb;
        a.qs += (size_t)done * k;
        g.scales += (size_t)done * hb;
        g.sums += (size_t)done * hb;
        g.totals += (size_t)done * hb;
        g.qs += (size_t)done * H;
        hipError_t err;
        uint32_t take;
        if (left >= 8 && glu_lds(8, nb) <= CU_LDS) err = launch_glu_nb<KIND, 8>(w, a, H, k, g, stream), take = 8;
        else if (left >= 4 && glu_lds(4, nb) <= CU_LDS) err = launch_glu_nb<KIND, 4>(w, a, H, k, g, stream), take = 4;
        else if (left >= 2 && glu_lds(2, nb) <= CU_LDS) err = launch_glu_nb<KIND, 2>(w, a, H, k, g, stream), take = 2;
        else err = launch_glu_nb<KIND, 1>(w, a, H, k, g, stream), take = 1;
        if (err != hipSuccess) return err;
        done += take;
    }
    return hipSuccess;
}

hipError_t launch_gate_up_swiglu(uint32_t kind, const uint8_t* w, Activations act, uint32_t rows, uint32_t H,
                                 uint32_t k, Activations glu, hipStream_t stream) {
    if (rows == 0 || H == 0) return hipSuccess;
    if (!lanes_fit(w, k) || rows >= MATRIX_ROWS) return hipErrorInvalidValue;
    const uint32_t nb = k >> 5, np = nb / 2u;
    if ((np & (np - 1u)) != 0 || H % glu_half(nb) != 0 || glu_lds(1, nb) > CU_LDS) return hipErrorInvalidValue;
    switch (kind) {
    case 0: return launch_glu<0>(w, act, rows, H, k, glu, stream);
    case 1: return launch_glu<1>(w, act, rows, H, k, glu, stream);
    default: return launch_glu<2>(w, act, rows, H, k, glu, stream);
    }
}

// ----------------------------------------- one row, weights in LDS: launchers

// LDS a k_matvec_one workgroup may take: one a compute unit (160 KB on
// gfx950, less 2 KB for the kernel's own LDS).
static constexpr size_t ONE_LDS_LIMIT = 158u * 1024u;

// Rows of whole pairs per pass, and rows of whole 16-byte pieces starting
// 16-byte aligned (the direct loads take 16 bytes a lane).
static bool one_fits(uint32_t kind, const uint8_t* w, uint32_t k) {
    const uint32_t nb = k >> 5, np = nb >> 1;
    return lanes_fit(w, k) && np > 0 && ONE_THREADS % np == 0 && (nb * block_bytes(kind)) % 16u == 0 &&
           ((uintptr_t)w & 15u) == 0;
}

// Rows a workgroup: about one workgroup a compute unit, within the LDS limit;
// when the rows take more than one round of workgroups, rounds of equal
// tiles (a last round of a few workgroups would take as long as a full one).
static uint32_t one_tile(uint32_t kind, uint32_t n, uint32_t k, bool norm, int compute_units, bool plain = false,
                         uint32_t xr = 1u) {
    const uint32_t nb = k >> 5, rb = nb * block_bytes(kind), stride = lanes_stride(nb);
    const uint32_t cus = (uint32_t)(compute_units > 0 ? compute_units : 256);
    uint32_t tr = std::max(1u, (n + cus - 1u) / cus);
    while (tr > 1 && one_lds(k, tr, rb, stride, norm, false, plain, xr).end > ONE_LDS_LIMIT) --tr;
    const uint64_t per_round = (uint64_t)cus * tr;
    const uint64_t rounds = (n + per_round - 1u) / per_round;
    return std::max(1u, (uint32_t)((n + cus * rounds - 1u) / (cus * rounds)));
}

template <int KIND, bool NORM, bool PLAIN = false, uint32_t XR = 1>
static hipError_t launch_one(const uint8_t* w, const float* x, const float* nw, float eps, Activations act, float* dst,
                             const float* bias, uint32_t n, uint32_t k, int compute_units, hipStream_t stream,
                             uint32_t ldx = 0) {
    const uint32_t nb = k >> 5, stride = lanes_stride(nb);
    const uint32_t tr = one_tile(KIND, n, k, NORM, compute_units, PLAIN, XR);
    const OneLds L = one_lds(k, tr, nb * Fmt<KIND>::BB, stride, NORM, false, PLAIN, XR);
    if (L.end > ONE_LDS_LIMIT) return hipErrorInvalidValue;
    if (tree_fold())
        TMH_LAUNCH((k_matvec_one<KIND, NORM, false, PLAIN, XR, true>), dim3((n + tr - 1u) / tr), dim3(ONE_THREADS),
                   L.end, stream, w, x, nw, eps, act, dst, bias, n, k, tr, stride, Activations{}, ldx);
    else
        TMH_LAUNCH((k_matvec_one<KIND, NORM, false, PLAIN, XR, false>), dim3((n + tr - 1u) / tr), dim3(ONE_THREADS),
                   L.end, stream, w, x, nw, eps, act, dst, bias, n, k, tr, stride, Activations{}, ldx);
    return hipGetLastError();
}

bool rms_product_fits(const uint8_t* w, uint32_t k, const float* x, uint32_t ldx, const float* norm) {
    (void)ldx;
    return k <= 2048u && norm && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)norm & 15u) == 0;
}

hipError_t launch_product_rms(uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, const float* norm,
                              float eps, float* dst, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                              hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (rows != 1 || !rms_product_fits(w, k, x, ldx, norm) || !one_fits(kind, w, k)) return hipErrorInvalidValue;
    switch (kind) {
    case 0: return launch_one<0, true>(w, x, norm, eps, Activations{}, dst, nullptr, n, k, compute_units, stream);
    case 1: return launch_one<1, true>(w, x, norm, eps, Activations{}, dst, nullptr, n, k, compute_units, stream);
    default: return launch_one<2, true>(w, x, norm, eps, Activations{}, dst, nullptr, n, k, compute_units, stream);
    }
}

hipError_t launch_product_one(uint32_t kind, const uint8_t* w, Activations act, float* dst, const float* bias,
                              uint32_t n, uint32_t k, int compute_units, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    if (!one_fits(kind, w, k) || ((uintptr_t)act.qs & 15u) != 0) return hipErrorInvalidValue;
    switch (kind) {
    case 0: return launch_one<0, false>(w, nullptr, nullptr, 0.0f, act, dst, bias, n, k, compute_units, stream);
    case 1: return launch_one<1, false>(w, nullptr, nullptr, 0.0f, act, dst, bias, n, k, compute_units, stream);
    default: return launch_one<2, false>(w, nullptr, nullptr, 0.0f, act, dst, bias, n, k, compute_units, stream);
    }
}

// One or two f32 rows x (ldx apart), quantised by every workgroup in its
// prologue (no norm): one launch, no scratch. k at most 8192 (the staged
// rows and the tile in LDS), rows 16-byte aligned; hipErrorInvalidValue,
// nothing launched, else.
hipError_t launch_product_f32_one(uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, float* dst,
                                  const float* bias, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                                  hipStream_t stream) {
    if (n == 0) return hipSuccess;
    if (rows < 1u || rows > 2u || k > 8192u || !one_fits(kind, w, k) || ((uintptr_t)x & 15u) != 0 ||
        (rows == 2u && ldx % 4u != 0))
        return hipErrorInvalidValue;
#define TMH_F32_ONE(KIND)                                                                                          \
    return rows == 1u ? launch_one<KIND, true, true>(w, x, nullptr, 0.0f, Activations{}, dst, bias, n, k,          \
                                                     compute_units, stream)                                       \
                      : launch_one<KIND, true, true, 2>(w, x, nullptr, 0.0f, Activations{}, dst, bias, n, k,       \
                                                        compute_units, stream, ldx);
    switch (kind) {
    case 0: TMH_F32_ONE(0)
    case 1: TMH_F32_ONE(1)
    default: TMH_F32_ONE(2)
    }
#undef TMH_F32_ONE
}

template <int KIND>
static hipError_t launch_glu_one(const uint8_t* w, const float* x, const float* norm, float eps, uint32_t H,
                                 uint32_t k, Activations glu, hipStream_t stream) {
    const uint32_t nb = k >> 5, h = glu_half(nb), stride = lanes_stride(nb);
    const OneLds L = one_lds(k, 2u * h, nb * Fmt<KIND>::BB, stride, true, true);
    if (L.end > ONE_LDS_LIMIT || H % h != 0) return hipErrorInvalidValue;
    if (tree_fold())
        TMH_LAUNCH((k_matvec_one<KIND, true, true, false, 1u, true>), dim3(H / h), dim3(ONE_THREADS), L.end, stream, w,
                   x, norm, eps, Activations{}, nullptr, nullptr, 2u * H, k, 2u * h, stride, glu, 0u);
    else
        TMH_LAUNCH((k_matvec_one<KIND, true, true, false, 1u, false>), dim3(H / h), dim3(ONE_THREADS), L.end, stream,
                   w, x, norm, eps, Activations{}, nullptr, nullptr, 2u * H, k, 2u * h, stride, glu, 0u);
    return hipGetLastError();
}

hipError_t launch_gate_up_swiglu_rms(uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, const float* norm,
                                     float eps, uint32_t rows, uint32_t H, uint32_t k, Activations glu,
                                     hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (rows != 1 || !rms_product_fits(w, k, x, ldx, norm) || !one_fits(kind, w, k)) return hipErrorInvalidValue;
    const uint32_t np = (k >> 5) / 2u;
    if ((np & (np - 1u)) != 0) return hipErrorInvalidValue;
    switch (kind) {
    case 0: return launch_glu_one<0>(w, x, norm, eps, H, k, glu, stream);
    case 1: return launch_glu_one<1>(w, x, norm, eps, H, k, glu, stream);
    default: return launch_glu_one<2>(w, x, norm, eps, H, k, glu, stream);
    }
}

// ----------------------------------- a few rows, weights in LDS: launchers

// k a multiple of 256 (whole groups of 8 blocks a wave), weight rows of
// whole 16-byte pieces starting 16-byte aligned (the direct loads); QUANT: rows and tables 16-byte aligned; F32/NORM: at most 2048
// values a row (a block a lane), rows and norm weights 16-byte aligned. A
// last single row of QUANT or NORM takes the one-row kernel, whose own
// limits apply then.
static bool nb_fits(uint32_t kind, uint32_t mode, const uint8_t* w, uint32_t rows, uint32_t k, const float* x,
                    uint32_t ldx, const float* nw, const Activations& act) {
    const uint32_t nb = k >> 5;
    if (nb == 0 || k % 256u != 0 || (nb * block_bytes(kind)) % 16u != 0 || ((uintptr_t)w & 15u) != 0) return false;
    if (mode != NB_F32 && rows % 2u == 1u && !one_fits(kind, w, k)) return false;
    if (mode == NB_QUANT) {
        const uintptr_t extra = kind == 1 ? (uintptr_t)act.totals : kind == 2 ? (uintptr_t)act.sums : 0;
        return act.qs && act.scales && (((uintptr_t)act.qs | (uintptr_t)act.scales | extra) & 15u) == 0;
    }
    if (k > 2048u || !x || ((uintptr_t)x & 15u) != 0 || ldx % 4u != 0) return false;
    return mode != NB_NORM || (nw && ((uintptr_t)nw & 15u) == 0);
}

// Weight rows a workgroup: about one workgroup a compute unit, within the
// LDS limit; rounds of equal tiles when the rows take more than one round.
template <int KIND, uint32_t MODE, int NB>
static uint32_t nb_tile(uint32_t n, uint32_t k, int compute_units) {
    const uint32_t nb = k >> 5, rb = nb * Fmt<KIND>::BB;
    const uint32_t cus = (uint32_t)(compute_units > 0 ? compute_units : 256);
    uint32_t tr = std::max(1u, (n + cus - 1u) / cus);
    while (tr > 1 && nb_lds(NB, KIND, k, tr, rb, MODE, false).end > ONE_LDS_LIMIT) --tr;
    const uint64_t per_round = (uint64_t)cus * tr;
    const uint64_t rounds = (n + per_round - 1u) / per_round;
    return std::max(1u, (uint32_t)((n + cus * rounds - 1u) / (cus * rounds)));
}

// Tiles of 16 weight rows a phase of k_matvec_nb: two (every wave's pairs
// of both, one barrier pair and one fold pass for both) up to 8 rows where
// the tile has more than 16 rows and the second contributions region fits
// the LDS limit, else one. TMH_NB_TPP=1 keeps one, for measurement.
static uint32_t nb_tpp(int nbatch, uint32_t kind, uint32_t k, uint32_t tr, uint32_t row_bytes, uint32_t mode,
                       bool glu) {
    static const bool on = [] {
        const char* env = getenv("TMH_NB_TPP");
        return !(env && strcmp(env, "1") == 0);
    }();
    return on && nbatch <= 8 && tr > 16u && nb_lds(nbatch, kind, k, tr, row_bytes, mode, glu, 2u).end <= ONE_LDS_LIMIT
               ? 2u
               : 1u;
}

// Contributions buffers of k_matvec_nb: two (each phase's fold behind the
// next phase's contributions, one barrier a phase) where a launch has two
// phases or more and the second buffer fits the LDS limit, else one.
// TMH_NB_BUFS=1 keeps one, for measurement.
static uint32_t nb_bufs(int nbatch, uint32_t kind, uint32_t k, uint32_t tr, uint32_t row_bytes, uint32_t mode,
                        bool glu, uint32_t tpp) {
    static const bool on = [] {
        const char* env = getenv("TMH_NB_BUFS");
        return !(env && strcmp(env, "1") == 0);
    }();
    const uint32_t tiles = (tr + 15u) / 16u, phases = (tiles + tpp - 1u) / tpp * ((k / 32u + NB_CHUNK - 1u) / NB_CHUNK);
    return on && phases >= 2u && nb_lds(nbatch, kind, k, tr, row_bytes, mode, glu, tpp, 2u).end <= ONE_LDS_LIMIT ? 2u
                                                                                                            : 1u;
}

template <int KIND, uint32_t MODE, int NB>
static hipError_t launch_nb(const uint8_t* w, const float* x, uint32_t ldx, const float* nw, float eps,
                            Activations act, float* dst, const float* bias, uint32_t bias_ld, uint32_t n, uint32_t k,
                            int compute_units, hipStream_t stream) {
    const uint32_t nb = k >> 5;
    const uint32_t tr = nb_tile<KIND, MODE, NB>(n, k, compute_units);
    const uint32_t tpp = nb_tpp(NB, KIND, k, tr, nb * Fmt<KIND>::BB, MODE, false);
    const uint32_t bufs = nb_bufs(NB, KIND, k, tr, nb * Fmt<KIND>::BB, MODE, false, tpp);
    const NbLds L = nb_lds(NB, KIND, k, tr, nb * Fmt<KIND>::BB, MODE, false, tpp, bufs);
    if (L.end > ONE_LDS_LIMIT) return hipErrorInvalidValue;
    if (tree_fold())
        TMH_LAUNCH((k_matvec_nb<KIND, MODE, false, NB, true>), dim3((n + tr - 1u) / tr), dim3(NbShape<NB>::THREADS),
                   L.end, stream, w, x, ldx, nw, eps, act, dst, bias, bias_ld, n, k, tr, tpp, bufs, Activations{});
    else
        TMH_LAUNCH((k_matvec_nb<KIND, MODE, false, NB, false>), dim3((n + tr - 1u) / tr), dim3(NbShape<NB>::THREADS),
                   L.end, stream, w, x, ldx, nw, eps, act, dst, bias, bias_ld, n, k, tr, tpp, bufs, Activations{});
    return hipGetLastError();
}

// Activation rows in groups of 8, 4 and 2 (each output depends on its own
// row only, so the grouping changes no bits); a last single row takes the
// one-row kernel (F32: k_matvec_nb of one row).
template <int KIND, uint32_t MODE>
static hipError_t launch_nb_rows(const uint8_t* w, const float* x, uint32_t ldx, const float* nw, float eps,
                                 Activations act, float* dst, const float* bias, uint32_t bias_ld, uint32_t rows,
                                 uint32_t n, uint32_t k, int compute_units, hipStream_t stream) {
    const uint32_t nb = k >> 5;
    uint32_t done = 0;
    while (done < rows) {
        const uint32_t left = rows - done;
        Activations a = act;
        if (MODE == NB_QUANT) {
            a.scales += (size_t)done * nb;
            a.sums += (size_t)done * nb;
            a.totals += (size_t)done * nb;
            a.qs += (size_t)done * k;
        }
        const float* xr = MODE == NB_QUANT ? nullptr : x + (size_t)done * ldx;
        float* d = dst + (size_t)done * n;
        const float* bi = bias ? bias + (size_t)done * bias_ld : nullptr;
        hipError_t err;
        uint32_t take;
        if (left >= 8) {
            err = launch_nb<KIND, MODE, 8>(w, xr, ldx, nw, eps, a, d, bi, bias_ld, n, k, compute_units, stream), take = 8;
        } else if (left >= 4) {
            err = launch_nb<KIND, MODE, 4>(w, xr, ldx, nw, eps, a, d, bi, bias_ld, n, k, compute_units, stream), take = 4;
        } else if (left >= 2) {
            err = launch_nb<KIND, MODE, 2>(w, xr, ldx, nw, eps, a, d, bi, bias_ld, n, k, compute_units, stream), take = 2;
        } else {
            take = 1;
            if constexpr (MODE == NB_F32)
                err = launch_nb<KIND, NB_F32, 1>(w, xr, ldx, nullptr, 0.0f, a, d, bi, 0, n, k, compute_units, stream);
            else if constexpr (MODE == NB_NORM)
                err = bi ? hipErrorInvalidValue
                         : launch_one<KIND, true>(w, xr, nw, eps, Activations{}, d, nullptr, n, k, compute_units, stream);
            else
                err = launch_one<KIND, false>(w, nullptr, nullptr, 0.0f, a, d, bi, n, k, compute_units, stream);
        }
        if (err != hipSuccess) return err;
        done += take;
    }
    return hipSuccess;
}

hipError_t launch_rows_product(uint32_t kind, uint32_t mode, const uint8_t* w, const float* x, uint32_t ldx,
                               const float* nw, float eps, Activations act, float* dst, const float* bias,
                               uint32_t bias_ld, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                               hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (mode > NB_NORM || !nb_fits(kind, mode, w, rows, k, x, ldx, nw, act) || (mode == NB_NORM && bias))
        return hipErrorInvalidValue;
#define TMH_NB_MODES(KIND)                                                                                          \
    switch (mode) {                                                                                                 \
    case NB_QUANT:                                                                                                  \
        return launch_nb_rows<KIND, NB_QUANT>(w, x, ldx, nw, eps, act, dst, bias, bias_ld, rows, n, k,              \
                                              compute_units, stream);                                               \
    case NB_F32:                                                                                                    \
        return launch_nb_rows<KIND, NB_F32>(w, x, ldx, nw, eps, act, dst, bias, bias_ld, rows, n, k, compute_units, \
                                            stream);                                                                \
    default:                                                                                                        \
        return launch_nb_rows<KIND, NB_NORM>(w, x, ldx, nw, eps, act, dst, bias, bias_ld, rows, n, k,               \
                                             compute_units, stream);                                                \
    }
    switch (kind) {
    case 0: TMH_NB_MODES(0)
    case 1: TMH_NB_MODES(1)
    default: TMH_NB_MODES(2)
    }
#undef TMH_NB_MODES
}

// The GLU tile of k_matvec_nb: 32 gate rows and the 32 up rows of the same
// indices (one quantisation block of outputs).
static constexpr uint32_t NB_GLU_HALF = 32;

template <int KIND, uint32_t MODE, int NB>
static hipError_t launch_nb_glu(const uint8_t* w, const float* x, uint32_t ldx, const float* nw, float eps,
                                Activations act, uint32_t H, uint32_t k, Activations glu, hipStream_t stream) {
    const uint32_t nb = k >> 5, h = NB_GLU_HALF;
    const uint32_t tpp = nb_tpp(NB, KIND, k, 2u * h, nb * Fmt<KIND>::BB, MODE, true);
    const uint32_t bufs = nb_bufs(NB, KIND, k, 2u * h, nb * Fmt<KIND>::BB, MODE, true, tpp);
    const NbLds L = nb_lds(NB, KIND, k, 2u * h, nb * Fmt<KIND>::BB, MODE, true, tpp, bufs);
    if (tree_fold())
        TMH_LAUNCH((k_matvec_nb<KIND, MODE, true, NB, true>), dim3(H / h), dim3(NbShape<NB>::THREADS), L.end, stream,
                   w, x, ldx, nw, eps, act, nullptr, nullptr, 0, 2u * H, k, 2u * h, tpp, bufs, glu);
    else
        TMH_LAUNCH((k_matvec_nb<KIND, MODE, true, NB, false>), dim3(H / h), dim3(NbShape<NB>::THREADS), L.end, stream,
                   w, x, ldx, nw, eps, act, nullptr, nullptr, 0, 2u * H, k, 2u * h, tpp, bufs, glu);
    return hipGetLastError();
}

template <int KIND, uint32_t MODE>
static hipError_t launch_nb_glu_rows(const uint8_t* w, const float* x, uint32_t ldx, const float* nw, float eps,
                                     Activations act, uint32_t rows, uint32_t H, uint32_t k, Activations glu,
                                     hipStream_t stream) {
    const uint32_t nb = k >> 5, hb = H >> 5;
    uint32_t done = 0;
    while (done < rows) {
        const uint32_t left = rows - done;
        Activations g = glu, a = act;
        g.scales += (size_t)done * hb;
        g.sums += (size_t)done * hb;
        g.totals += (size_t)done * hb;
        g.qs += (size_t)done * H;
        if (MODE == NB_QUANT) {
            a.scales += (size_t)done * nb;
            a.sums += (size_t)done * nb;
            a.totals += (size_t)done * nb;
            a.qs += (size_t)done * k;
        }
        const float* xr = MODE == NB_QUANT ? nullptr : x + (size_t)done * ldx;
        hipError_t err;
        uint32_t take;
        if (left >= 8) {
            err = launch_nb_glu<KIND, MODE, 8>(w, xr, ldx, nw, eps, a, H, k, g, stream), take = 8;
        } else if (left >= 4) {
            err = launch_nb_glu<KIND, MODE, 4>(w, xr, ldx, nw, eps, a, H, k, g, stream), take = 4;
        } else if (left >= 2) {
            err = launch_nb_glu<KIND, MODE, 2>(w, xr, ldx, nw, eps, a, H, k, g, stream), take = 2;
        } else {
            take = 1;
            if constexpr (MODE == NB_NORM) err = launch_glu_one<KIND>(w, xr, nw, eps, H, k, g, stream);
            else err = launch_glu_nb<KIND, 1>(w, a, H, k, g, stream);
        }
        if (err != hipSuccess) return err;
        done += take;
    }
    return hipSuccess;
}

hipError_t launch_rows_gate_up(uint32_t kind, uint32_t mode, const uint8_t* w, const float* x, uint32_t ldx,
                               const float* nw, float eps, Activations act, uint32_t rows, uint32_t H, uint32_t k,
                               Activations glu, hipStream_t stream) {
    if (rows == 0 || H == 0) return hipSuccess;
    if ((mode != NB_NORM && mode != NB_QUANT) || !nb_fits(kind, mode, w, rows, k, x, ldx, nw, act) ||
        H % NB_GLU_HALF != 0)
        return hipErrorInvalidValue;
    const uint32_t nb = k >> 5, np = nb / 2u;
    // the tile in LDS at the largest group (a last single row: the one-row
    // kernel's own limits under NORM, the lanes GLU kernel's under QUANT)
    const uint32_t group = rows >= 8 ? 8u : rows >= 4 ? 4u : rows >= 2 ? 2u : 1u;
    if (nb_lds(group, kind, k, 2u * NB_GLU_HALF, nb * block_bytes(kind), mode, true).end > ONE_LDS_LIMIT)
        return hipErrorInvalidValue;
    if (rows % 2u == 1u) {
        const uint32_t h1 = glu_half(nb);
        if ((np & (np - 1u)) != 0 || H % h1 != 0 || glu_lds(1, nb) > CU_LDS ||
            (mode == NB_NORM && one_lds(k, 2u * h1, nb * block_bytes(kind), lanes_stride(nb), true, true).end >
                                    ONE_LDS_LIMIT))
            return hipErrorInvalidValue;
    }
#define TMH_NB_GLU(KIND)                                                                                                return mode == NB_QUANT ? launch_nb_glu_rows<KIND, NB_QUANT>(w, x, ldx, nw, eps, act, rows, H, k, glu, stream)                             : launch_nb_glu_rows<KIND, NB_NORM>(w, x, ldx, nw, eps, act, rows, H, k, glu, stream);
    switch (kind) {
    case 0: TMH_NB_GLU(0)
    case 1: TMH_NB_GLU(1)
    default: TMH_NB_GLU(2)
    }
#undef TMH_NB_GLU
}

hipError_t launch_gather(uint32_t kind, const uint8_t* table, int32_t table_rows, uint32_t width, const int32_t* ids,
                         uint32_t count, float* dst, int32_t* errors, hipStream_t stream) {
    const uint32_t total = count * width;
    if (total == 0) return hipSuccess;
    const uint32_t grid = (total + 255u) / 256u;
    if (kind == 0)
        TMH_LAUNCH(k_gather_blocks<0>, dim3(grid), dim3(256), 0, stream, table, ids, dst, errors, table_rows,
                           width, total);
    else if (kind == 1)
        TMH_LAUNCH(k_gather_blocks<1>, dim3(grid), dim3(256), 0, stream, table, ids, dst, errors, table_rows,
                           width, total);
    else
        TMH_LAUNCH(k_gather_blocks<2>, dim3(grid), dim3(256), 0, stream, table, ids, dst, errors, table_rows,
                           width, total);
    return hipGetLastError();
}

}  // namespace tmh
