// Kernels for the rest of tensomite's Llama decode graph on gfx950, each
// computing what the reference's host kernels compute, operation for
// operation and in their order, so a GPU forward has the host's bits:
//
//   RMSNorm      host.cr:374-386  Σx² folded from 0 in index order, root =
//                                  sqrt(Σx²/n + ε), then x / root · w
//   RoPE         host.cr:448-466  x·cos + rotate_half(x)·sin, the partner
//                                  of a first-half column times -1
//   cache write  host.cr:586-597  each token's keys and values into its
//                                  row and position of [rows, kv heads,
//                                  capacity, width] (Op::WriteRows)
//   attention    host.cr:408-440  per query row: dot products in column
//                                  order, ·scale, causal mask, the first
//                                  highest score, Maths.exp(x - top), the
//                                  total in position order, then Σ_p
//                                  (e_p / total)·v_p in position order
//   SwiGLU       kernels.cr:18    gate / (Maths.exp(-gate) + 1) · value
//   add          host.cr:159-180  a + b
//   argmax       sampler.cr:35-36 the first index of the highest value
//
// The fold orders are sequential by definition, so the kernels keep them
// sequential: one lane walks each ordered sum (every lane of a wave walks
// the same one, reading LDS by broadcast), while everything that is not
// ordered -- loads, squares, dot products of different positions, the
// exponentials, divisions -- runs across the workgroup.
//
// Built, like every source of the library, with -ffp-contract=off and
// correctly rounded f32 division and square root.
#include "tmh_device.h"
#include "tmh_internal.h"

namespace tmh {


__device__ __forceinline__ void report(int32_t* errors, int32_t value, int32_t limit) {
    if (atomicAdd(&errors[0], 1) == 0) {
        errors[1] = value;
        errors[2] = limit;
    }
}

// One workgroup per row: the row staged in LDS, the ordered sum of its
// squares by wave 0, then x / root · w in parallel.
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x, uint32_t ldx,
                                                 const float* __restrict__ w, uint32_t n, float eps,
                                                 float* __restrict__ dst, uint32_t ld_dst) {
    extern __shared__ float4 lds4[];
    float* row = reinterpret_cast<float*>(lds4);
    const float root = stage_root(x + (size_t)blockIdx.x * ldx, n, eps, row);
    float* out = dst + (size_t)blockIdx.x * ld_dst;
    if (w) {
        for (uint32_t j = threadIdx.x; j < n; j += 256u) {
            const float v = row[j] / root;
            out[j] = v * w[j];
        }
    } else {
        for (uint32_t j = threadIdx.x; j < n; j += 256u) out[j] = row[j] / root;
    }
}

// RMSNorm then the activation quantiser, one workgroup per row (see
// rmsnorm_quantise_row).
__global__ __launch_bounds__(256) void k_rmsnorm_quantise(const float* __restrict__ x, uint32_t ldx,
                                                          const float* __restrict__ w, uint32_t n, float eps,
                                                          Activations act) {
    extern __shared__ float4 lds4[];
    float* row = reinterpret_cast<float*>(lds4);
    rmsnorm_quantise_row(x + (size_t)blockIdx.x * ldx, n, w, eps, act, blockIdx.x, row);
}

// RMSNorm then the activation quantiser, one workgroup per row, with Σx²
// folded by speculation (ordered_sum_wave): wave 0's lane c loads and
// squares values [c·M, c·M + M) of the row while every thread loads its own
// values and weights; then each 8-lane group normalises and quantises its
// blocks of 32 as rmsnorm_quantise_row does (the same bits: the squares
// each rounded, their sum in index order from 0, sqrtf(Σ/n + ε)).
template <int M>
__global__ __launch_bounds__(256) void k_rmsnorm_quantise_wave(const float* __restrict__ x, uint32_t ldx,
                                                               const float* __restrict__ w, uint32_t n, float eps,
                                                               Activations act) {
    __shared__ float root_slot;
    constexpr uint32_t PASSES = RMSNORM_LDS_ROW / 1024u;
    const uint32_t r = blockIdx.x, nb = n >> 5, sub = threadIdx.x & 7u;
    const float* xr = x + (size_t)r * ldx;
    float4 xv[PASSES], wv[PASSES];
#pragma unroll
    for (uint32_t pass = 0; pass < PASSES; ++pass) {
        const uint32_t blk = (threadIdx.x >> 3) + 32u * pass;
        const uint32_t j = blk * 32u + sub * 4u;
        xv[pass] = blk < nb ? *reinterpret_cast<const float4*>(xr + j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        wv[pass] = (w && blk < nb) ? *reinterpret_cast<const float4*>(w + j) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
    if (threadIdx.x < 64u) {
        float v[M];
        const uint32_t c0 = threadIdx.x * (uint32_t)M;
#pragma unroll
        for (int i = 0; i < M; i += 4) {
            const float4 q = c0 + i < n ? *reinterpret_cast<const float4*>(xr + c0 + i)
                                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            v[i] = q.x * q.x;
            v[i + 1] = q.y * q.y;
            v[i + 2] = q.z * q.z;
            v[i + 3] = q.w * q.w;
        }
        const float total = ordered_sum_wave<M>(v);
        if (threadIdx.x == 0) root_slot = __builtin_sqrtf(total / (float)n + eps);
    }
    __syncthreads();
    const float root = root_slot;
#pragma unroll
    for (uint32_t pass = 0; pass < PASSES; ++pass) {
        const uint32_t blk = (threadIdx.x >> 3) + 32u * pass;
        if (blk >= nb) break;
        const uint32_t j = blk * 32u + sub * 4u;
        const float xj[4] = {xv[pass].x, xv[pass].y, xv[pass].z, xv[pass].w};
        const float wj[4] = {wv[pass].x, wv[pass].y, wv[pass].z, wv[pass].w};
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q = xj[i] / root;
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

// Rows too wide for LDS: the fold reads the row from memory (one cache line
// feeds 32 steps of every lane).
__global__ __launch_bounds__(256) void k_rmsnorm_wide(const float* __restrict__ x, uint32_t ldx,
                                                      const float* __restrict__ w, uint32_t n, float eps,
                                                      float* __restrict__ dst, uint32_t ld_dst) {
    const float* xr = x + (size_t)blockIdx.x * ldx;
    float squares = 0.0f;
    for (uint32_t j = 0; j < n; ++j) squares += xr[j] * xr[j];
    const float root = __builtin_sqrtf(squares / (float)n + eps);
    float* out = dst + (size_t)blockIdx.x * ld_dst;
    for (uint32_t j = threadIdx.x; j < n; j += 256u) {
        const float v = xr[j] / root;
        out[j] = w ? v * w[j] : v;
    }
}

hipError_t launch_rmsnorm(const float* x, uint32_t ldx, const float* w, uint32_t rows, uint32_t n, float eps,
                          float* dst, uint32_t ld_dst, hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (n <= RMSNORM_LDS_ROW) {
        const size_t lds = (((size_t)n + 3u) & ~(size_t)3u) * sizeof(float);
        TMH_LAUNCH(k_rmsnorm, dim3(rows), dim3(256), lds, stream, x, ldx, w, n, eps, dst, ld_dst);
    } else {
        TMH_LAUNCH(k_rmsnorm_wide, dim3(rows), dim3(256), 0, stream, x, ldx, w, n, eps, dst, ld_dst);
    }
    return hipGetLastError();
}

bool rmsnorm_quantise_fits(uint32_t n) { return n > 0 && n % 32u == 0 && n <= RMSNORM_LDS_ROW; }

hipError_t launch_rmsnorm_quantise(const float* x, uint32_t ldx, const float* w, uint32_t rows, uint32_t n, float eps,
                                   Activations act, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (!rmsnorm_quantise_fits(n)) return hipErrorInvalidValue;
    if (ldx % 4u == 0 && ((uintptr_t)x & 15u) == 0 && (!w || ((uintptr_t)w & 15u) == 0)) {
        if (n <= 64u * 8u)
            TMH_LAUNCH(k_rmsnorm_quantise_wave<8>, dim3(rows), dim3(256), 0, stream, x, ldx, w, n, eps, act);
        else if (n <= 64u * 32u)
            TMH_LAUNCH(k_rmsnorm_quantise_wave<32>, dim3(rows), dim3(256), 0, stream, x, ldx, w, n, eps, act);
        else
            TMH_LAUNCH(k_rmsnorm_quantise_wave<128>, dim3(rows), dim3(256), 0, stream, x, ldx, w, n, eps, act);
        return hipGetLastError();
    }
    TMH_LAUNCH(k_rmsnorm_quantise, dim3(rows), dim3(256), (size_t)n * sizeof(float), stream, x, ldx, w,
                       n, eps, act);
    return hipGetLastError();
}

// ------------------------------------------------------- RoPE + cache write

// One thread per output element of `tokens` rows of [q heads | k heads |
// v heads], each `width` wide: q heads rotated into q_dst [tokens, heads,
// width]; k heads rotated and v heads copied into the caches
// [cache_rows, kv_heads, capacity, width] at the token's slot
// (row·capacity + position), whose position also picks the table row.
__global__ __launch_bounds__(256) void k_rope_write(RopeWrite a, uint32_t total) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t units = a.heads + 2u * a.kv_heads;
    const uint32_t col = i % a.width;
    const uint32_t rest = i / a.width;
    const uint32_t unit = rest % units;
    const uint32_t t = rest / units;
    const int32_t slot = a.slots[t];
    const int32_t cap = (int32_t)a.capacity;
    if (slot < 0 || slot >= (int32_t)a.cache_rows * cap) {
        if (col == 0 && unit == 0) report(a.errors, slot, (int32_t)a.cache_rows * cap);
        return;
    }
    const uint32_t row = (uint32_t)slot / a.capacity;
    const uint32_t pos = (uint32_t)slot - row * a.capacity;
    const float* src = a.x + (size_t)t * a.ldx + (size_t)unit * a.width;
    if (unit >= a.heads + a.kv_heads) {
        const uint32_t head = unit - a.heads - a.kv_heads;
        a.values[(((size_t)row * a.kv_heads + head) * a.capacity + pos) * a.width + col] = src[col];
        return;
    }
    const uint32_t half = a.width >> 1;
    const float partner = src[col < half ? col + half : col - half];
    const float rotated = col < half ? partner * -1.0f : partner;
    const float c = a.cos[(size_t)pos * a.width + col];
    const float s = a.sin[(size_t)pos * a.width + col];
    const float left = src[col] * c;
    const float right = rotated * s;
    const float v = left + right;
    if (unit < a.heads) {
        a.q_dst[((size_t)t * a.heads + unit) * a.width + col] = v;
    } else {
        const uint32_t head = unit - a.heads;
        a.keys[(((size_t)row * a.kv_heads + head) * a.capacity + pos) * a.width + col] = v;
    }
}

hipError_t launch_rope_write(const RopeWrite& a, uint32_t tokens, hipStream_t stream) {
    const uint64_t total = (uint64_t)tokens * (a.heads + 2u * a.kv_heads) * a.width;
    if (total == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)((total + 255u) / 256u);
    TMH_LAUNCH(k_rope_write, dim3(grid), dim3(256), 0, stream, a, (uint32_t)total);
    return hipGetLastError();
}

// ---------------------------------------------------------------- attention

// Wave-wide maximum that never takes a NaN (`o > top`).
__device__ __forceinline__ float wave_top(float top) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const float o = __shfl_xor(top, s, 64);
        top = o > top ? o : top;
    }
    return top;
}

// Floats of one staged chunk of values (positions × width), at most; two
// are staged in turn, in what the LDS (160 KB a workgroup on gfx950) leaves
// after q, the current key and value, the outputs and the scores. Small
// chunks leave room for several workgroups a compute unit (prefill runs
// one per query row and head).
constexpr uint32_t ATT_CHUNK_FLOATS = 4096;
constexpr size_t ATT_LDS_LIMIT = 160u * 1024u;

__host__ __device__ inline uint32_t att_chunk_positions(uint32_t width, uint32_t capacity) {
    const uint32_t w4 = (width + 3u) & ~3u;
    // 64 floats left for the kernel's own LDS (its tops and total)
    const size_t fixed = 4u * (size_t)w4 + ((capacity + 3u) & ~3u) + 64u;
    const size_t avail = ATT_LDS_LIMIT / 4u > fixed ? ATT_LDS_LIMIT / 4u - fixed : 0u;
    size_t ch = std::min<size_t>(ATT_CHUNK_FLOATS / width, avail / (2u * (size_t)width));
    ch &= ~(size_t)3u;
    return ch >= 4u ? (uint32_t)ch : 4u;
}

// LDS layout of the attention kernels, in floats: q, the current key and
// value, the row's attended outputs, the scores, then two value chunks.
struct AttLds {
    float *q, *kcur, *vcur, *out, *sc, *vbuf;
    uint32_t ch;  // positions of one value chunk
};

__device__ __forceinline__ AttLds att_lds(float* base, uint32_t width, uint32_t capacity) {
    const uint32_t w4 = (width + 3u) & ~3u;
    AttLds l;
    l.q = base;
    l.kcur = base + w4;
    l.vcur = base + 2u * w4;
    l.out = base + 3u * w4;
    l.sc = base + 4u * w4;
    l.vbuf = l.sc + ((capacity + 3u) & ~3u);
    l.ch = att_chunk_positions(width, capacity);
    return l;
}

size_t attention_lds(uint32_t width, uint32_t capacity) {
    const size_t w4 = (width + 3u) & ~3u;
    const size_t ch = att_chunk_positions(width, capacity);
    return (4u * w4 + ((capacity + 3u) & ~3u) + 2u * ch * width) * sizeof(float);
}

// Writes the products weight_p · v_p[c] of value positions [p0, p0 + count)
// of one head into `dst`, rows of `width` (each product rounded once, as
// the host's `scores[p] / total * v` rounds it), position `cur` (if in range)
// from `vcur` instead of the cache; threads from `first` on, `stride` apart,
// take float4s.
__device__ __forceinline__ void stage_products(float* dst, const float* __restrict__ vb, const float* wts,
                                               uint32_t width, uint32_t p0, uint32_t count, int32_t cur,
                                               const float* vcur, uint32_t first, uint32_t stride) {
    const uint32_t per = width >> 2;
    const uint32_t total = count * per;
    constexpr int U = 8;  // loads in flight per thread before any store
    for (uint32_t i0 = threadIdx.x - first; i0 < total; i0 += U * stride) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t i = i0 + u * stride;
            const uint32_t p = p0 + i / per, c = (i % per) * 4u;
            if (i < total)
                v[u] = *reinterpret_cast<const float4*>((int32_t)p == cur ? vcur + c : vb + (size_t)p * width + c);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t i = i0 + u * stride;
            if (i < total) {
                const uint32_t p = p0 + i / per, c = (i % per) * 4u;
                const float w = wts[p];
                float4 prod;
                prod.x = w * v[u].x;
                prod.y = w * v[u].y;
                prod.z = w * v[u].z;
                prod.w = w * v[u].w;
                *reinterpret_cast<float4*>(dst + (size_t)(p - p0) * width + c) = prod;
            }
        }
    }
}

// acc + Σ_{p < cnt} pc[p·stride], in order: the reads of the next 16 values
// are issued before the adds of the current 16, from two register buffers.
__device__ __forceinline__ float fold_column(float acc, const float* pc, uint32_t stride, uint32_t cnt) {
    float a[16], b[16];
    uint32_t p = 0;
    if (cnt >= 32u) {
#pragma unroll
        for (int i = 0; i < 16; ++i) a[i] = pc[(size_t)i * stride];
        for (; p + 48u <= cnt; p += 32u) {
#pragma unroll
            for (int i = 0; i < 16; ++i) b[i] = pc[(size_t)(p + 16u + i) * stride];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc += a[i];
#pragma unroll
            for (int i = 0; i < 16; ++i) a[i] = pc[(size_t)(p + 32u + i) * stride];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc += b[i];
        }
        // a holds [p, p + 16)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc += a[i];
        p += 16u;
    }
    for (; p < cnt; ++p) acc += pc[(size_t)p * stride];
    return acc;
}

// The attention of one query row and head, with the host's bits
// (host.cr:408-440): q in l.q; keys and values of positions [0, n) in the
// cache at kb/vb, but position `cur` (if ≥ 0) in l.kcur/l.vcur; positions
// past `last` masked. Leaves the outputs in l.out. Every thread calls it.
__device__ void attend(const AttLds& l, const float* __restrict__ kb, const float* __restrict__ vb, uint32_t width,
                       uint32_t n, int32_t last, int32_t cur, float scale) {
    __shared__ float tops[4];
    const uint32_t tid = threadIdx.x;
    const uint32_t w4n = width >> 2;
    const float4* q4 = reinterpret_cast<const float4*>(l.q);

    // scores, one position a thread: q·k in column order, ·scale, mask
    float top = -__builtin_inff();
    for (uint32_t p = tid; p < n; p += 256u) {
        const float4* k4 = reinterpret_cast<const float4*>((int32_t)p == cur ? l.kcur : kb + (size_t)p * width);
        float dot = 0.0f;
        // the key row in pieces of 16 float4, each piece's loads issued together
        for (uint32_t c0 = 0; c0 < w4n; c0 += 16u) {
            float4 k[16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (c0 + u < w4n) k[u] = k4[c0 + u];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (c0 + u < w4n) {
                    const float4 q = q4[c0 + u];
                    dot += q.x * k[u].x;
                    dot += q.y * k[u].y;
                    dot += q.z * k[u].z;
                    dot += q.w * k[u].w;
                }
            }
        }
        float x = dot * scale;
        // The causal mask adds -inf past the last position seen; its 0
        // elsewhere only turns a -0 score into +0, which changes no later bit.
        if ((int32_t)p > last) x = x + -__builtin_inff();
        l.sc[p] = x;
        top = x > top ? x : top;
    }
    top = wave_top(top);
    if ((tid & 63u) == 0) tops[tid >> 6] = top;
    __syncthreads();
    top = tops[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) top = tops[i] > top ? tops[i] : top;
    if (l.sc[0] != l.sc[0]) top = l.sc[0];  // the host's top is a NaN at position 0

    for (uint32_t p = tid; p < n; p += 256u) l.sc[p] = maths_exp(l.sc[p] - top);
    __syncthreads();
    const float total = shared_sum(l.sc, n);
    for (uint32_t p = tid; p < n; p += 256u) l.sc[p] = l.sc[p] / total;
    __syncthreads();

    // Σ_p weight_p · v_p[c] in position order, one lane per column: the
    // products are formed in parallel as the values stage through LDS in
    // chunks (the waves not folding stage the next chunk while the folding
    // waves add up this one), so the fold is a chain of adds.
    const uint32_t ch = l.ch;
    const uint32_t chunks = (n + ch - 1u) / ch;
    const uint32_t folding = ((width + 63u) >> 6) << 6;  // threads of the folding waves
    const bool overlap = folding < 256u;
    const uint32_t first_loader = overlap ? folding : 0u;
    stage_products(l.vbuf, vb, l.sc, width, 0, min(ch, n), cur, l.vcur, 0, 256u);
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t k = 0; k < chunks; ++k) {
        const uint32_t p0 = k * ch, cnt = min(ch, n - p0);
        const float* buf = l.vbuf + (size_t)(k & 1u) * ch * width;
        if (k + 1u < chunks && (!overlap || tid >= first_loader)) {
            const uint32_t q0 = p0 + ch;
            stage_products(l.vbuf + (size_t)((k + 1u) & 1u) * ch * width, vb, l.sc, width, q0, min(ch, n - q0), cur,
                           l.vcur, first_loader, 256u - first_loader);
        }
        if (!overlap) __syncthreads();
        if (tid < width) acc = fold_column(acc, buf + tid, width, cnt);
        __syncthreads();
    }
    if (tid < width) l.out[tid] = acc;
    __syncthreads();
}

// Writes the row's attended outputs (l.out, `width`) for token t, head h:
// the F32 values, and, when act.qs is set, their quantised blocks as
// quantize_activations makes them for the o product's row (width a
// multiple of 32; the row holds heads · width values).
__device__ __forceinline__ void emit(const float* lout, float* out, uint32_t width, Activations act, uint32_t t,
                                     uint32_t h, uint32_t heads) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t c = tid; c < width; c += 256u) out[c] = lout[c];
    if (!act.qs) return;
    const uint32_t blocks = width >> 5;
    const uint32_t k = heads * width, nb = k >> 5;
    const uint32_t blk = tid >> 3, sub = tid & 7u;
    if (blk < blocks) {
        const float4 v = *reinterpret_cast<const float4*>(lout + blk * 32u + sub * 4u);
        const Q8Quad q = quantize_quad(v.x, v.y, v.z, v.w);
        const uint32_t g = h * blocks + blk;
        *(uint32_t*)((int8_t*)act.qs + (size_t)t * k + g * 32u + sub * 4u) = q.packed;
        if (sub == 0) {
            ((float*)act.scales)[(size_t)t * nb + g] = q.scale;
            ((float*)act.sums)[(size_t)t * nb + g] = q.sum;
            ((int32_t*)act.totals)[(size_t)t * nb + g] = q.total;
        }
    }
}

// One workgroup per (query token, head) of cached keys and values.
__global__ __launch_bounds__(256) void k_attention(Attention a) {
    extern __shared__ float4 lds4[];
    const AttLds l = att_lds(reinterpret_cast<float*>(lds4), a.width, a.capacity);
    const uint32_t tid = threadIdx.x;
    const uint32_t t = blockIdx.x / a.heads;
    const uint32_t h = blockIdx.x - t * a.heads;
    const int32_t row = a.table[3u * t], last = a.table[3u * t + 1u], length = a.table[3u * t + 2u];
    float* out = a.dst + (size_t)t * a.ld_dst + (size_t)h * a.width;
    if (row < 0 || row >= (int32_t)a.cache_rows || length <= 0 || length > (int32_t)a.capacity || last < 0 ||
        last >= length) {
        for (uint32_t c = tid; c < a.width; c += 256u) out[c] = 0.0f;
        if (tid == 0 && h == 0) report(a.errors, row < 0 || row >= (int32_t)a.cache_rows ? row : length, (int32_t)a.capacity);
        return;
    }
    const uint32_t kv = h / (a.heads / a.kv_heads);
    const size_t base = ((size_t)row * a.kv_heads + kv) * a.capacity * a.width;
    const float* qh = a.q + (size_t)t * a.ldq + (size_t)h * a.width;
    for (uint32_t c = tid; c < a.width; c += 256u) l.q[c] = qh[c];
    __syncthreads();
    attend(l, a.keys + base, a.values + base, a.width, (uint32_t)length, last, -1, a.scale);
    emit(l.out, out, a.width, a.act, t, h, a.heads);
}

hipError_t launch_attention(const Attention& a, uint32_t tokens, hipStream_t stream) {
    if (tokens == 0 || a.heads == 0) return hipSuccess;
    const size_t lds = attention_lds(a.width, a.capacity);
    TMH_LAUNCH(k_attention, dim3(tokens * a.heads), dim3(256), lds, stream, a);
    return hipGetLastError();
}

// A decode step's attention with its RoPE and cache write fused: token t
// is its cache row's one new position (slot = row·capacity + position,
// table (row, position, position + 1)). The workgroup of query head h
// rotates its q head and its kv head's new key, takes the new value, and --
// the first query head of the group only -- writes both into the caches;
// the new position is attended from LDS, earlier ones from the caches.
// ------------------------------------------- decode attention, direct loads

// The decode kernel brings everything it reads into LDS by direct loads
// issued together at its start -- the head's q, k and v rows and RoPE
// tables, the first chunk of keys and the first chunk of values -- so their
// latencies overlap instead of following one another (one workgroup per
// head has a compute unit to itself, and it is those latencies that bound
// it). LDS, in floats: five staged rows of W64 (width rounded up to 64), q,
// the current key and value, the outputs (w4 each), the scores (capacity),
// a key chunk as rows, 16 bytes of pad after every 1 KB (a 16-byte direct
// load a kilobyte: contiguous reads, few loads; the pad shifts each
// kilobyte by four banks, so threads reading their positions' rows 16 bytes
// at a time meet at most 1024 / (4·width)-way conflicts), and a value chunk
// as rows.
struct AttDecodeLds {
    float *stage, *q, *kcur, *vcur, *out, *sc, *kt, *vrows;
    uint32_t cp;  // positions of a chunk
};

__host__ __device__ inline uint32_t att_decode_fixed_floats(uint32_t width, uint32_t capacity) {
    const uint32_t w64 = (width + 63u) & ~63u, w4 = (width + 3u) & ~3u;
    return 5u * w64 + 4u * w4 + ((capacity + 3u) & ~3u);
}

__host__ __device__ inline uint32_t att_key_stride(uint32_t width);

// Positions of a chunk: at most 256 (and the capacity), a key row (padded)
// and a value row each, in what the fixed part leaves of 160 KB (less 2 KB: the value
// chunk's last direct load and the kernel's own LDS).
__host__ __device__ inline uint32_t att_decode_chunk(uint32_t width, uint32_t capacity) {
    const size_t fixed = att_decode_fixed_floats(width, capacity);
    const size_t avail = ATT_LDS_LIMIT / 4u > fixed + 512u ? ATT_LDS_LIMIT / 4u - fixed - 512u : 0u;
    size_t cp = std::min<size_t>(std::min<size_t>(256u, (capacity + 3u) & ~3u),
                                 avail / ((size_t)att_key_stride(width) + width));
    cp &= ~(size_t)3u;
    return cp >= 4u ? (uint32_t)cp : 4u;
}

// Floats a key row takes in LDS on average (width, plus its share of the
// pad), of a key chunk (whole 1 KB direct loads, 1040 bytes apart), and of
// a value chunk (whole 256-float direct loads).
__host__ __device__ inline uint32_t att_key_stride(uint32_t width) { return width + (width + 63u) / 64u; }
__host__ __device__ inline uint32_t att_kt_floats(uint32_t width, uint32_t cp) {
    return ((cp * width + 255u) >> 8) * 260u;
}
// The LDS float offset of key float f (position · width + column) of a chunk.
__device__ __forceinline__ uint32_t att_key_at(uint32_t f) { return (f >> 8) * 260u + (f & 255u); }
__host__ __device__ inline uint32_t att_v_floats(uint32_t width, uint32_t cp) { return (cp * width + 255u) & ~255u; }

__device__ __forceinline__ AttDecodeLds att_decode_lds(float* base, uint32_t width, uint32_t capacity) {
    const uint32_t w64 = (width + 63u) & ~63u, w4 = (width + 3u) & ~3u;
    AttDecodeLds l;
    l.cp = att_decode_chunk(width, capacity);
    l.stage = base;
    l.q = base + 5u * w64;
    l.kcur = l.q + w4;
    l.vcur = l.kcur + w4;
    l.out = l.vcur + w4;
    l.sc = l.out + w4;
    l.kt = l.sc + ((capacity + 3u) & ~3u);
    l.vrows = l.kt + att_kt_floats(width, l.cp);
    return l;
}

size_t attention_decode_lds(uint32_t width, uint32_t capacity) {
    const uint32_t cp = att_decode_chunk(width, capacity);
    return ((size_t)att_decode_fixed_floats(width, capacity) + att_kt_floats(width, cp) + att_v_floats(width, cp)) *
           sizeof(float);
}

// Direct loads of `width` floats at src into LDS at `to` by one wave, 64 a
// load (lanes past the row read its last value again); returns the loads.
__device__ __forceinline__ uint32_t stage_row(const float* src, uint32_t width, uint32_t to) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t loads = 0;
    for (uint32_t c0 = 0; c0 < width; c0 += 64u, ++loads)
        lds_load4(src + min(c0 + lane, width - 1u), to + c0 * 4u);
    return loads;
}

// Direct loads of the keys of positions [p0, p0 + cnt) into `to`, 1 KB a
// load, 1040 bytes apart (att_key_at), loads wave, wave + 4, ...; returns
// this wave's loads. Lanes past the chunk read its last piece again.
__device__ __forceinline__ uint32_t stage_keys(const float* kb, uint32_t width, uint32_t p0, uint32_t cnt,
                                               uint32_t to, uint32_t wave) {
    const uint32_t lane = threadIdx.x & 63u;
    const uintptr_t base = (uintptr_t)(kb + (size_t)p0 * width);
    const uintptr_t last = base + (uintptr_t)cnt * width * 4u - 16u;
    const uint32_t loads = (cnt * width + 255u) >> 8;
    uint32_t mine = 0;
    for (uint32_t i = wave; i < loads; i += 4u, ++mine) {
        const uintptr_t a = base + (uintptr_t)i * 1024u + lane * 16u;
        lds_load16((const void*)(a < last ? a : last), to + i * 1040u);
    }
    return mine;
}

// Direct loads of the value rows of positions [p0, p0 + cnt) into `to` (as
// rows), loads i = wave, wave + 4, ...; returns this wave's loads. Lanes
// past the chunk read its last piece again.
__device__ __forceinline__ uint32_t stage_values(const float* vb, uint32_t width, uint32_t p0, uint32_t cnt,
                                                 uint32_t to, uint32_t wave) {
    const uint32_t lane = threadIdx.x & 63u;
    const uintptr_t base = (uintptr_t)(vb + (size_t)p0 * width);
    const uintptr_t last = base + (uintptr_t)cnt * width * 4u - 16u;
    const uint32_t loads = (cnt * width + 255u) >> 8;
    uint32_t mine = 0;
    for (uint32_t i = wave; i < loads; i += 4u, ++mine) {
        const uintptr_t a = base + (uintptr_t)i * 1024u + lane * 16u;
        lds_load16((const void*)(a < last ? a : last), to + i * 1024u);
    }
    return mine;
}

// acc += Σ_p w[p] · v[p · stride] over p in [0, cnt), each product rounded
// before its add, in position order (one column of a value chunk; one lane
// each). 16 positions a batch: a batch's values and weights are read into
// registers before the previous batch is folded (two sets of registers in
// turn). S: the row stride when fixed at compile time (reads then take
// immediate offsets), else 0 and `stride` holds it.
template <uint32_t S>
__device__ __forceinline__ void fold_values(const float* vr, const float* wr, uint32_t cnt, uint32_t stride,
                                            float& acc) {
    const uint32_t width = S ? S : stride;
    auto read = [&](uint32_t pl, float (&v)[16], float4 (&w)[4]) {
        const float* vp = vr + (size_t)pl * width;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = vp[(size_t)i * width];
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = *reinterpret_cast<const float4*>(wr + pl + 4u * q);
    };
    auto fold = [&](float (&v)[16], const float4 (&w)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float w4[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float prod = w4[e] * v[4 * q + e];
                acc += prod;
            }
        }
    };
    uint32_t pl = 0;
    if (cnt >= 32u) {
        float va[16], vb[16];
        float4 wa[4], wb[4];
        read(0, va, wa);
        for (; pl + 48u <= cnt; pl += 32u) {
            read(pl + 16u, vb, wb);
            fold(va, wa);
            read(pl + 32u, va, wa);
            fold(vb, wb);
        }
        // va holds [pl, pl + 16)
        if (pl + 32u <= cnt) {
            read(pl + 16u, vb, wb);
            fold(va, wa);
            fold(vb, wb);
            pl += 32u;
        } else {
            fold(va, wa);
            pl += 16u;
        }
    }
    for (; pl < cnt; ++pl) {
        const float prod = wr[pl] * vr[(size_t)pl * width];
        acc += prod;
    }
}

// attend() of one decode row from the staged chunks: the scores of chunk
// after chunk (the first staged already), the softmax, then the weighted
// values chunk after chunk, each product rounded before it is added, in
// position order. `vloads`: this wave's loads of the first value chunk,
// issued after its first key chunk. Barriers leave direct loads in flight
// until they are waited for.
__device__ void attend_staged(const AttDecodeLds& l, const float* __restrict__ kb, const float* __restrict__ vb,
                              uint32_t width, uint32_t n, int32_t last, int32_t cur, float scale, uint32_t vloads) {
    __shared__ float tops[4];
    __shared__ float total_slot;
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t cols = width >> 2, cp = l.cp;
    const float4* q4 = reinterpret_cast<const float4*>(l.q);


    // width 64: q held in registers for every score
    float4 qr[16];
    if (width == 64u) {
#pragma unroll
        for (uint32_t c4 = 0; c4 < 16u; ++c4) qr[c4] = q4[c4];
    }
    float top = -__builtin_inff();
    for (uint32_t p0 = 0; p0 < n; p0 += cp) {
        const uint32_t cnt = min(cp, n - p0);
        if (p0 == 0) {
            wait_vm_lds_upto(vloads);  // the first key chunk (the value chunk after it may fly)
        } else {
            lds_sync();  // the last chunk's keys are read
            stage_keys(kb, width, p0, cnt, lds_address(l.kt), wave);
            wait_vm_lds<0>();
        }
        lds_sync();
        // the current position's key (rotated here, not yet in what was
        // staged) into its row of the chunk: the host reads it from its cache
        if (cur >= (int32_t)p0 && cur < (int32_t)(p0 + cnt)) {
            for (uint32_t c = tid; c < width; c += 256u) l.kt[att_key_at((uint32_t)(cur - (int32_t)p0) * width + c)] = l.kcur[c];
            lds_sync();
        }
        // Thread -> position: lane l of a wave takes position 4 (l % 16) +
        // l / 16 of the wave's 64, so the 16 lanes an LDS pass serves read
        // 16 different 1 KB pieces (1040 bytes apart: distinct 4-bank
        // groups); lane l -> position l would put a piece's four rows, 256
        // bytes apart and so on the same banks, in one pass. Any order of
        // the positions gives the same scores.
        const uint32_t mine = (tid & ~63u) + 4u * (tid & 15u) + ((tid >> 4) & 3u);
        for (uint32_t pl = mine; pl < cnt; pl += 256u) {
            const uint32_t p = p0 + pl;
            float dot = 0.0f;
            if (width == 64u) {
                // q in registers; a position's 64 keys lie in one 1 KB piece
                // (four rows a piece), read at immediate offsets, all before
                // the first add (one LDS round trip, then a chain of adds)
                const float4* k4 = reinterpret_cast<const float4*>(l.kt + (pl >> 2) * 260u + (pl & 3u) * 64u);
                float4 kr[16];
#pragma unroll
                for (uint32_t c4 = 0; c4 < 16u; ++c4) kr[c4] = k4[c4];
#pragma unroll
                for (uint32_t c4 = 0; c4 < 16u; ++c4) asm volatile("" : "+v"(kr[c4].x), "+v"(kr[c4].y), "+v"(kr[c4].z), "+v"(kr[c4].w));
#pragma unroll
                for (uint32_t c4 = 0; c4 < 16u; ++c4) {
                    const float4 q = qr[c4];
                    const float4 k = kr[c4];
                    dot += q.x * k.x;
                    dot += q.y * k.y;
                    dot += q.z * k.z;
                    dot += q.w * k.w;
                }
            } else {
                for (uint32_t c4 = 0; c4 < cols; ++c4) {
                    const float4 q = q4[c4];
                    const float4 k = *reinterpret_cast<const float4*>(l.kt + att_key_at(pl * width + 4u * c4));
                    dot += q.x * k.x;
                    dot += q.y * k.y;
                    dot += q.z * k.z;
                    dot += q.w * k.w;
                }
            }
            float x = dot * scale;
            // The causal mask adds -inf past the last position seen; its 0
            // elsewhere only turns a -0 score into +0, which changes no later bit.
            if ((int32_t)p > last) x = x + -__builtin_inff();
            l.sc[p] = x;
            top = x > top ? x : top;
        }
    }
    // Width 64, chunks of 256 positions, the current position last: the
    // values of the first chunk's positions but the current one are folded
    // from registers, 64 positions a wave (wave w: positions 64w ... 64w +
    // 63, lane c: column c), read from LDS while the softmax runs (waves
    // 1-3 while wave 0 takes the total). Rows from nreg on are zeroed first
    // (and their weights below), so each of them adds +0.0, which leaves a
    // running sum from +0.0 unchanged.
    const bool regs = width == 64u && cp == 256u && cur == (int32_t)n - 1;
    const uint32_t nreg = regs ? (n <= cp ? n - 1u : cp) : 0u;
    float vreg[64];
    auto preload = [&]() {
        const uint32_t lane = tid & 63u, q0 = wave * 64u;
#pragma unroll
        for (uint32_t i = 0; i < 64u; ++i) vreg[i] = l.vrows[(q0 + i) * 64u + lane];
    };
    if (regs) wait_vm_lds<0>();  // this wave's loads of the first value chunk
    top = wave_top(top);
    if ((tid & 63u) == 0) tops[tid >> 6] = top;
    lds_sync();  // (and every wave's values are in)
    top = tops[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) top = tops[i] > top ? tops[i] : top;
    if (l.sc[0] != l.sc[0]) top = l.sc[0];  // the host's top is a NaN at position 0
    if (regs)
        for (uint32_t i = nreg * 16u + tid; i < cp * 16u; i += 256u)
            reinterpret_cast<float4*>(l.vrows)[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t p = tid; p < n; p += 256u) l.sc[p] = maths_exp(l.sc[p] - top);
    lds_sync();
    if (tid < 64u) {
        const float sum = n <= WAVE_SUM_MAX ? ordered_sum_by_wave(l.sc, n) : ordered_sum(l.sc, n);
        if (tid == 0) total_slot = sum;
    } else if (regs) {
        preload();
    }
    lds_sync();
    const float total = total_slot;
    for (uint32_t p = tid; p < n; p += 256u) l.sc[p] = l.sc[p] / total;
    if (regs) {
        // past the last position (capacity ≥ cp), by the thread whose wave
        // reads the weight below, as the divisions above are for p < 256
        if (tid >= n) l.sc[tid] = 0.0f;
        if (wave == 0) preload();
    }

    // Σ_p weight_p · v_p[c] in position order, one lane per column.
    float acc = 0.0f;
    uint32_t from = 0;  // the first position the chunk loop folds
    if (regs) {
        // Every wave its 64 products (each rounded once) together, from
        // weights that its own threads wrote (LDS operations of a wave take
        // effect in order, so no barrier is needed); then wave after wave
        // adds its products in order to the running sums it receives
        // through l.out, a chain of adds from registers.
        const uint32_t lane = tid & 63u, q0 = wave * 64u;
        float pr[64];
#pragma unroll
        for (uint32_t i = 0; i < 64u; i += 4u) {
            const float4 w4 = *reinterpret_cast<const float4*>(l.sc + q0 + i);
            pr[i] = w4.x * vreg[i];
            pr[i + 1u] = w4.y * vreg[i + 1u];
            pr[i + 2u] = w4.z * vreg[i + 2u];
            pr[i + 3u] = w4.w * vreg[i + 3u];
        }
        for (uint32_t v = 0; v < 4u; ++v) {
            if (wave == v) {
                float a = v == 0 ? 0.0f : l.out[lane];
                if (q0 < nreg) {
#pragma unroll
                    for (uint32_t i = 0; i < 64u; ++i) a += pr[i];
                }
                l.out[lane] = a;
            }
            lds_sync();
        }
        if (tid < 64u) {
            acc = l.out[tid];
            // the current position last, from LDS (not yet in the cache)
            if (n <= cp) {
                const float prod = l.sc[n - 1u] * l.vcur[tid];
                acc += prod;
            }
        }
        from = n <= cp ? n : cp;
    }
    for (uint32_t p0 = from; p0 < n; p0 += cp) {
        const uint32_t cnt = min(cp, n - p0);
        if (p0 > 0) {
            lds_sync();  // the last chunk's values are read
            stage_values(vb, width, p0, cnt, lds_address(l.vrows), wave);
        }
        wait_vm_lds<0>();
        lds_sync();  // the chunk's values and the weights are in
        if (cur >= (int32_t)p0 && cur < (int32_t)(p0 + cnt)) {
            // the current position's value row, as for its key
            for (uint32_t c = tid; c < width; c += 256u) l.vrows[(size_t)(cur - (int32_t)p0) * width + c] = l.vcur[c];
            lds_sync();
        }
        if (tid < width) {
            if (width == 64u)
                fold_values<64>(l.vrows + tid, l.sc + p0, cnt, width, acc);
            else
                fold_values<0>(l.vrows + tid, l.sc + p0, cnt, width, acc);
        }
    }
    if (tid < width) l.out[tid] = acc;
    lds_sync();
}

__global__ __launch_bounds__(256) void k_attention_decode(Attention a, RopeWrite r) {
    extern __shared__ float4 lds4[];
    const AttDecodeLds l = att_decode_lds(reinterpret_cast<float*>(lds4), a.width, a.capacity);
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t t = blockIdx.x / a.heads;
    const uint32_t h = blockIdx.x - t * a.heads;
    const uint32_t width = a.width;
    const int32_t slot = r.slots[t];
    const int32_t row = a.table[3u * t], last = a.table[3u * t + 1u], length = a.table[3u * t + 2u];
    const int32_t cap = (int32_t)a.capacity;
    float* out = a.dst + (size_t)t * a.ld_dst + (size_t)h * width;
    if (slot < 0 || slot >= (int32_t)a.cache_rows * cap || row != slot / cap || last != slot % cap ||
        length != last + 1) {
        for (uint32_t c = tid; c < width; c += 256u) out[c] = 0.0f;
        if (tid == 0 && h == 0) report(a.errors, slot, (int32_t)a.cache_rows * cap);
        return;
    }
    const uint32_t group = a.heads / a.kv_heads, kv = h / group;
    const uint32_t pos = (uint32_t)last, half = width >> 1, w64 = (width + 63u) & ~63u;
    const float* src = r.x + (size_t)t * r.ldx;
    const size_t base = ((size_t)row * a.kv_heads + kv) * a.capacity * width;
    const float* kb = a.keys + base;
    const float* vb = a.values + base;
    const uint32_t n = (uint32_t)length, cp = l.cp;

    // Every load at once: wave 0 the head's rows and tables, then every
    // wave its share of the first key chunk, then of the first value chunk.
    const uint32_t stage = lds_address(l.stage);
    if (wave == 0) {
        stage_row(src + (size_t)h * width, width, stage);
        stage_row(src + (size_t)(a.heads + kv) * width, width, stage + w64 * 4u);
        stage_row(src + (size_t)(a.heads + a.kv_heads + kv) * width, width, stage + 2u * w64 * 4u);
        stage_row(r.cos + (size_t)pos * width, width, stage + 3u * w64 * 4u);
        stage_row(r.sin + (size_t)pos * width, width, stage + 4u * w64 * 4u);
    }
    const uint32_t kloads = stage_keys(kb, width, 0, min(cp, n), lds_address(l.kt), wave);
    const uint32_t vloads = stage_values(vb, width, 0, min(cp, n), lds_address(l.vrows), wave);
    wait_vm_lds_upto(kloads + vloads);  // wave 0: its staged rows
    lds_sync();

    // RoPE of q and k from the staged rows, the cache write of k and v by
    // the first head of the group (host order: x·cos + (partner·-1 or
    // partner)·sin).
    const float* qs = l.stage;
    const float* ks = l.stage + w64;
    const float* vs = l.stage + 2u * w64;
    const float* cs = l.stage + 3u * w64;
    const float* sn = l.stage + 4u * w64;
    for (uint32_t c = tid; c < width; c += 256u) {
        const uint32_t o = c < half ? c + half : c - half;
        const float qp = qs[o], kp = ks[o];
        const float qr = c < half ? qp * -1.0f : qp;
        const float kr = c < half ? kp * -1.0f : kp;
        const float ql = qs[c] * cs[c], qg = qr * sn[c];
        const float kl = ks[c] * cs[c], kg = kr * sn[c];
        l.q[c] = ql + qg;
        const float k = kl + kg, v = vs[c];
        l.kcur[c] = k;
        l.vcur[c] = v;
        if (h % group == 0) {
            r.keys[base + (size_t)pos * width + c] = k;
            r.values[base + (size_t)pos * width + c] = v;
        }
    }
    lds_sync();
    attend_staged(l, kb, vb, width, n, last, last, a.scale, vloads);
    emit(l.out, out, width, a.act, t, h, a.heads);
}

hipError_t launch_attention_decode(const Attention& a, const RopeWrite& r, uint32_t tokens, hipStream_t stream) {
    if (tokens == 0 || a.heads == 0) return hipSuccess;
    const size_t lds = attention_decode_lds(a.width, a.capacity);
    TMH_LAUNCH(k_attention_decode, dim3(tokens * a.heads), dim3(256), lds, stream, a, r);
    return hipGetLastError();
}

// ------------------------------------------------------- SwiGLU, add

// dst[r, j] = gate[r, j] / (Maths.exp(-gate[r, j]) + 1) · value[r, j].
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ gate, const float* __restrict__ value,
                                                uint32_t ld, uint32_t n, uint32_t total, float* __restrict__ dst) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t r = i / n, j = i - r * n;
    dst[i] = swiglu_value(gate[(size_t)r * ld + j], value[(size_t)r * ld + j]);
}

// SwiGLU then the activation quantiser: each 8-lane group takes a block of
// 32 outputs of a row (4 a lane) and quantises it into `act` (n a multiple
// of 32), as the quantise pass would quantise SwiGLU's output.
__global__ __launch_bounds__(256) void k_swiglu_quantise(const float* __restrict__ gate,
                                                         const float* __restrict__ value, uint32_t ld, uint32_t n,
                                                         uint32_t blocks, Activations act) {
    const uint32_t g = (blockIdx.x * 256u + threadIdx.x) >> 3;
    const uint32_t sub = threadIdx.x & 7u;
    if (g >= blocks) return;  // all 8 lanes of a block leave together
    const uint32_t nb = n >> 5;
    const uint32_t r = g / nb, blk = g - r * nb;
    const uint32_t j = blk * 32u + sub * 4u;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = swiglu_value(gate[(size_t)r * ld + j + i], value[(size_t)r * ld + j + i]);
    const Q8Quad q = quantize_quad(v[0], v[1], v[2], v[3]);
    *(uint32_t*)((int8_t*)act.qs + (size_t)r * n + j) = q.packed;
    if (sub == 0) {
        ((float*)act.scales)[g] = q.scale;
        ((float*)act.sums)[g] = q.sum;
        ((int32_t*)act.totals)[g] = q.total;
    }
}

hipError_t launch_swiglu_quantise(const float* gate, const float* value, uint32_t ld, uint32_t rows, uint32_t n,
                                  Activations act, hipStream_t stream) {
    const uint64_t blocks = (uint64_t)rows * (n >> 5);
    if (blocks == 0) return hipSuccess;
    if (n % 32u != 0) return hipErrorInvalidValue;
    TMH_LAUNCH(k_swiglu_quantise, dim3((uint32_t)((blocks * 8u + 255u) / 256u)), dim3(256), 0, stream, gate,
                       value, ld, n, (uint32_t)blocks, act);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* gate, const float* value, uint32_t ld, uint32_t rows, uint32_t n, float* dst,
                         hipStream_t stream) {
    const uint64_t total = (uint64_t)rows * n;
    if (total == 0) return hipSuccess;
    TMH_LAUNCH(k_swiglu, dim3((uint32_t)((total + 255u) / 256u)), dim3(256), 0, stream, gate, value, ld, n,
                       (uint32_t)total, dst);
    return hipGetLastError();
}

// dst may be a or b: each element is read, then written, by one thread.
__global__ __launch_bounds__(256) void k_add(const float* a, const float* b, float* dst, uint32_t total) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < total) dst[i] = a[i] + b[i];
}

hipError_t launch_add(const float* a, const float* b, float* dst, uint32_t count, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    TMH_LAUNCH(k_add, dim3((count + 255u) / 256u), dim3(256), 0, stream, a, b, dst, count);
    return hipGetLastError();
}

// ------------------------------------------------------------------- argmax

// Candidate order of the first highest value: higher wins, then the lower
// index; no candidate (-1) loses to any.
__device__ __forceinline__ void better(float& v, int32_t& i, float ov, int32_t oi) {
    if (oi < 0) return;
    if (i < 0 || ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

// The first highest of elements [j0, j1) of row xr across the workgroup
// (NaNs are no candidates: the host's `x[i] > x[best]` never moves to one).
__device__ __forceinline__ void block_best(const float* __restrict__ xr, uint32_t j0, uint32_t j1, float& v,
                                           int32_t& i) {
    __shared__ float vs[4];
    __shared__ int32_t is[4];
    v = 0.0f;
    i = -1;
    for (uint32_t j = j0 + threadIdx.x; j < j1; j += 256u) {
        const float e = xr[j];
        if (e == e && (i < 0 || e > v)) {
            v = e;
            i = (int32_t)j;
        }
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const float ov = __shfl_xor(v, s, 64);
        const int32_t oi = __shfl_xor(i, s, 64);
        better(v, i, ov, oi);
    }
    if ((threadIdx.x & 63u) == 0) {
        vs[threadIdx.x >> 6] = v;
        is[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    for (int k = 0; k < 4; ++k) better(v, i, vs[k], is[k]);
}

// One workgroup per row: as the host's loop, a NaN at index 0 keeps index 0.
__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, uint32_t ldx, uint32_t n,
                                                int32_t* __restrict__ ids) {
    const float* xr = x + (size_t)blockIdx.x * ldx;
    float v;
    int32_t i;
    block_best(xr, 0, n, v, i);
    if (threadIdx.x == 0) {
        const float first = xr[0];
        ids[blockIdx.x] = (first != first || i < 0) ? 0 : i;
    }
}

hipError_t launch_argmax(const float* x, uint32_t ldx, uint32_t rows, uint32_t n, int32_t* ids, hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    TMH_LAUNCH(k_argmax, dim3(rows), dim3(256), 0, stream, x, ldx, n, ids);
    return hipGetLastError();
}

// Elements of a row per workgroup of the split argmax.
constexpr uint32_t ARGMAX_CHUNK = 2048;

uint32_t argmax_chunks(uint32_t n) { return (n + ARGMAX_CHUNK - 1u) / ARGMAX_CHUNK; }

// Split argmax, first half: workgroup (row, chunk) writes the first highest
// of its chunk (value, index or -1).
__global__ __launch_bounds__(256) void k_argmax_chunks(const float* __restrict__ x, uint32_t ldx, uint32_t n,
                                                       uint32_t chunks, float* __restrict__ values,
                                                       int32_t* __restrict__ index) {
    const uint32_t r = blockIdx.x / chunks, c = blockIdx.x - r * chunks;
    const uint32_t j0 = c * ARGMAX_CHUNK, j1 = min(n, j0 + ARGMAX_CHUNK);
    float v;
    int32_t i;
    block_best(x + (size_t)r * ldx, j0, j1, v, i);
    if (threadIdx.x == 0) {
        values[blockIdx.x] = v;
        index[blockIdx.x] = i;
    }
}

// ------------------------------------------------------------- decode step

// After a decode step over `rows` sequences (token r of the step belongs to
// cache row r): picks each row's token from the split argmax's chunks (in
// chunk order, so ties keep the lower index; a NaN logit at index 0 keeps
// index 0), logs it, and moves the row's slot and attention entry one
// position on. A row whose cache is full gets a slot of -1 and an entry one
// past its capacity, so a step that would run it anyway is reported by the
// RoPE and attention kernels instead of writing into the next row.
// One wave per row: the lanes load the chunks' bests together and reduce
// them by `better` (highest value, then lowest index: a maximum under a
// total order, so any reduction order gives the chunk-order result).
__global__ __launch_bounds__(64) void k_advance(uint32_t rows, const float* __restrict__ logits, uint32_t vocab,
                                                uint32_t chunks, const float* __restrict__ values,
                                                const int32_t* __restrict__ index, int32_t* __restrict__ ids,
                                                int32_t* __restrict__ log, uint32_t log_stride,
                                                int32_t* __restrict__ steps, int32_t* __restrict__ slots,
                                                int32_t* __restrict__ table, uint32_t capacity) {
    const uint32_t r = blockIdx.x;
    float v = 0.0f;
    int32_t i = -1;
    for (uint32_t c = threadIdx.x; c < chunks; c += 64u) better(v, i, values[r * chunks + c], index[r * chunks + c]);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const float ov = __shfl_xor(v, s, 64);
        const int32_t oi = __shfl_xor(i, s, 64);
        better(v, i, ov, oi);
    }
    if (threadIdx.x != 0) return;
    const float first = logits[(size_t)r * vocab];
    const int32_t chosen = (first != first || i < 0) ? 0 : i;
    ids[r] = chosen;
    const int32_t step = steps[r];
    if (step >= 0 && step < (int32_t)log_stride) log[(size_t)r * log_stride + step] = chosen;
    steps[r] = step + 1;
    const int32_t length = table[3u * r + 2u];
    const bool full = length < 0 || length >= (int32_t)capacity;
    slots[r] = full ? -1 : slots[r] + 1;
    table[3u * r + 1u] = full ? 0 : length;
    table[3u * r + 2u] = full ? (int32_t)capacity + 1 : length + 1;
}

hipError_t launch_choose_advance(const float* logits, uint32_t rows, uint32_t vocab, float* values, int32_t* index,
                                 int32_t* ids, int32_t* log, uint32_t log_stride, int32_t* steps, int32_t* slots,
                                 int32_t* table, uint32_t capacity, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    const uint32_t chunks = argmax_chunks(vocab);
    TMH_LAUNCH(k_argmax_chunks, dim3(rows * chunks), dim3(256), 0, stream, logits, vocab, vocab, chunks, values,
                       index);
    TMH_LAUNCH(k_advance, dim3(rows), dim3(64), 0, stream, rows, logits, vocab, chunks, values,
                       index, ids, log, log_stride, steps, slots, table, capacity);
    return hipGetLastError();
}

}  // namespace tmh
