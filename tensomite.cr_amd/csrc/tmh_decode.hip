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
#include "tmh_internal.h"

namespace tmh {

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

__device__ __forceinline__ void report(int32_t* errors, int32_t value, int32_t limit) {
    if (atomicAdd(&errors[0], 1) == 0) {
        errors[1] = value;
        errors[2] = limit;
    }
}

// ------------------------------------------------------------------ RMSNorm

// One workgroup per row. The row is staged in LDS; every wave then folds
// the squares in index order (ds_read_b128 broadcasts, four adds each), so
// each wave holds the root without another barrier.
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x, uint32_t ldx,
                                                 const float* __restrict__ w, uint32_t n, float eps,
                                                 float* __restrict__ dst, uint32_t ld_dst) {
    extern __shared__ float4 row4[];
    float* row = reinterpret_cast<float*>(row4);
    const float* xr = x + (size_t)blockIdx.x * ldx;
    for (uint32_t j = threadIdx.x; j < n; j += 256u) row[j] = xr[j];
    __syncthreads();
    float squares = 0.0f;
    const uint32_t n4 = n >> 2;
#pragma unroll 8
    for (uint32_t j = 0; j < n4; ++j) {
        const float4 v = row4[j];
        squares += v.x * v.x;
        squares += v.y * v.y;
        squares += v.z * v.z;
        squares += v.w * v.w;
    }
    for (uint32_t j = n4 << 2; j < n; ++j) squares += row[j] * row[j];
    const float root = __builtin_sqrtf(squares / (float)n + eps);
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

// Largest row the LDS kernel stages (64 KB).
constexpr uint32_t RMSNORM_LDS_ROW = 16384;

hipError_t launch_rmsnorm(const float* x, uint32_t ldx, const float* w, uint32_t rows, uint32_t n, float eps,
                          float* dst, uint32_t ld_dst, hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (n <= RMSNORM_LDS_ROW) {
        const size_t lds = ((size_t)n + 3u) / 4u * 16u;
        hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), lds, stream, x, ldx, w, n, eps, dst, ld_dst);
    } else {
        hipLaunchKernelGGL(k_rmsnorm_wide, dim3(rows), dim3(256), 0, stream, x, ldx, w, n, eps, dst, ld_dst);
    }
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
    hipLaunchKernelGGL(k_rope_write, dim3(grid), dim3(256), 0, stream, a, (uint32_t)total);
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

// One workgroup per (query token, head). Scores of all positions in
// parallel (each a column-order dot product), the top by a tree of
// comparisons (a maximum is exact in any order; a NaN only counts at
// position 0, as the host's `position == 0 || x > top` has it), the
// exponentials in parallel, then the total and the weighted values as
// position-order folds.
__global__ __launch_bounds__(256) void k_attention(Attention a) {
    extern __shared__ float4 lds4[];
    float* qv = reinterpret_cast<float*>(lds4);
    const uint32_t w4 = (a.width + 3u) & ~3u;
    float* sc = qv + w4;
    __shared__ float tops[4];
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
    const float* kb = a.keys + base;
    const float* vb = a.values + base;
    const float* qh = a.q + (size_t)t * a.ldq + (size_t)h * a.width;
    for (uint32_t c = tid; c < a.width; c += 256u) qv[c] = qh[c];
    __syncthreads();

    const uint32_t n = (uint32_t)length;
    const float4* q4 = reinterpret_cast<const float4*>(qv);
    float top = -__builtin_inff();
    for (uint32_t p = tid; p < n; p += 256u) {
        const float4* k4 = reinterpret_cast<const float4*>(kb + (size_t)p * a.width);
        float dot = 0.0f;
        for (uint32_t c = 0; c < (a.width >> 2); ++c) {
            const float4 q = q4[c];
            const float4 k = k4[c];
            dot += q.x * k.x;
            dot += q.y * k.y;
            dot += q.z * k.z;
            dot += q.w * k.w;
        }
        float x = dot * a.scale;
        // The causal mask adds -inf past the row's last position; its 0
        // elsewhere only turns a -0 score into +0, which changes no later bit.
        if ((int32_t)p > last) x = x + -__builtin_inff();
        sc[p] = x;
        top = x > top ? x : top;
    }
    top = wave_top(top);
    if ((tid & 63u) == 0) tops[tid >> 6] = top;
    __syncthreads();
    top = tops[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) top = tops[i] > top ? tops[i] : top;
    if (sc[0] != sc[0]) top = sc[0];

    for (uint32_t p = tid; p < n; p += 256u) sc[p] = maths_exp(sc[p] - top);
    __syncthreads();

    // The total, in position order, by every wave.
    const float4* s4 = reinterpret_cast<const float4*>(sc);
    float total = 0.0f;
    const uint32_t n4 = n >> 2;
#pragma unroll 8
    for (uint32_t j = 0; j < n4; ++j) {
        const float4 e = s4[j];
        total += e.x;
        total += e.y;
        total += e.z;
        total += e.w;
    }
    for (uint32_t j = n4 << 2; j < n; ++j) total += sc[j];
    __syncthreads();
    for (uint32_t p = tid; p < n; p += 256u) sc[p] = sc[p] / total;
    __syncthreads();

    // Σ_p weight_p · v_p[c], in position order: one lane per column.
    for (uint32_t c = tid; c < a.width; c += 256u) {
        const float* vc = vb + c;
        float acc = 0.0f;
        uint32_t p = 0;
        for (; p + 8u <= n; p += 8u) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = vc[(size_t)(p + i) * a.width];
            const float4 w0 = s4[p >> 2], w1 = s4[(p >> 2) + 1u];
            acc += w0.x * v[0];
            acc += w0.y * v[1];
            acc += w0.z * v[2];
            acc += w0.w * v[3];
            acc += w1.x * v[4];
            acc += w1.y * v[5];
            acc += w1.z * v[6];
            acc += w1.w * v[7];
        }
        for (; p < n; ++p) acc += sc[p] * vc[(size_t)p * a.width];
        out[c] = acc;
    }
}

size_t attention_lds(uint32_t width, uint32_t capacity) {
    return ((size_t)((width + 3u) & ~3u) + ((capacity + 3u) & ~3u)) * sizeof(float);
}

hipError_t launch_attention(const Attention& a, uint32_t tokens, hipStream_t stream) {
    if (tokens == 0 || a.heads == 0) return hipSuccess;
    const size_t lds = attention_lds(a.width, a.capacity);
    hipLaunchKernelGGL(k_attention, dim3(tokens * a.heads), dim3(256), lds, stream, a);
    return hipGetLastError();
}

// ------------------------------------------------------- SwiGLU, add

// dst[r, j] = gate[r, j] / (Maths.exp(-gate[r, j]) + 1) · value[r, j].
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ gate, const float* __restrict__ value,
                                                uint32_t ld, uint32_t n, uint32_t total, float* __restrict__ dst) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t r = i / n, j = i - r * n;
    const float g = gate[(size_t)r * ld + j];
    const float e = maths_exp(-g);
    const float d = e + 1.0f;
    const float q = g / d;
    dst[i] = q * value[(size_t)r * ld + j];
}

hipError_t launch_swiglu(const float* gate, const float* value, uint32_t ld, uint32_t rows, uint32_t n, float* dst,
                         hipStream_t stream) {
    const uint64_t total = (uint64_t)rows * n;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_swiglu, dim3((uint32_t)((total + 255u) / 256u)), dim3(256), 0, stream, gate, value, ld, n,
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
    hipLaunchKernelGGL(k_add, dim3((count + 255u) / 256u), dim3(256), 0, stream, a, b, dst, count);
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

// One workgroup per row: each thread the first highest of its strided
// elements, then a tree over candidates. As the host's loop (`x[i] >
// x[best]` from best = 0) never moves to a NaN, NaNs are no candidates, and
// a NaN at index 0 keeps index 0.
__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, uint32_t ldx, uint32_t n,
                                                int32_t* __restrict__ ids) {
    __shared__ float vs[4];
    __shared__ int32_t is[4];
    const float* xr = x + (size_t)blockIdx.x * ldx;
    float v = 0.0f;
    int32_t i = -1;
    for (uint32_t j = threadIdx.x; j < n; j += 256u) {
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
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k) better(v, i, vs[k], is[k]);
        const float first = xr[0];
        ids[blockIdx.x] = (first != first || i < 0) ? 0 : i;
    }
}

hipError_t launch_argmax(const float* x, uint32_t ldx, uint32_t rows, uint32_t n, int32_t* ids, hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(256), 0, stream, x, ldx, n, ids);
    return hipGetLastError();
}

// ------------------------------------------------------------- decode step

// After a decode step over `rows` sequences (token r of the step belongs to
// cache row r): logs each chosen id, and moves each row's slot and
// attention entry one position on. A row whose cache is full gets a slot
// of -1 and an entry one past its capacity, so a step that would run it
// anyway is reported by the RoPE and attention kernels instead of writing
// into the next row.
__global__ void k_advance(uint32_t rows, const int32_t* __restrict__ chosen, int32_t* __restrict__ log,
                          uint32_t log_stride, int32_t* __restrict__ steps, int32_t* __restrict__ slots,
                          int32_t* __restrict__ table, uint32_t capacity) {
    const uint32_t r = blockIdx.x * 64u + threadIdx.x;
    if (r >= rows) return;
    const int32_t step = steps[r];
    if (step >= 0 && step < (int32_t)log_stride) log[(size_t)r * log_stride + step] = chosen[r];
    steps[r] = step + 1;
    const int32_t length = table[3u * r + 2u];
    const bool full = length < 0 || length >= (int32_t)capacity;
    slots[r] = full ? -1 : slots[r] + 1;
    table[3u * r + 1u] = full ? 0 : length;
    table[3u * r + 2u] = full ? (int32_t)capacity + 1 : length + 1;
}

hipError_t launch_advance(uint32_t rows, const int32_t* chosen, int32_t* log, uint32_t log_stride, int32_t* steps,
                          int32_t* slots, int32_t* table, uint32_t capacity, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(k_advance, dim3((rows + 63u) / 64u), dim3(64), 0, stream, rows, chosen, log, log_stride, steps,
                       slots, table, capacity);
    return hipGetLastError();
}

}  // namespace tmh
