// Declarations shared by the runtime (tmh_runtime.hip) and the kernels
// (tmh_kernels.hip) of libtensomite_hip.so. Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tmh {

// Bytes of one block of 32 values, by kind (dtype.cr:237-244).
constexpr uint32_t block_bytes(uint32_t kind) { return kind == 0 ? 34u : kind == 1 ? 18u : 20u; }

// Quantised activations in device memory, as the quantise pass writes them:
// per block of 32 its F16-rounded scale, F16(d·Σq), Σq; and the int8 values.
struct Activations {
    const float* scales;
    const float* sums;
    const int32_t* totals;
    const int8_t* qs;
};

// Launches the quantise pass over `rows` rows of `k` values, `ldx` apart.
hipError_t launch_quantize(const float* x, uint32_t ldx, uint32_t rows, uint32_t k, float* scales, float* sums,
                           int32_t* totals, int8_t* qs, hipStream_t stream);

// Launches dst[rows, n] = x · wᵀ (+ bias) over quantised activations, in the
// kernel `mode` asks for (TMH_MODE_*). `w` points at the first weight row.
hipError_t launch_block_matmul(uint32_t kind, uint32_t mode, const uint8_t* w, Activations act, float* dst,
                               const float* bias, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                               hipStream_t stream);

// Whether one activation row of this weight can take the one-row kernel,
// which quantises the activations itself (no separate quantise pass).
bool row_kernel_fits(uint32_t mode, const uint8_t* w, uint32_t k);

// Launches dst[n] = x · wᵀ (+ bias) for one f32 activation row x.
hipError_t launch_row(uint32_t kind, const uint8_t* w, const float* x, float* dst, const float* bias, uint32_t n,
                      uint32_t k, int compute_units, hipStream_t stream);

// One product of a grouped launch of one-row products: its operands, then
// the tiling the launcher chose (rows per workgroup, LDS stride, tiles) and
// the first workgroup of the launch that runs it.
struct RowProduct {
    const uint8_t* w;
    const float* x;
    float* dst;
    const float* bias;
    uint32_t n, k;
    uint32_t tr, stride, tiles, first;
};

// Fills in p's tiling (tr, stride, tiles).
void plan_row(uint32_t kind, RowProduct& p, int compute_units);

// LDS a workgroup needs for p's activations, and for p's contributions.
size_t row_act_bytes(const RowProduct& p);
size_t row_part_bytes(const RowProduct& p);

// Launches the persistent one-row kernel over a device table of products
// holding `tiles` tiles, tile t belonging to product owner[t], all of kind
// `kind`, with LDS for the largest activations and contributions among them.
hipError_t launch_rows(uint32_t kind, const RowProduct* table, const uint32_t* owner, uint32_t tiles,
                       size_t act_bytes, size_t part_bytes, int compute_units, hipStream_t stream);

// Launches the block gather; ids out of range go to `errors` (count, id, rows).
hipError_t launch_gather(uint32_t kind, const uint8_t* table, int32_t table_rows, uint32_t width, const int32_t* ids,
                         uint32_t count, float* dst, int32_t* errors, hipStream_t stream);

}  // namespace tmh
