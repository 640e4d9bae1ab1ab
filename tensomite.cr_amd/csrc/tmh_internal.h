// Declarations shared by the sources of libtensomite_hip.so: the runtime
// (tmh_runtime.hip), the product kernels (tmh_kernels.hip), the decode-graph
// kernels (tmh_decode.hip) and the decoder (tmh_llama.hip). Not part of the
// C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace tmh {

// Counts one kernel launch on the calling thread's current device (the
// counters' `launches`, as CUDA's Context#launches, cuda.cr:463-475). Every
// launch site goes through TMH_LAUNCH; a captured graph's replays launch
// its kernels without counting them again.
void count_launch();
#define TMH_LAUNCH(...)              \
    do {                             \
        ::tmh::count_launch();       \
        hipLaunchKernelGGL(__VA_ARGS__); \
    } while (0)

// Whether the product launches this thread queues fold each row's
// contributions in UNORDERED's order (Fold4: four running sums) rather than the
// host's block order: set, for the launches of one call, by tmh_block_matmul
// in TMH_MODE_UNORDERED and by plans and decoders set to that mode
// (measurement only). The launchers pass it to the kernels.
bool tree_fold();
struct TreeFold {
    bool saved;
    explicit TreeFold(bool on);
    ~TreeFold();
};

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

// One product of the streamed one-row kernel: operands; the address of the
// last 16-byte piece of its weight rows (direct loads never read past it);
// its steps first ... first + steps - 1 of the launch, each `rows`
// consecutive weight rows (the last may hold fewer), step_bytes apart;
// pairs per row np, bytes per row, LDS floats between two rows'
// contributions.
// How a streamed product's activation row arrives: f32 x, quantised by the
// kernel; f32 x under an RMSNorm (x / sqrt(Σx²/k + eps) · norm, the host's
// order) then quantised; or already quantised by the quantise pass (its
// int8 values at x, scales at aux0, and at aux1 the block extras the kind
// reads: Q4_0 totals, Q4_1 sums).
constexpr uint32_t STREAM_X_F32 = 0, STREAM_X_RMSNORM = 1, STREAM_X_QUANTISED = 2;

struct StreamProduct {
    const uint8_t* w;
    const float* x;
    float* dst;
    const float* bias;
    uint64_t wlast;
    uint32_t n, k, first, steps;
    uint32_t np, rows, row_bytes, stride;
    uint32_t step_bytes, mode;
    float eps;
    uint32_t unused;
    const float* aux0;  // STREAM_X_RMSNORM: the norm's weights; STREAM_X_QUANTISED: scales
    const void* aux1;   // STREAM_X_QUANTISED: totals (Q4_0) or sums (Q4_1)
};

// What one workgroup of the streamed kernel starts from, in one record so
// that its first loads (its first product's activation row, the first
// step's weights) need one scalar round trip: its steps s_begin ... s_end - 1,
// its first product, that product's input mode and arrays (x0, a0, a1, K in
// k0), the x and K of its second product when both take f32 x (x1 null
// otherwise: a later product is prepared in the loop), and the issue cursor
// at its first step (weight address, the product's last 16-byte piece, bias
// or a stand-in with has 0, steps left, bytes and rows per step, first row, n).
struct StreamStart {
    uint64_t src, wlast;
    const float* bias;
    const float* x0;
    const float* x1;
    const float* a0;
    const void* a1;
    uint32_t k0, k1, s_begin, s_end, first_pi, left, step_bytes, rows, row, n, has, mode0;
};

// The shape of a streamed launch: the product table and each workgroup's
// start (device memory), steps in all, workgroups, ring slots,
// whether any product has a bias, LDS of one activation buffer and of one
// buffer of contributions (floats), floats of one staged x, the
// activations' LDS offset, LDS in all.
struct StreamLaunch {
    const StreamProduct* table;
    const StreamStart* starts;
    uint32_t total, grid, ring, has_bias, act_bytes, part_floats, x_floats, act_offset;
    size_t lds;
    uint32_t tree;  // UNORDERED's fold
};

// Host side: fills in each product's geometry and steps (w, x, dst, bias, n,
// k set by the caller), the launch's shape, and each workgroup's first
// product. False when the products do not fit the kernel (rows of an odd
// number of blocks, or LDS).
// wgs_per_cu: workgroups per compute unit (0: the default, 6, or TMH_STREAM_WGS);
// the ring gets the LDS they leave.
bool plan_stream(uint32_t kind, std::vector<StreamProduct>& products, int compute_units, StreamLaunch& launch,
                 std::vector<StreamStart>& starts, uint32_t wgs_per_cu = 0);

// Builds a streamed launch for `products` and uploads its product table and
// workgroup starts into one device allocation (*mem, freed by the caller).
// hipErrorInvalidValue, nothing allocated, when the products do not fit
// the kernel.
hipError_t make_stream(uint32_t kind, std::vector<StreamProduct>& products, int compute_units, StreamLaunch& launch,
                       void** mem, uint32_t wgs_per_cu = 0);

// Launches the streamed one-row kernel (table and starts in device memory).
hipError_t launch_stream(uint32_t kind, const StreamLaunch& launch, hipStream_t stream);

// dst[rows, n] = residual[rows, n] + act · wᵀ for a few activation rows
// (fewer than the matrix cores take), the residual added in the product's
// fold as a bias row per activation row: the host's `x + product`, one
// rounding. hipErrorInvalidValue when the shape is not for that kernel.
hipError_t launch_product_residual(uint32_t kind, const uint8_t* w, Activations act, float* dst, const float* residual,
                                   uint32_t rows, uint32_t n, uint32_t k, int compute_units, hipStream_t stream);

// SwiGLU(act · gateᵀ, act · upᵀ) quantised into `glu` ([rows, H] as the
// quantise pass lays it out), one launch per group of rows: w is the merged
// [gate | up] matrix of 2·H rows, the lanes product folds each output in
// block order and its epilogue applies SwiGLU and the quantiser, with the
// bits of a product, k_swiglu_quantise's arithmetic and a quantise pass.
// hipErrorInvalidValue when the shape is not for that kernel.
hipError_t launch_gate_up_swiglu(uint32_t kind, const uint8_t* w, Activations act, uint32_t rows, uint32_t H,
                                 uint32_t k, Activations glu, hipStream_t stream);

// One-row products over an f32 row x that each workgroup first takes through
// RMSNorm (weights `norm`, eps) and the activation quantiser, with the bits
// of the norm+quantise launch then the lanes product: dst[n]; and gate_up
// with SwiGLU and the quantiser in its epilogue, as launch_gate_up_swiglu.
// hipErrorInvalidValue when the shape is not for them (rows other than 1, k
// above 2048, rows of an odd number of blocks, x or norm not 16-byte aligned).
bool rms_product_fits(const uint8_t* w, uint32_t k, const float* x, uint32_t ldx, const float* norm);
hipError_t launch_product_rms(uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, const float* norm,
                              float eps, float* dst, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                              hipStream_t stream);
hipError_t launch_gate_up_swiglu_rms(uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, const float* norm,
                                     float eps, uint32_t rows, uint32_t H, uint32_t k, Activations glu,
                                     hipStream_t stream);

// Input modes of the few-rows products with weights in LDS.
constexpr uint32_t NB_QUANT = 0;  // rows quantised already (act, as the quantise pass lays them out)
constexpr uint32_t NB_F32 = 1;    // f32 rows x, quantised by each workgroup
constexpr uint32_t NB_NORM = 2;   // f32 rows x through RMSNorm (weights nw, eps), then quantised

// dst[rows, n] = rows of activations times w (n rows), + bias[b · bias_ld +
// row] as a separate rounding: groups of 8, 4 and 2 rows a launch, each
// workgroup's weight tile direct-loaded into LDS at its start and, for
// F32/NORM, the rows quantised (NORM: through RMSNorm first) by every
// workgroup in its prologue; the bits of the quantise pass (or norm +
// quantise) then the product. hipErrorInvalidValue, nothing launched, when
// the shape is not for it (F32/NORM: k above 2048; rows of an odd number of
// blocks; x, norm or the activations not 16-byte aligned).
hipError_t launch_rows_product(uint32_t kind, uint32_t mode, const uint8_t* w, const float* x, uint32_t ldx,
                               const float* nw, float eps, Activations act, float* dst, const float* bias,
                               uint32_t bias_ld, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                               hipStream_t stream);

// gate_up of rows (NORM: x through RMSNorm; QUANT: act) with SwiGLU and
// the quantiser in the epilogue, as launch_gate_up_swiglu_rms for several
// rows: glu receives [rows, H] quantised as the quantise pass lays them out.
hipError_t launch_rows_gate_up(uint32_t kind, uint32_t mode, const uint8_t* w, const float* x, uint32_t ldx,
                               const float* nw, float eps, Activations act, uint32_t rows, uint32_t H, uint32_t k,
                               Activations glu, hipStream_t stream);

// One quantised activation row times w (n rows), dst[row] = Σ (+ bias[row]):
// the weights of each workgroup's tile direct-loaded into LDS at its start.
// hipErrorInvalidValue when the shape is not for it.
hipError_t launch_product_one(uint32_t kind, const uint8_t* w, Activations act, float* dst, const float* bias,
                              uint32_t n, uint32_t k, int compute_units, hipStream_t stream);
// One or two f32 rows (ldx apart) quantised in each workgroup's prologue
// (no norm), k <= 8192.
hipError_t launch_product_f32_one(uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, float* dst,
                                  const float* bias, uint32_t rows, uint32_t n, uint32_t k, int compute_units,
                                  hipStream_t stream);

// dst[i] = the F16 bits of the float with word first + i, i < count.
hipError_t launch_f16_words(uint32_t first, uint32_t count, uint16_t* dst, hipStream_t stream);

// The read-rate hook: `workgroups` workgroups read bytes / 16 pieces at src
// grid-stride, out[b] the XOR of workgroup b's.
hipError_t launch_read(const void* src, uint64_t bytes, uint32_t workgroups, uint32_t* out, hipStream_t stream);

// Launches the block gather; ids out of range go to `errors` (count, id, rows).
hipError_t launch_gather(uint32_t kind, const uint8_t* table, int32_t table_rows, uint32_t width, const int32_t* ids,
                         uint32_t count, float* dst, int32_t* errors, hipStream_t stream);

// ------------------------------------------------- the rest of the decode graph
// (tmh_decode.hip)

// RMSNorm of `rows` rows of n (x rows ldx apart, dst rows ld_dst apart);
// `w` may be null (no weight).
hipError_t launch_rmsnorm(const float* x, uint32_t ldx, const float* w, uint32_t rows, uint32_t n, float eps,
                          float* dst, uint32_t ld_dst, hipStream_t stream);

// RoPE of q and k heads and the cache write of k and v, for tokens whose
// rows of `x` hold [heads q | kv_heads k | kv_heads v] of `width` each.
struct RopeWrite {
    const float* x;
    uint32_t ldx;
    uint32_t heads, kv_heads, width;
    const float* cos;  // [capacity or more, width]
    const float* sin;
    const int32_t* slots;  // per token: cache row · capacity + position
    uint32_t cache_rows, capacity;
    float* q_dst;   // [tokens, heads, width]
    float* keys;    // [cache_rows, kv_heads, capacity, width]
    float* values;  // likewise
    int32_t* errors;
};
hipError_t launch_rope_write(const RopeWrite& a, uint32_t tokens, hipStream_t stream);

// Attention of `tokens` query rows of `heads` heads against the cache; per
// token the table holds (cache row, last position it sees, positions held).
struct Attention {
    const float* q;
    uint32_t ldq;  // token t's heads start at q + t·ldq
    const float* keys;
    const float* values;
    uint32_t cache_rows, kv_heads, capacity, width, heads;
    const int32_t* table;
    float scale;
    float* dst;
    uint32_t ld_dst;
    int32_t* errors;
    Activations act;  // with qs set, the outputs are also quantised here (width a multiple of 32)
};
size_t attention_lds(uint32_t width, uint32_t capacity);
size_t attention_decode_lds(uint32_t width, uint32_t capacity);  // of launch_attention_decode
hipError_t launch_attention(const Attention& a, uint32_t tokens, hipStream_t stream);
// A decode step's attention with the RoPE and cache write of `r` fused: each
// token is its cache row's one new position.
hipError_t launch_attention_decode(const Attention& a, const RopeWrite& r, uint32_t tokens, hipStream_t stream);

// RMSNorm then quantisation into `act`, one launch; for n a multiple of 32
// up to the LDS limit.
bool rmsnorm_quantise_fits(uint32_t n);
hipError_t launch_rmsnorm_quantise(const float* x, uint32_t ldx, const float* w, uint32_t rows, uint32_t n, float eps,
                                   Activations act, hipStream_t stream);
hipError_t launch_swiglu_quantise(const float* gate, const float* value, uint32_t ld, uint32_t rows, uint32_t n,
                                  Activations act, hipStream_t stream);

hipError_t launch_swiglu(const float* gate, const float* value, uint32_t ld, uint32_t rows, uint32_t n, float* dst,
                         hipStream_t stream);
hipError_t launch_add(const float* a, const float* b, float* dst, uint32_t count, hipStream_t stream);
hipError_t launch_argmax(const float* x, uint32_t ldx, uint32_t rows, uint32_t n, int32_t* ids, hipStream_t stream);
// The greedy choice of every row of a decode step and the move to the next
// position: a split argmax over `logits` [rows, vocab] through values/index
// (rows · argmax_chunks(vocab) entries each), then ids, the log and the
// device-held slots and attention entries.
uint32_t argmax_chunks(uint32_t n);
hipError_t launch_choose_advance(const float* logits, uint32_t rows, uint32_t vocab, float* values, int32_t* index,
                                 int32_t* ids, int32_t* log, uint32_t log_stride, int32_t* steps, int32_t* slots,
                                 int32_t* table, uint32_t capacity, hipStream_t stream);

// ------------------------------------------------- the runtime, for other sources

// The calling thread's device: its ordered stream, compute units and error
// buffer; returns a TMH_* code (0 on success).
struct DeviceContext {
    int index;
    hipStream_t stream;
    int compute_units;
    int32_t* errors;
};
int device_context(DeviceContext* out, bool kernels);
// Marks the error buffer as possibly written, for the next sync to check,
// and counts `ops` kernel ops.
void note_launch(int index, int ops, bool errors);
// Device allocation honouring the allocation-failure test hook.
hipError_t device_malloc(void** p, size_t bytes);
// Bytes the quantise pass writes for `rows` rows of k, and its carving.
size_t scratch_need(uint32_t rows, uint32_t k);
Activations carve_scratch(uint8_t* base, uint32_t rows, uint32_t k);

// ------------------------------------------------- GGUF files (tmh_gguf.hip)

// Tensor kinds by ggml's numbering (gguf.cr:29-36).
constexpr uint32_t GGUF_F32 = 0, GGUF_F16 = 1, GGUF_Q4_0 = 2, GGUF_Q4_1 = 3, GGUF_Q8_0 = 8, GGUF_BF16 = 30;

struct GgufValue {
    uint32_t type = 0;  // GGUF value type
    int64_t i = 0;      // integers and bools
    double f = 0.0;     // float32 (widened) and float64
    std::string s;      // strings
};

struct GgufTensor {
    std::string name;
    uint32_t kind;
    std::vector<int64_t> shape;  // outermost first
    uint64_t offset, bytes;      // within the file
};

// A GGUF file, memory-mapped and parsed (metadata scalars and the tensor
// directory); tensors are read from the mapping on demand.
struct Gguf {
    std::string path;
    const uint8_t* map = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, GgufValue> metadata;
    std::vector<GgufTensor> tensors;
    std::unordered_map<std::string, int> index;

    ~Gguf();
    int open(const char* file);  // a TMH_* code
    const GgufTensor* find(const std::string& name) const;
    const GgufValue* value(const std::string& key) const;
};

uint64_t gguf_bytes_for(uint32_t kind, int64_t count);
// Rows rows[0..count) of t (every row, in order, when rows is null) into out.
bool gguf_rows(const Gguf& g, const GgufTensor& t, const int32_t* rows, uint32_t count, std::vector<uint8_t>& out);

}  // namespace tmh
