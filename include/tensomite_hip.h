/*
 * tensomite_hip.h -- the C ABI of libtensomite_hip.so, an MI355X (gfx950)
 * backend for tensomite's quantised products (Op::BlockMatMul) and block
 * gathers (Op::Gather on a block table).
 *
 * It replaces, for this device, the native seam the reference's CUDA device
 * binds through `lib LibCUDA` / `lib LibNVRTC` (src/tensomite/cuda/lib.cr:48-110)
 * and the host-side pieces of `CUDA < HostDevice` that manage device memory
 * (src/tensomite/cuda.cr). Conventions follow that seam so a Crystal `lib`
 * binding is a line per function:
 *
 *   - every entry point returns an int: 0 on success, a HIP runtime error
 *     code (1..999, hipError_t's numbering) or a library code (TMH_ERROR_*);
 *     tmh_error_name/tmh_error_string describe it (cuda/lib.cr:51-52,
 *     cuda.cr:1069-1075);
 *   - device memory is a uint64_t address (LibCUDA::DevicePtr, cuda/lib.cr:49);
 *   - no run-time compilation: the kernels are built offline for gfx950.
 *
 * Threads: any thread may call. Each thread addresses the device it last
 * passed to tmh_set_device (device 0 if none), as the reference's
 * Context#bind makes its context current per thread (cuda.cr:1118-1125).
 * All work for a device -- kernels and copies -- is queued on ONE ordered
 * stream, so it runs in submission order (the reference's single default
 * stream, cuda.cr:1176-1196).
 */
#ifndef TENSOMITE_HIP_H
#define TENSOMITE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ result codes */

#define TMH_SUCCESS 0
/* 1..999: hipError_t values, passed through. */
#define TMH_ERROR_INVALID_VALUE 1000 /* an argument out of range (null pointer, size) */
#define TMH_ERROR_SHAPE 1001         /* shapes disagree: ShapeError (errors.cr) */
#define TMH_ERROR_DTYPE 1002         /* not a block kind: DTypeError (errors.cr) */
#define TMH_ERROR_NO_KERNELS 1003    /* kernels unavailable: the caller runs its host kernel
                                        (cuda.cr:1164-1172, CUDA_ERROR_NOT_SUPPORTED) */
#define TMH_ERROR_OUT_OF_MEMORY 1004 /* device allocation failed */
#define TMH_ERROR_EXECUTION 1005     /* a kernel found an index out of range: ExecutionError,
                                        reported at tmh_sync (cuda.cr:967-983) */
#define TMH_ERROR_NO_DEVICE 1006     /* no GPU, or a device index out of range */
#define TMH_ERROR_BUSY 1007          /* the retired list is busy or full (buffer_pool.cr:101-111) */
#define TMH_ERROR_NOT_READY 1008     /* tmh_block_matmul_fixed before tmh_init set the device up */
#define TMH_ERROR_SCRATCH_LIMIT 1009 /* tmh_block_matmul_fixed: more than TMH_FIXED_SCRATCH_BYTES of
                                        quantised activations */

/* Bytes of quantised activations tmh_block_matmul_fixed can hold: per row,
 * k int8 values and three 4-byte values per block of 32 (each of the four
 * parts rounded up to 256 bytes over all rows), e.g. 512 rows of k = 2048. */
#define TMH_FIXED_SCRATCH_BYTES (8u << 20)

/* Block kinds, numbered as the reference's kernels number them (cuda.cr:774-781). */
#define TMH_Q8_0 0 /* F16 d, 32 int8: x = q·d                      (34 bytes) */
#define TMH_Q4_0 1 /* F16 d, 16 bytes of nibbles: x = (q - 8)·d     (18 bytes) */
#define TMH_Q4_1 2 /* F16 d, F16 m, 16 bytes of nibbles: x = q·d + m (20 bytes) */

/* How a product divides its work: BlockMatMulMode (quant.cr:5-28). AUTO,
 * THREAD, LANES and MATRIX give the host's bits. UNORDERED is for
 * measurement only (quant.cr:14-17 prices the ordered sum the same way):
 * from 32 activation rows, where k is a multiple of 256, it runs the
 * matrix-core kernel with each block's contribution added by one fused
 * multiply-add; below that it runs AUTO's kernels with each row's
 * contributions summed as four running sums instead of in block order (as
 * block_matmul_unordered_f32, cuda/kernels.cu:1334-1375, prices the lanes
 * product); its results may differ in the last bits. LOADS, STREAM and STREAM_ACTIVATIONS are Metal measurement
 * modes the reference runs as LANES elsewhere; so does this device. MATRIX
 * has no counterpart in the reference: the int8 matrix-core path for many
 * activation rows. */
#define TMH_MODE_AUTO 0
#define TMH_MODE_THREAD 1
#define TMH_MODE_LANES 2
#define TMH_MODE_UNORDERED 3
#define TMH_MODE_LOADS 4
#define TMH_MODE_STREAM 5
#define TMH_MODE_STREAM_ACTIVATIONS 6
#define TMH_MODE_MATRIX 7

typedef struct tmh_device_info {
    char name[256];          /* marketing name, as GPU#name (cuda.cr:316) */
    char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint64_t memory;         /* global memory in bytes, as GPU#memory */
    int32_t compute_units;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width;
    int32_t l2_bytes;
    int32_t lds_bytes_per_block;
} tmh_device_info;

/* Device counters, as CUDA#uploads/#downloads/#gpu_ops/#device_bytes and
 * BufferPool#hits/#misses/#held/#limit (cuda.cr:214-230, buffer_pool.cr:14-35);
 * `frees` counts device memory freed because the pool was full, `launches`
 * the kernels queued (Context#launches, cuda.cr:463-475; a captured graph's
 * replays are not counted again). */
typedef struct tmh_counters {
    int64_t uploads;
    int64_t downloads;
    int64_t gpu_ops;
    int64_t device_bytes;
    int64_t pool_held;
    int64_t pool_limit;
    int64_t pool_hits;
    int64_t pool_misses;
    int64_t frees;
    int64_t launches;
} tmh_counters;

/* ------------------------------------------------------------ devices */

/* Starts the runtime and counts the GPUs: CUDA.init + gpu_count
 * (cuda.cr:985-1000; cuInit/cuDeviceGetCount, cuda/lib.cr:53-54). */
int tmh_init(int32_t* count);

/* Name, memory and shape of a GPU (GPU record, cuda.cr:310-320;
 * cuDeviceGetName/cuDeviceTotalMem/cuDeviceGetAttribute, cuda/lib.cr:55-58). */
int tmh_device_info_get(int32_t device, tmh_device_info* out);

/* Makes `device` current on the calling thread (Context#bind, cuda.cr:1118-1125;
 * cuCtxSetCurrent, cuda/lib.cr:61). */
int tmh_set_device(int32_t device);
int tmh_get_device(int32_t* device);

/* ------------------------------------------------------------ memory */

/* Raw device memory: Context#alloc/#free (cuda.cr:1128-1137; cuMemAlloc/cuMemFree,
 * cuda/lib.cr:65-66). At least 4 bytes are allocated, as CUDA#alloc does. */
int tmh_malloc(uint64_t* ptr, uint64_t bytes);
int tmh_free(uint64_t ptr);

/* Frees from any thread, never failing the caller: Context#free_from_any_thread
 * (cuda.cr:1139-1143), for finalizers. Returns 0. */
int tmh_free_any_thread(uint64_t ptr);

/* Copies host memory into device memory and returns when the bytes are on
 * the device: Context#upload (cuda.cr:1146-1149; cuMemcpyHtoD, cuda/lib.cr:67). */
int tmh_upload(uint64_t dst, const void* src, uint64_t bytes);

/* Queues a copy into device memory and returns once `src` has been copied
 * into the library's pinned staging ring, so the caller may free or reuse it
 * at once. Ordered with kernels and copies like every other call. No
 * counterpart in the reference, whose uploads are synchronous (cuda.cr:360-370):
 * it overlaps the host-side copy of one chunk with the DMA of the last. */
int tmh_upload_async(uint64_t dst, const void* src, uint64_t bytes);

/* Copies device memory to the host after all queued work has finished:
 * Context#download (cuda.cr:1151-1154; cuMemcpyDtoH, cuda/lib.cr:68). */
int tmh_download(void* dst, uint64_t src, uint64_t bytes);

/* Device-to-device copy, queued in order (Tensor#take_rows/.cat_rows on a
 * device, tensor/quantised.cr:32-55, without the host round trip). */
int tmh_copy(uint64_t dst, uint64_t src, uint64_t bytes);

/* Waits for all queued work: Context#synchronize (cuda.cr:1156-1158;
 * cuCtxSynchronize, cuda/lib.cr:62). */
int tmh_synchronize(void);

/* ------------------------------------------------------- the buffer layer */

/* Device memory of exactly `bytes`, from the pool when a buffer of that size
 * is free, else newly allocated: CUDA#alloc (cuda.cr:339-353) over
 * BufferPool#take (buffer_pool.cr:38-51). */
int tmh_alloc(uint64_t* ptr, uint64_t bytes);

/* Gives memory back, from any thread and never waiting: CUDA#retire
 * (cuda.cr:439-444) over RetiredList#push (buffer_pool.cr:101-111). When the
 * list is busy or full, the memory is freed at once instead. Returns 0. */
int tmh_retire(uint64_t ptr, uint64_t bytes);

/* Waits for the GPU, moves retired memory into the pool (freeing what it
 * cannot hold), then reports a kernel's index error, if any, as
 * TMH_ERROR_EXECUTION: CUDA#sync (cuda.cr:419-428), #recycle_retired
 * (447-454), #check_errors (972-983). */
int tmh_sync(void);

/* The pool's limit in bytes (default max(1 GiB, a quarter of device memory),
 * cuda.cr:319). */
int tmh_pool_set_limit(int64_t bytes);

int tmh_counters_get(tmh_counters* out);

/* ------------------------------------------------------------ errors */

/* hipGetErrorName/hipGetErrorString for HIP codes; the library's own names
 * for TMH_ERROR_* (cuGetErrorName/cuGetErrorString, cuda/lib.cr:51-52). */
const char* tmh_error_name(int code);
const char* tmh_error_string(int code);

/* The first index error a gather kernel reported since the last call:
 * out[0] = reports, out[1] = the id, out[2] = the table's rows; clears it
 * (the error buffer of cuda.cr:961-983). */
int tmh_error_report(int32_t out[3]);

/* Test hook: makes the next `count` device allocations fail with
 * TMH_ERROR_OUT_OF_MEMORY (the stub driver's malloc failure,
 * scripts/cuda_stub/libcuda.c:100-106). */
int tmh_debug_fail_allocations(int32_t count);

/* Test hook: with `off` non-zero, every kernel entry point returns
 * TMH_ERROR_NO_KERNELS, as when the reference's module cannot load
 * (cuda.cr:1164-1172). */
int tmh_debug_disable_kernels(int32_t off);

/* Test hook: dst[i] (uint16, device) = the F16 bits the device's kernels
 * round the float with bit pattern first + i to (F16.new, f16.cr:29-41),
 * for i < count: lets a test sweep every f32 word through the device's own
 * conversion (the activation scales and sums use it). Queued on the stream. */
int tmh_debug_f16_words(uint32_t first, uint32_t count, uint64_t dst);

/* Measurement hook (no counterpart in the reference): `workgroups`
 * workgroups of 256 threads read `bytes` (a multiple of 16, src 16-byte
 * aligned) grid-stride, 16 bytes a lane a load and four loads in flight,
 * non-temporal, and write the XOR of what each read to out[workgroup]
 * (uint32, device). Timed with tmh_event_*, it gives the HBM read rate the
 * product kernels are measured against. Queued on the stream. */
int tmh_debug_read(uint64_t src, uint64_t bytes, uint32_t workgroups, uint64_t out);

/* ------------------------------------------------------------ events */

/* Timing on the library's stream: cuEventCreate/Record/ElapsedTime
 * (cuda/lib.cr:80-86; CUDA::Profile per-kernel timing, cuda.cr:463-481). */
int tmh_event_create(uint64_t* event);
int tmh_event_record(uint64_t event);
int tmh_event_elapsed_ms(uint64_t start, uint64_t stop, float* ms);
int tmh_event_destroy(uint64_t event);

/* ------------------------------------------------------------ kernels */

/* Quantises `rows` rows of `k` activations (k a multiple of 32, rows `ldx`
 * floats apart) to 8 bits per block of 32, as quantize_rows_q8_f32
 * (cuda/kernels.cu:1190-1207) and the host's quantize_activations
 * (quant.cr:424-442) do: per block d = amax/127, q = round-half-away(x/d),
 * scales[b] = F16(d), sums[b] = F16(Σq·d), totals[b] = Σq; qs is [rows, k]
 * int8, the others [rows, k/32]. */
int tmh_quantize_rows_q8(uint64_t x, uint32_t rows, uint32_t k, uint32_t ldx, uint64_t scales, uint64_t sums,
                         uint64_t totals, uint64_t qs);

/* dst[rows, n] = x[rows, k] · wᵀ (+ bias[n]) for a block-format weight w of n
 * rows of k values, the weight's first row `w_byte_offset` bytes into its
 * buffer (a row slice, as `bytes_for(view.offset)`): Op::BlockMatMul as
 * CUDA#launch_blocks queues it (cuda.cr:736-756) -- the activations
 * quantised into library scratch, then the product, every output summing its
 * blocks in order with the host's expressions, so the bits equal
 * Quant.matmul_reference's (quant.cr:122-142) and do not depend on `rows`.
 * Rows of x are `ldx` floats apart; dst is dense [rows, n]; bias may be 0.
 * `mode` is a TMH_MODE_*. */
int tmh_block_matmul(uint32_t kind, uint64_t w, uint64_t w_byte_offset, uint64_t x, uint32_t ldx, uint64_t dst,
                     uint64_t bias, uint32_t rows, uint32_t n, uint32_t k, uint32_t mode);

/* tmh_block_matmul without any allocation: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, hosts that forbid it). Same arguments, kernels
 * and bits as tmh_block_matmul, but the quantised activations live in a
 * fixed per-GPU array of TMH_FIXED_SCRATCH_BYTES that the library holds
 * until the process ends (one-row products the one-row kernel takes need
 * none). tmh_init must have run first (it sets every device up):
 * TMH_ERROR_NOT_READY otherwise; more than the array holds is
 * TMH_ERROR_SCRATCH_LIMIT. Every call on a GPU shares its array and the
 * library's one stream: calls are queued in order, but work captured from
 * them into a graph and replayed later races with any other call of this
 * entry point that overlaps it on that GPU. */
int tmh_block_matmul_fixed(uint32_t kind, uint64_t w, uint64_t w_byte_offset, uint64_t x, uint32_t ldx, uint64_t dst,
                           uint64_t bias, uint32_t rows, uint32_t n, uint32_t k, uint32_t mode);

/* The product of tmh_block_matmul from activations already quantised by
 * tmh_quantize_rows_q8 (its four outputs), for callers that share one
 * quantisation between products. */
int tmh_block_matmul_quantised(uint32_t kind, uint64_t w, uint64_t w_byte_offset, uint64_t scales, uint64_t sums,
                               uint64_t totals, uint64_t qs, uint64_t dst, uint64_t bias, uint32_t rows, uint32_t n,
                               uint32_t k, uint32_t mode);

/* dst[count, width] = rows ids[0..count) of a block table of `table_rows`
 * rows of `width` values, dequantised: gather_blocks_f32
 * (cuda/kernels.cu:1172-1185) for Op::Gather on a block table. An id out of
 * range writes zeros and is reported at the next tmh_sync as
 * TMH_ERROR_EXECUTION (HostDevice#block_gather raises ExecutionError,
 * host.cr:648-658). */
int tmh_gather_blocks(uint32_t kind, uint64_t table, uint64_t table_byte_offset, int32_t table_rows, uint32_t width,
                      uint64_t ids, uint32_t count, uint64_t dst);

/* Quantises `count` host f32 values (a whole number of blocks of 32) into
 * host block bytes `out`: Quant.quantize (quant.cr:77-90, 497-535), the step
 * Tensor#quantize runs on the host for every device (tensor/quantised.cr:11-19).
 * Blocks are split over `threads` host threads (0: every core); the bytes do
 * not depend on the split. Needs no GPU. */
int tmh_quantize_weights(uint32_t kind, const float* values, uint64_t count, uint8_t* out, int32_t threads);

/* ------------------------------------------------------------ plans */

/* How a plan product's activation row arrives (tmh_product.x_mode). */
enum {
    TMH_X_F32 = 0,       /* x: f32 [k], quantised by the launch as tmh_block_matmul does */
    TMH_X_RMSNORM = 1,   /* x: f32 [k], taken through Op::RMSNorm (host.cr:374-386) with
                          * weights `norm` [k] and `eps` first: one launch for what
                          * tmh_rmsnorm then the product would do, with the same bits */
    TMH_X_QUANTISED = 2  /* x: int8 [k] values of tmh_quantize_rows_q8 (one row), with
                          * its scales, sums and totals: as tmh_block_matmul_quantised */
};

/* One product of a plan: Op::BlockMatMul with ONE activation row,
 * dst[n] = x[k] · w[n, k]ᵀ (+ bias[n]). */
typedef struct tmh_product {
    uint64_t w;             /* weight buffer */
    uint64_t w_byte_offset; /* byte offset of the first row (a row slice) */
    uint64_t x;             /* the activation row, as x_mode says */
    uint64_t dst;           /* f32 [n] */
    uint64_t bias;          /* f32 [n], or 0 */
    uint32_t n;
    uint32_t k;
    uint32_t x_mode;        /* TMH_X_F32 (0), TMH_X_RMSNORM or TMH_X_QUANTISED */
    float eps;              /* TMH_X_RMSNORM */
    uint64_t norm;          /* TMH_X_RMSNORM: f32 [k] */
    uint64_t scales, sums, totals; /* TMH_X_QUANTISED: f32 [k/32], f32 [k/32], i32 [k/32] */
} tmh_product;

/* Records `count` independent products of one block kind to run as ONE
 * kernel launch, each with the bits tmh_block_matmul gives it. The products
 * must not write what another reads. No counterpart in the reference, which
 * launches products one by one (cuda.cr:736-756): it is the batched launch
 * that small decode products need to stream weights at HBM speed rather
 * than at the launch rate. Rows must hold an even number of blocks and start
 * 4-byte aligned (TMH_ERROR_SHAPE otherwise). */
int tmh_plan_create(uint32_t kind, const tmh_product* products, uint32_t count, uint64_t* plan);
/* Products with x_mode other than TMH_X_F32 need the streamed kernel (rows of
 * at most 512 blocks and LDS for their staging); TMH_ERROR_SHAPE otherwise. */

/* Queues the plan's launch on the device's stream. */
int tmh_plan_run(uint64_t plan);

int tmh_plan_destroy(uint64_t plan);

/* Writes a one-line description of the plan's launch (kernel, grid, LDS)
 * into text (at most size bytes, NUL-terminated). No counterpart in the
 * reference: it names the kernel for profilers and benchmarks. */
int tmh_plan_describe(uint64_t plan, char* text, uint32_t size);

/* The plan's BlockMatMulMode (quant.cr:5-28): TMH_MODE_AUTO (the host's
 * block-order fold, the default) or TMH_MODE_UNORDERED (the same kernel and
 * loads, each row's contributions summed as four running sums: results may
 * differ in the last bits; a measurement mode, as block_matmul_unordered_f32
 * is for the reference's lanes products, cuda/kernels.cu:1334-1375). */
int tmh_plan_set_mode(uint64_t plan, uint32_t mode);

/* ------------------------------------------------- the rest of the decode graph
 *
 * The F32 ops a Llama decode step runs besides its products, each with the
 * bits of the reference's host kernel for the op (the ops the reference's GPU
 * devices leave to that host kernel, cuda.cr:395-415). All arrays are F32 in
 * device memory unless stated; rows are dense unless a leading dimension is
 * given. Kernel-detected index errors are reported at tmh_sync, as a gather's. */

/* Op::RMSNorm, host.cr:374-386: dst[r] = x[r] / sqrt(Σ_j x[r,j]² / n + eps) · weight,
 * the sum folded from 0 in index order. `weight` may be 0 (no weight). x rows
 * are `ldx` apart; dst must not overlap x. */
int tmh_rmsnorm(uint64_t x, uint32_t ldx, uint64_t weight, uint32_t rows, uint32_t n, float eps, uint64_t dst);

/* Op::Rope (host.cr:448-466) of the q and k heads and Op::WriteRows
 * (host.cr:586-597) of the rotated k and the v heads, for `tokens` rows of x
 * (`ldx` apart) each holding [heads q | kv_heads k | kv_heads v] heads of
 * `width` (a merged qkv product's output, modules.cr:484-493). Token t sits at
 * slots[t] (int32, device) = cache row · capacity + position; its rotation is
 * row `position` of the cos/sin tables ([table_rows, width], RotaryEmbedding,
 * modules.cr:344-351). Writes q_dst [tokens, heads, width] and the caches
 * keys/values [cache_rows, kv_heads, capacity, width]. A slot out of range is
 * an index error. */
int tmh_rope_write(uint64_t x, uint32_t ldx, uint32_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t width,
                   uint64_t cos, uint64_t sin, uint32_t table_rows, uint64_t slots, uint32_t cache_rows,
                   uint32_t capacity, uint64_t q_dst, uint64_t keys, uint64_t values);

/* Attention of `tokens` query rows against the caches, with the bits of
 * host.cr:408-440 (Op::Attention; the composite of composite.cr:190-199 and
 * Op::RaggedAttention have the same): per token and head, scores q·k_p in
 * column order, · scale, -inf past the token's last position, the first
 * highest, Maths.exp(x - top), their total in position order, then
 * Σ_p (e_p / total)·v_p in position order. Query head h reads kv head
 * h / (heads / kv_heads). `table` (int32, device) holds per token its cache
 * row, the last position it sees and the positions its row holds
 * (composite.cr:201-212). q rows are `ldq` apart ([heads, width] each), dst
 * rows `ld_dst` apart. width must be a multiple of 4, and the positions and
 * staged values must fit the kernel's 64 KB of LDS: (4·width + capacity +
 * 8192) floats (capacity up to 7,936 at width 64). */
int tmh_attention(uint64_t q, uint32_t ldq, uint32_t tokens, uint32_t heads, uint64_t keys, uint64_t values,
                  uint32_t cache_rows, uint32_t kv_heads, uint32_t capacity, uint32_t width, uint64_t table,
                  float scale, uint64_t dst, uint32_t ld_dst);

/* SwiGLU, kernels.cr:18: dst[r, j] = gate[r, j] / (Maths.exp(-gate[r, j]) + 1) · value[r, j];
 * gate and value rows `ld` apart (the two halves of a merged gate_up row,
 * modules.cr:515-522), dst dense [rows, n]. */
int tmh_swiglu(uint64_t gate, uint64_t value, uint32_t ld, uint32_t rows, uint32_t n, uint64_t dst);

/* Binary Add of two dense F32 arrays, host.cr:159-180: dst = a + b (dst may be a). */
int tmh_add(uint64_t a, uint64_t b, uint64_t dst, uint64_t count);

/* Sampler.greedy, sampler.cr:35-36: ids[r] (int32, device) = the first index
 * of the highest value of row r (rows `ldx` apart). */
int tmh_argmax(uint64_t x, uint32_t ldx, uint32_t rows, uint32_t n, uint64_t ids);

/* ------------------------------------------------------------ Llama decoding
 *
 * A Llama whose forward runs entirely on the device: Llama#forward /
 * #forward_last and Generative#generate with the greedy sampler
 * (llama.cr:256-303, generative.cr:155-190) over `rows` sequences, each with
 * a KV cache row of `capacity` positions. Every product and op is one of the
 * entry points above (tmh_block_matmul's kernels, tmh_gather_blocks,
 * tmh_rmsnorm, tmh_rope_write, tmh_attention, tmh_swiglu, tmh_add,
 * tmh_argmax), so the logits and tokens are the host's bits. A decode step
 * keeps its state (ids, slots, attention table) on the device, so steps can
 * be replayed from one captured HIP graph without host round trips. */

typedef struct tmh_llama_config {
    int32_t layers, width, heads, kv_heads, head_width, hidden, vocab, context;
    float eps;    /* RMSNorm epsilon */
    double theta; /* RoPE base */
    uint32_t kind; /* TMH_Q8_0 / TMH_Q4_0 / TMH_Q4_1: every matrix and the embedding table */
} tmh_llama_config;

/* Device addresses of the weights, which stay the caller's: the embedding
 * table [vocab, width] blocks; the head [vocab, width] blocks (0: tied to the
 * embedding); the final norm [width]; and per layer (arrays of `layers`
 * addresses) the norms [width], the merged qkv [(heads + 2·kv_heads)·head_width,
 * width] with q and k rows in Hugging Face order (llama.cr:226-235), o
 * [width, heads·head_width], the merged gate_up [2·hidden, width] and down
 * [width, hidden]. The norms must be 16-byte aligned. The arrays are read
 * during tmh_llama_create only. */
typedef struct tmh_llama_weights {
    uint64_t embed, head, norm;
    const uint64_t* attn_norm;
    const uint64_t* ffn_norm;
    const uint64_t* qkv;
    const uint64_t* o;
    const uint64_t* gate_up;
    const uint64_t* down;
} tmh_llama_weights;

/* Makes a decoder for `rows` sequences of at most `capacity` positions
 * (≤ context), its buffers sized for `max_tokens` tokens a forward (a longer
 * forward runs as forwards of `max_tokens` in turn, with the same bits). Allocates its
 * caches, activations and rotation tables (RotaryEmbedding's, in F32 by
 * powf/cosf/sinf). */
int tmh_llama_create(const tmh_llama_config* config, const tmh_llama_weights* weights, uint32_t rows,
                     uint32_t capacity, uint32_t max_tokens, uint64_t* model);

/* Runs `count` ids (host int32) of sequence `row` at the positions after its
 * cached ones and appends their keys and values (Generative#forward,
 * generative.cr:155-160); with `last_only`, only the last position's final
 * norm and head run (#forward_last, 162-172). Writes the logits, [count or 1,
 * vocab], to `logits` (host) unless it is null. Waits for the device. */
int tmh_llama_forward(uint64_t model, uint32_t row, const int32_t* ids, uint32_t count, uint32_t last_only,
                      float* logits);

/* Greedy generation for every row at once (Generative#generate with
 * Sampler.greedy, generative.cr:177-190): from each row's last forward's
 * logits, `steps` tokens per row, each chosen then run as the row's next
 * position (the last one chosen is not run). Writes tokens[row·steps + i]
 * (host). With `graph`, each decode step is one launch of a HIP graph
 * captured on first use. Every row must have run a forward first. */
int tmh_llama_generate(uint64_t model, uint32_t steps, int32_t* tokens, uint32_t graph);

/* Positions held by `row`'s cache; and emptying it (Cache#reset, modules.cr:157-161). */
int tmh_llama_length(uint64_t model, uint32_t row, int32_t* length);
int tmh_llama_reset(uint64_t model, uint32_t row);

/* Queues one decode step of every row with the device-held state, for timing
 * (the step tmh_llama_generate repeats); `graph` as there. Does not wait. */
int tmh_llama_step(uint64_t model, uint32_t graph);

/* The BlockMatMulMode of the decoder's products: TMH_MODE_AUTO (default:
 * the host's bits) or TMH_MODE_UNORDERED (each product folds in its own
 * order, as tmh_plan_set_mode; a measurement mode that prices the host's
 * order in a decode step, as the reference's CUDA device does with
 * block_mode = Unordered, cuda.cr:750-756). A captured step graph is
 * dropped when the mode changes. */
int tmh_llama_set_mode(uint64_t model, uint32_t mode);

int tmh_llama_destroy(uint64_t model);

/* ------------------------------------------------------------ GGUF files
 *
 * The reference's GGUF reader (gguf.cr) for this device: the file is mapped
 * once; a tensor's bytes reach the device through the pinned staging ring
 * (tmh_upload_async), optionally as a list of its rows in any order, so a row
 * reorder (Tensor#take_rows, tensor/quantised.cr:32-43, as Llama.unpermute
 * uses it) or a join of several tensors into one buffer (Linear.merge's
 * cat_rows, modules.cr:36-56) happens on the host before the upload, not as
 * a download and re-upload (quantised.cr:45-55). */

/* Maps and parses a GGUF file of version 2 or 3 (gguf.cr:289-329). Unknown
 * tensor kinds are TMH_ERROR_DTYPE; a damaged file TMH_ERROR_INVALID_VALUE. */
int tmh_gguf_open(const char* path, uint64_t* file);
int tmh_gguf_close(uint64_t file);

/* A tensor's kind (ggml numbering: F32 0, F16 1, Q4_0 2, Q4_1 3, Q8_0 8,
 * BF16 30), shape outermost first (up to 4 dimensions) and byte size: the
 * file's Entry (gguf.cr:85-98). Any output pointer may be null. */
int tmh_gguf_tensor(uint64_t file, const char* name, uint32_t* kind, int64_t* shape, uint32_t* dims,
                    uint64_t* bytes);

/* Queues the upload of tensor `name` to device address dst, as stored (rows
 * null) or as its rows rows[0..count) in that order (GGUF#[], gguf.cr:112-136,
 * then take_rows). Returns once the bytes are in the staging ring. */
int tmh_gguf_upload(uint64_t file, const char* name, const int32_t* rows, uint32_t count, uint64_t dst);

/* Llama.load of a GGUF file onto the device (llama.cr:184-235): the config
 * from its llama.* metadata (Llama.config, llama.cr:57-77), then every
 * weight uploaded once, the q and k rows put back in Hugging Face order
 * (Llama.unpermute) and the projections joined (qkv, gate_up) on the way;
 * a decoder as tmh_llama_create makes, owning the weights. Every matrix and
 * the embedding table must share one block kind (the file's token_embd);
 * norms may be F32, F16 or BF16 (widened, as GGUF#[] widens them). A file
 * with tensors the model lacks is refused, as the reference refuses it.
 * `capacity` 0 means the model's context. Writes the config it read. */
int tmh_llama_load_gguf(const char* path, uint32_t rows, uint32_t capacity, uint32_t max_tokens,
                        tmh_llama_config* config, uint64_t* model);

#ifdef __cplusplus
}
#endif

#endif /* TENSOMITE_HIP_H */
