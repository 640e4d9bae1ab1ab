// The C ABI of the decode-graph ops (tmh_rmsnorm ... tmh_argmax) and the
// device-resident Llama decoder (tmh_llama_*): Llama#forward,
// #forward_last and Generative#generate (src/tensomite/models/llama.cr:256-303,
// generative.cr:155-190) as a fixed sequence of this library's launches.
//
// The decoder keeps everything a step reads on the device -- the ids to run,
// each token's cache slot and attention entry -- and a step ends by choosing
// the next ids and moving those entries on, so consecutive steps need no host
// round trip and one captured HIP graph replays any number of them.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/tensomite_hip.h"
#include "tmh_internal.h"

namespace {

using tmh::DeviceContext;

int code(hipError_t e) { return e == hipErrorOutOfMemory ? TMH_ERROR_OUT_OF_MEMORY : (int)e; }



int check_rope(uint32_t heads, uint32_t kv_heads, uint32_t width, uint32_t table_rows, uint32_t capacity) {
    if (width == 0 || width % 2u != 0 || heads == 0 || kv_heads == 0 || capacity == 0) return TMH_ERROR_SHAPE;
    if (capacity > table_rows) return TMH_ERROR_SHAPE;
    return TMH_SUCCESS;
}

int check_attention(uint32_t heads, uint32_t kv_heads, uint32_t width, uint32_t capacity) {
    if (width == 0 || width % 4u != 0 || heads == 0 || kv_heads == 0 || heads % kv_heads != 0) return TMH_ERROR_SHAPE;
    // the attention kernels' dynamic LDS plus their own (256 bytes; decode:
    // 2 KB, also covering its last direct load) within a CU's 160 KB
    if (capacity == 0 || tmh::attention_lds(width, capacity) + 256u > 160u * 1024u ||
        tmh::attention_decode_lds(width, capacity) + 2048u > 160u * 1024u)
        return TMH_ERROR_SHAPE;
    return TMH_SUCCESS;
}

// ------------------------------------------------------------------ decoder

struct Llama {
    int device = 0;
    tmh_llama_config c{};
    uint32_t rows = 0, capacity = 0, max_tokens = 0;
    uint32_t qn = 0, kvn = 0, nqkv = 0;
    size_t row_bytes = 0;  // bytes of one weight row of `width` inputs

    // weights (the caller's)
    const uint8_t* embed = nullptr;
    const uint8_t* head = nullptr;
    const float* norm = nullptr;
    std::vector<const float*> attn_norm, ffn_norm;
    std::vector<const uint8_t*> qkv, o, gate_up, down;

    // device memory (one allocation), carved below
    uint8_t* memory = nullptr;
    float* x[2] = {nullptr, nullptr};  // the residual stream, ping-ponged by one-row residual products
    float *h = nullptr, *qkv_out = nullptr, *q = nullptr, *att = nullptr, *o_out = nullptr;
    float *gu = nullptr, *act = nullptr, *logits = nullptr;
    float *cos = nullptr, *sin = nullptr;
    float *keys = nullptr, *values = nullptr;  // [layers][rows][kv_heads][capacity][head_width]
    int32_t *ids = nullptr, *slots = nullptr, *table = nullptr, *steps = nullptr, *log = nullptr;
    float* best_values = nullptr;  // the split argmax's chunks
    int32_t* best_index = nullptr;
    uint8_t* scratch[2] = {nullptr, nullptr};  // quantised activations: a product's input, and the next one's
    size_t layer_cache = 0;  // floats of one layer's keys

    std::vector<int32_t> length;   // positions held, per row
    std::vector<char> has_logits;  // whether row r's logits row holds its last forward's
    bool generating = false;       // the device state continues a generation

    hipGraphExec_t graph = nullptr;
    // The step graph is captured on this stream of the model's own, so that
    // no other call (another thread's product on the device's stream) can
    // enqueue into the capture; the graph then runs on the device's stream.
    hipStream_t capture = nullptr;
    void* owned = nullptr;  // weights this decoder loaded itself (tmh_llama_load_gguf)
    uint32_t mode = TMH_MODE_AUTO;  // the products' BlockMatMulMode: AUTO, or UNORDERED (tmh_llama_set_mode)
};

// Rows a forward takes through the products whose workgroups stage their
// weight tile into LDS and run the norm and quantiser in their prologue
// (one row: k_matvec_one; 2 to 8: k_matvec_nb), five launches a layer.
constexpr uint32_t FEW_ROWS = 8;

// How a forward of 2 to FEW_ROWS rows takes RMSNorm: in a launch of its own
// (k_rmsnorm_quantise_wave) before the products, which then take the
// quantised rows -- the default: every workgroup of a fused product would
// normalise and quantise every row again, VALU work that outweighs the
// launch at 8 rows -- or in each product's prologue (TMH_FEW_ROWS_NORM=fused,
// for comparisons).
bool few_rows_norm_fused() {
    static const bool fused = [] {
        const char* env = getenv("TMH_FEW_ROWS_NORM");
        return env && strcmp(env, "fused") == 0;
    }();
    return fused;
}

// dst[rows, n] = act · wᵀ (+ bias) over quantised activations.
hipError_t product(const Llama& m, const DeviceContext& ctx, const uint8_t* w, tmh::Activations act, uint32_t rows,
                   uint32_t n, uint32_t k, float* dst, const float* bias) {
    return tmh::launch_block_matmul(m.c.kind, TMH_MODE_AUTO, w, act, dst, bias, rows, n, k, ctx.compute_units,
                                    ctx.stream);
}

// dst[rows, n] = act · wᵀ with no bias: up to FEW_ROWS rows the product
// with weights in LDS, else (or where its shape does not fit) product().
hipError_t few_product(const Llama& m, const DeviceContext& ctx, const uint8_t* w, tmh::Activations act, uint32_t rows,
                       uint32_t n, uint32_t k, float* dst) {
    hipError_t e = rows <= FEW_ROWS ? tmh::launch_rows_product(m.c.kind, tmh::NB_QUANT, w, nullptr, 0, nullptr, 0.0f,
                                                               act, dst, nullptr, 0, rows, n, k, ctx.compute_units,
                                                               ctx.stream)
                                    : hipErrorInvalidValue;
    return e == hipErrorInvalidValue ? product(m, ctx, w, act, rows, n, k, dst, nullptr) : e;
}

// Quantises rows of f32 activations into act.
hipError_t quantise(const DeviceContext& ctx, const float* x, uint32_t rows, uint32_t k, tmh::Activations act) {
    return tmh::launch_quantize(x, k, rows, k, (float*)act.scales, (float*)act.sums, (int32_t*)act.totals,
                                (int8_t*)act.qs, ctx.stream);
}

// RMSNorm of x's rows, quantised into act: one launch where the row fits.
hipError_t norm_quantise(const Llama& m, const DeviceContext& ctx, const float* x, const float* w, uint32_t rows,
                         tmh::Activations act) {
    const uint32_t W = (uint32_t)m.c.width;
    if (tmh::rmsnorm_quantise_fits(W)) return tmh::launch_rmsnorm_quantise(x, W, w, rows, W, m.c.eps, act, ctx.stream);
    hipError_t e = tmh::launch_rmsnorm(x, W, w, rows, W, m.c.eps, m.h, W, ctx.stream);
    return e == hipSuccess ? quantise(ctx, m.h, rows, W, act) : e;
}

// The residual update x += act · wᵀ, as the host's `x + product` (one
// rounding per element either way round): for fewer rows than the matrix
// cores take, the product (weights in LDS up to FEW_ROWS rows, else the
// lanes or few-rows kernel) adds each row's x as its bias and writes the
// other residual buffer; else one row is a product with x as bias, and more
// rows a product and an add.
hipError_t residual(const Llama& m, const DeviceContext& ctx, const uint8_t* w, tmh::Activations act, uint32_t rows,
                    uint32_t k, int& cur) {
    const uint32_t W = (uint32_t)m.c.width;
    if (rows <= FEW_ROWS) {
        // up to 8 rows: the weights of each workgroup's tile staged into LDS at once
        hipError_t r = rows == 1 ? tmh::launch_product_one(m.c.kind, w, act, m.x[cur ^ 1], m.x[cur], W, k,
                                                           ctx.compute_units, ctx.stream)
                                 : tmh::launch_rows_product(m.c.kind, tmh::NB_QUANT, w, nullptr, 0, nullptr, 0.0f, act,
                                                            m.x[cur ^ 1], m.x[cur], W, rows, W, k, ctx.compute_units,
                                                            ctx.stream);
        if (r != hipErrorInvalidValue) {
            cur ^= 1;
            return r;
        }
    }
    hipError_t r = tmh::launch_product_residual(m.c.kind, w, act, m.x[cur ^ 1], m.x[cur], rows, W, k,
                                                ctx.compute_units, ctx.stream);
    if (r != hipErrorInvalidValue) {
        cur ^= 1;
        return r;
    }
    if (rows == 1) {
        hipError_t e = product(m, ctx, w, act, 1, W, k, m.x[cur ^ 1], m.x[cur]);
        cur ^= 1;
        return e;
    }
    hipError_t e = product(m, ctx, w, act, rows, W, k, m.o_out, nullptr);
    return e == hipSuccess ? tmh::launch_add(m.x[cur], m.o_out, m.x[cur], rows * W, ctx.stream) : e;
}

// The forward of `tokens` ids already on the device (m.ids), whose slots
// and attention entries are on the device too; then the final norm and the
// head over `final_rows` rows from row `final_from`, into logits rows from
// `logits_row`. With `decode`, token t is cache row t's one new position, and
// its RoPE and cache write run inside the attention launch.
hipError_t forward_tokens(const Llama& m, const DeviceContext& ctx, uint32_t tokens, uint32_t final_from,
                          uint32_t final_rows, uint32_t logits_row, bool decode) {
    const tmh::TreeFold order(m.mode == TMH_MODE_UNORDERED);
    const tmh_llama_config& c = m.c;
    const uint32_t W = (uint32_t)c.width, H = (uint32_t)c.hidden, hw = (uint32_t)c.head_width;
    const float scale = (float)(1.0 / std::sqrt((double)hw));
    const bool quant_att = hw % 32u == 0;
    const bool rows_fused = tokens <= FEW_ROWS;
    int cur = 0;
    hipError_t e = tmh::launch_gather(c.kind, m.embed, c.vocab, W, m.ids, tokens, m.x[cur], ctx.errors, ctx.stream);
    const tmh::Activations a_in = tmh::carve_scratch(m.scratch[0], tokens, W);
    for (int32_t l = 0; l < c.layers && e == hipSuccess; ++l) {
        float* keys = m.keys + (size_t)l * m.layer_cache;
        float* values = m.values + (size_t)l * m.layer_cache;
        // one row (or up to FEW_ROWS with the fused norm): the norm and
        // quantiser in the product's prologue (one launch); else
        // RMSNorm+quantise, then the product
        hipError_t f = !rows_fused ? hipErrorInvalidValue
                       : tokens == 1
                           ? tmh::launch_product_rms(c.kind, m.qkv[l], m.x[cur], W, m.attn_norm[l], c.eps, m.qkv_out,
                                                     tokens, m.nqkv, W, ctx.compute_units, ctx.stream)
                       : few_rows_norm_fused()
                           ? tmh::launch_rows_product(c.kind, tmh::NB_NORM, m.qkv[l], m.x[cur], W, m.attn_norm[l],
                                                      c.eps, tmh::Activations{}, m.qkv_out, nullptr, 0, tokens,
                                                      m.nqkv, W, ctx.compute_units, ctx.stream)
                           : hipErrorInvalidValue;
        if (f == hipErrorInvalidValue) {
            e = norm_quantise(m, ctx, m.x[cur], m.attn_norm[l], tokens, a_in);
            if (e == hipSuccess) e = few_product(m, ctx, m.qkv[l], a_in, tokens, m.nqkv, W, m.qkv_out);
        } else {
            e = f;
        }
        const tmh::Activations a_att = tmh::carve_scratch(m.scratch[1], tokens, m.qn);
        tmh::RopeWrite r{m.qkv_out, m.nqkv, (uint32_t)c.heads, (uint32_t)c.kv_heads, hw, m.cos, m.sin,
                         m.slots, m.rows, m.capacity, m.q, keys, values, ctx.errors};
        tmh::Attention a{m.q, m.qn, keys, values, m.rows, (uint32_t)c.kv_heads, m.capacity, hw,
                         (uint32_t)c.heads, m.table, scale, m.att, m.qn, ctx.errors,
                         quant_att ? a_att : tmh::Activations{}};
        if (e == hipSuccess) {
            if (decode) {
                e = tmh::launch_attention_decode(a, r, tokens, ctx.stream);
            } else {
                e = tmh::launch_rope_write(r, tokens, ctx.stream);
                if (e == hipSuccess) e = tmh::launch_attention(a, tokens, ctx.stream);
            }
        }
        if (e == hipSuccess && !quant_att) e = quantise(ctx, m.att, tokens, m.qn, a_att);
        if (e == hipSuccess) e = residual(m, ctx, m.o[l], a_att, tokens, m.qn, cur);
        const tmh::Activations a_hid = tmh::carve_scratch(m.scratch[1], tokens, H);
        // up to FEW_ROWS rows: RMSNorm in gate_up's prologue, SwiGLU and the
        // quantiser in its epilogue (one launch)
        hipError_t fg = !(e == hipSuccess && rows_fused) ? hipErrorInvalidValue
                        : tokens == 1 ? tmh::launch_gate_up_swiglu_rms(c.kind, m.gate_up[l], m.x[cur], W, m.ffn_norm[l],
                                                                       c.eps, tokens, H, W, a_hid, ctx.stream)
                        : few_rows_norm_fused()
                            ? tmh::launch_rows_gate_up(c.kind, tmh::NB_NORM, m.gate_up[l], m.x[cur], W, m.ffn_norm[l],
                                                       c.eps, tmh::Activations{}, tokens, H, W, a_hid, ctx.stream)
                            : hipErrorInvalidValue;
        if (fg != hipErrorInvalidValue) {
            e = fg;
        } else if (e == hipSuccess) {
            e = norm_quantise(m, ctx, m.x[cur], m.ffn_norm[l], tokens, a_in);
        }
        if (e == hipSuccess && fg == hipErrorInvalidValue) {
            // gate_up with SwiGLU and the quantiser in its epilogue where the
            // shape allows (weights in LDS up to FEW_ROWS rows, else the
            // lanes kernel), else the product then SwiGLU+quantise
            hipError_t g = tokens <= FEW_ROWS
                               ? tmh::launch_rows_gate_up(c.kind, tmh::NB_QUANT, m.gate_up[l], nullptr, 0, nullptr,
                                                          0.0f, a_in, tokens, H, W, a_hid, ctx.stream)
                               : hipErrorInvalidValue;
            if (g == hipErrorInvalidValue)
                g = tmh::launch_gate_up_swiglu(c.kind, m.gate_up[l], a_in, tokens, H, W, a_hid, ctx.stream);
            if (g == hipErrorInvalidValue) {
                e = product(m, ctx, m.gate_up[l], a_in, tokens, 2u * H, W, m.gu, nullptr);
                if (e == hipSuccess)
                    e = tmh::launch_swiglu_quantise(m.gu, m.gu + H, 2u * H, tokens, H, a_hid, ctx.stream);
            } else {
                e = g;
            }
        }
        if (e == hipSuccess) e = residual(m, ctx, m.down[l], a_hid, tokens, H, cur);
    }
    const tmh::Activations a_fin = tmh::carve_scratch(m.scratch[0], final_rows, W);
    float* logits = m.logits + (size_t)logits_row * c.vocab;
    const float* x_fin = m.x[cur] + (size_t)final_from * W;
    hipError_t fh = !(e == hipSuccess && final_rows <= FEW_ROWS) ? hipErrorInvalidValue
                    : final_rows == 1
                        ? tmh::launch_product_rms(c.kind, m.head, x_fin, W, m.norm, c.eps, logits, final_rows,
                                                  (uint32_t)c.vocab, W, ctx.compute_units, ctx.stream)
                    : few_rows_norm_fused()
                        ? tmh::launch_rows_product(c.kind, tmh::NB_NORM, m.head, x_fin, W, m.norm, c.eps,
                                                   tmh::Activations{}, logits, nullptr, 0, final_rows,
                                                   (uint32_t)c.vocab, W, ctx.compute_units, ctx.stream)
                        : hipErrorInvalidValue;
    if (fh != hipErrorInvalidValue) return fh;
    if (e == hipSuccess) e = norm_quantise(m, ctx, x_fin, m.norm, final_rows, a_fin);
    if (e == hipSuccess) e = few_product(m, ctx, m.head, a_fin, final_rows, (uint32_t)c.vocab, W, logits);
    return e;
}

// Chooses each row's next token from logits rows 0..rows-1, logs it and
// moves the row on.
hipError_t choose(const Llama& m, const DeviceContext& ctx) {
    return tmh::launch_choose_advance(m.logits, m.rows, (uint32_t)m.c.vocab, m.best_values, m.best_index, m.ids, m.log,
                                      m.capacity, m.steps, m.slots, m.table, m.capacity, ctx.stream);
}

// One decode step of every row from the device-held state: run each row's
// chosen id, choose the next, log it and move the row on.
hipError_t decode_step(const Llama& m, const DeviceContext& ctx) {
    hipError_t e = forward_tokens(m, ctx, m.rows, 0, m.rows, 0, true);
    return e == hipSuccess ? choose(m, ctx) : e;
}

int run_step(Llama& m, const DeviceContext& ctx, bool graph) {
    if (!graph) return code(decode_step(m, ctx));
    if (!m.graph) {
        if (!m.capture) {
            hipError_t e = hipStreamCreateWithFlags(&m.capture, hipStreamNonBlocking);
            if (e != hipSuccess) {
                m.capture = nullptr;
                return code(e);
            }
        }
        DeviceContext cap = ctx;
        cap.stream = m.capture;
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamBeginCapture(cap.stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return code(e);
        hipError_t step = decode_step(m, cap);
        e = hipStreamEndCapture(cap.stream, &g);
        if (step != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return code(step);
        }
        if (e != hipSuccess) return code(e);
        e = hipGraphInstantiate(&m.graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            m.graph = nullptr;
            return code(e);
        }
    }
    return code(hipGraphLaunch(m.graph, ctx.stream));
}

Llama* model_of(uint64_t handle, const DeviceContext& ctx, int* err) {
    Llama* m = (Llama*)handle;
    if (!m) {
        *err = TMH_ERROR_INVALID_VALUE;
        return nullptr;
    }
    if (m->device != ctx.index) {
        *err = TMH_ERROR_INVALID_VALUE;
        return nullptr;
    }
    *err = TMH_SUCCESS;
    return m;
}

size_t align256(size_t v) { return (v + 255u) & ~(size_t)255u; }

}  // namespace

extern "C" {

// ----------------------------------------------------------------- the ops

int tmh_rmsnorm(uint64_t x, uint32_t ldx, uint64_t weight, uint32_t rows, uint32_t n, float eps, uint64_t dst) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    if (n == 0 || ldx < n) return TMH_ERROR_SHAPE;
    if (rows == 0) return TMH_SUCCESS;
    if (!x || !dst) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)rows * ldx > 0x7fffffffull) return TMH_ERROR_SHAPE;
    hipError_t e = tmh::launch_rmsnorm((const float*)x, ldx, (const float*)weight, rows, n, eps, (float*)dst, n,
                                       ctx.stream);
    if (e == hipSuccess) tmh::note_launch(ctx.index, 1, false);
    return code(e);
}

int tmh_rope_write(uint64_t x, uint32_t ldx, uint32_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t width,
                   uint64_t cos, uint64_t sin, uint32_t table_rows, uint64_t slots, uint32_t cache_rows,
                   uint32_t capacity, uint64_t q_dst, uint64_t keys, uint64_t values) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    if ((err = check_rope(heads, kv_heads, width, table_rows, capacity)) != TMH_SUCCESS) return err;
    if (ldx < (heads + 2u * kv_heads) * width || cache_rows == 0) return TMH_ERROR_SHAPE;
    if (tokens == 0) return TMH_SUCCESS;
    if (!x || !cos || !sin || !slots || !q_dst || !keys || !values) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)tokens * (heads + 2u * kv_heads) * width > 0x7fffffffull ||
        (uint64_t)cache_rows * capacity > 0x7fffffffull)
        return TMH_ERROR_SHAPE;
    tmh::RopeWrite a{(const float*)x, ldx, heads, kv_heads, width, (const float*)cos, (const float*)sin,
                     (const int32_t*)slots, cache_rows, capacity, (float*)q_dst, (float*)keys, (float*)values,
                     ctx.errors};
    hipError_t e = tmh::launch_rope_write(a, tokens, ctx.stream);
    if (e == hipSuccess) tmh::note_launch(ctx.index, 1, true);
    return code(e);
}

int tmh_attention(uint64_t q, uint32_t ldq, uint32_t tokens, uint32_t heads, uint64_t keys, uint64_t values,
                  uint32_t cache_rows, uint32_t kv_heads, uint32_t capacity, uint32_t width, uint64_t table,
                  float scale, uint64_t dst, uint32_t ld_dst) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    if ((err = check_attention(heads, kv_heads, width, capacity)) != TMH_SUCCESS) return err;
    if (ldq < heads * width || ld_dst < heads * width || cache_rows == 0) return TMH_ERROR_SHAPE;
    if (tokens == 0) return TMH_SUCCESS;
    if (!q || !keys || !values || !table || !dst) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)tokens * heads > 0x7fffffffull) return TMH_ERROR_SHAPE;
    tmh::Attention a{(const float*)q, ldq, (const float*)keys, (const float*)values, cache_rows, kv_heads, capacity,
                     width, heads, (const int32_t*)table, scale, (float*)dst, ld_dst, ctx.errors};
    hipError_t e = tmh::launch_attention(a, tokens, ctx.stream);
    if (e == hipSuccess) tmh::note_launch(ctx.index, 1, true);
    return code(e);
}

int tmh_swiglu(uint64_t gate, uint64_t value, uint32_t ld, uint32_t rows, uint32_t n, uint64_t dst) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    if (ld < n) return TMH_ERROR_SHAPE;
    if (rows == 0 || n == 0) return TMH_SUCCESS;
    if (!gate || !value || !dst) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)rows * ld > 0x7fffffffull) return TMH_ERROR_SHAPE;
    hipError_t e = tmh::launch_swiglu((const float*)gate, (const float*)value, ld, rows, n, (float*)dst, ctx.stream);
    if (e == hipSuccess) tmh::note_launch(ctx.index, 1, false);
    return code(e);
}

int tmh_add(uint64_t a, uint64_t b, uint64_t dst, uint64_t count) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    if (count == 0) return TMH_SUCCESS;
    if (!a || !b || !dst) return TMH_ERROR_INVALID_VALUE;
    if (count > 0x7fffffffull) return TMH_ERROR_SHAPE;
    hipError_t e = tmh::launch_add((const float*)a, (const float*)b, (float*)dst, (uint32_t)count, ctx.stream);
    if (e == hipSuccess) tmh::note_launch(ctx.index, 1, false);
    return code(e);
}

int tmh_argmax(uint64_t x, uint32_t ldx, uint32_t rows, uint32_t n, uint64_t ids) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    if (n == 0 || ldx < n) return TMH_ERROR_SHAPE;
    if (rows == 0) return TMH_SUCCESS;
    if (!x || !ids) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)rows * ldx > 0x7fffffffull) return TMH_ERROR_SHAPE;
    hipError_t e = tmh::launch_argmax((const float*)x, ldx, rows, n, (int32_t*)ids, ctx.stream);
    if (e == hipSuccess) tmh::note_launch(ctx.index, 1, false);
    return code(e);
}

// ------------------------------------------------------------- the decoder

int tmh_llama_create(const tmh_llama_config* config, const tmh_llama_weights* weights, uint32_t rows,
                     uint32_t capacity, uint32_t max_tokens, uint64_t* model) {
    if (!config || !weights || !model) return TMH_ERROR_INVALID_VALUE;
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    const tmh_llama_config& c = *config;
    if (c.kind > 2u) return TMH_ERROR_DTYPE;
    if (c.layers <= 0 || c.width <= 0 || c.width % 32 != 0 || c.hidden <= 0 || c.hidden % 32 != 0 || c.heads <= 0 ||
        c.kv_heads <= 0 || c.heads % c.kv_heads != 0 || c.head_width <= 0 || c.vocab <= 0 || c.context <= 0)
        return TMH_ERROR_SHAPE;
    if ((c.heads * c.head_width) % 32 != 0) return TMH_ERROR_SHAPE;
    if (rows == 0 || max_tokens == 0 || capacity == 0 || capacity > (uint32_t)c.context) return TMH_ERROR_SHAPE;
    if ((err = check_rope(c.heads, c.kv_heads, c.head_width, capacity, capacity)) != TMH_SUCCESS) return err;
    if ((err = check_attention(c.heads, c.kv_heads, c.head_width, capacity)) != TMH_SUCCESS) return err;
    if (!weights->embed || !weights->norm || !weights->attn_norm || !weights->ffn_norm || !weights->qkv ||
        !weights->o || !weights->gate_up || !weights->down || weights->norm % 16u != 0)
        return TMH_ERROR_INVALID_VALUE;

    Llama* m = new Llama();
    m->device = ctx.index;
    m->c = c;
    m->rows = rows;
    m->capacity = capacity;
    m->max_tokens = max_tokens;
    m->qn = (uint32_t)(c.heads * c.head_width);
    m->kvn = (uint32_t)(c.kv_heads * c.head_width);
    m->nqkv = m->qn + 2u * m->kvn;
    m->row_bytes = (size_t)c.width / 32u * tmh::block_bytes(c.kind);
    m->embed = (const uint8_t*)weights->embed;
    m->head = (const uint8_t*)(weights->head ? weights->head : weights->embed);
    m->norm = (const float*)weights->norm;
    for (int32_t l = 0; l < c.layers; ++l) {
        if (!weights->attn_norm[l] || !weights->ffn_norm[l] || !weights->qkv[l] || !weights->o[l] ||
            !weights->gate_up[l] || !weights->down[l] || weights->attn_norm[l] % 16u != 0 ||
            weights->ffn_norm[l] % 16u != 0) {
            delete m;
            return TMH_ERROR_INVALID_VALUE;
        }
        m->attn_norm.push_back((const float*)weights->attn_norm[l]);
        m->ffn_norm.push_back((const float*)weights->ffn_norm[l]);
        m->qkv.push_back((const uint8_t*)weights->qkv[l]);
        m->o.push_back((const uint8_t*)weights->o[l]);
        m->gate_up.push_back((const uint8_t*)weights->gate_up[l]);
        m->down.push_back((const uint8_t*)weights->down[l]);
    }
    m->length.assign(rows, 0);
    m->has_logits.assign(rows, 0);

    // One allocation, carved 256-byte aligned.
    const size_t R = std::max(rows, max_tokens);
    const size_t W = (size_t)c.width, H = (size_t)c.hidden, hw = (size_t)c.head_width;
    m->layer_cache = (size_t)rows * c.kv_heads * capacity * hw;
    const uint32_t widest = (uint32_t)std::max<size_t>({W, H, (size_t)m->qn});
    struct Part {
        void** at;
        size_t bytes;
    } parts[] = {
        {(void**)&m->x[0], R * W * 4},
        {(void**)&m->x[1], R * W * 4},
        {(void**)&m->h, R * W * 4},
        {(void**)&m->qkv_out, R * m->nqkv * 4},
        {(void**)&m->q, R * m->qn * 4},
        {(void**)&m->att, R * m->qn * 4},
        {(void**)&m->o_out, R * W * 4},
        {(void**)&m->gu, R * 2 * H * 4},
        {(void**)&m->act, R * H * 4},
        {(void**)&m->logits, R * (size_t)c.vocab * 4},
        {(void**)&m->cos, (size_t)capacity * hw * 4},
        {(void**)&m->sin, (size_t)capacity * hw * 4},
        {(void**)&m->ids, R * 4},
        {(void**)&m->slots, R * 4},
        {(void**)&m->table, R * 3 * 4},
        {(void**)&m->steps, (size_t)rows * 4},
        {(void**)&m->log, (size_t)rows * capacity * 4},
        {(void**)&m->scratch[0], tmh::scratch_need((uint32_t)R, widest)},
        {(void**)&m->scratch[1], tmh::scratch_need((uint32_t)R, widest)},
        {(void**)&m->best_values, R * tmh::argmax_chunks((uint32_t)c.vocab) * 4},
        {(void**)&m->best_index, R * tmh::argmax_chunks((uint32_t)c.vocab) * 4},
        {(void**)&m->keys, m->layer_cache * c.layers * 4},
        {(void**)&m->values, m->layer_cache * c.layers * 4},
    };
    size_t total = 0;
    for (const Part& p : parts) total += align256(p.bytes);
    void* mem = nullptr;
    hipError_t e = tmh::device_malloc(&mem, total);
    if (e != hipSuccess) {
        delete m;
        return code(e);
    }
    m->memory = (uint8_t*)mem;
    size_t at = 0;
    for (const Part& p : parts) {
        *p.at = m->memory + at;
        at += align256(p.bytes);
    }

    // RotaryEmbedding's tables (modules.cr:344-351), in F32 as there:
    // frequency i = 1 / θ^(2i/width) by powf, then cosf/sinf of p·frequency.
    const uint32_t half = (uint32_t)hw / 2u;
    std::vector<float> freq(half), cs((size_t)capacity * hw), sn((size_t)capacity * hw);
    const float theta = (float)c.theta;
    for (uint32_t i = 0; i < half; ++i) freq[i] = 1.0f / powf(theta, (float)(2u * i) / (float)hw);
    for (uint32_t p = 0; p < capacity; ++p)
        for (uint32_t i = 0; i < hw; ++i) {
            const float angle = (float)p * freq[i % half];
            cs[(size_t)p * hw + i] = cosf(angle);
            sn[(size_t)p * hw + i] = sinf(angle);
        }
    e = hipMemcpyAsync(m->cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, ctx.stream);
    if (e == hipSuccess) e = hipMemcpyAsync(m->sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, ctx.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx.stream);
    if (e != hipSuccess) {
        (void)hipFree(m->memory);
        delete m;
        return code(e);
    }
    *model = (uint64_t)m;
    return TMH_SUCCESS;
}

int tmh_llama_forward(uint64_t model, uint32_t row, const int32_t* ids, uint32_t count, uint32_t last_only,
                      float* logits) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    Llama* m = model_of(model, ctx, &err);
    if (!m) return err;
    if (row >= m->rows || !ids) return TMH_ERROR_INVALID_VALUE;
    if (count == 0) return TMH_ERROR_SHAPE;
    const int32_t past = m->length[row];
    if ((uint64_t)past + count > m->capacity) return TMH_ERROR_SHAPE;
    for (uint32_t i = 0; i < count; ++i)
        if (ids[i] < 0 || ids[i] >= m->c.vocab) return TMH_ERROR_INVALID_VALUE;
    if (count > m->max_tokens) {
        // More ids than one forward's buffers hold: forwards of max_tokens
        // ids in turn, each after the positions the ones before it cached.
        // Every position reads the cache by position, so its bits are those
        // of one forward over all the ids (as prefill equals one-by-one
        // decode); the logits of each part land at its offset, or with
        // last_only only the last id's.
        const size_t vocab = (size_t)m->c.vocab;
        for (uint32_t off = 0; off < count; off += m->max_tokens) {
            const uint32_t part = std::min(m->max_tokens, count - off);
            const bool last = off + part == count;
            float* out = !logits ? nullptr : last_only ? (last ? logits : nullptr) : logits + (size_t)off * vocab;
            if ((err = tmh_llama_forward(model, row, ids + off, part, last_only, out)) != TMH_SUCCESS) return err;
        }
        return TMH_SUCCESS;
    }
    // ids, slots, then the attention table, in one upload
    std::vector<int32_t> host((size_t)count * 5);
    for (uint32_t i = 0; i < count; ++i) {
        host[i] = ids[i];
        host[count + i] = (int32_t)(row * m->capacity) + past + (int32_t)i;
        host[2 * count + 3 * i] = (int32_t)row;
        host[2 * count + 3 * i + 1] = past + (int32_t)i;
        host[2 * count + 3 * i + 2] = past + (int32_t)count;
    }
    m->generating = false;
    hipError_t e = hipMemcpyAsync(m->ids, host.data(), (size_t)count * 4, hipMemcpyHostToDevice, ctx.stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->slots, host.data() + count, (size_t)count * 4, hipMemcpyHostToDevice, ctx.stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->table, host.data() + 2 * count, (size_t)count * 12, hipMemcpyHostToDevice, ctx.stream);
    const uint32_t final_rows = last_only ? 1u : count;
    // A last-only forward leaves its logits in the row's logits row, where
    // generation starts from.
    const uint32_t logits_row = last_only ? row : 0u;
    if (e == hipSuccess)
        e = forward_tokens(*m, ctx, count, last_only ? count - 1u : 0u, final_rows, logits_row, false);
    if (e != hipSuccess) return code(e);
    tmh::note_launch(ctx.index, 0, true);
    m->length[row] = past + (int32_t)count;
    const size_t vocab = (size_t)m->c.vocab;
    if (logits) {
        e = hipMemcpyAsync(logits, m->logits + (size_t)logits_row * vocab, (size_t)final_rows * vocab * 4,
                           hipMemcpyDeviceToHost, ctx.stream);
        if (e != hipSuccess) return code(e);
    }
    if (!last_only) {
        // The logits filled rows 0..count-1, over other rows' last logits;
        // the last one moves to the row's own logits row.
        for (uint32_t r = 0; r < std::min(count, m->rows); ++r) m->has_logits[r] = 0;
        if (count - 1u != row) {
            e = hipMemcpyAsync(m->logits + (size_t)row * vocab, m->logits + (size_t)(count - 1u) * vocab, vocab * 4,
                               hipMemcpyDeviceToDevice, ctx.stream);
            if (e != hipSuccess) return code(e);
        }
    }
    m->has_logits[row] = 1;
    return tmh_sync();
}

int tmh_llama_generate(uint64_t model, uint32_t steps, int32_t* tokens, uint32_t graph) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    Llama* m = model_of(model, ctx, &err);
    if (!m) return err;
    if (steps == 0) return TMH_SUCCESS;
    if (!tokens) return TMH_ERROR_INVALID_VALUE;
    for (uint32_t r = 0; r < m->rows; ++r) {
        if (!m->has_logits[r]) return TMH_ERROR_INVALID_VALUE;
        if ((uint64_t)m->length[r] + steps - 1u > m->capacity) return TMH_ERROR_SHAPE;
    }
    if (steps > m->capacity) return TMH_ERROR_SHAPE;
    // Each row as if its last forward's token had just been run: the step's
    // advance then points it at its next position.
    std::vector<int32_t> host((size_t)m->rows * 5);
    for (uint32_t r = 0; r < m->rows; ++r) {
        const int32_t len = m->length[r];
        host[r] = (int32_t)(r * m->capacity) + len - 1;
        host[m->rows + 3 * r] = (int32_t)r;
        host[m->rows + 3 * r + 1] = len - 1;
        host[m->rows + 3 * r + 2] = len;
        host[4 * m->rows + r] = 0;
    }
    hipError_t e = hipMemcpyAsync(m->slots, host.data(), (size_t)m->rows * 4, hipMemcpyHostToDevice, ctx.stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->table, host.data() + m->rows, (size_t)m->rows * 12, hipMemcpyHostToDevice, ctx.stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->steps, host.data() + 4 * m->rows, (size_t)m->rows * 4, hipMemcpyHostToDevice, ctx.stream);
    // the first token of each row from its last forward's logits
    if (e == hipSuccess) e = choose(*m, ctx);
    if (e != hipSuccess) return code(e);
    tmh::note_launch(ctx.index, 0, true);
    for (uint32_t i = 1; i < steps; ++i) {
        if ((err = run_step(*m, ctx, graph != 0)) != TMH_SUCCESS) return err;
        for (uint32_t r = 0; r < m->rows; ++r) m->length[r] += 1;
    }
    std::fill(m->has_logits.begin(), m->has_logits.end(), 1);
    m->generating = true;
    std::vector<int32_t> log((size_t)m->rows * m->capacity);
    e = hipMemcpyAsync(log.data(), m->log, log.size() * 4, hipMemcpyDeviceToHost, ctx.stream);
    if (e != hipSuccess) return code(e);
    if ((err = tmh_sync()) != TMH_SUCCESS) return err;
    for (uint32_t r = 0; r < m->rows; ++r)
        std::memcpy(tokens + (size_t)r * steps, log.data() + (size_t)r * m->capacity, (size_t)steps * 4);
    return TMH_SUCCESS;
}

int tmh_llama_step(uint64_t model, uint32_t graph) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    Llama* m = model_of(model, ctx, &err);
    if (!m) return err;
    if (!m->generating) return TMH_ERROR_INVALID_VALUE;
    for (uint32_t r = 0; r < m->rows; ++r)
        if ((uint64_t)m->length[r] + 1u > m->capacity) return TMH_ERROR_SHAPE;
    if ((err = run_step(*m, ctx, graph != 0)) != TMH_SUCCESS) return err;
    for (uint32_t r = 0; r < m->rows; ++r) m->length[r] += 1;
    tmh::note_launch(ctx.index, 0, true);
    return TMH_SUCCESS;
}

int tmh_llama_length(uint64_t model, uint32_t row, int32_t* length) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, false);
    if (err) return err;
    Llama* m = model_of(model, ctx, &err);
    if (!m) return err;
    if (row >= m->rows || !length) return TMH_ERROR_INVALID_VALUE;
    *length = m->length[row];
    return TMH_SUCCESS;
}

int tmh_llama_reset(uint64_t model, uint32_t row) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, false);
    if (err) return err;
    Llama* m = model_of(model, ctx, &err);
    if (!m) return err;
    if (row >= m->rows) return TMH_ERROR_INVALID_VALUE;
    m->length[row] = 0;
    m->has_logits[row] = 0;
    m->generating = false;
    return TMH_SUCCESS;
}

int tmh_llama_set_mode(uint64_t model, uint32_t mode) {
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, false);
    if (err) return err;
    Llama* m = model_of(model, ctx, &err);
    if (!m) return err;
    if (mode != TMH_MODE_AUTO && mode != TMH_MODE_UNORDERED) return TMH_ERROR_INVALID_VALUE;
    if (mode != m->mode && m->graph) {
        // the captured step holds the old mode's kernel arguments
        (void)hipStreamSynchronize(ctx.stream);
        (void)hipGraphExecDestroy(m->graph);
        m->graph = nullptr;
    }
    m->mode = mode;
    return TMH_SUCCESS;
}

int tmh_llama_destroy(uint64_t model) {
    if (!model) return TMH_SUCCESS;
    DeviceContext ctx;
    Llama* m = (Llama*)model;
    if (tmh::device_context(&ctx, false) == TMH_SUCCESS) (void)hipStreamSynchronize(ctx.stream);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    if (m->capture) (void)hipStreamDestroy(m->capture);
    if (m->memory) (void)hipFree(m->memory);
    if (m->owned) (void)hipFree(m->owned);
    delete m;
    return TMH_SUCCESS;
}

}  // extern "C"

// ---------------------------------------------------------- GGUF loading

namespace {

// Llama.unpermute's row order for block weights (llama.cr:226-235): each
// head's rows from llama.cpp's rotary pairing (2i, 2i+1) to (i, i + half).
std::vector<int32_t> unpermute_order(int32_t heads, int32_t head_width) {
    const int32_t half = head_width / 2;
    std::vector<int32_t> order;
    order.reserve((size_t)heads * head_width);
    for (int32_t h = 0; h < heads; ++h)
        for (int32_t pair = 0; pair < 2; ++pair)
            for (int32_t i = 0; i < half; ++i) order.push_back(h * 2 * half + 2 * i + pair);
    return order;
}

bool meta_int(const tmh::Gguf& g, const std::string& key, int64_t* out) {
    const tmh::GgufValue* v = g.value(key);
    if (!v || !(v->type <= 5 || v->type == 10 || v->type == 11)) return false;
    *out = v->i;
    return true;
}

bool meta_float(const tmh::Gguf& g, const std::string& key, double* out) {
    const tmh::GgufValue* v = g.value(key);
    if (!v) return false;
    if (v->type == 6 || v->type == 12) *out = v->f;
    else if (v->type <= 5 || v->type == 10 || v->type == 11) *out = (double)v->i;
    else return false;
    return true;
}

// Llama.config (llama.cr:57-77) from the llama.* metadata.
int gguf_config(const tmh::Gguf& g, tmh_llama_config* c) {
    const tmh::GgufValue* arch = g.value("general.architecture");
    if (!arch || arch->type != 8 || arch->s != "llama") return TMH_ERROR_INVALID_VALUE;
    const tmh::GgufValue* scaling = g.value("llama.rope.scaling.type");
    if (scaling && !(scaling->type == 8 && scaling->s == "none")) return TMH_ERROR_INVALID_VALUE;
    int64_t layers, width, heads, hidden, context, kv, hw, vocab;
    double eps, theta = 10000.0;
    if (!meta_int(g, "llama.block_count", &layers) || !meta_int(g, "llama.embedding_length", &width) ||
        !meta_int(g, "llama.attention.head_count", &heads) || !meta_int(g, "llama.feed_forward_length", &hidden) ||
        !meta_int(g, "llama.context_length", &context) ||
        !meta_float(g, "llama.attention.layer_norm_rms_epsilon", &eps))
        return TMH_ERROR_INVALID_VALUE;
    if (heads <= 0 || width <= 0) return TMH_ERROR_SHAPE;
    if (!meta_int(g, "llama.attention.head_count_kv", &kv)) kv = heads;
    if (!meta_int(g, "llama.rope.dimension_count", &hw)) hw = width / heads;
    if (!meta_int(g, "llama.vocab_size", &vocab)) {
        const tmh::GgufTensor* e = g.find("token_embd.weight");
        if (!e || e->shape.size() != 2) return TMH_ERROR_INVALID_VALUE;
        vocab = e->shape[0];
    }
    (void)meta_float(g, "llama.rope.freq_base", &theta);
    const tmh::GgufTensor* e = g.find("token_embd.weight");
    if (!e) return TMH_ERROR_INVALID_VALUE;
    uint32_t kind;
    switch (e->kind) {
    case tmh::GGUF_Q8_0: kind = TMH_Q8_0; break;
    case tmh::GGUF_Q4_0: kind = TMH_Q4_0; break;
    case tmh::GGUF_Q4_1: kind = TMH_Q4_1; break;
    default: return TMH_ERROR_DTYPE;
    }
    const int64_t limit = 1ll << 30;
    if (layers <= 0 || layers > 4096 || heads > limit || kv <= 0 || hw <= 0 || hidden <= 0 || vocab <= 0 ||
        context <= 0 || width > limit || hidden > limit || vocab > limit || context > limit)
        return TMH_ERROR_SHAPE;
    c->layers = (int32_t)layers;
    c->width = (int32_t)width;
    c->heads = (int32_t)heads;
    c->kv_heads = (int32_t)kv;
    c->head_width = (int32_t)hw;
    c->hidden = (int32_t)hidden;
    c->vocab = (int32_t)vocab;
    c->context = (int32_t)context;
    c->eps = (float)eps;
    c->theta = theta;
    c->kind = kind;
    return TMH_SUCCESS;
}

// Widens an F16 or BF16 tensor to F32 on the host, as GGUF#[] does.
bool widen(const tmh::Gguf& g, const tmh::GgufTensor& t, std::vector<float>& out) {
    const int64_t count = (int64_t)(t.kind == tmh::GGUF_F32 ? t.bytes / 4 : t.bytes / 2);
    out.resize((size_t)count);
    const uint8_t* p = g.map + t.offset;
    for (int64_t i = 0; i < count; ++i) {
        if (t.kind == tmh::GGUF_F32) {
            std::memcpy(&out[i], p + 4 * i, 4);
        } else {
            uint16_t h;
            std::memcpy(&h, p + 2 * i, 2);
            if (t.kind == tmh::GGUF_BF16) {
                const uint32_t bits = (uint32_t)h << 16;
                std::memcpy(&out[i], &bits, 4);
            } else {
                _Float16 f;
                std::memcpy(&f, &h, 2);
                out[i] = (float)f;
            }
        }
    }
    return true;
}

}  // namespace

extern "C" {

int tmh_llama_load_gguf(const char* path, uint32_t rows, uint32_t capacity, uint32_t max_tokens,
                        tmh_llama_config* config, uint64_t* model) {
    if (!path || !model) return TMH_ERROR_INVALID_VALUE;
    *model = 0;
    DeviceContext ctx;
    int err = tmh::device_context(&ctx, true);
    if (err) return err;
    tmh::Gguf g;
    if ((err = g.open(path)) != TMH_SUCCESS) return err;
    tmh_llama_config c{};
    if ((err = gguf_config(g, &c)) != TMH_SUCCESS) return err;
    const uint32_t gkind = c.kind == TMH_Q8_0 ? tmh::GGUF_Q8_0 : c.kind == TMH_Q4_0 ? tmh::GGUF_Q4_0 : tmh::GGUF_Q4_1;
    const int64_t W = c.width, H = c.hidden, qn = (int64_t)c.heads * c.head_width, kvn = (int64_t)c.kv_heads * c.head_width;

    // The tensors the model has, by GGUF name, with their shapes; a block
    // matrix or an F32-like vector each.
    struct Want {
        std::string name;
        std::vector<int64_t> shape;
        bool matrix;
    };
    std::vector<Want> wants = {{"token_embd.weight", {c.vocab, W}, true}, {"output_norm.weight", {W}, false}};
    const bool tied = g.find("output.weight") == nullptr;
    if (!tied) wants.push_back({"output.weight", {c.vocab, W}, true});
    for (int32_t l = 0; l < c.layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        wants.push_back({b + "attn_norm.weight", {W}, false});
        wants.push_back({b + "attn_q.weight", {qn, W}, true});
        wants.push_back({b + "attn_k.weight", {kvn, W}, true});
        wants.push_back({b + "attn_v.weight", {kvn, W}, true});
        wants.push_back({b + "attn_output.weight", {W, qn}, true});
        wants.push_back({b + "ffn_norm.weight", {W}, false});
        wants.push_back({b + "ffn_gate.weight", {H, W}, true});
        wants.push_back({b + "ffn_up.weight", {H, W}, true});
        wants.push_back({b + "ffn_down.weight", {W, H}, true});
    }
    for (const Want& w : wants) {
        const tmh::GgufTensor* t = g.find(w.name);
        if (!t) return TMH_ERROR_INVALID_VALUE;
        if (t->shape != w.shape) return TMH_ERROR_SHAPE;
        if (w.matrix ? t->kind != gkind
                     : !(t->kind == tmh::GGUF_F32 || t->kind == tmh::GGUF_F16 || t->kind == tmh::GGUF_BF16))
            return TMH_ERROR_DTYPE;
    }
    if (wants.size() != g.tensors.size()) return TMH_ERROR_INVALID_VALUE;  // tensors the model lacks

    // One device allocation for every weight, carved 256-byte aligned.
    const uint64_t row = tmh::gguf_bytes_for(gkind, W);
    const uint64_t embed_bytes = (uint64_t)c.vocab * row;
    const uint64_t qkv_bytes = (uint64_t)(qn + 2 * kvn) * row, o_bytes = (uint64_t)W * tmh::gguf_bytes_for(gkind, qn);
    const uint64_t gu_bytes = (uint64_t)(2 * H) * row, down_bytes = (uint64_t)W * tmh::gguf_bytes_for(gkind, H);
    const uint64_t norm_bytes = (uint64_t)W * 4;
    const uint64_t per_layer = align256(qkv_bytes) + align256(o_bytes) + align256(gu_bytes) + align256(down_bytes) +
                               2 * align256(norm_bytes);
    const uint64_t total = align256(embed_bytes) + (tied ? 0 : align256(embed_bytes)) + align256(norm_bytes) +
                           per_layer * (uint64_t)c.layers;
    void* mem = nullptr;
    hipError_t e = tmh::device_malloc(&mem, total);
    if (e != hipSuccess) return code(e);
    uint8_t* base = (uint8_t*)mem;
    uint64_t at = 0;
    auto carve = [&](uint64_t bytes) {
        uint64_t p = (uint64_t)(base + at);
        at += align256(bytes);
        return p;
    };
    auto upload = [&](const std::string& name, const int32_t* order, uint32_t count, uint64_t dst) {
        return tmh_gguf_upload((uint64_t)&g, name.c_str(), order, count, dst);
    };
    auto upload_norm = [&](const std::string& name, uint64_t dst) {
        const tmh::GgufTensor* t = g.find(name);
        if (t->kind == tmh::GGUF_F32) return upload(name, nullptr, 0, dst);
        std::vector<float> wide;
        widen(g, *t, wide);
        return tmh_upload_async(dst, wide.data(), wide.size() * 4);
    };
    std::vector<uint64_t> attn_norm(c.layers), ffn_norm(c.layers), qkv(c.layers), o(c.layers), gate_up(c.layers),
        down(c.layers);
    const std::vector<int32_t> q_order = unpermute_order(c.heads, c.head_width);
    const std::vector<int32_t> k_order = unpermute_order(c.kv_heads, c.head_width);
    tmh_llama_weights w{};
    w.embed = carve(embed_bytes);
    err = upload("token_embd.weight", nullptr, 0, w.embed);
    if (!err && !tied) {
        w.head = carve(embed_bytes);
        err = upload("output.weight", nullptr, 0, w.head);
    }
    if (!err) {
        w.norm = carve(norm_bytes);
        err = upload_norm("output_norm.weight", w.norm);
    }
    for (int32_t l = 0; l < c.layers && !err; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        attn_norm[l] = carve(norm_bytes);
        ffn_norm[l] = carve(norm_bytes);
        qkv[l] = carve(qkv_bytes);
        o[l] = carve(o_bytes);
        gate_up[l] = carve(gu_bytes);
        down[l] = carve(down_bytes);
        err = upload_norm(b + "attn_norm.weight", attn_norm[l]);
        if (!err) err = upload_norm(b + "ffn_norm.weight", ffn_norm[l]);
        if (!err) err = upload(b + "attn_q.weight", q_order.data(), (uint32_t)q_order.size(), qkv[l]);
        if (!err) err = upload(b + "attn_k.weight", k_order.data(), (uint32_t)k_order.size(), qkv[l] + qn * row);
        if (!err) err = upload(b + "attn_v.weight", nullptr, 0, qkv[l] + (qn + kvn) * row);
        if (!err) err = upload(b + "attn_output.weight", nullptr, 0, o[l]);
        if (!err) err = upload(b + "ffn_gate.weight", nullptr, 0, gate_up[l]);
        if (!err) err = upload(b + "ffn_up.weight", nullptr, 0, gate_up[l] + H * row);
        if (!err) err = upload(b + "ffn_down.weight", nullptr, 0, down[l]);
    }
    if (!err) {
        w.attn_norm = attn_norm.data();
        w.ffn_norm = ffn_norm.data();
        w.qkv = qkv.data();
        w.o = o.data();
        w.gate_up = gate_up.data();
        w.down = down.data();
        err = tmh_llama_create(&c, &w, rows, capacity ? capacity : (uint32_t)c.context, max_tokens, model);
    }
    if (!err) err = tmh_synchronize();  // the staged uploads have landed
    if (err) {
        if (*model) {
            (void)tmh_llama_destroy(*model);
            *model = 0;
        }
        (void)hipFree(mem);
        return err;
    }
    ((Llama*)*model)->owned = mem;
    if (config) *config = c;
    return TMH_SUCCESS;
}

}  // extern "C"
