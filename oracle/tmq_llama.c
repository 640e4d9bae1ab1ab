/*
 * tmq_llama.c -- CPU restatement of tensomite's Llama forward on a host
 * device, for decode parity: every op rounded as the reference's host kernels
 * round it, in their order.
 *
 * TEST INFRASTRUCTURE ONLY (see tmq_oracle.c's header). Built into the same
 * libtmq_oracle*.so; compiled with -ffp-contract=off, no fast math.
 *
 * The graph (src/tensomite/models/llama.cr:113-124, 256-303; modules.cr):
 *   x = gather(embed, ids)                          Quant.gather, quant.cr:417-422
 *   per layer:
 *     h = rmsnorm(x) · w                            host.cr:374-386
 *     qkv = h · Wqkvᵀ (one merged product)          Quant.matmul, quant.cr:155-182
 *     q, k = rope(q), rope(k) at their positions    host.cr:448-466; tables modules.cr:344-351
 *     cache[past...] = k, v                         Tensor#write (Cache#append, modules.cr:164-176)
 *     scores = q · kᵀ (index order), softmax(scale, mask), · v
 *                                                   the Attention op, host.cr:408-440 (the composite
 *                                                   of composite.cr:190-199 rounds alike: matmul
 *                                                   host.cr:700-721, softmax host.cr:363-383)
 *     x = x + attended · Woᵀ                        binary Add, host.cr:159-180
 *     h = rmsnorm(x) · w2; gu = h · Wguᵀ
 *     x = x + swiglu(gate, up) · Wdownᵀ             kernels.cr:18 (gate / (exp(-gate) + 1) · up)
 *   logits = rmsnorm(x) · headᵀ                     llama.cr:294-303
 *   greedy token = the first highest logit          sampler.cr:35-36
 *
 * Parity pins (tests/test_oracle_llama.py): Maths.exp against its stated
 * error bound and special values (maths.cr:1-54, spec/maths_spec.cr); the
 * tiny_llama GGUF fixtures' F32 logits (block_matmul_spec.cr:275-284: Q8_0
 * error < Q4_0 error / 4); prefill == one-by-one decode bits
 * (block_matmul_spec.cr:253-260); a row alone == in a batch.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int tmo_block_bytes(int kind);
int tmo_matmul(int kind, const float* x, const uint8_t* w, int32_t rows, int32_t n, int32_t k, float* dst);
int tmo_dequantize(int kind, const uint8_t* bytes, int64_t count, float* values);
void tmo_parallel_for(int32_t count, void (*fn)(void*, int32_t, int32_t), void* ctx);

/* ------------------------------------------------------------ Maths.exp */

static inline float bits_float(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Maths.exp, maths.cr:36-54: range reduction x = n·ln2 + r, a degree-6
 * polynomial, 2^n as two exponent halves; 0 below -87.34, inf above 88.72. */
float tmo_exp(float x) {
    const float LOG2E = 1.44269504088896341f, LN2_HI = 0.693359375f, LN2_LO = -2.12194440e-4f;
    const float EXP_HI = 88.72283905f, EXP_LO = -87.3365447f, ROUNDER = 12582912.0f;
    float clamped = (x > EXP_HI || x < EXP_LO) ? 0.0f : x;
    float n = clamped * LOG2E;
    n = n + ROUNDER;
    n = n - ROUNDER;
    float r = clamped - n * LN2_HI;
    r = r - n * LN2_LO;
    float z = r * r;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * z + r;
    p = p + 1.0f;
    int32_t whole = isnan(n) ? INT32_MIN : (int32_t)n; /* n is clamped: only NaN is out of range */
    int32_t half = whole >> 1;
    float result = p * bits_float((uint32_t)(half + 127) << 23);
    result = result * bits_float((uint32_t)(whole - half + 127) << 23);
    result = x > EXP_HI ? INFINITY : result;
    result = x < EXP_LO ? 0.0f : result;
    return isnan(x) ? x : result;
}

void tmo_exp_many(const float* x, int64_t count, float* out) {
    for (int64_t i = 0; i < count; i++) out[i] = tmo_exp(x[i]);
}

/* ------------------------------------------------------------ row ops */

/* rmsnorm_row, host.cr:374-386: Σx² folded from zero, root = sqrt(Σx²/n + ε),
 * then x / root · w. */
void tmo_rmsnorm(const float* x, const float* w, int32_t rows, int32_t n, float eps, float* out) {
    for (int32_t r = 0; r < rows; r++) {
        const float* xr = x + (int64_t)r * n;
        float squares = 0.0f;
        for (int32_t j = 0; j < n; j++) squares += xr[j] * xr[j];
        float root = sqrtf(squares / (float)n + eps);
        for (int32_t j = 0; j < n; j++) {
            float v = xr[j] / root;
            out[(int64_t)r * n + j] = w ? v * w[j] : v;
        }
    }
}

/* RotaryEmbedding tables, modules.cr:344-351: frequency i = 1 / θ^(2i/width)
 * in Float32 (powf), cos/sin of p·frequency (cosf, sinf). */
void tmo_rope_tables(int32_t width, int32_t context, double theta, float* cos_out, float* sin_out) {
    int32_t half = width / 2;
    float* freq = malloc(sizeof(float) * (size_t)half);
    for (int32_t i = 0; i < half; i++) freq[i] = 1.0f / powf((float)theta, (float)(2 * i) / (float)width);
    for (int32_t p = 0; p < context; p++)
        for (int32_t i = 0; i < width; i++) {
            float angle = (float)p * freq[i % half];
            cos_out[(int64_t)p * width + i] = cosf(angle);
            sin_out[(int64_t)p * width + i] = sinf(angle);
        }
    free(freq);
}

/* rope, host.cr:448-466, one row of n at a table row: x·cos + rotate_half(x)·sin. */
static void rope_row(const float* x, int32_t n, const float* c, const float* s, float* out) {
    int32_t half = n / 2;
    for (int32_t col = 0; col < n; col++) {
        float partner = x[col < half ? col + half : col - half];
        float rotated = col < half ? partner * -1.0f : partner;
        float a = x[col] * c[col];
        float b = rotated * s[col];
        out[col] = a + b;
    }
}

/* The gate of SwiGLU, kernels.cr:18: gate / (exp(-gate) + 1) · value. */
static inline float swiglu(float gate, float value) {
    float e = tmo_exp(-gate);
    float d = e + 1.0f;
    float q = gate / d;
    return q * value;
}

void tmo_swiglu_many(const float* gate, const float* value, int64_t count, float* out) {
    for (int64_t i = 0; i < count; i++) out[i] = swiglu(gate[i], value[i]);
}

/* SwiGLU of each row's gate and up halves (rows of 2·hidden), a[r, j] =
 * swiglu(gu[r, j], gu[r, hidden + j]), in spans of elements on the
 * spinning pool (elementwise, so any split gives the same bits). */
typedef struct {
    const float* gu;
    float* a;
    int32_t hidden;
} swiglu_job;

static void swiglu_items(void* arg, int32_t first, int32_t stop) {
    const swiglu_job* j = arg;
    for (int32_t e = first; e < stop; e++) {
        const int32_t r = e / j->hidden, c = e - r * j->hidden;
        j->a[e] = swiglu(j->gu[(size_t)r * 2 * j->hidden + c], j->gu[(size_t)r * 2 * j->hidden + j->hidden + c]);
    }
}

/* ------------------------------------------------------------ the model */

typedef struct {
    int32_t layers, width, heads, kv_heads, head_width, hidden, vocab, context;
    float eps;
    double theta;
    int32_t kind; /* block kind of every matrix (and the embedding table) */
} tmo_llama_config;

typedef struct {
    const uint8_t* embed;      /* [vocab, width] blocks */
    const uint8_t* head;       /* [vocab, width] blocks: the embedding table when tied */
    const float* norm;         /* [width] */
    const float* const* attn_norm; /* per layer [width] */
    const float* const* ffn_norm;
    const uint8_t* const* qkv;     /* per layer [(heads + 2·kv_heads)·head_width, width]; q and k rows in HF order */
    const uint8_t* const* o;       /* per layer [width, heads·head_width] */
    const uint8_t* const* gate_up; /* per layer [2·hidden, width] */
    const uint8_t* const* down;    /* per layer [width, hidden] */
} tmo_llama_weights;

typedef struct {
    tmo_llama_config c;
    tmo_llama_weights w;
    float *cos, *sin;
    float *keys, *values; /* per layer [kv_heads, context, head_width] */
    int32_t length;
} tmo_llama;

tmo_llama* tmo_llama_new(const tmo_llama_config* c, const tmo_llama_weights* w) {
    tmo_llama* m = calloc(1, sizeof(tmo_llama));
    m->c = *c;
    m->w = *w;
    m->cos = malloc(sizeof(float) * (size_t)c->context * c->head_width);
    m->sin = malloc(sizeof(float) * (size_t)c->context * c->head_width);
    tmo_rope_tables(c->head_width, c->context, c->theta, m->cos, m->sin);
    size_t cache = (size_t)c->layers * c->kv_heads * c->context * c->head_width;
    m->keys = calloc(cache, sizeof(float));
    m->values = calloc(cache, sizeof(float));
    return m;
}

void tmo_llama_free(tmo_llama* m) {
    if (!m) return;
    free(m->cos);
    free(m->sin);
    free(m->keys);
    free(m->values);
    free(m);
}

void tmo_llama_reset(tmo_llama* m) { m->length = 0; }

int32_t tmo_llama_length(const tmo_llama* m) { return m->length; }

/* The rope tables, for the device to upload the same values. */
const float* tmo_llama_cos(const tmo_llama* m) { return m->cos; }
const float* tmo_llama_sin(const tmo_llama* m) { return m->sin; }

typedef struct {
    const float *q, *keys, *values;
    int32_t heads, kv_heads, capacity, width;
    const int32_t* table;
    float scale;
    float* out;
} attention_job;

/* Items first .. stop - 1 (item = token · heads + head), each with its own
 * scores. */
static void attention_items(void* arg, int32_t first, int32_t stop) {
    const attention_job* j = arg;
    const int32_t group = j->heads / j->kv_heads, width = j->width;
    float* scores = malloc(sizeof(float) * (size_t)j->capacity);
    for (int32_t item = first; item < stop; item++) {
        const int32_t t = item / j->heads, h = item - t * j->heads;
        const int32_t row = j->table[3 * t], last = j->table[3 * t + 1], positions = j->table[3 * t + 2];
        const int32_t kv = h / group;
        const float* kh = j->keys + ((size_t)row * j->kv_heads + kv) * j->capacity * width;
        const float* vh = j->values + ((size_t)row * j->kv_heads + kv) * j->capacity * width;
        const float* qi = j->q + ((size_t)t * j->heads + h) * width;
        float top = 0.0f;
        for (int32_t p = 0; p < positions; p++) {
            float dot = 0.0f;
            for (int32_t col = 0; col < width; col++) dot += qi[col] * kh[(size_t)p * width + col];
            float x = dot * j->scale;
            float mask = p > last ? -INFINITY : 0.0f;
            x = x + mask;
            scores[p] = x;
            if (p == 0 || x > top) top = x;
        }
        float total = 0.0f;
        for (int32_t p = 0; p < positions; p++) total += (scores[p] = tmo_exp(scores[p] - top));
        float* oi = j->out + ((size_t)t * j->heads + h) * width;
        for (int32_t col = 0; col < width; col++) {
            float acc = 0.0f;
            for (int32_t p = 0; p < positions; p++) acc += scores[p] / total * vh[(size_t)p * width + col];
            oi[col] = acc;
        }
    }
    free(scores);
}

/* The Attention op on a host device, host.cr:408-440, for `tokens` packed
 * query rows q [tokens, heads, width] against caches [rows, kv_heads,
 * capacity, width]: token t reads cache row table[3t] up to table[3t+2]
 * positions and sees positions up to table[3t+1] (the causal mask,
 * composite.cr:282-290). Per head h (kv head h / group): scores[p] = (q · k_p)
 * in column order, · scale, + mask (-inf past the last seen position), top =
 * the first highest, e_p = Maths.exp(scores[p] - top), total in position
 * order, out[c] = Σ_p (e_p / total) · v_p[c] in position order. The
 * reference walks the (token, head) items on one thread; here they run on
 * the spinning pool, each item's arithmetic the same sequence, so the bits
 * are the same. */
void tmo_attention(const float* q, int32_t tokens, int32_t heads, const float* keys, const float* values,
                   int32_t kv_heads, int32_t capacity, int32_t width, const int32_t* table, float scale, float* out) {
    attention_job j = {q, keys, values, heads, kv_heads, capacity, width, table, scale, out};
    tmo_parallel_for(tokens * heads, attention_items, &j);
}

/* The Rope op, host.cr:448-466, on `heads` heads of `width` per token (token
 * rows `ldx` apart), token t rotated by table row positions[t]; out is
 * [tokens, heads, width]. */
void tmo_rope(const float* x, int32_t ldx, int32_t tokens, int32_t heads, int32_t width, const float* cos,
              const float* sin, const int32_t* positions, float* out) {
    for (int32_t t = 0; t < tokens; t++)
        for (int32_t h = 0; h < heads; h++)
            rope_row(x + (size_t)t * ldx + (size_t)h * width, width, cos + (size_t)positions[t] * width,
                     sin + (size_t)positions[t] * width, out + ((size_t)t * heads + h) * width);
}

/* Llama#logits then #head (llama.cr:265-303) for `count` new ids after the
 * cached positions; writes [count, vocab] logits, or with `last_only` the
 * last row's [vocab] (forward_last, generative.cr:168-172). Returns 0, or -1
 * when the positions exceed the context. */
int tmo_llama_forward(tmo_llama* m, const int32_t* ids, int32_t count, int32_t last_only, float* logits) {
    const tmo_llama_config* c = &m->c;
    int32_t past = m->length;
    if (count <= 0 || past + count > c->context) return -1;
    for (int32_t i = 0; i < count; i++)
        if (ids[i] < 0 || ids[i] >= c->vocab) return -2;
    int32_t W = c->width, hw = c->head_width, H = c->hidden;
    int32_t qn = c->heads * hw, kvn = c->kv_heads * hw, nqkv = qn + 2 * kvn;
    int64_t row_bytes = (int64_t)W / 32 * tmo_block_bytes(c->kind);
    float* x = malloc(sizeof(float) * (size_t)count * W);
    float* h = malloc(sizeof(float) * (size_t)count * W);
    float* qkv = malloc(sizeof(float) * (size_t)count * nqkv);
    float* q = malloc(sizeof(float) * (size_t)count * qn);
    float* att = malloc(sizeof(float) * (size_t)count * qn);
    float* o = malloc(sizeof(float) * (size_t)count * W);
    float* gu = malloc(sizeof(float) * (size_t)count * 2 * H);
    float* a = malloc(sizeof(float) * (size_t)count * H);
    int32_t* table = malloc(sizeof(int32_t) * 3 * (size_t)count);
    float scale = (float)(1.0 / sqrt((double)hw));
    for (int32_t i = 0; i < count; i++) {
        table[3 * i] = 0;
        table[3 * i + 1] = past + i;
        table[3 * i + 2] = past + count;
        tmo_dequantize(c->kind, m->w.embed + ids[i] * row_bytes, W, x + (size_t)i * W);
    }
    for (int32_t layer = 0; layer < c->layers; layer++) {
        tmo_rmsnorm(x, m->w.attn_norm[layer], count, W, c->eps, h);
        tmo_matmul(c->kind, h, m->w.qkv[layer], count, nqkv, W, qkv);
        float* keys = m->keys + (size_t)layer * c->kv_heads * c->context * hw;
        float* values = m->values + (size_t)layer * c->kv_heads * c->context * hw;
        for (int32_t i = 0; i < count; i++) {
            int32_t pos = past + i;
            const float* cr = m->cos + (size_t)pos * hw;
            const float* sr = m->sin + (size_t)pos * hw;
            const float* row = qkv + (size_t)i * nqkv;
            for (int32_t hd = 0; hd < c->heads; hd++) rope_row(row + hd * hw, hw, cr, sr, q + (size_t)i * qn + hd * hw);
            for (int32_t kv = 0; kv < c->kv_heads; kv++) {
                rope_row(row + qn + kv * hw, hw, cr, sr, keys + ((size_t)kv * c->context + pos) * hw);
                memcpy(values + ((size_t)kv * c->context + pos) * hw, row + qn + kvn + kv * hw, sizeof(float) * hw);
            }
        }
        tmo_attention(q, count, c->heads, keys, values, c->kv_heads, c->context, hw, table, scale, att);
        tmo_matmul(c->kind, att, m->w.o[layer], count, W, qn, o);
        for (int64_t j = 0; j < (int64_t)count * W; j++) x[j] = x[j] + o[j];
        tmo_rmsnorm(x, m->w.ffn_norm[layer], count, W, c->eps, h);
        tmo_matmul(c->kind, h, m->w.gate_up[layer], count, 2 * H, W, gu);
        swiglu_job sj = {gu, a, H};
        tmo_parallel_for(count * H, swiglu_items, &sj);
        tmo_matmul(c->kind, a, m->w.down[layer], count, W, H, o);
        for (int64_t j = 0; j < (int64_t)count * W; j++) x[j] = x[j] + o[j];
    }
    const float* last = last_only ? x + (size_t)(count - 1) * W : x;
    int32_t rows = last_only ? 1 : count;
    tmo_rmsnorm(last, m->w.norm, rows, W, c->eps, h);
    tmo_matmul(c->kind, h, m->w.head, rows, c->vocab, W, logits);
    m->length = past + count;
    free(x);
    free(h);
    free(qkv);
    free(q);
    free(att);
    free(o);
    free(gu);
    free(a);
    free(table);
    return 0;
}

/* Sampler.greedy, sampler.cr:35-36: the first index of the highest logit. */
int32_t tmo_argmax(const float* logits, int32_t n) {
    int32_t best = 0;
    for (int32_t i = 1; i < n; i++)
        if (logits[i] > logits[best]) best = i;
    return best;
}
