/* ThreadSanitizer driver for the oracle's spinning pool (test
 * infrastructure: the CPU baselines' threads): products of every format and
 * the Attention op on 8 threads, 20 and 50 times, each equal bit for bit to
 * the same call on one thread. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
int tmo_quantize(int kind, const float* values, int64_t count, uint8_t* out);
int tmo_matmul(int kind, const float* x, const uint8_t* w, int32_t rows, int32_t n, int32_t k, float* dst);
void tmo_set_threads(int threads);
void tmo_attention(const float* q, int32_t tokens, int32_t heads, const float* keys, const float* values,
                   int32_t kv_heads, int32_t capacity, int32_t width, const int32_t* table, float scale, float* out);
static float frand(unsigned* s) { *s = *s * 1103515245u + 12345u; return ((*s >> 8) & 0xffff) / 32768.0f - 1.0f; }
int main(void) {
    unsigned s = 1;
    const int n = 3000, k = 2048, rows = 3;
    float* w = malloc(sizeof(float) * n * k); float* x = malloc(sizeof(float) * rows * k);
    for (int i = 0; i < n * k; i++) w[i] = frand(&s) * 0.02f;
    for (int i = 0; i < rows * k; i++) x[i] = frand(&s);
    int bad = 0;
    for (int kind = 0; kind < 3; kind++) {
        uint8_t* wq = malloc((size_t)n * (k / 32) * 34);
        tmo_quantize(kind, w, (int64_t)n * k, wq);
        float* a = malloc(sizeof(float) * rows * n); float* b = malloc(sizeof(float) * rows * n);
        tmo_set_threads(1); tmo_matmul(kind, x, wq, rows, n, k, a);
        tmo_set_threads(8);
        for (int rep = 0; rep < 20; rep++) { tmo_matmul(kind, x, wq, rows, n, k, b); bad += memcmp(a, b, sizeof(float) * rows * n) != 0; }
        free(wq); free(a); free(b);
    }
    const int heads = 8, cap = 300, hw = 64, p = 250;
    float* q = malloc(sizeof(float) * 2 * heads * hw); float* kk = malloc(sizeof(float) * 2 * heads * cap * hw); float* vv = malloc(sizeof(float) * 2 * heads * cap * hw);
    for (int i = 0; i < 2 * heads * hw; i++) q[i] = frand(&s);
    for (int i = 0; i < 2 * heads * cap * hw; i++) { kk[i] = frand(&s); vv[i] = frand(&s); }
    int32_t table[6] = {0, p - 1, p, 1, p - 10, p - 9};
    float* o1 = malloc(sizeof(float) * 2 * heads * hw); float* o8 = malloc(sizeof(float) * 2 * heads * hw);
    tmo_set_threads(1); tmo_attention(q, 2, heads, kk, vv, heads, cap, hw, table, 0.125f, o1);
    tmo_set_threads(8);
    for (int rep = 0; rep < 50; rep++) { tmo_attention(q, 2, heads, kk, vv, heads, cap, hw, table, 0.125f, o8); bad += memcmp(o1, o8, sizeof(float) * 2 * heads * hw) != 0; }
    printf("mismatches %d\n", bad);
    return bad != 0;
}
