// Host-only robustness driver for the GGUF reader (AddressSanitizer build):
// opens each fixture, then every truncation of its first 64 KB and random
// byte mutations of its header region, querying a few tensors when a
// variant opens. Any out-of-bounds access aborts with a sanitizer report.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>
#include "tensomite_hip.h"

static std::vector<unsigned char> slurp(const char* p) {
    FILE* f = fopen(p, "rb");
    std::vector<unsigned char> v;
    if (!f) return v;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    v.resize(n);
    if (fread(v.data(), 1, n, f) != (size_t)n) v.clear();
    fclose(f);
    return v;
}

static int try_open(const std::vector<unsigned char>& d, size_t len, const char* tmp) {
    FILE* f = fopen(tmp, "wb");
    fwrite(d.data(), 1, len, f);
    fclose(f);
    uint64_t h = 0;
    int e = tmh_gguf_open(tmp, &h);
    if (e == 0) {
        const char* names[] = {"token_embd.weight", "blk.0.attn_q.weight", "blk.1.ffn_down.weight", "output_norm.weight",
                               "nope"};
        for (const char* nm : names) {
            uint32_t kind, dims;
            int64_t shape[4];
            uint64_t bytes;
            tmh_gguf_tensor(h, nm, &kind, shape, &dims, &bytes);
        }
        tmh_gguf_close(h);
    }
    return e;
}

int main(int argc, char** argv) {
    const char* tmp = "/tmp/gguf_fuzz.gguf";
    long opened = 0, refused = 0;
    for (int a = 1; a < argc; ++a) {
        std::vector<unsigned char> good = slurp(argv[a]);
        if (good.empty()) { fprintf(stderr, "cannot read %s\n", argv[a]); return 2; }
        if (try_open(good, good.size(), tmp) != 0) { fprintf(stderr, "fixture refused: %s\n", argv[a]); return 3; }
        const size_t lim = good.size() < 65536 ? good.size() : 65536;
        for (size_t len = 0; len < lim; ++len) (try_open(good, len, tmp) == 0 ? opened : refused)++;
        std::mt19937_64 rng(12345 + a);
        const size_t head = good.size() < 8192 ? good.size() : 8192;
        for (int i = 0; i < 20000; ++i) {
            std::vector<unsigned char> d = good;
            const int flips = 1 + (int)(rng() % 4);
            for (int j = 0; j < flips; ++j) {
                const size_t at = rng() % head;
                switch (rng() % 3) {
                case 0: d[at] ^= (unsigned char)(1u << (rng() % 8)); break;
                case 1: d[at] = (unsigned char)rng(); break;
                default: d[at] = (rng() % 2) ? 0xff : 0x00; break;
                }
            }
            (try_open(d, d.size(), tmp) == 0 ? opened : refused)++;
        }
        printf("%s: done\n", argv[a]);
    }
    printf("variants opened %ld, refused %ld\n", opened, refused);
    return 0;
}
