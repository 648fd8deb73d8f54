/* Host fuzz driver for the GGUF reader (qwenqwen3.js_amd/csrc/gguf.cpp), run
 * under AddressSanitizer + UBSan.  It mutates a valid GGUF file (random
 * truncation and up to three bit flips past the magic) and, for every file
 * the reader accepts, walks every accessor: header, each tensor record (its
 * name is read byte by byte), each KV (number, string bytes, last array
 * element), lookups by the names just read, and the MoE block binding of
 * block 0.  Files the reader refuses must leave no allocation behind.
 *
 * usage: gguf_fuzz <file.gguf> <iterations> <seed>
 * prints "ok N refused M" and exits 0; a sanitizer report exits non-zero. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/qq_gguf.h"

static uint64_t rng_state;

/* xorshift64 (Marsaglia, "Xorshift RNGs", 2003) */
static uint64_t next_u64(void)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return rng_state;
}

static unsigned touch(const char *s, uint64_t n)
{
    unsigned h = 0;
    for (uint64_t i = 0; i < n; i++) h = h * 31u + (unsigned char)s[i];
    return h;
}

static unsigned walk(const qq_gguf *g)
{
    unsigned h = 0;
    qq_gguf_header_info hd;
    if (qq_gguf_header(g, &hd)) return h;
    for (uint64_t i = 0; i < hd.tensor_count; i++) {
        qq_gguf_tensor t;
        if (qq_gguf_tensor_info(g, i, &t)) continue;
        h += touch(t.name, strlen(t.name));
        h += (unsigned)qq_gguf_find_tensor(g, t.name);
    }
    for (uint64_t i = 0; i < hd.kv_count; i++) {
        const char *key;
        uint32_t type, et;
        uint64_t n, len;
        const char *s;
        double v;
        if (qq_gguf_kv_info(g, i, &key, &type)) continue;
        h += touch(key, strlen(key)) + (unsigned)qq_gguf_find_key(g, key);
        if (qq_gguf_kv_number(g, i, &v) == 0) h += (unsigned)(v != v);
        if (qq_gguf_kv_string(g, i, &s, &len) == 0) h += touch(s, len);
        if (qq_gguf_kv_array(g, i, &et, &n) == 0 && n)
            if (qq_gguf_kv_array_number(g, i, n - 1, &v) == 0) h += (unsigned)(v != v);
    }
    qq_gguf_moe_info mi;
    if (qq_gguf_moe_params(g, 0, 0, -1, &mi) == 0) h += (unsigned)(mi.H + mi.F + mi.E + mi.K);
    return h;
}

int main(int argc, char **argv)
{
    if (argc != 4) {
        fprintf(stderr, "usage: %s <file.gguf> <iterations> <seed>\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "rb");
    if (!f) {
        perror(argv[1]);
        return 2;
    }
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    uint8_t *base = (uint8_t *)malloc(n ? (size_t)n : 1);
    if (!base || fread(base, 1, (size_t)n, f) != (size_t)n) {
        fprintf(stderr, "cannot read %s\n", argv[1]);
        return 2;
    }
    fclose(f);
    long iters = atol(argv[2]);
    rng_state = (uint64_t)strtoull(argv[3], NULL, 10) * 0x9E3779B97F4A7C15ull + 1;

    /* the header and tables (everything before the data section) are where
     * the parser branches: most cuts and flips land there */
    uint64_t head = (uint64_t)n;
    {
        qq_gguf *g0 = NULL;
        qq_gguf_header_info hd;
        if (qq_gguf_open_memory(base, (size_t)n, &g0) != 0 || qq_gguf_header(g0, &hd) != 0) {
            fprintf(stderr, "%s: the unmutated file is refused: %s\n", argv[1], qq_gguf_last_error());
            return 2;
        }
        head = hd.data_offset < (uint64_t)n ? hd.data_offset : (uint64_t)n;
        qq_gguf_close(g0);
    }

    long ok = 0, refused = 0;
    unsigned h = 0;
    for (long it = 0; it < iters; it++) {
        /* exact-size copies, so a read past the end is a heap overflow */
        uint64_t span = (next_u64() & 1) ? head + 1 : (uint64_t)n + 1;
        size_t len = (next_u64() & 3) ? (size_t)n : (size_t)(next_u64() % span);
        uint8_t *b = (uint8_t *)malloc(len ? len : 1);
        memcpy(b, base, len);
        int flips = (int)(next_u64() % 4);
        for (int i = 0; i < flips && len > 4; i++) {
            uint64_t lim = (next_u64() % 4 && head > 4 && head < len) ? head : len;
            b[4 + next_u64() % (lim - 4)] ^= (uint8_t)(1u << (next_u64() % 8));
        }
        qq_gguf *g = NULL;
        if (qq_gguf_open_memory(b, len, &g) == 0) {
            ok++;
            h += walk(g);
            qq_gguf_close(g);
        } else {
            refused++;
        }
        free(b);
    }
    free(base);
    printf("ok %ld refused %ld (walk hash %08x)\n", ok, refused, h);
    return 0;
}
