/* Host-only driver for the GGUF reader under AddressSanitizer and UBSan
 * (built and run by tests/test_gguf_reader.py with gcc; no GPU involved).
 *
 *   gguf_fuzz <seed file> <scratch path> <iterations> <span>
 *
 * Each iteration corrupts a copy of the seed file (byte writes and u64
 * writes within its first <span> bytes, truncation anywhere), opens it with
 * orn_gguf_open and, when that succeeds, walks every accessor and reads
 * every tensor.  The sanitizers turn any out-of-bounds access, overflow or
 * leak into a non-zero exit.  The entry points of the rest of the library
 * that gguf_file.c calls are stubbed. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../ornith-flight_amd/csrc/host/internal.h"

/* ---- stubs: the device side is not part of this driver ------------------ */
int orn_set_err(gpu_context *ctx, int code, const char *fmt, ...) { return code; }
const ornith_moe_shape *orn_store_shape(const ornith_moe_store *st) { return NULL; }
float orn_quirk_half(uint16_t h) { return (float)h; }
bool gpu_dequantize_tensor_from_buf(gpu_context *c, const void *d, const orn_tensor_info *t,
                                    float *o) { return false; }
bool gpu_dequantize_expert_slice_from_buf(gpu_context *c, const void *d, const orn_tensor_info *t,
                                          int e, float *o) { return false; }
int gpu_moe_store_set_experts(gpu_context *c, ornith_moe_store *s, int l, int m, int f, int n,
                              const void *b) { return 0; }
int gpu_moe_store_set_router(gpu_context *c, ornith_moe_store *s, int l, const float *w,
                             const float *b) { return 0; }
int gpu_moe_store_set_norm(gpu_context *c, ornith_moe_store *s, int l, const float *w) { return 0; }
int gpu_moe_store_set_shexp_gate(gpu_context *c, ornith_moe_store *s, int l, const float *w) { return 0; }

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next(void)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return rng_state;
}

static volatile unsigned sink;

static void touch(const void *p, size_t n)
{
    const unsigned char *b = (const unsigned char *)p;
    for (size_t i = 0; i < n; ++i) sink += b[i];
}

static void walk(const orn_gguf *g)
{
    sink += orn_gguf_version(g) + (unsigned)orn_gguf_tensor_count(g) +
            (unsigned)orn_gguf_metadata_count(g) + (unsigned)orn_gguf_alignment(g);
    const char *a = orn_gguf_architecture(g);
    if (a) touch(a, strlen(a));
    orn_gguf_value v;
    static const char *const keys[] = {"general.architecture", "general.alignment", "tok", "x"};
    for (int i = 0; i < 4; ++i)
        if (orn_gguf_find_metadata(g, keys[i], &v)) {
            if (v.type == 8) touch(v.value.string.data, v.value.string.len);
            if (v.type == 9 && v.value.array.elem_type == 6)
                touch(v.value.array.data, v.value.array.count * 4);
        }
    uint32_t u;
    sink += orn_gguf_get_param_u32(g, "block_count", &u);
    const uint64_t n = orn_gguf_list_tensors(g, NULL, 0);
    const orn_tensor_info **list = (const orn_tensor_info **)calloc(n ? n : 1, sizeof *list);
    const uint64_t got = orn_gguf_list_tensors(g, list, n);
    for (uint64_t i = 0; i < got; ++i) {
        const orn_tensor_info *t = list[i];
        touch(t->name, strlen(t->name));
        if (orn_gguf_find_tensor(g, t->name) == NULL) abort();
        if (t->size_bytes && t->size_bytes < (1u << 24)) {
            unsigned char *buf = (unsigned char *)malloc(t->size_bytes);
            if (orn_gguf_read_tensor_data(g, t, buf, t->size_bytes)) touch(buf, t->size_bytes);
            if (orn_gguf_read_tensor_bytes(g, t, t->size_bytes / 2, buf, t->size_bytes / 4))
                touch(buf, t->size_bytes / 4);
            free(buf);
            const void *p = orn_gguf_tensor_data_from_info(g, t);
            if (p) touch(p, t->size_bytes);
        }
    }
    free(list);
}

int main(int argc, char **argv)
{
    if (argc != 5) return 2;
    FILE *f = fopen(argv[1], "rb");
    if (!f) return 2;
    fseek(f, 0, SEEK_END);
    const long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    unsigned char *seed = (unsigned char *)malloc((size_t)len);
    if (fread(seed, 1, (size_t)len, f) != (size_t)len) return 2;
    fclose(f);
    unsigned char *b = (unsigned char *)malloc((size_t)len);
    const long iters = atol(argv[3]);
    long span = atol(argv[4]);
    if (span <= 0 || span > len) span = len;
    long opened = 0;
    char err[128];
    for (long it = 0; it < iters; ++it) {
        memcpy(b, seed, (size_t)len);
        long n = len;
        const int edits = 1 + (int)(next() % 3);
        for (int e = 0; e < edits; ++e) {
            const long pos = (long)(next() % (uint64_t)span);
            if (next() & 1) {
                b[pos] = (unsigned char)next();
            } else {
                const uint64_t v = next() >> (next() % 64);
                for (int k = 0; k < 8 && pos + k < len; ++k) b[pos + k] = (unsigned char)(v >> (8 * k));
            }
        }
        if (next() % 5 == 0) n = (long)(next() % (uint64_t)len);
        FILE *o = fopen(argv[2], "wb");
        if (!o || fwrite(b, 1, (size_t)n, o) != (size_t)n) return 2;
        fclose(o);
        orn_gguf *g = orn_gguf_open(argv[2], err, sizeof err);
        if (!g) continue;
        ++opened;
        walk(g);
        orn_gguf_close(g);
    }
    printf("opened %ld of %ld\n", opened, iters);
    free(seed);
    free(b);
    return 0;
}
