/* SPDX-License-Identifier: MIT
 *
 * GGUF container reader (C99), and the upload of a model file's MoE tensors
 * into a resident store.
 *
 * Container, as the reference parses it (engine/src/gguf.c:289-404):
 *   "GGUF" | u32 version (<= 3) | u64 tensor_count | u64 metadata_count |
 *   metadata:     (string key, u32 value_type, value)*
 *   tensor infos: (string name, u32 n_dims, u64 dims[n_dims], u32 type,
 *                  u64 offset)*
 *   data section, starting at the header's end rounded up to
 *   general.alignment (default 32) when there are tensors.
 * Strings are (u64 length, bytes); everything is little-endian.  Value types
 * 0..12: uint8, int8, uint16, int16, uint32, int32, float32, bool, string,
 * array (u32 element type, u64 count, elements), uint64, int64, float64.
 * Tensor offsets are relative to the data section; dims past n_dims read as
 * 1, n_elems is their product and size_bytes = ggml_row_size(type, n_elems).
 * Tensors are kept sorted by name and found by binary search
 * (gguf.c:378-380, 481-487).
 *
 * How this reader differs, all on inputs the reference does not parse
 * correctly: it reads the header region with pread into memory the handle
 * owns, and checks every length and count against the file size before
 * using it; it rejects n_dims > 4 (the reference keeps reading 4 dims and
 * misparses the rest) and a general.alignment that is not a power of two
 * (the reference's round-up needs one); it skips the contents of nested
 * arrays (the reference skips only their 12-byte header, gguf.c:233-234).
 * The file is also mapped read-only, only so that orn_gguf_tensor_data can
 * hand out addresses as gguf_tensor_data does; nothing here touches the
 * mapping.
 */
#define _XOPEN_SOURCE 700
#include "internal.h"

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

typedef struct {
    size_t key, key_len; /* offset of the key bytes in hdr, and their count */
    size_t data;         /* offset of a string's bytes / an array's elements */
    orn_gguf_value val;
} meta_rec;

struct orn_gguf {
    int fd;
    size_t file_size;
    const uint8_t *map;       /* read-only mapping of the file (or NULL) */
    uint8_t *hdr;             /* file bytes [0, hdr_len) read so far */
    size_t hdr_len, hdr_cap;
    uint32_t version;
    uint64_t n_tensors, n_meta;
    size_t alignment, data_offset;
    meta_rec *meta;
    orn_tensor_info *tensors; /* sorted by name */
    char **names;             /* NUL-terminated names, in file order */
    char arch[64];
    int has_arch;
};

/* ---- cursor over the file, reading the header on demand ----------------- */
typedef struct {
    orn_gguf *g;
    size_t pos;
    char *err;
    size_t err_len;
} cursor;

static int fail(cursor *c, const char *msg)
{
    if (c->err && c->err_len) snprintf(c->err, c->err_len, "%s (at byte %zu)", msg, c->pos);
    return 0;
}

static size_t pread_all(int fd, void *buf, size_t n, size_t off)
{
    size_t got = 0;
    while (got < n) {
        const ssize_t r = pread(fd, (uint8_t *)buf + got, n - got, (off_t)(off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) break;
        got += (size_t)r;
    }
    return got;
}

/* Make hdr[pos, pos + n) valid, reading more of the file when needed. */
static int need(cursor *c, size_t n)
{
    orn_gguf *g = c->g;
    if (n > g->file_size || c->pos > g->file_size - n) return fail(c, "truncated file");
    const size_t end = c->pos + n;
    if (end <= g->hdr_len) return 1;
    if (end > g->hdr_cap) {
        size_t cap = g->hdr_cap ? g->hdr_cap : 4096;
        while (cap < end) cap *= 2;
        if (cap > g->file_size) cap = g->file_size;
        uint8_t *p = (uint8_t *)realloc(g->hdr, cap);
        if (!p) return fail(c, "out of memory");
        g->hdr = p;
        g->hdr_cap = cap;
    }
    g->hdr_len += pread_all(g->fd, g->hdr + g->hdr_len, g->hdr_cap - g->hdr_len, g->hdr_len);
    if (end > g->hdr_len) return fail(c, "short read");
    return 1;
}

static int rd(cursor *c, void *out, size_t n)
{
    if (!need(c, n)) return 0;
    memcpy(out, c->g->hdr + c->pos, n);
    c->pos += n;
    return 1;
}

static int rd_str(cursor *c, size_t *off, size_t *len)
{
    uint64_t n;
    if (!rd(c, &n, 8)) return 0;
    if (n > c->g->file_size || !need(c, (size_t)n)) return fail(c, "string past the end of the file");
    *off = c->pos;
    *len = (size_t)n;
    c->pos += (size_t)n;
    return 1;
}

static size_t scalar_size(uint32_t t)
{
    switch (t) {
    case 0: case 1: case 7: return 1;    /* uint8, int8, bool */
    case 2: case 3: return 2;            /* uint16, int16 */
    case 4: case 5: case 6: return 4;    /* uint32, int32, float32 */
    case 10: case 11: case 12: return 8; /* uint64, int64, float64 */
    default: return 0;
    }
}

/* Skip `count` elements of type `et` (nested arrays with their contents). */
static int skip_elems(cursor *c, uint32_t et, uint64_t count, int depth)
{
    const size_t es = scalar_size(et);
    if (es) {
        if (count > (c->g->file_size - c->pos) / es) return fail(c, "array past the end of the file");
        c->pos += (size_t)count * es;
        return 1;
    }
    if (et != 8 && et != 9) return fail(c, "unknown array element type");
    if (et == 9 && depth > 8) return fail(c, "arrays nested too deeply");
    for (uint64_t i = 0; i < count; ++i) {
        if (et == 8) {
            size_t off, len;
            if (!rd_str(c, &off, &len)) return 0;
        } else {
            uint32_t it;
            uint64_t n;
            if (!rd(c, &it, 4) || !rd(c, &n, 8) || !skip_elems(c, it, n, depth + 1)) return 0;
        }
    }
    return 1;
}

static int rd_value(cursor *c, uint32_t t, meta_rec *m)
{
    orn_gguf_value *v = &m->val;
    memset(v, 0, sizeof *v);
    v->type = (int)t;
    const size_t sz = scalar_size(t);
    if (sz) {
        uint8_t b[8];
        if (!rd(c, b, sz)) return 0;
        switch (t) {
        case 0: v->value.uint8 = b[0]; break;
        case 1: memcpy(&v->value.int8, b, 1); break;
        case 2: memcpy(&v->value.uint16, b, 2); break;
        case 3: memcpy(&v->value.int16, b, 2); break;
        case 4: memcpy(&v->value.uint32, b, 4); break;
        case 5: memcpy(&v->value.int32, b, 4); break;
        case 6: memcpy(&v->value.float32, b, 4); break;
        case 7: v->value.boolean = b[0] != 0; break;
        case 10: memcpy(&v->value.uint64, b, 8); break;
        case 11: memcpy(&v->value.int64, b, 8); break;
        default: memcpy(&v->value.float64, b, 8); break;
        }
        return 1;
    }
    if (t == 8) {
        size_t len;
        if (!rd_str(c, &m->data, &len)) return 0;
        v->value.string.len = len;
        return 1;
    }
    if (t == 9) {
        uint32_t et;
        uint64_t count;
        if (!rd(c, &et, 4) || !rd(c, &count, 8)) return 0;
        m->data = c->pos;
        v->value.array.elem_type = (int)et;
        v->value.array.count = (size_t)count;
        if (!skip_elems(c, et, count, 0)) return 0;
        /* the elements are addressed through hdr: have them all read */
        const size_t span = c->pos - m->data;
        c->pos = m->data;
        if (!need(c, span)) return 0;
        c->pos += span;
        return 1;
    }
    return fail(c, "unknown metadata value type");
}

static int cmp_tensor(const void *a, const void *b)
{
    return strcmp(((const orn_tensor_info *)a)->name, ((const orn_tensor_info *)b)->name);
}

void orn_gguf_close(orn_gguf *g)
{
    if (!g) return;
    if (g->map) munmap((void *)g->map, g->file_size);
    if (g->fd >= 0) close(g->fd);
    if (g->names) {
        for (uint64_t i = 0; i < g->n_tensors; ++i) free(g->names[i]);
        free(g->names);
    }
    free(g->tensors);
    free(g->meta);
    free(g->hdr);
    free(g);
}

static int parse(orn_gguf *g, cursor *c)
{
    uint8_t magic[4];
    if (g->file_size < 4) return fail(c, "too small");
    if (!rd(c, magic, 4)) return 0;
    if (memcmp(magic, "GGUF", 4) != 0) return fail(c, "bad magic");
    if (!rd(c, &g->version, 4)) return 0;
    if (g->version > 3) return fail(c, "bad version");
    if (!rd(c, &g->n_tensors, 8) || !rd(c, &g->n_meta, 8)) return 0;
    /* each entry takes at least 12 bytes of the file */
    if (g->n_meta > g->file_size / 12 || g->n_tensors > g->file_size / 12)
        return fail(c, "entry count past the end of the file");
    g->alignment = 32;
    if (g->n_meta) {
        g->meta = (meta_rec *)calloc((size_t)g->n_meta, sizeof(meta_rec));
        if (!g->meta) return fail(c, "out of memory");
    }
    for (uint64_t i = 0; i < g->n_meta; ++i) {
        meta_rec *m = &g->meta[i];
        uint32_t t;
        if (!rd_str(c, &m->key, &m->key_len) || !rd(c, &t, 4) || !rd_value(c, t, m)) return 0;
    }
    if (g->n_tensors) {
        g->tensors = (orn_tensor_info *)calloc((size_t)g->n_tensors, sizeof(orn_tensor_info));
        g->names = (char **)calloc((size_t)g->n_tensors, sizeof(char *));
        if (!g->tensors || !g->names) return fail(c, "out of memory");
    }
    for (uint64_t i = 0; i < g->n_tensors; ++i) {
        orn_tensor_info *t = &g->tensors[i];
        size_t noff, nlen;
        uint32_t nd, ty;
        if (!rd_str(c, &noff, &nlen) || !rd(c, &nd, 4)) return 0;
        if (nd > 4) return fail(c, "tensor with more than 4 dimensions");
        if (!(g->names[i] = (char *)malloc(nlen + 1))) return fail(c, "out of memory");
        memcpy(g->names[i], g->hdr + noff, nlen);
        g->names[i][nlen] = '\0';
        t->name = g->names[i];
        t->n_dims = nd;
        uint64_t n = 1;
        for (uint32_t d = 0; d < 4; ++d) {
            uint64_t v = 1;
            if (d < nd && !rd(c, &v, 8)) return 0;
            if (v && n > UINT64_MAX / v) return fail(c, "tensor element count overflows");
            t->dims[d] = v;
            n *= v;
        }
        if (!rd(c, &ty, 4) || !rd(c, &t->offset, 8)) return 0;
        t->type = (int)ty;
        /* F32 / F16 byte sizes are 4n / 2n: refuse counts where that wraps
         * (the wrapped size would pass the checks against the file size) */
        if ((ty == ORN_TYPE_F32 && n > SIZE_MAX / 4) || (ty == ORN_TYPE_F16 && n > SIZE_MAX / 2))
            return fail(c, "tensor byte size overflows");
        t->n_elems = (size_t)n;
        t->size_bytes = orn_row_size((int)ty, n);
    }
    /* hdr has its final address now: point the values at it, and take the
     * two keys the reader interprets itself (gguf.c:336-352) */
    for (uint64_t i = 0; i < g->n_meta; ++i) {
        meta_rec *m = &g->meta[i];
        const char *key = (const char *)(g->hdr + m->key);
        if (m->val.type == 8) m->val.value.string.data = (const char *)(g->hdr + m->data);
        if (m->val.type == 9) m->val.value.array.data = g->hdr + m->data;
        if (m->key_len == 20 && !memcmp(key, "general.architecture", 20) && m->val.type == 8) {
            size_t n = m->val.value.string.len;
            if (n > sizeof g->arch - 1) n = sizeof g->arch - 1;
            memcpy(g->arch, m->val.value.string.data, n);
            g->arch[n] = '\0';
            g->has_arch = 1;
        }
        if (m->key_len == 17 && !memcmp(key, "general.alignment", 17) && m->val.type == 4) {
            const uint32_t a = m->val.value.uint32;
            if (a == 0 || (a & (a - 1))) return fail(c, "general.alignment is not a power of two");
            g->alignment = a;
        }
    }
    g->data_offset = g->n_tensors ? (c->pos + g->alignment - 1) & ~(g->alignment - 1) : c->pos;
    if (g->n_tensors)
        qsort(g->tensors, (size_t)g->n_tensors, sizeof(orn_tensor_info), cmp_tensor);
    return 1;
}

orn_gguf *orn_gguf_open(const char *path, char *err, size_t err_len)
{
    if (err && err_len) err[0] = '\0';
    if (!path) {
        if (err && err_len) snprintf(err, err_len, "NULL path");
        return NULL;
    }
    orn_gguf *g = (orn_gguf *)calloc(1, sizeof *g);
    if (!g) return NULL;
    g->fd = open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        if (err && err_len) snprintf(err, err_len, "cannot open %s", path);
        orn_gguf_close(g);
        return NULL;
    }
    g->file_size = (size_t)st.st_size;
    cursor c = {g, 0, err, err_len};
    if (!parse(g, &c)) {
        orn_gguf_close(g);
        return NULL;
    }
    void *p = mmap(NULL, g->file_size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    g->map = p == MAP_FAILED ? NULL : (const uint8_t *)p;
    return g;
}

uint32_t orn_gguf_version(const orn_gguf *g) { return g ? g->version : 0; }
uint64_t orn_gguf_tensor_count(const orn_gguf *g) { return g ? g->n_tensors : 0; }
uint64_t orn_gguf_metadata_count(const orn_gguf *g) { return g ? g->n_meta : 0; }
const char *orn_gguf_architecture(const orn_gguf *g) { return g && g->has_arch ? g->arch : NULL; }
size_t orn_gguf_alignment(const orn_gguf *g) { return g ? g->alignment : 32; }
size_t orn_gguf_data_offset(const orn_gguf *g) { return g ? g->data_offset : 0; }

bool orn_gguf_find_metadata(const orn_gguf *g, const char *key, orn_gguf_value *out)
{
    if (!g || !key || !out) return false;
    const size_t n = strlen(key);
    for (uint64_t i = 0; i < g->n_meta; ++i) {
        const meta_rec *m = &g->meta[i];
        if (m->key_len == n && !memcmp(g->hdr + m->key, key, n)) {
            *out = m->val;
            return true;
        }
    }
    return false;
}

bool orn_gguf_get_param_u32(const orn_gguf *g, const char *param, uint32_t *out)
{
    if (!g || !param || !out || !g->has_arch) return false;
    char key[192];
    if (snprintf(key, sizeof key, "%s.%s", g->arch, param) >= (int)sizeof key) return false;
    orn_gguf_value v;
    if (!orn_gguf_find_metadata(g, key, &v) || v.type != 4) return false;
    *out = v.value.uint32;
    return true;
}

const orn_tensor_info *orn_gguf_find_tensor(const orn_gguf *g, const char *name)
{
    if (!g || !name || !g->n_tensors) return NULL;
    orn_tensor_info k;
    memset(&k, 0, sizeof k);
    k.name = name;
    return (const orn_tensor_info *)bsearch(&k, g->tensors, (size_t)g->n_tensors,
                                            sizeof(orn_tensor_info), cmp_tensor);
}

uint64_t orn_gguf_list_tensors(const orn_gguf *g, const orn_tensor_info **out, uint64_t max)
{
    if (!g) return 0;
    if (!out) return g->n_tensors;
    const uint64_t n = g->n_tensors < max ? g->n_tensors : max;
    for (uint64_t i = 0; i < n; ++i) out[i] = &g->tensors[i];
    return n;
}

const void *orn_gguf_tensor_data_from_info(const orn_gguf *g, const orn_tensor_info *t)
{
    if (!g || !t || !g->map) return NULL;
    if (t->offset > g->file_size || g->data_offset > g->file_size - t->offset) return NULL;
    const size_t start = g->data_offset + t->offset;
    if (t->size_bytes > g->file_size - start) return NULL;
    return g->map + start;
}

const void *orn_gguf_tensor_data(const orn_gguf *g, const char *name)
{
    return orn_gguf_tensor_data_from_info(g, orn_gguf_find_tensor(g, name));
}

size_t orn_gguf_read_tensor_bytes(const orn_gguf *g, const orn_tensor_info *t, size_t byte_offset,
                                  void *buffer, size_t n)
{
    if (!g || !t || !buffer || g->fd < 0) return 0;
    if (byte_offset > t->size_bytes || n > t->size_bytes - byte_offset) return 0;
    if (t->offset > g->file_size || g->data_offset > g->file_size - t->offset) return 0;
    const size_t start = g->data_offset + t->offset + byte_offset;
    if (start > g->file_size || n > g->file_size - start) return 0;
    return pread_all(g->fd, buffer, n, start) == n ? n : 0;
}

size_t orn_gguf_read_tensor_data(const orn_gguf *g, const orn_tensor_info *t, void *buffer,
                                 size_t buffer_size)
{
    if (!t || buffer_size < t->size_bytes) return 0;
    return orn_gguf_read_tensor_bytes(g, t, 0, buffer, t->size_bytes);
}

/* gguf_dequantize_tensor / gguf_dequantize_expert_slice (gguf.c:641-648,
 * 714-722) with the tensor's bytes taken by pread rather than through the
 * mapping. */
static void *read_whole(const orn_gguf *g, const orn_tensor_info *t)
{
    if (!g || !t || !t->size_bytes) return NULL;
    void *b = malloc(t->size_bytes);
    if (b && orn_gguf_read_tensor_data(g, t, b, t->size_bytes) != t->size_bytes) {
        free(b);
        b = NULL;
    }
    return b;
}

bool gpu_dequantize_tensor_gguf(gpu_context *ctx, const orn_gguf *g, const orn_tensor_info *t,
                                float *output)
{
    if (!ctx || !output) return false;
    void *b = read_whole(g, t);
    if (!b) return false;
    const bool ok = gpu_dequantize_tensor_from_buf(ctx, b, t, output);
    free(b);
    return ok;
}

bool gpu_dequantize_expert_slice_gguf(gpu_context *ctx, const orn_gguf *g,
                                      const orn_tensor_info *t, int expert_idx, float *output)
{
    if (!ctx || !output) return false;
    void *b = read_whole(g, t);
    if (!b) return false;
    const bool ok = gpu_dequantize_expert_slice_from_buf(ctx, b, t, expert_idx, output);
    free(b);
    return ok;
}

/* ---------------------------------------------------------------------------
 * A model file's MoE tensors -> a file-orientation store
 * ------------------------------------------------------------------------- */
#define LOAD_CHUNK_EXPERTS 32 /* host staging: 32 experts of one matrix at a time */

/* The tensor blk.<l>.<suffix>, checked for type and dims (unused dims 1). */
static const orn_tensor_info *layer_tensor(gpu_context *ctx, const orn_gguf *g, int l,
                                           const char *suffix, int type, uint64_t d0,
                                           uint64_t d1, uint64_t d2, int *rc)
{
    char name[128];
    snprintf(name, sizeof name, "blk.%d.%s", l, suffix);
    const orn_tensor_info *t = orn_gguf_find_tensor(g, name);
    if (!t) {
        *rc = orn_set_err(ctx, ORN_EINVAL, "load_gguf: tensor %s not in the file", name);
        return NULL;
    }
    const uint64_t w[4] = {d0, d1, d2, 1};
    int ok = t->type == type;
    for (int i = 0; i < 4; ++i) ok = ok && t->dims[i] == w[i];
    if (!ok) {
        *rc = orn_set_err(ctx, ORN_EUNSUPPORTED,
                          "load_gguf: %s is type %d ne [%llu %llu %llu %llu]; this store takes "
                          "type %d ne [%llu %llu %llu]",
                          name, t->type, (unsigned long long)t->dims[0],
                          (unsigned long long)t->dims[1], (unsigned long long)t->dims[2],
                          (unsigned long long)t->dims[3], type, (unsigned long long)d0,
                          (unsigned long long)d1, (unsigned long long)d2);
        return NULL;
    }
    return t;
}

int gpu_moe_store_load_gguf(gpu_context *ctx, ornith_moe_store *st, const orn_gguf *g,
                            int file_first_layer, int store_first_layer, int n_layers)
{
    if (!ctx) return ORN_EINVAL;
    if (!st || !g || n_layers < 0 || file_first_layer < 0 || store_first_layer < 0)
        return orn_set_err(ctx, ORN_EINVAL, "load_gguf: bad arguments");
    const ornith_moe_shape *sh = orn_store_shape(st);
    if (!sh->file_layout)
        return orn_set_err(ctx, ORN_EUNSUPPORTED,
                           "load_gguf: a model file's expert tensors need a store created with "
                           "file_layout = 1");
    if (n_layers > sh->n_layers - store_first_layer)
        return orn_set_err(ctx, ORN_EINVAL, "load_gguf: layers past the end of the store");
    const uint64_t D = (uint64_t)sh->d_model, H = (uint64_t)sh->hidden,
                   E = (uint64_t)sh->n_experts;
    size_t stage = (size_t)(D * H / ORN_QK_K) * ORN_Q6K_BYTES * LOAD_CHUNK_EXPERTS;
    if (stage < (size_t)(D * E) * sizeof(float)) stage = (size_t)(D * E) * sizeof(float);
    uint8_t *buf = (uint8_t *)malloc(stage);
    float *fb = (float *)malloc((size_t)(D * E) * sizeof(float));
    if (!buf || !fb) {
        free(buf);
        free(fb);
        return orn_set_err(ctx, ORN_ENOMEM, "load_gguf: host staging");
    }
    /* routed experts: ne = [K, M, E], input index fastest, experts slowest
     * (names: model.c:707-711); shared expert: ne = [K, M] (model.c:847-852) */
    static const char *const exps[3] = {"ffn_gate_exps.weight", "ffn_up_exps.weight",
                                        "ffn_down_exps.weight"};
    static const char *const shexp[3] = {"ffn_gate_shexp.weight", "ffn_up_shexp.weight",
                                         "ffn_down_shexp.weight"};
    int rc = ORN_OK;
    for (int i = 0; i < n_layers && rc == ORN_OK; ++i) {
        const int fl = file_first_layer + i, sl = store_first_layer + i;
        for (int m = 0; m < 3 && rc == ORN_OK; ++m) {
            const int ty = m == ORN_MAT_DOWN ? ORN_TYPE_Q6_K : ORN_TYPE_Q4_K;
            const uint64_t K = m == ORN_MAT_DOWN ? H : D, M = m == ORN_MAT_DOWN ? D : H;
            const orn_tensor_info *t = layer_tensor(ctx, g, fl, exps[m], ty, K, M, E, &rc);
            if (!t) break;
            const size_t bpe = t->size_bytes / (size_t)E;
            for (uint64_t e0 = 0; e0 < E && rc == ORN_OK; e0 += LOAD_CHUNK_EXPERTS) {
                const int n = (int)(E - e0 < LOAD_CHUNK_EXPERTS ? E - e0 : LOAD_CHUNK_EXPERTS);
                if (orn_gguf_read_tensor_bytes(g, t, (size_t)e0 * bpe, buf, (size_t)n * bpe) !=
                    (size_t)n * bpe) {
                    rc = orn_set_err(ctx, ORN_EINVAL, "load_gguf: reading %s failed", t->name);
                    break;
                }
                rc = gpu_moe_store_set_experts(ctx, st, sl, m, (int)e0, n, buf);
            }
            if (rc || !sh->has_shared) continue;
            if (!(t = layer_tensor(ctx, g, fl, shexp[m], ty, K, M, 1, &rc))) break;
            if (orn_gguf_read_tensor_data(g, t, buf, stage) != t->size_bytes) {
                rc = orn_set_err(ctx, ORN_EINVAL, "load_gguf: reading %s failed", t->name);
                break;
            }
            rc = gpu_moe_store_set_experts(ctx, st, sl, m, (int)E, 1, buf);
        }
        if (rc) break;
        /* router ffn_gate_inp.weight, ne = [D, E]: W[e*D + d]; f32, or f16
         * decoded with the reference's rule (gguf.c:16-26) */
        char name[128];
        snprintf(name, sizeof name, "blk.%d.ffn_gate_inp.weight", fl);
        const orn_tensor_info *t = orn_gguf_find_tensor(g, name);
        const int rtype = t && t->type == ORN_TYPE_F16 ? ORN_TYPE_F16 : ORN_TYPE_F32;
        if (!(t = layer_tensor(ctx, g, fl, "ffn_gate_inp.weight", rtype, D, E, 1, &rc))) break;
        if (orn_gguf_read_tensor_data(g, t, buf, stage) != t->size_bytes) {
            rc = orn_set_err(ctx, ORN_EINVAL, "load_gguf: reading %s failed", name);
            break;
        }
        if (t->type == ORN_TYPE_F32) {
            memcpy(fb, buf, (size_t)(D * E) * sizeof(float));
        } else {
            for (uint64_t j = 0; j < D * E; ++j)
                fb[j] = orn_quirk_half((uint16_t)(buf[2 * j] | (buf[2 * j + 1] << 8)));
        }
        if ((rc = gpu_moe_store_set_router(ctx, st, sl, fb, NULL))) break;
        /* the rmsnorm weights in front of the MoE block (model.c:807, 996),
         * when the file has them */
        snprintf(name, sizeof name, "blk.%d.post_attention_norm.weight", fl);
        if ((t = orn_gguf_find_tensor(g, name))) {
            if (t->type != ORN_TYPE_F32 || t->n_elems != D ||
                orn_gguf_read_tensor_data(g, t, fb, (size_t)(D * E) * sizeof(float)) !=
                    t->size_bytes) {
                rc = orn_set_err(ctx, ORN_EUNSUPPORTED, "load_gguf: %s is not %llu f32", name,
                                 (unsigned long long)D);
                break;
            }
            rc = gpu_moe_store_set_norm(ctx, st, sl, fb);
            if (rc) break;
        }
        /* the shared-expert gate (Qwen-MoE files; the reference ignores it),
         * when the file has it: applied under ORN_MOE_SHEXP_GATE */
        snprintf(name, sizeof name, "blk.%d.ffn_gate_inp_shexp.weight", fl);
        if (sh->has_shared && (t = orn_gguf_find_tensor(g, name))) {
            if ((t->type != ORN_TYPE_F32 && t->type != ORN_TYPE_F16) || t->n_elems != D ||
                orn_gguf_read_tensor_data(g, t, buf, stage) != t->size_bytes) {
                rc = orn_set_err(ctx, ORN_EUNSUPPORTED, "load_gguf: %s is not %llu f32/f16", name,
                                 (unsigned long long)D);
                break;
            }
            if (t->type == ORN_TYPE_F32) {
                memcpy(fb, buf, (size_t)D * sizeof(float));
            } else {
                for (uint64_t j = 0; j < D; ++j)
                    fb[j] = orn_quirk_half((uint16_t)(buf[2 * j] | (buf[2 * j + 1] << 8)));
            }
            if ((rc = gpu_moe_store_set_shexp_gate(ctx, st, sl, fb))) break;
        }
    }
    free(buf);
    free(fb);
    return rc;
}
