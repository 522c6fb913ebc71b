/* SPDX-License-Identifier: MIT
 *
 * Resident routed-MoE layers and the per-layer forward (C99 host side).
 *
 * The forward replaces model.c:992-1144 for a batch of tokens:
 *   norm -> exact router logits + top-k -> dispatch -> gate/up -> mid ->
 *   down -> combine,
 * all enqueued on the context's stream; no host round trip between steps.
 */
#include "internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* A forward call as a HIP graph: everything the captured kernel arguments
 * depend on is in the key (buffers by address, the workspace base). */
#define ORN_GRAPH_SLOTS 32
typedef struct {
    int layer, n_layers, T, mode, ep_first, ep_count;
    unsigned flags;
    const void *x, *resid, *out, *idx, *w;
    void *ws;
} orn_graph_key;

typedef struct {
    int used;
    orn_graph_key key;
    hipGraphExec_t exec;
    int *ctl; /* the call's device counters (for gpu_moe_last_stats) */
    float *logits; /* and its last layer's router logits (gpu_moe_last_logits) */
    int lT, lE;
    unsigned long long tick;
} orn_graph;

struct ornith_moe_store {
    ornith_moe_shape sh;
    size_t blocks_per_matrix; /* D*H/256 */
    uint8_t *gate, *up;       /* [L][E+1][H/256][D] * 144 B */
    uint8_t *down_body;       /* [L][E+1][D/256][H] * 208 B */
    uint16_t *down_d;         /* [L][E+1][D/256][H] */
    float *router_q;          /* [L][D/4][E][4]: W(d, e) at ((d/4)*E + e)*4 + d%4 */
    float *bias;              /* [L][E] */
    int *has_bias;            /* host [L] */
    float *norm;              /* [L][D] */
    float *shexp_gate;        /* [L][D] shared-expert gate vectors */
    unsigned char *has_shexp_gate; /* host [L] */
    /* Prefill (MFMA) layouts, present when sh.prefill_layout is set (built
     * by prefill_pack.c; per layer and expert slot):
     *   pq[m]  gate/up nibbles [D/32][H/256][4][64][4] u32   (D*H/2 bytes)
     *   psc[m] sub-block scales [D/32][H/256][8][32] fp16      (D*H/16)
     *   pmn[m] sub-block mins, same shape                       (D*H/16)
     *   pd[m], pdm[m]  d and dmin [H/256][D] fp32               (D*H/64 each)
     *   dq     down q + 32, 6-bit [H/32][D/256] x ORNK_DQ_UNIT   (D*H*3/4)
     *   dsc    down sub-block scales [H/32][D/256][16][32] fp16   (D*H/8)
     *   dd     down d [D/256][H] fp32                             (D*H/64)
     *   dmax   [3]: max |d|,|dmin| of gate and of up, max |d| of down */
    uint32_t *pq[2];
    uint16_t *psc[2], *pmn[2];
    float *pd[2], *pdm[2];
    uint8_t *dq;
    uint16_t *dsc;
    float *dd;
    float *dmax;
    float *dmax_host;         /* host mirror of dmax, [L][E+1][3] */
    int *q6_scmax;            /* host [L]: largest |Q6_K sub-scale| uploaded */
    int *dev_scmax;           /* device [1]: the same, computed by the device packer */
    size_t bytes;
    /* shape.cache_slots > 0: the experts live in this cache's host tier and
     * device slots; gate/up/down_body/down_d and the prefill arrays above
     * are then unused (NULL) */
    orn_cache *cache;
    /* HIP graphs of earlier calls made with ORN_MOE_GRAPH (least recently
     * used replaced first); any upload to the store drops them all. */
    orn_graph graphs[ORN_GRAPH_SLOTS];
    unsigned long long graph_tick;
};

/* prefill_pack.c */
void orn_pack_q4k_prefill(const uint8_t *blocks, int K, int M, uint32_t *qn, uint16_t *sc,
                          uint16_t *mn, float *d, float *dm, float *dmax);
int orn_pack_q6k_prefill(const uint8_t *blocks, int K, int M, uint8_t *qb, uint16_t *sc, float *d,
                         float *dmax);

/* ---------------------------------------------------------------------------
 * Workspace (grow-only device scratch owned by the context)
 * ------------------------------------------------------------------------- */
void *orn_ws_get(gpu_context *ctx, size_t bytes)
{
    if (bytes <= ctx->ws.bytes) return ctx->ws.base;
    hipStreamSynchronize(ctx->stream);
    if (ctx->ws.base) hipFree(ctx->ws.base);
    ctx->ws.base = NULL;
    ctx->ws.bytes = 0;
    ctx->last_ctl = NULL;
    ctx->last_logits = NULL;
    size_t want = bytes + (bytes >> 3);
    if (hipMalloc(&ctx->ws.base, want) != hipSuccess) {
        orn_set_err(ctx, ORN_ENOMEM, "workspace allocation of %zu bytes failed", want);
        ctx->ws.base = NULL;
        return NULL;
    }
    ctx->ws.bytes = want;
    return ctx->ws.base;
}

/* The certified routing kernel's counter area: allocated on first use and
 * zeroed by a fill kernel on the context's stream (ordered before the
 * kernels that use it; a null-stream memset would not be). */
static int *ctx_sync(gpu_context *ctx)
{
    if (ctx->sync) return ctx->sync;
    void *p = NULL;
    if (hipMalloc(&p, ORNK_SYNC_BYTES) != hipSuccess) {
        orn_set_err(ctx, ORN_ENOMEM, "allocation of the routing counters failed");
        return NULL;
    }
    if (ornk_fill_f32((float *)p, 0.0f, ORNK_SYNC_BYTES / 4, ctx->stream) != hipSuccess) {
        hipFree(p);
        orn_set_err(ctx, ORN_EHIP, "routing counter initialisation failed");
        return NULL;
    }
    ctx->sync = (int *)p;
    return ctx->sync;
}

void orn_ws_release(gpu_context *ctx)
{
    if (ctx->ws.base) hipFree(ctx->ws.base);
    ctx->ws.base = NULL;
    ctx->ws.bytes = 0;
}

/* ---------------------------------------------------------------------------
 * Profiling: HIP events around each launch on the context's stream
 * ------------------------------------------------------------------------- */
static void prof_collect(gpu_context *ctx)
{
    if (!ctx->prof_n_pending) return;
    hipStreamSynchronize(ctx->stream);
    for (int i = 0; i < ctx->prof_n_pending; ++i) {
        orn_prof_rec *r = &ctx->prof_pending[i];
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r->start, r->stop) == hipSuccess) {
            ctx->prof_total_ms[r->name_id] += ms;
            ctx->prof_calls[r->name_id] += 1;
        }
    }
    ctx->prof_n_pending = 0;
    ctx->prof_pool_used = 0;
}

int gpu_profile_enable(gpu_context *ctx, int on)
{
    if (!ctx) return ORN_EINVAL;
    if (on && !ctx->prof_pool) {
        ctx->prof_pool_n = 2 * ORN_PROF_MAX_PENDING;
        ctx->prof_pool = (hipEvent_t *)calloc((size_t)ctx->prof_pool_n, sizeof(hipEvent_t));
        ctx->prof_pending = (orn_prof_rec *)calloc(ORN_PROF_MAX_PENDING, sizeof(orn_prof_rec));
        if (!ctx->prof_pool || !ctx->prof_pending) return ORN_ENOMEM;
        for (int i = 0; i < ctx->prof_pool_n; ++i)
            if (hipEventCreate(&ctx->prof_pool[i]) != hipSuccess) return ORN_EHIP;
    }
    if (!on && ctx->prof_pool) {
        prof_collect(ctx);
        for (int i = 0; i < ctx->prof_pool_n; ++i) hipEventDestroy(ctx->prof_pool[i]);
        free(ctx->prof_pool);
        free(ctx->prof_pending);
        ctx->prof_pool = NULL;
        ctx->prof_pending = NULL;
        ctx->prof_pool_n = 0;
    }
    ctx->prof_on = on ? 1 : 0;
    return ORN_OK;
}

void gpu_profile_reset(gpu_context *ctx)
{
    if (!ctx) return;
    prof_collect(ctx);
    for (int i = 0; i < ORN_PROF_MAX_NAMES; ++i) {
        ctx->prof_total_ms[i] = 0.0;
        ctx->prof_calls[i] = 0;
    }
}

int gpu_profile_count(gpu_context *ctx)
{
    if (!ctx) return 0;
    prof_collect(ctx);
    return ctx->prof_n_names;
}

const char *gpu_profile_name(gpu_context *ctx, int i)
{
    return (ctx && i >= 0 && i < ctx->prof_n_names) ? ctx->prof_names[i] : "";
}

double gpu_profile_total_ms(gpu_context *ctx, int i)
{
    if (!ctx || i < 0 || i >= ctx->prof_n_names) return 0.0;
    prof_collect(ctx);
    return ctx->prof_total_ms[i];
}

long gpu_profile_calls(gpu_context *ctx, int i)
{
    if (!ctx || i < 0 || i >= ctx->prof_n_names) return 0;
    prof_collect(ctx);
    return ctx->prof_calls[i];
}

int orn_prof_begin(gpu_context *ctx, const char *name)
{
    if (!ctx->prof_on) return -1;
    if (ctx->prof_n_pending >= ORN_PROF_MAX_PENDING || ctx->prof_pool_used + 2 > ctx->prof_pool_n)
        prof_collect(ctx);
    int id = -1;
    for (int i = 0; i < ctx->prof_n_names; ++i)
        if (strcmp(ctx->prof_names[i], name) == 0) { id = i; break; }
    if (id < 0) {
        if (ctx->prof_n_names >= ORN_PROF_MAX_NAMES) return -1;
        id = ctx->prof_n_names++;
        snprintf(ctx->prof_names[id], sizeof ctx->prof_names[id], "%s", name);
    }
    orn_prof_rec *r = &ctx->prof_pending[ctx->prof_n_pending];
    r->name_id = id;
    r->start = ctx->prof_pool[ctx->prof_pool_used++];
    r->stop = ctx->prof_pool[ctx->prof_pool_used++];
    hipEventRecord(r->start, ctx->stream);
    return ctx->prof_n_pending++;
}

void orn_prof_end(gpu_context *ctx, int slot)
{
    if (slot < 0) return;
    hipEventRecord(ctx->prof_pending[slot].stop, ctx->stream);
}

/* A record whose events the caller hands to hipExtLaunchKernel (which stamps
 * a kernel's own start and end into them) instead of recording them around
 * the launch; *start = *stop = NULL when profiling is off. */
int orn_prof_kernel(gpu_context *ctx, const char *name, hipEvent_t *start, hipEvent_t *stop)
{
    *start = *stop = NULL;
    if (!ctx->prof_on) return -1;
    if (ctx->prof_n_pending >= ORN_PROF_MAX_PENDING || ctx->prof_pool_used + 2 > ctx->prof_pool_n)
        prof_collect(ctx);
    int id = -1;
    for (int i = 0; i < ctx->prof_n_names; ++i)
        if (strcmp(ctx->prof_names[i], name) == 0) { id = i; break; }
    if (id < 0) {
        if (ctx->prof_n_names >= ORN_PROF_MAX_NAMES) return -1;
        id = ctx->prof_n_names++;
        snprintf(ctx->prof_names[id], sizeof ctx->prof_names[id], "%s", name);
    }
    orn_prof_rec *r = &ctx->prof_pending[ctx->prof_n_pending];
    r->name_id = id;
    r->start = *start = ctx->prof_pool[ctx->prof_pool_used++];
    r->stop = *stop = ctx->prof_pool[ctx->prof_pool_used++];
    return ctx->prof_n_pending++;
}

/* ---------------------------------------------------------------------------
 * Store
 * ------------------------------------------------------------------------- */
/* The matvec kernels spread a wave's 64 lanes over 8 lanes per 256-wide
 * block: D / 256 and H / 256 must divide 64 (powers of two), or D / 256 be a
 * multiple of 8 (whole column groups). */
static int widths_ok(int D, int H)
{
    const int nd = D / 256, nh = H / 256;
    return D > 0 && D % 256 == 0 && ((nd & (nd - 1)) == 0 || nd % 8 == 0) && H > 0 &&
           H % 256 == 0 && H <= 1024 && (nh & (nh - 1)) == 0;
}

static int shape_ok(const ornith_moe_shape *s)
{
    return s && s->n_layers > 0 && widths_ok(s->d_model, s->hidden) && s->n_experts > 0 &&
           s->n_experts <= 256 && s->top_k > 0 && s->top_k <= 16 && s->top_k <= s->n_experts &&
           (s->has_shared == 0 || s->has_shared == 1) && s->d_model % 128 == 0 &&
           (s->prefill_layout >= 0 && s->prefill_layout <= 2) &&
           (s->prefill_layout != 2 || s->cache_slots == 0) &&
           (s->file_layout == 0 || (s->file_layout == 1 && !s->prefill_layout &&
                                    ornk_file_supported(s->d_model, s->hidden))) &&
           s->cache_slots >= 0;
}

static void graphs_clear(ornith_moe_store *st)
{
    for (int i = 0; i < ORN_GRAPH_SLOTS; ++i) {
        if (st->graphs[i].used) hipGraphExecDestroy(st->graphs[i].exec);
        st->graphs[i].used = 0;
    }
}

static void store_free(ornith_moe_store *st)
{
    if (!st) return;
    graphs_clear(st);
    hipFree(st->gate);
    hipFree(st->up);
    hipFree(st->down_body);
    hipFree(st->down_d);
    hipFree(st->router_q);
    hipFree(st->bias);
    hipFree(st->norm);
    hipFree(st->shexp_gate);
    free(st->has_shexp_gate);
    for (int m = 0; m < 2; ++m) {
        hipFree(st->pq[m]);
        hipFree(st->psc[m]);
        hipFree(st->pmn[m]);
        hipFree(st->pd[m]);
        hipFree(st->pdm[m]);
    }
    hipFree(st->dq);
    hipFree(st->dsc);
    hipFree(st->dd);
    hipFree(st->dmax);
    hipFree(st->dev_scmax);
    orn_cache_destroy(st->cache);
    free(st->dmax_host);
    free(st->q6_scmax);
    free(st->has_bias);
    free(st);
}

ornith_moe_store *gpu_moe_store_create(gpu_context *ctx, const ornith_moe_shape *shape)
{
    if (!ctx) return NULL;
    if (!shape_ok(shape)) {
        orn_set_err(ctx, ORN_EINVAL, "unsupported MoE shape");
        return NULL;
    }
    ornith_moe_store *st = (ornith_moe_store *)calloc(1, sizeof *st);
    if (!st) return NULL;
    st->sh = *shape;
    const size_t L = (size_t)shape->n_layers, E1 = (size_t)shape->n_experts + 1;
    const size_t D = (size_t)shape->d_model, H = (size_t)shape->hidden,
                 E = (size_t)shape->n_experts;
    st->blocks_per_matrix = D * H / 256;
    const size_t nb = L * E1 * st->blocks_per_matrix;
    size_t sizes[8] = {nb * 144, nb * 144, nb * 208, nb * 2, L * E * D * 4, L * E * 4, L * D * 4,
                       L * D * 4};
    void **ptrs[8] = {(void **)&st->gate, (void **)&st->up, (void **)&st->down_body,
                      (void **)&st->down_d, (void **)&st->router_q, (void **)&st->bias,
                      (void **)&st->norm, (void **)&st->shexp_gate};
    const int cached = shape->cache_slots > 0;
    /* prefill_layout = 2: the experts live in the MFMA layouts alone (the
     * GGUF blocks are packed as they arrive and not kept) */
    const int lean = shape->prefill_layout == 2;
    st->has_shexp_gate = (unsigned char *)calloc(L, 1);
    if (!st->has_shexp_gate) {
        orn_set_err(ctx, ORN_ENOMEM, "store tables");
        store_free(st);
        return NULL;
    }
    for (int i = cached || lean ? 4 : 0; i < 8; ++i) {
        if (hipMalloc(ptrs[i], sizes[i]) != hipSuccess ||
            hipMemsetAsync(*ptrs[i], 0, sizes[i], ctx->stream) != hipSuccess) {
            orn_set_err(ctx, ORN_ENOMEM, "store allocation of %zu bytes failed", sizes[i]);
            store_free(st);
            return NULL;
        }
        st->bytes += sizes[i];
    }
    if (cached) {
        st->cache = orn_cache_create(ctx, shape);
        st->q6_scmax = (int *)calloc(L, sizeof(int));
        if (!st->cache || !st->q6_scmax) {
            if (st->cache) orn_set_err(ctx, ORN_ENOMEM, "store allocation failed");
            store_free(st);
            return NULL;
        }
        st->bytes += orn_cache_device_bytes(st->cache);
    } else if (shape->prefill_layout) {
        const size_t LE = L * E1, DH = D * H;
        size_t psz[14] = {LE * DH / 2, LE * DH / 2, LE * DH / 16, LE * DH / 16, LE * DH / 16,
                          LE * DH / 16, LE * DH / 64, LE * DH / 64, LE * DH / 64, LE * DH / 64,
                          LE * ORNK_DQ_BYTES(DH), LE * DH / 8, LE * DH / 64,
                          LE * 3 * sizeof(float)};
        void **pp[14] = {(void **)&st->pq[0], (void **)&st->pq[1], (void **)&st->psc[0],
                         (void **)&st->psc[1], (void **)&st->pmn[0], (void **)&st->pmn[1],
                         (void **)&st->pd[0], (void **)&st->pd[1], (void **)&st->pdm[0],
                         (void **)&st->pdm[1], (void **)&st->dq, (void **)&st->dsc,
                         (void **)&st->dd, (void **)&st->dmax};
        for (int i = 0; i < 14; ++i) {
            if (hipMalloc(pp[i], psz[i]) != hipSuccess ||
                hipMemsetAsync(*pp[i], 0, psz[i], ctx->stream) != hipSuccess) {
                orn_set_err(ctx, ORN_ENOMEM, "store allocation of %zu bytes failed", psz[i]);
                store_free(st);
                return NULL;
            }
            st->bytes += psz[i];
        }
        st->dmax_host = (float *)calloc(LE * 3, sizeof(float));
        st->q6_scmax = (int *)calloc(L, sizeof(int));
        if (hipMalloc((void **)&st->dev_scmax, sizeof(int)) != hipSuccess) st->dev_scmax = NULL;
        if (!st->dmax_host || !st->q6_scmax || !st->dev_scmax) {
            store_free(st);
            return NULL;
        }
    }
    st->has_bias = (int *)calloc(L, sizeof(int));
    float *ones = (float *)malloc(D * sizeof(float));
    if (!st->has_bias || !ones) {
        free(ones);
        store_free(st);
        return NULL;
    }
    for (size_t i = 0; i < D; ++i) ones[i] = 1.0f;
    for (size_t l = 0; l < L; ++l)
        hipMemcpyAsync(st->norm + l * D, ones, D * sizeof(float), hipMemcpyHostToDevice,
                       ctx->stream);
    hipStreamSynchronize(ctx->stream);
    free(ones);
    return st;
}

void gpu_moe_store_destroy(gpu_context *ctx, ornith_moe_store *store)
{
    if (ctx) hipStreamSynchronize(ctx->stream);
    store_free(store);
}

size_t gpu_moe_store_bytes(const ornith_moe_store *store) { return store ? store->bytes : 0; }

const ornith_moe_shape *orn_store_shape(const ornith_moe_store *st) { return &st->sh; }

/* Where the experts' decode-layout blocks live: the device arrays of a
 * resident store, or the host tier of a streamed one (same [L][E+1]
 * layout; copies to and from either use hipMemcpyDefault). */
static void expert_arrays(ornith_moe_store *st, uint8_t **g, uint8_t **u, uint8_t **b,
                          uint16_t **d)
{
    if (st->cache) {
        orn_cache_host_tier(st->cache, g, u, b, d);
        return;
    }
    *g = st->gate;
    *u = st->up;
    *b = st->down_body;
    *d = st->down_d;
}

/* Largest |Q6_K sub-scale| of n experts' down bodies (208-byte bodies, the
 * 16 int8 scales at offset 192). */
static int q6_scmax_of(const uint8_t *body, size_t n_bodies)
{
    int mx = 0;
    for (size_t i = 0; i < n_bodies; ++i)
        for (int j = 0; j < 16; ++j) {
            const int v = (int8_t)body[i * 208 + 192 + j];
            if (v > mx) mx = v;
            if (-v > mx) mx = -v;
        }
    return mx;
}

/* Permute one expert's GGUF block stream (row-major: block (k, c) at
 * k*NBc + c) into the device's block-column-major order (c*K + k). */
static void permute_q4k(const uint8_t *src, uint8_t *dst, int K, int NBc)
{
    for (int k = 0; k < K; ++k)
        for (int c = 0; c < NBc; ++c)
            memcpy(dst + ((size_t)c * K + k) * 144, src + ((size_t)k * NBc + c) * 144, 144);
}

static void permute_q6k(const uint8_t *src, uint8_t *body, uint16_t *dv, int K, int NBc)
{
    for (int k = 0; k < K; ++k)
        for (int c = 0; c < NBc; ++c) {
            const uint8_t *b = src + ((size_t)k * NBc + c) * ORN_Q6K_BYTES;
            const size_t o = (size_t)c * K + k;
            memcpy(body + o * 208, b, 208);
            dv[o] = (uint16_t)(b[ORN_Q6K_OFF_D] | (b[ORN_Q6K_OFF_D + 1] << 8));
        }
}

/* Pack and upload the prefill layouts of n experts (one matrix). */
static int upload_q4k_prefill(gpu_context *ctx, ornith_moe_store *st, int layer, int matrix,
                              int first, int n, const void *blocks)
{
    const size_t D = (size_t)st->sh.d_model, H = (size_t)st->sh.hidden, DH = D * H;
    const size_t E1 = (size_t)st->sh.n_experts + 1, nb = st->blocks_per_matrix;
    const int m = matrix == ORN_MAT_GATE ? 0 : 1;
    uint32_t *qn = (uint32_t *)malloc(DH / 2);
    uint16_t *sc = (uint16_t *)malloc(DH / 16), *mn = (uint16_t *)malloc(DH / 16);
    float *d = (float *)malloc(DH / 64), *dm = (float *)malloc(DH / 64);
    int rc = ORN_OK;
    if (!qn || !sc || !mn || !d || !dm) rc = orn_set_err(ctx, ORN_ENOMEM, "host staging");
    hipStream_t s = ctx->stream;
    for (int i = 0; i < n && !rc; ++i) {
        const size_t slot = (size_t)layer * E1 + (size_t)(first + i);
        float dmax;
        orn_pack_q4k_prefill((const uint8_t *)blocks + (size_t)i * nb * ORN_Q4K_BYTES, (int)D,
                             (int)H, qn, sc, mn, d, dm, &dmax);
        st->dmax_host[slot * 3 + m] = dmax;
        rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->pq[m] + slot * (DH / 2), qn, DH / 2,
                                               hipMemcpyHostToDevice, s), "upload prefill q4k");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->psc[m] + slot * (DH / 16), sc,
                                                   DH / 16, hipMemcpyHostToDevice, s), "upload sc");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->pmn[m] + slot * (DH / 16), mn,
                                                   DH / 16, hipMemcpyHostToDevice, s), "upload mn");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->pd[m] + slot * (DH / 64), d,
                                                   DH / 64, hipMemcpyHostToDevice, s), "upload d");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->pdm[m] + slot * (DH / 64), dm,
                                                   DH / 64, hipMemcpyHostToDevice, s), "upload dm");
        hipStreamSynchronize(s);
    }
    if (!rc) {
        const size_t slot0 = (size_t)layer * E1 + (size_t)first;
        rc = orn_hip_check(ctx, hipMemcpyAsync(st->dmax + slot0 * 3, st->dmax_host + slot0 * 3,
                                               (size_t)n * 3 * sizeof(float),
                                               hipMemcpyHostToDevice, s), "upload dmax");
        hipStreamSynchronize(s);
    }
    free(qn);
    free(sc);
    free(mn);
    free(d);
    free(dm);
    return rc;
}

static int upload_q6k_prefill(gpu_context *ctx, ornith_moe_store *st, int layer, int first, int n,
                              const void *blocks)
{
    const size_t D = (size_t)st->sh.d_model, H = (size_t)st->sh.hidden, DH = D * H;
    const size_t E1 = (size_t)st->sh.n_experts + 1, nb = st->blocks_per_matrix;
    uint8_t *qb = (uint8_t *)malloc(ORNK_DQ_BYTES(DH));
    uint16_t *sc = (uint16_t *)malloc(DH / 8);
    float *d = (float *)malloc(DH / 64);
    int rc = ORN_OK;
    if (!qb || !sc || !d) rc = orn_set_err(ctx, ORN_ENOMEM, "host staging");
    hipStream_t s = ctx->stream;
    for (int i = 0; i < n && !rc; ++i) {
        const size_t slot = (size_t)layer * E1 + (size_t)(first + i);
        float dmax;
        const int scmax = orn_pack_q6k_prefill((const uint8_t *)blocks +
                                                   (size_t)i * nb * ORN_Q6K_BYTES,
                                               (int)H, (int)D, qb, sc, d, &dmax);
        if (scmax > st->q6_scmax[layer]) st->q6_scmax[layer] = scmax;
        st->dmax_host[slot * 3 + 2] = dmax;
        rc = orn_hip_check(ctx, hipMemcpyAsync(st->dq + slot * ORNK_DQ_BYTES(DH), qb,
                                               ORNK_DQ_BYTES(DH), hipMemcpyHostToDevice, s),
                           "upload prefill q6k");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->dsc + slot * (DH / 8), sc, DH / 8,
                                                   hipMemcpyHostToDevice, s), "upload q6k sc");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync((uint8_t *)st->dd + slot * (DH / 64), d, DH / 64,
                                                   hipMemcpyHostToDevice, s), "upload q6k d");
        hipStreamSynchronize(s);
    }
    if (!rc) {
        const size_t slot0 = (size_t)layer * E1 + (size_t)first;
        rc = orn_hip_check(ctx, hipMemcpyAsync(st->dmax + slot0 * 3, st->dmax_host + slot0 * 3,
                                               (size_t)n * 3 * sizeof(float),
                                               hipMemcpyHostToDevice, s), "upload dmax");
        hipStreamSynchronize(s);
    }
    free(qb);
    free(sc);
    free(d);
    return rc;
}

int gpu_moe_store_set_experts(gpu_context *ctx, ornith_moe_store *st, int layer, int matrix,
                              int expert_first, int n, const void *blocks)
{
    if (!ctx || !st || !blocks) return ORN_EINVAL;
    const int E1 = st->sh.n_experts + 1;
    if (layer < 0 || layer >= st->sh.n_layers || expert_first < 0 || n < 0 ||
        expert_first + n > E1 || matrix < 0 || matrix > 2)
        return orn_set_err(ctx, ORN_EINVAL, "set_experts: bad layer/expert range/matrix");
    if (n == 0) return ORN_OK;
    graphs_clear(st);  /* the path choice depends on the uploaded scales */
    const int D = st->sh.d_model, H = st->sh.hidden;
    const size_t nb = st->blocks_per_matrix;
    const size_t slot0 = (size_t)layer * E1 + (size_t)expert_first;
    hipStream_t s = ctx->stream;
    int rc = ORN_OK;
    uint8_t *a_gate, *a_up, *a_body;
    uint16_t *a_d;
    expert_arrays(st, &a_gate, &a_up, &a_body, &a_d);
    if (st->cache) {  /* the host tier is rewritten: no copy may read it now */
        if ((rc = orn_cache_quiesce(ctx, st->cache))) return rc;
        if ((rc = orn_hip_check(ctx, hipStreamSynchronize(s), "set_experts"))) return rc;
        orn_cache_invalidate(st->cache, layer, expert_first, n);
    }
    if (st->sh.prefill_layout == 2) {  /* no GGUF copy: packed from the host blocks */
        rc = matrix != ORN_MAT_DOWN
                 ? upload_q4k_prefill(ctx, st, layer, matrix, expert_first, n, blocks)
                 : upload_q6k_prefill(ctx, st, layer, expert_first, n, blocks);
    } else if (matrix != ORN_MAT_DOWN) {
        uint8_t *tmp = (uint8_t *)malloc((size_t)n * nb * 144);
        if (!tmp) return orn_set_err(ctx, ORN_ENOMEM, "host staging");
        for (int i = 0; i < n; ++i) {
            const uint8_t *src = (const uint8_t *)blocks + (size_t)i * nb * ORN_Q4K_BYTES;
            if (st->sh.file_layout) memcpy(tmp + i * nb * 144, src, nb * 144);  /* file order */
            else permute_q4k(src, tmp + i * nb * 144, D, H / 256);
        }
        uint8_t *dst = (matrix == ORN_MAT_GATE ? a_gate : a_up) + slot0 * nb * 144;
        rc = orn_hip_check(ctx, hipMemcpyAsync(dst, tmp, (size_t)n * nb * 144, hipMemcpyDefault,
                                               s), "upload q4k");
        hipStreamSynchronize(s);
        free(tmp);
        if (!rc && st->sh.prefill_layout && !st->cache)
            rc = upload_q4k_prefill(ctx, st, layer, matrix, expert_first, n, blocks);
    } else {
        uint8_t *body = (uint8_t *)malloc((size_t)n * nb * 208);
        uint16_t *dv = (uint16_t *)malloc((size_t)n * nb * 2);
        if (!body || !dv) {
            free(body);
            free(dv);
            return orn_set_err(ctx, ORN_ENOMEM, "host staging");
        }
        for (int i = 0; i < n; ++i) {
            /* file order is D rows of H/256 blocks: the same split with the
             * roles of the two block indices exchanged leaves it in place */
            const uint8_t *src = (const uint8_t *)blocks + (size_t)i * nb * ORN_Q6K_BYTES;
            if (st->sh.file_layout) permute_q6k(src, body + i * nb * 208, dv + i * nb, (int)nb, 1);
            else permute_q6k(src, body + i * nb * 208, dv + i * nb, H, D / 256);
        }
        rc = orn_hip_check(ctx, hipMemcpyAsync(a_body + slot0 * nb * 208, body,
                                               (size_t)n * nb * 208, hipMemcpyDefault, s),
                           "upload q6k");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(a_d + slot0 * nb, dv, (size_t)n * nb * 2,
                                                   hipMemcpyDefault, s), "upload q6k d");
        hipStreamSynchronize(s);
        if (!rc && st->cache) {
            /* the MFMA layouts are packed on the device when an expert is
             * loaded into a slot; the path choice needs the scale range now */
            const int scmax = q6_scmax_of(body, (size_t)n * nb);
            if (scmax > st->q6_scmax[layer]) st->q6_scmax[layer] = scmax;
        }
        free(body);
        free(dv);
        if (!rc && st->sh.prefill_layout && !st->cache)
            rc = upload_q6k_prefill(ctx, st, layer, expert_first, n, blocks);
    }
    return rc;
}

int gpu_moe_store_set_router(gpu_context *ctx, ornith_moe_store *st, int layer, const float *W,
                             const float *bias)
{
    if (!ctx || !st || !W) return ORN_EINVAL;
    if (layer < 0 || layer >= st->sh.n_layers) return orn_set_err(ctx, ORN_EINVAL, "bad layer");
    graphs_clear(st);  /* the bias pointer is a kernel argument */
    const size_t D = (size_t)st->sh.d_model, E = (size_t)st->sh.n_experts;
    float *t = (float *)malloc(D * E * sizeof(float));
    if (!t) return orn_set_err(ctx, ORN_ENOMEM, "host staging");
    for (size_t d = 0; d < D; ++d)
        for (size_t e = 0; e < E; ++e)
            t[((d >> 2) * E + e) * 4 + (d & 3)] = st->sh.file_layout ? W[e * D + d] : W[d * E + e];
    hipStream_t s = ctx->stream;
    int rc = orn_hip_check(ctx, hipMemcpyAsync(st->router_q + (size_t)layer * E * D, t,
                                               D * E * sizeof(float), hipMemcpyHostToDevice, s),
                           "upload router");
    if (!rc) {
        if (bias)
            rc = orn_hip_check(ctx, hipMemcpyAsync(st->bias + (size_t)layer * E, bias,
                                                   E * sizeof(float), hipMemcpyHostToDevice, s),
                               "upload bias");
        st->has_bias[layer] = bias ? 1 : 0;
    }
    hipStreamSynchronize(s);
    free(t);
    return rc;
}

int gpu_moe_store_set_norm(gpu_context *ctx, ornith_moe_store *st, int layer, const float *w)
{
    if (!ctx || !st || !w) return ORN_EINVAL;
    if (layer < 0 || layer >= st->sh.n_layers) return orn_set_err(ctx, ORN_EINVAL, "bad layer");
    const size_t D = (size_t)st->sh.d_model;
    int rc = orn_hip_check(ctx, hipMemcpyAsync(st->norm + (size_t)layer * D, w, D * sizeof(float),
                                               hipMemcpyHostToDevice, ctx->stream),
                           "upload norm");
    hipStreamSynchronize(ctx->stream);
    return rc;
}

int gpu_moe_store_set_shexp_gate(gpu_context *ctx, ornith_moe_store *st, int layer,
                                 const float *w)
{
    if (!ctx || !st) return ORN_EINVAL;
    if (layer < 0 || layer >= st->sh.n_layers) return orn_set_err(ctx, ORN_EINVAL, "bad layer");
    if (w && !st->sh.has_shared)
        return orn_set_err(ctx, ORN_EINVAL, "shared-expert gate on a store without a shared expert");
    graphs_clear(st);
    st->has_shexp_gate[layer] = 0;
    if (!w) return ORN_OK;
    const size_t D = (size_t)st->sh.d_model;
    int rc = orn_hip_check(ctx, hipMemcpyAsync(st->shexp_gate + (size_t)layer * D, w,
                                               D * sizeof(float), hipMemcpyHostToDevice,
                                               ctx->stream),
                           "upload shared-expert gate");
    hipStreamSynchronize(ctx->stream);
    if (!rc) st->has_shexp_gate[layer] = 1;
    return rc;
}

/* The layer's synthetic experts and router are generated on the device
 * (synth.hip: the same bytes as the host generator orn_synth_*, written
 * into the store's order), and with prefill_layout the MFMA layouts are
 * built there too; only the Zipf bias (E floats) comes from the host. */
int gpu_moe_store_fill_synthetic(gpu_context *ctx, ornith_moe_store *st, int layer, uint64_t seed,
                                 float zipf_s)
{
    if (!ctx || !st) return ORN_EINVAL;
    if (layer < 0 || layer >= st->sh.n_layers) return orn_set_err(ctx, ORN_EINVAL, "bad layer");
    graphs_clear(st);
    const int E = st->sh.n_experts, E1 = E + st->sh.has_shared;
    const size_t S = (size_t)E + 1; /* slots per layer in the store */
    const size_t nb = st->blocks_per_matrix;
    const size_t D = (size_t)st->sh.d_model, H = (size_t)st->sh.hidden;
    const size_t slot0 = (size_t)layer * S;
    hipStream_t s = ctx->stream;
    ornk_synth_args g;
    memset(&g, 0, sizeof g);
    g.seed = seed;
    g.layer = layer;
    g.D = (int)D;
    g.H = (int)H;
    g.n_experts = E;
    g.has_shared = st->sh.has_shared;
    g.file = st->sh.file_layout;
    g.router = st->router_q + (size_t)layer * E * D;
    int rc;
    uint8_t *stage = NULL;  /* a lean store's one-layer staging, freed below */
    if (st->sh.prefill_layout == 2) {
        /* generated on the device into a one-layer staging area, packed
         * into the MFMA layouts below, then released */
        const size_t bytes = S * nb * 500;
        if (hipMalloc((void **)&stage, bytes) != hipSuccess)
            return orn_set_err(ctx, ORN_ENOMEM, "fill_synthetic: %zu bytes of staging", bytes);
        g.gate = stage;
        g.up = stage + S * nb * 144;
        g.down_body = stage + S * nb * 288;
        g.down_d = (uint16_t *)(stage + S * nb * 496);
        rc = orn_hip_check(ctx, (hipError_t)ornk_synth_layer(&g, s), "synthetic layer");
        if (rc) {
            hipStreamSynchronize(s);
            hipFree(stage);
            return rc;
        }
    } else if (st->cache) {
        /* generated on the device into a one-layer staging area, then
         * copied to the host tier */
        if ((rc = orn_cache_quiesce(ctx, st->cache))) return rc;
        orn_cache_invalidate(st->cache, layer, 0, E + 1);
        uint8_t *tmp = NULL;
        const size_t bytes = S * nb * 500;
        if (hipMalloc((void **)&tmp, bytes) != hipSuccess)
            return orn_set_err(ctx, ORN_ENOMEM, "fill_synthetic: %zu bytes of staging", bytes);
        g.gate = tmp;
        g.up = tmp + S * nb * 144;
        g.down_body = tmp + S * nb * 288;
        g.down_d = (uint16_t *)(tmp + S * nb * 496);
        rc = orn_hip_check(ctx, (hipError_t)ornk_synth_layer(&g, s), "synthetic layer");
        uint8_t *a_gate, *a_up, *a_body;
        uint16_t *a_d;
        expert_arrays(st, &a_gate, &a_up, &a_body, &a_d);
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(a_gate + slot0 * nb * 144, g.gate,
                                                   S * nb * 144, hipMemcpyDefault, s), "tier");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(a_up + slot0 * nb * 144, g.up, S * nb * 144,
                                                   hipMemcpyDefault, s), "tier");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(a_body + slot0 * nb * 208, g.down_body,
                                                   S * nb * 208, hipMemcpyDefault, s), "tier");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(a_d + slot0 * nb, g.down_d, S * nb * 2,
                                                   hipMemcpyDefault, s), "tier");
        if (!rc) rc = orn_hip_check(ctx, hipStreamSynchronize(s), "synthetic layer");
        hipFree(tmp);
        if (rc) return rc;
        st->q6_scmax[layer] = q6_scmax_of(a_body + slot0 * nb * 208, (size_t)E1 * nb);
    } else {
        g.gate = st->gate + slot0 * nb * 144;
        g.up = st->up + slot0 * nb * 144;
        g.down_body = st->down_body + slot0 * nb * 208;
        g.down_d = st->down_d + slot0 * nb;
        rc = orn_hip_check(ctx, (hipError_t)ornk_synth_layer(&g, s), "synthetic layer");
        if (rc) return rc;
    }
    if (zipf_s > 0.0f) {
        float *b = (float *)malloc((size_t)E * sizeof(float));
        if (!b) {
            hipStreamSynchronize(s);
            hipFree(stage);
            return orn_set_err(ctx, ORN_ENOMEM, "host staging");
        }
        orn_synth_zipf_bias(seed, orn_synth_stream(layer, ORN_SYN_ZIPF, 0), E, zipf_s, b);
        rc = orn_hip_check(ctx, hipMemcpyAsync(st->bias + (size_t)layer * E, b,
                                               (size_t)E * sizeof(float), hipMemcpyHostToDevice, s),
                           "upload bias");
        hipStreamSynchronize(s);
        free(b);
        if (rc) {
            hipFree(stage);
            return rc;
        }
    }
    st->has_bias[layer] = zipf_s > 0.0f ? 1 : 0;
    if (st->sh.prefill_layout && !st->cache) {
        const size_t DH = D * H;
        ornk_pack_args pa;
        memset(&pa, 0, sizeof pa);
        pa.D = (int)D;
        pa.H = (int)H;
        pa.n_e = E1;
        pa.gu[0] = g.gate;
        pa.gu[1] = g.up;
        pa.down_body = g.down_body;
        pa.down_d = g.down_d;
        for (int m = 0; m < 2; ++m) {
            pa.pq[m] = (uint32_t *)((uint8_t *)st->pq[m] + slot0 * (DH / 2));
            pa.psc[m] = (uint16_t *)((uint8_t *)st->psc[m] + slot0 * (DH / 16));
            pa.pmn[m] = (uint16_t *)((uint8_t *)st->pmn[m] + slot0 * (DH / 16));
            pa.pd[m] = (float *)((uint8_t *)st->pd[m] + slot0 * (DH / 64));
            pa.pdm[m] = (float *)((uint8_t *)st->pdm[m] + slot0 * (DH / 64));
        }
        pa.dq = st->dq + slot0 * ORNK_DQ_BYTES(DH);
        pa.dsc = (uint16_t *)((uint8_t *)st->dsc + slot0 * (DH / 8));
        pa.dd = (float *)((uint8_t *)st->dd + slot0 * (DH / 64));
        pa.dmax = st->dmax + slot0 * 3;
        pa.scmax = st->dev_scmax;
        rc = orn_hip_check(ctx, (hipError_t)ornk_pack_prefill(&pa, s), "prefill layouts");
        /* host mirrors: the per-slot maxima (re-uploaded by later partial
         * uploads of the layer) and the layer's largest Q6_K sub-scale */
        int scmax = 0;
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(st->dmax_host + slot0 * 3, pa.dmax,
                                                   (size_t)E1 * 3 * sizeof(float),
                                                   hipMemcpyDeviceToHost, s), "dmax copy");
        if (!rc)
            rc = orn_hip_check(ctx, hipMemcpyAsync(&scmax, st->dev_scmax, sizeof(int),
                                                   hipMemcpyDeviceToHost, s), "scmax copy");
        if (!rc) rc = orn_hip_check(ctx, hipStreamSynchronize(s), "prefill layouts");
        hipStreamSynchronize(s);
        hipFree(stage);  /* NULL unless lean */
        if (rc) return rc;
        st->q6_scmax[layer] = scmax;
    }
    return orn_hip_check(ctx, hipStreamSynchronize(s), "synthetic layer");
}

/* Inverse of gpu_moe_store_set_experts: the GGUF block stream of n experts
 * of one matrix, in the orientation set_experts takes. */
int gpu_moe_store_get_experts(gpu_context *ctx, ornith_moe_store *st, int layer, int matrix,
                              int expert_first, int n, void *blocks)
{
    if (!ctx || !st || !blocks) return ORN_EINVAL;
    const int E1 = st->sh.n_experts + 1;
    if (layer < 0 || layer >= st->sh.n_layers || expert_first < 0 || n < 0 ||
        expert_first + n > E1 || matrix < 0 || matrix > 2)
        return orn_set_err(ctx, ORN_EINVAL, "get_experts: bad layer/expert range/matrix");
    if (n == 0) return ORN_OK;
    if (st->sh.prefill_layout == 2)
        return orn_set_err(ctx, ORN_EUNSUPPORTED,
                           "get_experts: a store with prefill_layout = 2 keeps no GGUF blocks");
    const int D = st->sh.d_model, H = st->sh.hidden, file = st->sh.file_layout;
    const size_t nb = st->blocks_per_matrix;
    const size_t slot0 = (size_t)layer * E1 + (size_t)expert_first;
    hipStream_t s = ctx->stream;
    uint8_t *out = (uint8_t *)blocks;
    int rc;
    uint8_t *a_gate, *a_up, *a_body;
    uint16_t *a_d;
    expert_arrays(st, &a_gate, &a_up, &a_body, &a_d);
    if (matrix != ORN_MAT_DOWN) {
        const uint8_t *src = (matrix == ORN_MAT_GATE ? a_gate : a_up) + slot0 * nb * 144;
        uint8_t *tmp = (uint8_t *)malloc((size_t)n * nb * 144);
        if (!tmp) return orn_set_err(ctx, ORN_ENOMEM, "host staging");
        rc = orn_hip_check(ctx, hipMemcpyAsync(tmp, src, (size_t)n * nb * 144, hipMemcpyDefault,
                                               s), "download q4k");
        if (!rc) rc = orn_hip_check(ctx, hipStreamSynchronize(s), "download q4k");
        const int K = D, NBc = H / 256;
        for (int i = 0; i < n && !rc; ++i) {
            const uint8_t *t = tmp + (size_t)i * nb * 144;
            uint8_t *o = out + (size_t)i * nb * ORN_Q4K_BYTES;
            if (file) {
                memcpy(o, t, nb * 144);
                continue;
            }
            for (int k = 0; k < K; ++k)
                for (int c = 0; c < NBc; ++c)
                    memcpy(o + ((size_t)k * NBc + c) * 144, t + ((size_t)c * K + k) * 144, 144);
        }
        free(tmp);
        return rc;
    }
    uint8_t *body = (uint8_t *)malloc((size_t)n * nb * 208);
    uint16_t *dv = (uint16_t *)malloc((size_t)n * nb * 2);
    if (!body || !dv) {
        free(body);
        free(dv);
        return orn_set_err(ctx, ORN_ENOMEM, "host staging");
    }
    rc = orn_hip_check(ctx, hipMemcpyAsync(body, a_body + slot0 * nb * 208, (size_t)n * nb * 208,
                                           hipMemcpyDefault, s), "download q6k");
    if (!rc)
        rc = orn_hip_check(ctx, hipMemcpyAsync(dv, a_d + slot0 * nb, (size_t)n * nb * 2,
                                               hipMemcpyDefault, s), "download q6k d");
    if (!rc) rc = orn_hip_check(ctx, hipStreamSynchronize(s), "download q6k");
    const int K = file ? (int)nb : H, NBc = file ? 1 : D / 256;
    for (int i = 0; i < n && !rc; ++i)
        for (int k = 0; k < K; ++k)
            for (int c = 0; c < NBc; ++c) {
                const size_t q = (size_t)i * nb + (size_t)c * K + k;
                uint8_t *o = out + ((size_t)i * nb + (size_t)k * NBc + c) * ORN_Q6K_BYTES;
                memcpy(o, body + q * 208, 208);
                o[ORN_Q6K_OFF_D] = (uint8_t)dv[q];
                o[ORN_Q6K_OFF_D + 1] = (uint8_t)(dv[q] >> 8);
            }
    free(body);
    free(dv);
    return rc;
}

/* ---------------------------------------------------------------------------
 * Forward
 * ------------------------------------------------------------------------- */
#define ALIGN256(x) (((x) + 255u) & ~(size_t)255u)

typedef struct {
    int ks_gu, ks_dn, rows_max, items_max, tchunk;
    int use_dec; /* MFMA path with the decode-shaped kernels (items <= 16 rows) */
} plan_t;

static int pow2_floor(int v)
{
    int p = 1;
    while (p * 2 <= v) p *= 2;
    return p;
}

/* Work decomposition for T tokens.  Work items hold up to `tchunk` token rows
 * of one expert; the gate/up and down kernels split the reduction dimension
 * into ks slices so the grid holds ~2048 blocks (8 per CU).  Slices keep at
 * least 32 rows (gate/up) and 32 rows (down) so the split-K partials stay a
 * small fraction of the weight bytes. */
static plan_t make_plan(const ornith_moe_shape *sh, int T, int use_mfma)
{
    plan_t p;
    p.use_dec = 0;
    const int k = sh->top_k, E = sh->n_experts;
    const int D = sh->d_model, H = sh->hidden;
    /* MFMA work items hold at most one 16-row tile (the decode kernels) at
     * decode sizes, two (the decode kernels' two-tile instances) above 64
     * tokens wherever the batch averages at most 16 rows per expert, four
     * (the prefill grouped GEMMs) beyond.  Skewed batches of the middle
     * kind (a few hot experts, many cold ones) then split each hot expert
     * into items of 32 rows instead of running every cold expert through a
     * 64-row tile: an item costs its weight conversion whatever its rows. */
    p.tchunk = use_mfma ? (T <= 64 ? 16 : T * k <= 16 * E ? 32 : 64) : (T <= 64 ? 2 : 8);
    p.rows_max = T * k + (sh->has_shared ? T : 0);
    const int max_slots = (T * k < E ? T * k : E) + (sh->has_shared ? 1 : 0);
    p.items_max = max_slots + (p.rows_max + p.tchunk - 1) / p.tchunk;
    int est_items = max_slots + p.rows_max / p.tchunk;
    if (est_items < 1) est_items = 1;
    /* gate/up: K = D rows; a wave covers RW rows per step, a block 4*RW */
    const int rw_gu = 64 / (8 * (H / 256));
    int ks = pow2_floor(2048 / est_items);
    if (ks < 1) ks = 1;
    if (ks > 64) ks = 64;
    while (ks > 1 && (D % ks || (D / ks) % (16 * rw_gu) || D / ks < 32)) ks /= 2;
    p.ks_gu = ks;
    /* down: K = H rows */
    const int cr = 8 * (D / 256);
    const int rw_dn = 64 / (cr < 64 ? cr : 64);
    int kd = pow2_floor(2048 / est_items);
    if (kd < 1) kd = 1;
    if (kd > 16) kd = 16;
    while (kd > 1 && (H % kd || (H / kd) % (16 * rw_dn) || H / kd < 32)) kd /= 2;
    p.ks_dn = kd;
    if (use_mfma) {
        /* split-K so that the grid holds ~2048 work groups: gate/up has
         * 2*(H/256) tiles per item and slice, down D/256 */
        int kg = pow2_floor(2048 / (est_items * 2 * (H / 256)) > 0
                                ? 2048 / (est_items * 2 * (H / 256)) : 1);
        /* the prefill gate/up kernel pipelines 4 steps per loop turn:
         * slices of a multiple of 4 steps, at most 64 */
        while (kg > 1 && ((D / 32) % kg || (D / 32 / kg) % 4)) kg /= 2;
        while (D / 32 / kg > 64) kg *= 2;
        int kdn = pow2_floor(2048 / (est_items * (D / 256)) > 0 ? 2048 / (est_items * (D / 256)) : 1);
        while (kdn > 1 && (H / 32) % kdn) kdn /= 2;
        if (kdn > H / 32) kdn = H / 32;
        if (kdn > 16) kdn = 16; /* the combine sums at most 16 slices */
        p.ks_gu = kg;
        p.ks_dn = kdn;
        if (p.tchunk <= 32) {
            /* Decode kernels (slices of 4..32 reduction steps compiled).
             * Gate/up: about 2048 work groups over the estimated items, slices
             * of 4..16 steps (measured best: 16 at 16 tokens, 4 at 1 token);
             * down: 8-step slices. */
            const int ng = 2048 / (est_items * 2 * (H / 256));
            int dg = pow2_floor(ng > 0 ? ng : 1);
            while (dg > 1 && (D / 32) % dg) dg /= 2;
            while (dg > 1 && D / 32 / dg < 4) dg /= 2;
            while ((D / 32) % (2 * dg) == 0 && D / 32 / dg > 16) dg *= 2;
            int dd = 1;
            while ((H / 32) % (2 * dd) == 0 && H / 32 / dd > 8) dd *= 2;
            /* Two-tile items (32 rows): down unsplit when a slice of all H
             * steps is compiled.  The combine then reads one partial per
             * row: Zipf T=256 combine 6.7 -> 4.4 us, down 32.0 -> 33.4. */
            if (p.tchunk == 32 && ornk_dec_supported(D / 32 / dg, H / 32)) dd = 1;
            if ((D / 32) % dg == 0 && (H / 32) % dd == 0 &&
                ornk_dec_supported(D / 32 / dg, H / 32 / dd)) {
                p.use_dec = 1;
                p.ks_gu = dg;
                p.ks_dn = dd;
            }
        }
    }
    return p;
}

/* File-orientation path: items of <= 16 rows (one MFMA row tile); the
 * reduction is split, in whole super-blocks, so that gate/up has about
 * 8192 work groups (2H/256 per item and slice) and down about 8192
 * (D / ornk_file_down_cols() per item and slice): these kernels need
 * several rounds of work groups to hide their memory latency, and a wave
 * that covers one super-block uses every byte of its blocks while they are
 * cached. */
static plan_t make_plan_file(const ornith_moe_shape *sh, int T)
{
    plan_t p;
    memset(&p, 0, sizeof p);
    const int k = sh->top_k, E = sh->n_experts, D = sh->d_model, H = sh->hidden;
    /* items of up to 64 rows (four row tiles per work group, each expert's
     * weights streamed once per 64 rows) once routed experts average 16
     * rows or more; 16 below, where most items hold a row or two */
    p.tchunk = T * k >= 16 * E ? 64 : 16;
    p.rows_max = T * k + (sh->has_shared ? T : 0);
    const int max_slots = (T * k < E ? T * k : E) + (sh->has_shared ? 1 : 0);
    p.items_max = max_slots + (p.rows_max + p.tchunk - 1) / p.tchunk;
    int est = max_slots + p.rows_max / p.tchunk;
    if (est < 1) est = 1;
    const int ng = 8192 / (est * (2 * H / 256)), nd = 8192 / (est * (D / ornk_file_down_cols()));
    int kg = pow2_floor(ng > 0 ? ng : 1), kd = pow2_floor(nd > 0 ? nd : 1);
    while (kg > 1 && (D / 256) % kg) kg /= 2;
    while (kd > 1 && (H / 256) % kd) kd /= 2;
    p.ks_gu = kg;
    p.ks_dn = kd;
    return p;
}

static int check_buf(const gpu_buffer *b, size_t bytes) { return b && b->size >= bytes; }

static int launch(gpu_context *ctx, const char *name, int (*fn)(const ornk_moe_args *, hipStream_t),
                  const ornk_moe_args *a)
{
    int slot = orn_prof_begin(ctx, name);
    int e = fn(a, ctx->stream);
    orn_prof_end(ctx, slot);
    if (e != hipSuccess)
        return orn_set_err(ctx, ORN_EHIP, "%s: %s", name, hipGetErrorString((hipError_t)e));
    return ORN_OK;
}

/* A step whose launcher takes its profiling events: under profiling its
 * kernel carries the record's events (the kernel's own duration, as a
 * kernel trace measures it, rather than the span between two event packets
 * around the launch); a step of two kernels spans both. */
static int launch_k(gpu_context *ctx, const char *name,
                         int (*fn)(const ornk_moe_args *, hipStream_t), const ornk_moe_args *a)
{
    ornk_moe_args b = *a;
    orn_prof_kernel(ctx, name, &b.ev_start, &b.ev_stop);
    int e = fn(&b, ctx->stream);
    if (e != hipSuccess)
        return orn_set_err(ctx, ORN_EHIP, "%s: %s", name, hipGetErrorString((hipError_t)e));
    return ORN_OK;
}

/* fixed_ws: NULL = the context's grow-only workspace; else the device's
 * fixed scratch of ORNK_SCRATCH_BYTES (gpu_moe_forward_noalloc), and the
 * call then allocates nothing. */
static int moe_forward_dev(gpu_context *ctx, ornith_moe_store *st, int layer, const float *x,
                           int T, const float *resid, float *out, uint32_t *idx_out, float *w_out,
                           const ornith_moe_opts *opts, void *fixed_ws)
{
    const ornith_moe_shape *sh = &st->sh;
    const int D = sh->d_model, H = sh->hidden, E = sh->n_experts, k = sh->top_k;
    const int E1 = E + 1;
    const unsigned flags = opts ? opts->flags : 0u;
    const int mode = opts ? opts->route_mode : ORN_ROUTE_RENORM;
    if (mode != ORN_ROUTE_RENORM && mode != ORN_ROUTE_LITERAL)
        return orn_set_err(ctx, ORN_EINVAL, "bad route mode");
    const int ep_first = opts ? opts->ep_first : 0, ep_count = opts ? opts->ep_count : 0;
    if (ep_first < 0 || ep_count < 0 || (ep_count == 0 && ep_first != 0) ||
        ep_first + ep_count > E)
        return orn_set_err(ctx, ORN_EINVAL, "bad expert share [%d, %d)", ep_first,
                           ep_first + ep_count);
    if ((flags & ORN_MOE_PATH_VALU) && (flags & ORN_MOE_PATH_MFMA))
        return orn_set_err(ctx, ORN_EINVAL, "both expert paths forced");
    const int file = sh->file_layout;
    if (file && (flags & (ORN_MOE_PATH_VALU | ORN_MOE_PATH_MFMA)))
        return orn_set_err(ctx, ORN_EUNSUPPORTED,
                           "a file-layout store has one expert path; do not force one");
    /* The MFMA path needs the prefill layouts.  Q6_K sub-scales above 64 in
     * magnitude (real quantizers emit them up to 128) take the down kernels'
     * wide instances, which split sc * q in two exact fp16 operands. */
    const int mfma_ok = sh->prefill_layout;
    int use_mfma = mfma_ok && T >= ORN_MOE_MFMA_MIN_TOKENS;
    if (sh->prefill_layout == 2) {
        if (flags & ORN_MOE_PATH_VALU)
            return orn_set_err(ctx, ORN_EUNSUPPORTED,
                               "the VALU path reads GGUF blocks, which a store with "
                               "prefill_layout = 2 does not keep");
        use_mfma = 1;
    }
    if (flags & ORN_MOE_PATH_VALU) use_mfma = 0;
    if (flags & ORN_MOE_PATH_MFMA) {
        if (!mfma_ok)
            return orn_set_err(ctx, ORN_EUNSUPPORTED,
                               "MFMA path needs the prefill layout");
        use_mfma = 1;
    }
    if (file) use_mfma = 0;  /* the mid and combine steps run as on the VALU path */
    plan_t p = file ? make_plan_file(sh, T) : make_plan(sh, T, use_mfma);

    /* Certified routing of the smallest decode batches (router_cert.hip):
     * logits, top-k and dispatch in one launch.  Streamed stores keep it too
     * (the slot list is read back after the dispatch either way). */
    const int cert = !(flags & ORN_MOE_EXACT_LOGITS) && ornk_route_cert_supported(T, D, E, k);

    /* the fixed scratch keeps its first ORNK_SYNC_BYTES for the routing
     * counters (zeroed when the scratch is first resolved); otherwise they
     * have an allocation of their own */
    size_t off = fixed_ws ? ORNK_SYNC_BYTES : 0;
    int *sync = NULL;
    if (cert) {
        sync = fixed_ws ? (int *)fixed_ws : ctx_sync(ctx);
        if (!sync) return ORN_ENOMEM;
    }
#define CARVE(name, bytes)       \
    size_t name = off;           \
    off += ALIGN256((size_t)(bytes))
    CARVE(o_xn, (flags & ORN_MOE_NORM) ? (size_t)T * D * 4 : 0);
    CARVE(o_est, cert ? (size_t)T * (E + 1) * 8 : 0); /* tagged (S, B) words, rmsnorm scales */
    CARVE(o_logits, (size_t)T * E * 4);
    CARVE(o_idx, (size_t)T * k * 4);
    CARVE(o_w, (size_t)T * k * 4);
    CARVE(o_ctl, 64);
    CARVE(o_slot_e, (size_t)E1 * 4);
    CARVE(o_slot_off, (size_t)E1 * 4);
    CARVE(o_slot_cnt, (size_t)E1 * 4);
    CARVE(o_row_tok, (size_t)p.rows_max * 4);
    CARVE(o_pair_row, (size_t)T * k * 4);
    CARVE(o_items, (size_t)p.items_max * 16);
    CARVE(o_gu, (size_t)p.ks_gu * p.rows_max * 2 * H * 4);
    CARVE(o_mid, (size_t)p.rows_max * H * 4);
    CARVE(o_dn, (size_t)p.ks_dn * p.rows_max * D * 4);
    CARVE(o_xamax, use_mfma ? (size_t)T * 4 : 0);
    CARVE(o_midamax, use_mfma ? (size_t)p.rows_max * 4 : 0);
    CARVE(o_fxh, file ? (size_t)T * D * 2 : 0);
    CARVE(o_fxl, file ? (size_t)T * D * 2 : 0);
    CARVE(o_fsh, file ? (size_t)T * (D / 32) * 2 : 0);
    CARVE(o_fsl, file ? (size_t)T * (D / 32) * 2 : 0);
    CARVE(o_fxinv, file ? (size_t)T * 4 : 0);
    CARVE(o_fmh, file ? (size_t)p.rows_max * H * 2 : 0);
    CARVE(o_fml, file ? (size_t)p.rows_max * H * 2 : 0);
    CARVE(o_fminv, file ? (size_t)p.rows_max * 4 : 0);
#undef CARVE
    uint8_t *ws;
    if (fixed_ws) {
        if (off > ORNK_SCRATCH_BYTES)
            return orn_set_err(ctx, ORN_EINVAL,
                               "gpu_moe_forward_noalloc: %d tokens need %zu bytes of work "
                               "buffers; the fixed scratch holds %u",
                               T, off, (unsigned)ORNK_SCRATCH_BYTES);
        ws = (uint8_t *)fixed_ws;
    } else {
        ws = (uint8_t *)orn_ws_get(ctx, off);
        if (!ws) return ORN_ENOMEM;
    }

    const size_t E1nb = (size_t)E1 * st->blocks_per_matrix;
    ornk_moe_args a;
    memset(&a, 0, sizeof a);
    a.T = T;
    a.D = D;
    a.H = H;
    a.E = E;
    a.k = k;
    /* an expert-parallel share computes the shared expert iff it starts at 0 */
    a.has_shared = sh->has_shared && ep_first == 0;
    a.ep_lo = ep_first;
    a.ep_n = ep_count ? ep_count : E;
    a.mode = mode;
    a.apply_norm = (flags & ORN_MOE_NORM) ? 1 : 0;
    a.ks_gu = p.ks_gu;
    a.ks_dn = p.ks_dn;
    a.rows_max = p.rows_max;
    a.items_max = p.items_max;
    a.tchunk = p.tchunk;
    if (!st->cache && st->gate) {  /* a streamed store's slots are set after the dispatch */
        a.gate = st->gate + (size_t)layer * E1nb * 144;
        a.up = st->up + (size_t)layer * E1nb * 144;
        a.down_body = st->down_body + (size_t)layer * E1nb * 208;
        a.down_d = st->down_d + (size_t)layer * E1nb;
    }
    a.router = st->router_q + (size_t)layer * E * D;
    a.bias = st->has_bias[layer] ? st->bias + (size_t)layer * E : NULL;
    a.norm_w = st->norm + (size_t)layer * D;
    if (flags & ORN_MOE_SHEXP_GATE) {
        if (!st->has_shexp_gate[layer])
            return orn_set_err(ctx, ORN_EINVAL,
                               "ORN_MOE_SHEXP_GATE: layer %d has no shared-expert gate", layer);
        a.shexp_gate = st->shexp_gate + (size_t)layer * D;
    }
    a.x = x;
    a.resid = resid;
    a.out = out;
    a.xn = a.apply_norm ? (float *)(ws + o_xn) : (float *)x;
    a.logits = (float *)(ws + o_logits);
    a.sync = sync;
    a.route_est = cert ? (double *)(ws + o_est) : NULL;
    /* the selection is written straight into the caller's buffers if given */
    a.idx = idx_out ? idx_out : (uint32_t *)(ws + o_idx);
    a.w = w_out ? w_out : (float *)(ws + o_w);
    a.ctl = (int *)(ws + o_ctl);
    a.slot_expert = (int *)(ws + o_slot_e);
    a.slot_off = (int *)(ws + o_slot_off);
    a.slot_cnt = (int *)(ws + o_slot_cnt);
    a.row_token = (int *)(ws + o_row_tok);
    a.pair_row = (int *)(ws + o_pair_row);
    a.items = (int *)(ws + o_items);
    a.gu_part = (float *)(ws + o_gu);
    a.mid = (float *)(ws + o_mid);
    a.dn_part = (float *)(ws + o_dn);
    a.use_mfma = use_mfma;
    a.q6_wide = st->q6_scmax && st->q6_scmax[layer] > 64; /* held by MFMA-layout stores */
    if (use_mfma && !st->cache) {  /* a streamed store's slot arrays come from the cache */
        const size_t slot0 = (size_t)layer * E1, DH = (size_t)D * H;
        for (int m = 0; m < 2; ++m) {
            a.gu_pf.pq[m] = (const uint32_t *)((const uint8_t *)st->pq[m] + slot0 * (DH / 2));
            a.gu_pf.psc[m] = (const uint16_t *)((const uint8_t *)st->psc[m] + slot0 * (DH / 16));
            a.gu_pf.pmn[m] = (const uint16_t *)((const uint8_t *)st->pmn[m] + slot0 * (DH / 16));
            a.gu_pf.pd[m] = (const float *)((const uint8_t *)st->pd[m] + slot0 * (DH / 64));
            a.gu_pf.pdm[m] = (const float *)((const uint8_t *)st->pdm[m] + slot0 * (DH / 64));
        }
        a.gu_pf.dmax = st->dmax + slot0 * 3;
        a.dn_pf.dq = st->dq + slot0 * ORNK_DQ_BYTES(DH);
        a.dn_pf.dsc = (const uint16_t *)((const uint8_t *)st->dsc + slot0 * (DH / 8));
        a.dn_pf.dd = (const float *)((const uint8_t *)st->dd + slot0 * (DH / 64));
        a.dn_pf.dmax = st->dmax + slot0 * 3;
    }
    if (use_mfma) {
        a.x_amax = (float *)(ws + o_xamax);
        a.router_amax = 1;  /* every routing kernel writes the rows' max |x| */
        a.mid_amax = (float *)(ws + o_midamax);
    }

    if (file) {
        a.fw.xh = (uint32_t *)(ws + o_fxh);
        a.fw.xl = (uint32_t *)(ws + o_fxl);
        a.fw.xsh = (uint16_t *)(ws + o_fsh);
        a.fw.xsl = (uint16_t *)(ws + o_fsl);
        a.fw.xinv = (float *)(ws + o_fxinv);
        a.fw.mh = (uint32_t *)(ws + o_fmh);
        a.fw.ml = (uint32_t *)(ws + o_fml);
        a.fw.minv = (float *)(ws + o_fminv);
    }

    int rc;
    /* A separate norm kernel runs only where the router does not fuse the
     * norm (profiled only then, so that every recorded step is a kernel). */
    if (cert) {
        /* the norm, logits, selection and dispatch in one launch */
        if ((rc = launch_k(ctx, "moe_route", ornk_moe_route_cert, &a))) return rc;
    } else {
        if (a.apply_norm && !ornk_router_pc_supported(T, D) &&
            (rc = launch(ctx, "moe_norm", ornk_moe_norm, &a)))
            return rc;
        if ((rc = launch_k(ctx, "moe_route", ornk_moe_route, &a))) return rc;
        if ((rc = launch_k(ctx, "moe_dispatch", ornk_moe_dispatch, &a))) return rc;
    }
    /* streamed experts: read the dispatch's experts back, load the missing
     * ones into slots and renumber the work items (host round trip) */
    if (st->cache && (rc = orn_cache_prepare(ctx, st->cache, layer, &a))) return rc;
    if (file) {
        /* decode sizes: the exact router wrote the file kernels' activations */
        if ((cert || !ornk_router_pc_supported(T, D)) &&
            (rc = launch_k(ctx, "moe_file_prep_x", ornk_file_prep_x, &a)))
            return rc;
        if ((rc = launch_k(ctx, "moe_gateup_file", ornk_file_gateup, &a))) return rc;
        /* the mid step also writes the down kernel's hi/lo activations */
        if ((rc = launch_k(ctx, "moe_mid", ornk_moe_mid, &a))) return rc;
        if ((rc = launch_k(ctx, "moe_down_file", ornk_file_down, &a))) return rc;
        if ((rc = launch_k(ctx, "moe_combine", ornk_moe_combine, &a))) return rc;
        ctx->last_ctl = a.ctl;
        ctx->last_logits = a.logits;
        ctx->last_T = T;
        ctx->last_E = E;
        if (!(flags & ORN_MOE_ASYNC))
            return orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "moe forward");
        return ORN_OK;
    }
    if (p.use_dec) {
        if ((rc = launch_k(ctx, "moe_gateup_dec", ornk_moe_gateup_dec, &a))) return rc;
    } else if (use_mfma) {
        if ((rc = launch_k(ctx, "moe_gateup_mfma", ornk_moe_gateup_mfma, &a))) return rc;
    } else {
        if ((rc = launch_k(ctx, "moe_gateup", ornk_moe_gateup, &a))) return rc;
    }
    /* Up to 64 tokens the decode down kernel forms mid from the gate/up
     * partials (each of its work groups for its item's rows); above, where
     * a hot expert's rows span many items, mid is a step of its own. */
    const int fused_mid = p.use_dec && ornk_down_dec_fuses_mid(T, H, p.ks_gu, p.ks_dn);
    if (!fused_mid && (rc = launch_k(ctx, "moe_mid", ornk_moe_mid, &a))) return rc;
    if (p.use_dec) {
        if ((rc = launch_k(ctx, "moe_down_dec", ornk_moe_down_dec, &a))) return rc;
    } else if (use_mfma) {
        if ((rc = launch_k(ctx, "moe_down_mfma", ornk_moe_down_mfma, &a))) return rc;
    } else {
        if ((rc = launch_k(ctx, "moe_down", ornk_moe_down, &a))) return rc;
    }
    if ((rc = launch_k(ctx, "moe_combine", ornk_moe_combine, &a))) return rc;

    ctx->last_ctl = a.ctl;
    ctx->last_logits = a.logits;
    ctx->last_T = T;
    ctx->last_E = E;
    if (!(flags & ORN_MOE_ASYNC))
        return orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "moe forward");
    return ORN_OK;
}

/* ---------------------------------------------------------------------------
 * HIP graphs (ORN_MOE_GRAPH): the first call with a given key runs eagerly
 * (which also sizes the workspace), then records the same enqueue sequence
 * into a graph without executing it; later calls with the same key launch
 * the graph.  No memset or memcpy nodes: every step is a kernel.
 * ------------------------------------------------------------------------- */
typedef int (*orn_body_fn)(gpu_context *ctx, ornith_moe_store *st, const void *arg);

static orn_graph *graph_lookup(ornith_moe_store *st, const orn_graph_key *key)
{
    for (int i = 0; i < ORN_GRAPH_SLOTS; ++i)
        if (st->graphs[i].used && !memcmp(&st->graphs[i].key, key, sizeof *key))
            return &st->graphs[i];
    return NULL;
}

static int run_body(gpu_context *ctx, ornith_moe_store *st, orn_graph_key *key, orn_body_fn body,
                    const void *arg, int sync)
{
    int rc;
    if ((key->flags & ORN_MOE_GRAPH) && !ctx->prof_on) {
        key->ws = ctx->ws.base;
        orn_graph *g = graph_lookup(st, key);
        if (g) {
            g->tick = ++st->graph_tick;
            rc = orn_hip_check(ctx, hipGraphLaunch(g->exec, ctx->stream), "graph launch");
            if (rc) return rc;
            ctx->last_ctl = g->ctl;
            ctx->last_logits = g->logits;
            ctx->last_T = g->lT;
            ctx->last_E = g->lE;
        } else {
            if ((rc = body(ctx, st, arg))) return rc;
            key->ws = ctx->ws.base;
            hipGraph_t graph = NULL;
            rc = orn_hip_check(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal),
                               "begin capture");
            if (rc) return rc;
            const int brc = body(ctx, st, arg);
            const hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
            hipGraphExec_t exec = NULL;
            if (!brc && ce == hipSuccess && graph &&
                hipGraphInstantiate(&exec, graph, NULL, NULL, 0) == hipSuccess) {
                orn_graph *slot = &st->graphs[0];
                for (int i = 0; i < ORN_GRAPH_SLOTS; ++i) {
                    if (!st->graphs[i].used) { slot = &st->graphs[i]; break; }
                    if (st->graphs[i].tick < slot->tick) slot = &st->graphs[i];
                }
                if (slot->used) hipGraphExecDestroy(slot->exec);
                slot->used = 1;
                slot->key = *key;
                slot->exec = exec;
                slot->ctl = ctx->last_ctl;
                slot->logits = ctx->last_logits;
                slot->lT = ctx->last_T;
                slot->lE = ctx->last_E;
                slot->tick = ++st->graph_tick;
            }
            if (graph) hipGraphDestroy(graph);
            (void)hipGetLastError();  /* a failed capture leaves the eager result valid */
        }
    } else {
        if ((rc = body(ctx, st, arg))) return rc;
    }
    if (sync) return orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "moe forward");
    return ORN_OK;
}

typedef struct {
    int layer, T;
    const float *x, *resid;
    float *out;
    uint32_t *idx;
    float *w;
    ornith_moe_opts opts; /* ORN_MOE_ASYNC set */
} fwd_arg;

static int fwd_body(gpu_context *ctx, ornith_moe_store *st, const void *p)
{
    const fwd_arg *a = (const fwd_arg *)p;
    return moe_forward_dev(ctx, st, a->layer, a->x, a->T, a->resid, a->out, a->idx, a->w,
                           &a->opts, NULL);
}

/* Argument checks shared by the forward entry points (1: run, 0: nothing to
 * do, negative: error). */
static int forward_args_ok(gpu_context *ctx, const ornith_moe_store *st, int layer,
                           const gpu_buffer *x, int n_tokens, const gpu_buffer *resid,
                           const gpu_buffer *out, const gpu_buffer *idx_out,
                           const gpu_buffer *w_out, const char *who)
{
    if (!st || !x || !out || n_tokens < 0)
        return orn_set_err(ctx, ORN_EINVAL, "%s: NULL argument or negative T", who);
    if (layer < 0 || layer >= st->sh.n_layers)
        return orn_set_err(ctx, ORN_EINVAL, "%s: bad layer", who);
    if (n_tokens == 0) return 0;
    const size_t act = (size_t)n_tokens * st->sh.d_model * 4;
    const size_t sel = (size_t)n_tokens * st->sh.top_k * 4;
    if (!check_buf(x, act) || !check_buf(out, act) || (resid && !check_buf(resid, act)) ||
        (idx_out && !check_buf(idx_out, sel)) || (w_out && !check_buf(w_out, sel)))
        return orn_set_err(ctx, ORN_EINVAL, "%s: buffer too small", who);
    if (out == x || out == resid)
        return orn_set_err(ctx, ORN_EINVAL, "%s: out aliases an input", who);
    return 1;
}

int gpu_moe_forward(gpu_context *ctx, ornith_moe_store *st, int layer, const gpu_buffer *x,
                    int n_tokens, const gpu_buffer *resid, gpu_buffer *out, gpu_buffer *idx_out,
                    gpu_buffer *w_out, const ornith_moe_opts *opts)
{
    if (!ctx) return ORN_EINVAL;
    const int ok = forward_args_ok(ctx, st, layer, x, n_tokens, resid, out, idx_out, w_out,
                                   "gpu_moe_forward");
    if (ok <= 0) return ok;
    const unsigned flags = opts ? opts->flags : 0u;
    if (st->cache && (flags & ORN_MOE_GRAPH))
        return orn_set_err(ctx, ORN_EUNSUPPORTED,
                           "gpu_moe_forward: a streamed store reads its routing back on the "
                           "host; ORN_MOE_GRAPH cannot capture that");
    fwd_arg a = {layer,
                 n_tokens,
                 (const float *)x->dev,
                 resid ? (const float *)resid->dev : NULL,
                 (float *)out->dev,
                 idx_out ? (uint32_t *)idx_out->dev : NULL,
                 w_out ? (float *)w_out->dev : NULL,
                 {opts ? opts->route_mode : ORN_ROUTE_RENORM, flags | ORN_MOE_ASYNC,
                  opts ? opts->ep_first : 0, opts ? opts->ep_count : 0}};
    orn_graph_key key;
    memset(&key, 0, sizeof key);
    key.layer = layer;
    key.n_layers = 1;
    key.T = n_tokens;
    key.mode = a.opts.route_mode;
    key.ep_first = a.opts.ep_first;
    key.ep_count = a.opts.ep_count;
    key.flags = flags & ~ORN_MOE_ASYNC;
    key.x = a.x;
    key.resid = a.resid;
    key.out = a.out;
    key.idx = a.idx;
    key.w = a.w;
    return run_body(ctx, st, &key, fwd_body, &a, !(flags & ORN_MOE_ASYNC));
}

/* gpu_moe_forward with the work buffers in the device's fixed scratch: no
 * hipMalloc, hipFree, graph instantiation or other allocating call. */
int gpu_moe_forward_noalloc(gpu_context *ctx, ornith_moe_store *st, int layer,
                            const gpu_buffer *x, int n_tokens, const gpu_buffer *resid,
                            gpu_buffer *out, gpu_buffer *idx_out, gpu_buffer *w_out,
                            const ornith_moe_opts *opts)
{
    if (!ctx) return ORN_EINVAL;
    const int ok = forward_args_ok(ctx, st, layer, x, n_tokens, resid, out, idx_out, w_out,
                                   "gpu_moe_forward_noalloc");
    if (ok <= 0) return ok;
    if (!ctx->scratch) {
        /* first call on this context: this device's address of the scratch
         * array (looked up once per device, with the device current) */
        hipError_t e = hipSetDevice(ctx->device);
        if (e == hipSuccess) e = (hipError_t)ornk_scratch_resolve(ctx->device, &ctx->scratch);
        /* its first ORNK_SYNC_BYTES are counters that must start at zero (the
         * kernels that use them leave them zeroed); a fill kernel, not a
         * memset, so that a caller may capture this call into a graph */
        if (e == hipSuccess)
            e = (hipError_t)ornk_fill_f32((float *)ctx->scratch, 0.0f, ORNK_SYNC_BYTES / 4,
                                          ctx->stream);
        if (e != hipSuccess) {
            ctx->scratch = NULL;
            return orn_set_err(ctx, ORN_EUNSUPPORTED,
                               "gpu_moe_forward_noalloc: device scratch lookup failed: %s",
                               hipGetErrorString(e));
        }
    }
    const unsigned flags = opts ? opts->flags : 0u;
    if (flags & ORN_MOE_GRAPH)
        return orn_set_err(ctx, ORN_EINVAL,
                           "gpu_moe_forward_noalloc: ORN_MOE_GRAPH (graph instantiation "
                           "allocates)");
    return moe_forward_dev(ctx, st, layer, (const float *)x->dev, n_tokens,
                           resid ? (const float *)resid->dev : NULL, (float *)out->dev,
                           idx_out ? (uint32_t *)idx_out->dev : NULL,
                           w_out ? (float *)w_out->dev : NULL, opts, ctx->scratch);
}

typedef struct {
    int first, n, T;
    float *x, *tmp;
    ornith_moe_opts opts; /* ORN_MOE_NORM | ORN_MOE_ASYNC set */
} stack_arg;

/* Layers ping-pong between x and tmp; the last one writes x in place, which
 * is safe because its only reader of the residual input at the time of the
 * write is the combine kernel itself, element by element. */
static int stack_body(gpu_context *ctx, ornith_moe_store *st, const void *p)
{
    const stack_arg *a = (const stack_arg *)p;
    float *cur = a->x;
    for (int l = 0; l < a->n; ++l) {
        float *dst = (l == a->n - 1) ? a->x : (cur == a->x ? a->tmp : a->x);
        int rc = moe_forward_dev(ctx, st, a->first + l, cur, a->T, cur, dst, NULL, NULL, &a->opts,
                                 NULL);
        if (rc) return rc;
        cur = dst;
    }
    return ORN_OK;
}

int gpu_moe_forward_stack(gpu_context *ctx, ornith_moe_store *st, int first_layer, int n_layers,
                          gpu_buffer *x, gpu_buffer *tmp, int n_tokens, const ornith_moe_opts *opts)
{
    if (!ctx) return ORN_EINVAL;
    if (!st || !x || !tmp || n_tokens < 0 || n_layers < 0 || first_layer < 0 ||
        first_layer + n_layers > st->sh.n_layers)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_moe_forward_stack: bad arguments");
    const size_t act = (size_t)n_tokens * st->sh.d_model * 4;
    if (!check_buf(x, act) || !check_buf(tmp, act) || x == tmp)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_moe_forward_stack: buffer too small");
    if (n_tokens == 0 || n_layers == 0) return ORN_OK;
    const unsigned flags = opts ? opts->flags : 0u;
    if (st->cache && (flags & ORN_MOE_GRAPH))
        return orn_set_err(ctx, ORN_EUNSUPPORTED,
                           "gpu_moe_forward_stack: a streamed store reads its routing back on "
                           "the host; ORN_MOE_GRAPH cannot capture that");
    stack_arg a = {first_layer, n_layers, n_tokens, (float *)x->dev, (float *)tmp->dev,
                   {opts ? opts->route_mode : ORN_ROUTE_RENORM,
                    flags | ORN_MOE_NORM | ORN_MOE_ASYNC, 0, 0}};
    orn_graph_key key;
    memset(&key, 0, sizeof key);
    key.layer = first_layer;
    key.n_layers = n_layers;
    key.T = n_tokens;
    key.mode = a.opts.route_mode;
    key.ep_first = a.opts.ep_first;
    key.ep_count = a.opts.ep_count;
    key.flags = (flags & ~ORN_MOE_ASYNC) | 0x80000000u; /* stack calls never match a layer call */
    key.x = a.x;
    key.out = a.tmp;
    return run_body(ctx, st, &key, stack_body, &a, !(flags & ORN_MOE_ASYNC));
}

int gpu_moe_last_logits(gpu_context *ctx, float *out, size_t max_floats, size_t *n_floats)
{
    if (!ctx) return ORN_EINVAL;
    const size_t n = ctx->last_logits ? (size_t)ctx->last_T * (size_t)ctx->last_E : 0;
    if (n_floats) *n_floats = n;
    const size_t m = n < max_floats ? n : max_floats;
    if (m && !out) return orn_set_err(ctx, ORN_EINVAL, "gpu_moe_last_logits: NULL output");
    if (m) {
        int rc = orn_hip_check(ctx, hipMemcpyAsync(out, ctx->last_logits, m * sizeof(float),
                                                   hipMemcpyDeviceToHost, ctx->stream),
                               "logits copy");
        if (rc) return rc;
    }
    return orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "logits copy");
}

int gpu_moe_last_chained(gpu_context *ctx, int *n_chained)
{
    if (!ctx || !n_chained) return ORN_EINVAL;
    *n_chained = 0;
    if (!ctx->last_ctl) return ORN_OK;
    int rc = orn_hip_check(ctx, hipMemcpyAsync(ctx->ctl_host, ctx->last_ctl, 16 * sizeof(int),
                                               hipMemcpyDeviceToHost, ctx->stream),
                           "stats copy");
    if (rc) return rc;
    rc = orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "stats copy");
    if (!rc) *n_chained = ctx->ctl_host[4];
    return rc;
}

int gpu_moe_last_stats(gpu_context *ctx, int *n_slots, int *n_rows, int *n_literal)
{
    if (!ctx) return ORN_EINVAL;
    memset(ctx->ctl_host, 0, 16 * sizeof(int));
    if (ctx->last_ctl) {
        int rc = orn_hip_check(ctx, hipMemcpyAsync(ctx->ctl_host, ctx->last_ctl, 16 * sizeof(int),
                                                   hipMemcpyDeviceToHost, ctx->stream),
                               "stats copy");
        if (rc) return rc;
    }
    hipStreamSynchronize(ctx->stream);
    if (n_slots) *n_slots = ctx->ctl_host[0];
    if (n_rows) *n_rows = ctx->ctl_host[2];
    if (n_literal) *n_literal = ctx->ctl_host[3];
    return ORN_OK;
}

/* ---------------------------------------------------------------------------
 * Streamed experts (cache.c): prefetch, pinning, statistics
 * ------------------------------------------------------------------------- */
int gpu_moe_store_prefetch(gpu_context *ctx, ornith_moe_store *st, int layer, const int *experts,
                           int n)
{
    if (!ctx) return ORN_EINVAL;
    if (!st || !st->cache)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_moe_store_prefetch: not a streamed store");
    return orn_cache_prefetch(ctx, st->cache, layer, experts, n);
}

int gpu_moe_store_pin(gpu_context *ctx, ornith_moe_store *st, int layer, const int *experts, int n,
                      int pin)
{
    if (!ctx) return ORN_EINVAL;
    if (!st || !st->cache)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_moe_store_pin: not a streamed store");
    return orn_cache_pin(ctx, st->cache, layer, experts, n, pin);
}

int gpu_moe_store_cache_stats(gpu_context *ctx, ornith_moe_store *st, ornith_moe_cache_stats *out,
                              int reset)
{
    if (!ctx) return ORN_EINVAL;
    if (!st || !st->cache)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_moe_store_cache_stats: not a streamed store");
    orn_cache_stats(st->cache, out, reset);
    return ORN_OK;
}
