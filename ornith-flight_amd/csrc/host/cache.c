/* SPDX-License-Identifier: MIT
 *
 * Streamed experts: a store whose experts live in a host tier (pinned host
 * memory, in the device layout) and reach the GPU through a fixed pool of
 * device slots, for models whose experts do not all fit in HBM.
 *
 * The reference's tiering (memory.c:79-421, used by model.c:692-753 and
 * 913-937, 1150-1166) caches dequantized fp32 slices in host memory: a
 * hot-store of pinned experts (memory_hot_promote), an LRU of the rest
 * (memory_get: hit, or miss with the least recently used entry evicted),
 * and a pool of prefetch threads.  Here the same policy runs over device
 * slots holding *quantized* blocks:
 *   - key = (layer, expert), one slot holds the expert's three matrices
 *     (and their MFMA layouts, packed on the device after the copy);
 *   - a forward reads the experts its dispatch chose (and the shared
 *     expert) back from the device, loads the missing ones into free or
 *     least recently used slots (never a pinned one, never one this
 *     forward needs) and rewrites the expert ids of its work items into
 *     slot numbers.  A batch of loads is one kernel that reads the pinned
 *     tier over the host link (cache.hip) and one pack of the batch's MFMA
 *     layouts, whatever the number of experts;
 *   - pinning (memory_hot_promote) loads an expert and exempts it from
 *     eviction; prefetching (memory_prefetch_submit) loads experts ahead
 *     on a copy stream of its own, which the next forward waits for
 *     only if it has to.
 * Statistics follow cache_stats (memory.h:40-55) where they apply.
 */
#include "internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct orn_cache {
    int L, E1, C, prefill, D, H;
    size_t nb, DH;
    /* host tier, [L][E1] experts in the device layout (pinned, mapped), and
     * the device addresses of the same memory */
    uint8_t *h_gate, *h_up, *h_body;
    uint16_t *h_dv;
    void *dh[4];
    /* device slots, [C] experts */
    uint8_t *gate, *up, *body;
    uint16_t *dv;
    uint32_t *pq[2];
    uint16_t *psc[2], *pmn[2];
    float *pd[2], *pdm[2];
    uint8_t *dq;
    uint16_t *dsc;
    float *dd;
    float *dmax;
    int *scmax[2]; /* packer scratch, one per stream */
    /* slot state */
    int *slot_key;                 /* [C] layer*E1 + expert, or -1 */
    unsigned long long *slot_tick; /* [C] last use */
    unsigned long long *slot_fwd;  /* [C] forward that last needed it */
    unsigned char *slot_pin, *slot_need, *slot_pf; /* [C] */
    int *key_slot;                 /* [L*E1] slot, or -1 */
    unsigned long long tick, fwd;
    /* forward plumbing */
    int *h_ctl, *h_slot_e, *h_remap; /* pinned: [4], [E1], [E1] */
    int *d_remap;                    /* [E1] */
    /* load batches: (key, slot) pairs in mapped pinned memory and the slot
     * lists the packer reads; [0] forwards and pins, [1] prefetches */
    int *h_loads[2];
    void *dh_loads[2];
    int *d_slots[2];
    int n_loads[2];
    hipStream_t copy;
    hipEvent_t pf_ev;
    /* pf_pending: the compute stream has not yet been made to wait for the
     * last prefetch batch.  pf_list_busy: that batch's load list (list 1,
     * read by its gather kernel when the kernel runs) may still be unread;
     * cleared only once the host has waited for pf_ev (or quiesced the copy
     * stream), never by the compute stream's wait. */
    int pf_pending, pf_list_busy;
    ornith_moe_cache_stats stats;
    size_t dev_bytes, host_bytes;
};

void orn_cache_destroy(orn_cache *c)
{
    if (!c) return;
    if (c->copy) hipStreamSynchronize(c->copy);
    hipHostFree(c->h_gate);
    hipHostFree(c->h_up);
    hipHostFree(c->h_body);
    hipHostFree(c->h_dv);
    hipHostFree(c->h_ctl);
    hipHostFree(c->h_slot_e);
    hipHostFree(c->h_remap);
    hipHostFree(c->h_loads[0]);
    hipHostFree(c->h_loads[1]);
    void *dev[] = {c->gate, c->up, c->body, c->dv, c->pq[0], c->pq[1], c->psc[0], c->psc[1],
                   c->pmn[0], c->pmn[1], c->pd[0], c->pd[1], c->pdm[0], c->pdm[1], c->dq,
                   c->dsc, c->dd, c->dmax, c->scmax[0], c->scmax[1], c->d_remap,
                   c->d_slots[0], c->d_slots[1]};
    for (size_t i = 0; i < sizeof dev / sizeof dev[0]; ++i) hipFree(dev[i]);
    if (c->pf_ev) hipEventDestroy(c->pf_ev);
    if (c->copy) hipStreamDestroy(c->copy);
    free(c->slot_key);
    free(c->slot_tick);
    free(c->slot_fwd);
    free(c->slot_pin);
    free(c->slot_need);
    free(c->slot_pf);
    free(c->key_slot);
    free(c);
}

static int dev_alloc(gpu_context *ctx, orn_cache *c, void **p, size_t bytes)
{
    if (hipMalloc(p, bytes) != hipSuccess) {
        *p = NULL;
        return orn_set_err(ctx, ORN_ENOMEM, "expert cache: %zu device bytes", bytes);
    }
    c->dev_bytes += bytes;
    return ORN_OK;
}

static int host_alloc(gpu_context *ctx, orn_cache *c, void **p, size_t bytes)
{
    if (hipHostMalloc(p, bytes, hipHostMallocMapped) != hipSuccess) {
        *p = NULL;
        return orn_set_err(ctx, ORN_ENOMEM, "expert cache: %zu pinned host bytes", bytes);
    }
    memset(*p, 0, bytes);
    c->host_bytes += bytes;
    return ORN_OK;
}

orn_cache *orn_cache_create(gpu_context *ctx, const ornith_moe_shape *sh)
{
    orn_cache *c = (orn_cache *)calloc(1, sizeof *c);
    if (!c) return NULL;
    c->L = sh->n_layers;
    c->E1 = sh->n_experts + 1;
    c->C = sh->cache_slots;
    c->prefill = sh->prefill_layout;
    c->D = sh->d_model;
    c->H = sh->hidden;
    c->nb = (size_t)sh->d_model * sh->hidden / 256;
    c->DH = (size_t)sh->d_model * sh->hidden;
    const size_t LE = (size_t)c->L * c->E1, C = (size_t)c->C, nb = c->nb, DH = c->DH;
    int rc = host_alloc(ctx, c, (void **)&c->h_gate, LE * nb * 144);
    if (!rc) rc = host_alloc(ctx, c, (void **)&c->h_up, LE * nb * 144);
    if (!rc) rc = host_alloc(ctx, c, (void **)&c->h_body, LE * nb * 208);
    if (!rc) rc = host_alloc(ctx, c, (void **)&c->h_dv, LE * nb * 2);
    if (!rc) rc = host_alloc(ctx, c, (void **)&c->h_ctl, 4 * sizeof(int));
    if (!rc) rc = host_alloc(ctx, c, (void **)&c->h_slot_e, (size_t)c->E1 * sizeof(int));
    if (!rc) rc = host_alloc(ctx, c, (void **)&c->h_remap, (size_t)c->E1 * sizeof(int));
    for (int i = 0; i < 2 && !rc; ++i) {
        rc = host_alloc(ctx, c, (void **)&c->h_loads[i], (size_t)c->E1 * 2 * sizeof(int));
        if (!rc) rc = dev_alloc(ctx, c, (void **)&c->d_slots[i], (size_t)c->E1 * sizeof(int));
    }
    void *hp[4] = {c->h_gate, c->h_up, c->h_body, c->h_dv};
    for (int i = 0; i < 4 && !rc; ++i)
        if (hipHostGetDevicePointer(&c->dh[i], hp[i], 0) != hipSuccess)
            rc = orn_set_err(ctx, ORN_EHIP, "expert cache: host tier is not device-visible");
    for (int i = 0; i < 2 && !rc; ++i)
        if (hipHostGetDevicePointer(&c->dh_loads[i], c->h_loads[i], 0) != hipSuccess)
            rc = orn_set_err(ctx, ORN_EHIP, "expert cache: load list is not device-visible");
    if (!rc) rc = dev_alloc(ctx, c, (void **)&c->gate, C * nb * 144);
    if (!rc) rc = dev_alloc(ctx, c, (void **)&c->up, C * nb * 144);
    if (!rc) rc = dev_alloc(ctx, c, (void **)&c->body, C * nb * 208);
    if (!rc) rc = dev_alloc(ctx, c, (void **)&c->dv, C * nb * 2);
    if (!rc) rc = dev_alloc(ctx, c, (void **)&c->d_remap, (size_t)c->E1 * sizeof(int));
    for (int i = 0; i < 2 && !rc; ++i) rc = dev_alloc(ctx, c, (void **)&c->scmax[i], sizeof(int));
    if (!rc && c->prefill) {
        for (int m = 0; m < 2 && !rc; ++m) {
            rc = dev_alloc(ctx, c, (void **)&c->pq[m], C * DH / 2);
            if (!rc) rc = dev_alloc(ctx, c, (void **)&c->psc[m], C * DH / 16);
            if (!rc) rc = dev_alloc(ctx, c, (void **)&c->pmn[m], C * DH / 16);
            if (!rc) rc = dev_alloc(ctx, c, (void **)&c->pd[m], C * DH / 64);
            if (!rc) rc = dev_alloc(ctx, c, (void **)&c->pdm[m], C * DH / 64);
        }
        if (!rc) rc = dev_alloc(ctx, c, (void **)&c->dq, C * ORNK_DQ_BYTES(DH));
        if (!rc) rc = dev_alloc(ctx, c, (void **)&c->dsc, C * DH / 8);
        if (!rc) rc = dev_alloc(ctx, c, (void **)&c->dd, C * DH / 64);
        if (!rc) rc = dev_alloc(ctx, c, (void **)&c->dmax, C * 3 * sizeof(float));
    }
    if (!rc && (hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking) != hipSuccess ||
                hipEventCreateWithFlags(&c->pf_ev, hipEventDisableTiming) != hipSuccess))
        rc = orn_set_err(ctx, ORN_EHIP, "expert cache: copy stream");
    c->slot_key = (int *)malloc(C * sizeof(int));
    c->slot_tick = (unsigned long long *)calloc(C, sizeof(unsigned long long));
    c->slot_fwd = (unsigned long long *)calloc(C, sizeof(unsigned long long));
    c->slot_pin = (unsigned char *)calloc(C, 1);
    c->slot_need = (unsigned char *)calloc(C, 1);
    c->slot_pf = (unsigned char *)calloc(C, 1);
    c->key_slot = (int *)malloc(LE * sizeof(int));
    if (!rc && (!c->slot_key || !c->slot_tick || !c->slot_fwd || !c->slot_pin || !c->slot_need ||
                !c->slot_pf || !c->key_slot))
        rc = orn_set_err(ctx, ORN_ENOMEM, "expert cache: host tables");
    if (rc) {
        orn_cache_destroy(c);
        return NULL;
    }
    for (size_t i = 0; i < C; ++i) c->slot_key[i] = -1;
    for (size_t i = 0; i < LE; ++i) c->key_slot[i] = -1;
    c->fwd = 1; /* slot_fwd == fwd marks the slots of the last forward */
    c->stats.slots = c->C;
    return c;
}

size_t orn_cache_device_bytes(const orn_cache *c) { return c->dev_bytes; }
size_t orn_cache_host_bytes(const orn_cache *c) { return c->host_bytes; }

void orn_cache_host_tier(orn_cache *c, uint8_t **gate, uint8_t **up, uint8_t **body,
                         uint16_t **dv)
{
    *gate = c->h_gate;
    *up = c->h_up;
    *body = c->h_body;
    *dv = c->h_dv;
}

void orn_cache_slot_arrays(orn_cache *c, ornk_moe_args *a)
{
    a->gate = c->gate;
    a->up = c->up;
    a->down_body = c->body;
    a->down_d = c->dv;
    if (!c->prefill) return;
    for (int m = 0; m < 2; ++m) {
        a->gu_pf.pq[m] = c->pq[m];
        a->gu_pf.psc[m] = c->psc[m];
        a->gu_pf.pmn[m] = c->pmn[m];
        a->gu_pf.pd[m] = c->pd[m];
        a->gu_pf.pdm[m] = c->pdm[m];
    }
    a->gu_pf.dmax = c->dmax;
    a->dn_pf.dq = c->dq;
    a->dn_pf.dsc = c->dsc;
    a->dn_pf.dd = c->dd;
    a->dn_pf.dmax = c->dmax;
}

/* Before the host tier of a layer is rewritten: no copy may still read it. */
int orn_cache_quiesce(gpu_context *ctx, orn_cache *c)
{
    const int rc = orn_hip_check(ctx, hipStreamSynchronize(c->copy), "expert cache: copy stream");
    if (!rc) c->pf_pending = c->pf_list_busy = 0;
    return rc;
}

/* Experts [first, first + n) of a layer changed in the host tier: their
 * device copies are stale. */
void orn_cache_invalidate(orn_cache *c, int layer, int first, int n)
{
    for (int e = first; e < first + n; ++e) {
        const int key = layer * c->E1 + e, s = c->key_slot[key];
        if (s < 0) continue;
        c->key_slot[key] = -1;
        c->slot_key[s] = -1;
        c->slot_pin[s] = 0;
        c->slot_pf[s] = 0;
    }
}

/* Give slot s to expert `key` (evicting its holder) and add the load to
 * batch `which`; flush_loads copies and packs the batch. */
static void stage_load(orn_cache *c, int key, int s, int which)
{
    if (c->slot_key[s] >= 0) {
        c->key_slot[c->slot_key[s]] = -1;
        c->stats.evictions++;
    }
    c->slot_key[s] = key;
    c->key_slot[key] = s;
    c->slot_pin[s] = 0;
    int *l = c->h_loads[which] + 2 * c->n_loads[which]++;
    l[0] = key;
    l[1] = s;
    c->stats.bytes_uploaded += c->nb * 498; /* 144 + 144 + 208 + 2 per block */
}

/* The staged loads of batch `which`, on stream st: one gather kernel over
 * the host link, then the MFMA layouts of the loaded slots. */
static int flush_loads(gpu_context *ctx, orn_cache *c, hipStream_t st, int which)
{
    const int n = c->n_loads[which];
    c->n_loads[which] = 0;
    if (n == 0) return ORN_OK;
    ornk_gather_args g;
    memset(&g, 0, sizeof g);
    g.loads = (const int *)c->dh_loads[which];
    g.n = n;
    g.h_gate = (const uint8_t *)c->dh[0];
    g.h_up = (const uint8_t *)c->dh[1];
    g.h_body = (const uint8_t *)c->dh[2];
    g.h_d = (const uint16_t *)c->dh[3];
    g.gate = c->gate;
    g.up = c->up;
    g.body = c->body;
    g.d = c->dv;
    g.slots_out = c->d_slots[which];
    g.dmax = c->prefill ? c->dmax : NULL;
    g.nb = c->nb;
    int rc = orn_hip_check(ctx, (hipError_t)ornk_cache_gather(&g, st), "expert cache: load");
    if (rc || !c->prefill) return rc;
    ornk_pack_args pa;
    memset(&pa, 0, sizeof pa);
    pa.D = c->D;
    pa.H = c->H;
    pa.n_e = n;
    pa.gu[0] = c->gate;
    pa.gu[1] = c->up;
    pa.down_body = c->body;
    pa.down_d = c->dv;
    for (int m = 0; m < 2; ++m) {
        pa.pq[m] = c->pq[m];
        pa.psc[m] = c->psc[m];
        pa.pmn[m] = c->pmn[m];
        pa.pd[m] = c->pd[m];
        pa.pdm[m] = c->pdm[m];
    }
    pa.dq = c->dq;
    pa.dsc = c->dsc;
    pa.dd = c->dd;
    pa.dmax = c->dmax;
    pa.scmax = c->scmax[which];
    pa.slots = c->d_slots[which];
    return orn_hip_check(ctx, (hipError_t)ornk_pack_prefill(&pa, st), "expert cache: layouts");
}

/* A slot for a new expert: a free one, else the least recently used one
 * that is not pinned, not needed by the forward being prepared and (with
 * busy_fwd) not used by the forward still in flight. */
static int victim(const orn_cache *c, int busy_fwd)
{
    int best = -1;
    for (int s = 0; s < c->C; ++s) {
        if (c->slot_key[s] < 0) return s;
        if (c->slot_pin[s] || c->slot_need[s]) continue;
        if (busy_fwd && c->slot_fwd[s] == c->fwd) continue;
        if (best < 0 || c->slot_tick[s] < c->slot_tick[best]) best = s;
    }
    return best;
}

/* Wait (on the compute stream) for the prefetches issued so far. */
static int join_prefetch(gpu_context *ctx, orn_cache *c)
{
    if (!c->pf_pending) return ORN_OK;
    c->pf_pending = 0;
    return orn_hip_check(ctx, hipStreamWaitEvent(ctx->stream, c->pf_ev, 0),
                         "expert cache: prefetch wait");
}

/* After the dispatch of a forward of `layer`: make its experts resident and
 * turn the expert ids of its items and slots into slot numbers. */
int orn_cache_prepare(gpu_context *ctx, orn_cache *c, int layer, ornk_moe_args *a)
{
    const int E1 = c->E1;
    hipStream_t s = ctx->stream;
    int rc = orn_hip_check(ctx, hipMemcpyAsync(c->h_ctl, a->ctl, 4 * sizeof(int),
                                               hipMemcpyDeviceToHost, s), "expert cache: ctl");
    if (!rc)
        rc = orn_hip_check(ctx, hipMemcpyAsync(c->h_slot_e, a->slot_expert, (size_t)E1 * sizeof(int),
                                               hipMemcpyDeviceToHost, s), "expert cache: slots");
    if (!rc) rc = orn_hip_check(ctx, hipStreamSynchronize(s), "expert cache: read back");
    if (rc) return rc;
    const int n = c->h_ctl[0];
    if (n < 0 || n > E1) return orn_set_err(ctx, ORN_EHIP, "expert cache: %d slots read back", n);
    if (n > c->C)
        return orn_set_err(ctx, ORN_EINVAL,
                           "expert cache: this forward needs %d experts; the cache has %d slots",
                           n, c->C);
    c->fwd++;
    memset(c->slot_need, 0, (size_t)c->C);
    int misses[257], n_miss = 0;
    for (int i = 0; i < n; ++i) {
        const int e = c->h_slot_e[i];
        if (e < 0 || e >= E1) return orn_set_err(ctx, ORN_EHIP, "expert cache: expert id %d", e);
        const int key = layer * E1 + e, sl = c->key_slot[key];
        if (sl >= 0) {
            c->stats.hits++;
            if (c->slot_pf[sl]) c->stats.prefetch_hits++;
            c->slot_pf[sl] = 0;
            c->slot_need[sl] = 1;
            c->slot_tick[sl] = ++c->tick;
            c->slot_fwd[sl] = c->fwd;
        } else {
            misses[n_miss++] = key;
        }
    }
    /* a prefetch may still write a slot this forward reads or replaces */
    if ((rc = join_prefetch(ctx, c))) return rc;
    for (int i = 0; i < n_miss; ++i) {
        const int sl = victim(c, 0);
        if (sl < 0) {
            int held = 0;
            for (int j = 0; j < c->C; ++j) held += c->slot_pin[j] || c->slot_need[j];
            /* the slots already given to this forward's misses are loaded,
             * so that every slot holds the expert it is mapped to */
            flush_loads(ctx, c, s, 0);
            return orn_set_err(ctx, ORN_EINVAL,
                               "expert cache: no slot to evict (%d slots, %d pinned or needed "
                               "by this forward)", c->C, held);
        }
        c->stats.misses++;
        stage_load(c, misses[i], sl, 0);
        c->slot_pf[sl] = 0;
        c->slot_need[sl] = 1;
        c->slot_tick[sl] = ++c->tick;
        c->slot_fwd[sl] = c->fwd;
    }
    if ((rc = flush_loads(ctx, c, s, 0))) return rc;
    for (int i = 0; i < n; ++i) {
        const int e = c->h_slot_e[i];
        c->h_remap[e] = c->key_slot[layer * E1 + e];
    }
    rc = orn_hip_check(ctx, hipMemcpyAsync(c->d_remap, c->h_remap, (size_t)E1 * sizeof(int),
                                           hipMemcpyHostToDevice, s), "expert cache: remap");
    if (rc) return rc;
    rc = orn_hip_check(ctx, (hipError_t)ornk_remap_items(a->items, a->slot_expert, a->ctl,
                                                         c->d_remap, a->items_max, E1, s),
                       "expert cache: remap items");
    if (rc) return rc;
    orn_cache_slot_arrays(c, a);
    return ORN_OK;
}

static int check_ids(gpu_context *ctx, const orn_cache *c, int layer, const int *experts, int n)
{
    if (layer < 0 || layer >= c->L || n < 0 || (n && !experts))
        return orn_set_err(ctx, ORN_EINVAL, "expert cache: bad layer or expert list");
    for (int i = 0; i < n; ++i)
        if (experts[i] < 0 || experts[i] >= c->E1)
            return orn_set_err(ctx, ORN_EINVAL, "expert cache: expert %d out of range",
                               experts[i]);
    return ORN_OK;
}

int orn_cache_prefetch(gpu_context *ctx, orn_cache *c, int layer, const int *experts, int n)
{
    int rc = check_ids(ctx, c, layer, experts, n);
    if (rc) return rc;
    /* the previous prefetch batch's list must have been read, whether or not
     * a forward has joined that batch since (a join only orders the compute
     * stream; the gather may still be queued on the copy stream) */
    if (c->pf_list_busy) {
        if ((rc = orn_hip_check(ctx, hipEventSynchronize(c->pf_ev), "expert cache: prefetch")))
            return rc;
        c->pf_list_busy = 0;
    }
    memset(c->slot_need, 0, (size_t)c->C);
    for (int i = 0; i < n; ++i) {
        const int key = layer * c->E1 + experts[i];
        int sl = c->key_slot[key];
        if (sl >= 0) {
            c->slot_need[sl] = 1;
            continue;
        }
        sl = victim(c, 1);
        if (sl < 0) break; /* nothing evictable: a prefetch is only a hint */
        stage_load(c, key, sl, 1);
        c->stats.prefetches++;
        c->slot_pf[sl] = 1;
        c->slot_need[sl] = 1;
        c->slot_tick[sl] = ++c->tick;
    }
    memset(c->slot_need, 0, (size_t)c->C);
    if (c->n_loads[1] == 0) return ORN_OK;
    c->pf_list_busy = 1; /* list 1 is read by the gather when it runs */
    rc = flush_loads(ctx, c, c->copy, 1);
    if (!rc)
        rc = orn_hip_check(ctx, hipEventRecord(c->pf_ev, c->copy), "expert cache: prefetch event");
    if (!rc) {
        c->pf_pending = 1;
    } else {
        /* no event covers what was enqueued: wait for the copy stream */
        hipStreamSynchronize(c->copy);
        c->pf_list_busy = 0;
    }
    return rc;
}

int orn_cache_pin(gpu_context *ctx, orn_cache *c, int layer, const int *experts, int n, int pin)
{
    int rc = check_ids(ctx, c, layer, experts, n);
    if (rc) return rc;
    if ((rc = join_prefetch(ctx, c))) return rc;
    /* the load list is rewritten: the last forward's batch must be done */
    if ((rc = orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "expert cache: pin")))
        return rc;
    memset(c->slot_need, 0, (size_t)c->C);
    for (int i = 0; i < n; ++i) {
        const int key = layer * c->E1 + experts[i];
        int sl = c->key_slot[key];
        if (sl < 0 && pin) {
            sl = victim(c, 1);
            if (sl < 0) {  /* the slots already given are loaded below */
                rc = orn_set_err(ctx, ORN_EINVAL, "expert cache: no slot left to pin into");
                break;
            }
            stage_load(c, key, sl, 0);
            c->stats.misses++;
            c->slot_tick[sl] = ++c->tick;
        }
        if (sl >= 0) {
            c->slot_pin[sl] = (unsigned char)(pin != 0);
            c->slot_need[sl] = 1;
        }
    }
    memset(c->slot_need, 0, (size_t)c->C);
    const int frc = flush_loads(ctx, c, ctx->stream, 0);
    if (!rc) rc = frc;
    const int src = orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "expert cache: pin");
    return rc ? rc : src;
}

void orn_cache_stats(orn_cache *c, ornith_moe_cache_stats *out, int reset)
{
    ornith_moe_cache_stats s = c->stats;
    s.slots = c->C;
    s.resident = 0;
    s.pinned = 0;
    for (int i = 0; i < c->C; ++i) {
        s.resident += c->slot_key[i] >= 0;
        s.pinned += c->slot_pin[i] != 0;
    }
    s.device_bytes = c->dev_bytes;
    s.host_bytes = c->host_bytes;
    if (out) *out = s;
    if (reset) {
        memset(&c->stats, 0, sizeof c->stats);
        c->stats.slots = c->C;
    }
}
