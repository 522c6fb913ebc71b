/* SPDX-License-Identifier: MIT
 *
 * Internal definitions shared by the C99 host files of libornith_hip.
 */
#ifndef ORNITH_HOST_INTERNAL_H
#define ORNITH_HOST_INTERNAL_H

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include "../../../include/ornith/gpu.h"
#include "../../../include/ornith/ornith_hip.h"
#include "../kernels/launch.h"

#define ORN_PROF_MAX_NAMES 32
#define ORN_PROF_MAX_PENDING 8192

typedef struct {
    int name_id;
    hipEvent_t start, stop;
} orn_prof_rec;

struct gpu_buffer {
    void *dev;   /* device address used by kernels */
    void *host;  /* host address for GPU_BUF_SHARED (pinned, device-mapped) */
    size_t size;
    gpu_buffer_flags flags;
};

typedef struct {
    /* grow-only device workspace for the MoE forward */
    void *base;
    size_t bytes;
} orn_workspace;

struct gpu_context {
    int device;
    hipStream_t stream;
    size_t used_memory;
    char err[256];
    orn_workspace ws;
    /* this device's fixed scratch, resolved by the first
     * gpu_moe_forward_noalloc call on the context (NULL until then) */
    void *scratch;
    /* counters and the generation word of the certified routing kernel
     * (ORNK_SYNC_BYTES, zeroed on the stream at allocation; the kernel keeps
     * its counter at zero between launches).  Its own allocation: the
     * workspace is shared with other ops and is reallocated as it grows. */
    int *sync;
    /* device counters read back after a forward */
    int *ctl_host; /* pinned mirror of the last forward's counters */
    int *last_ctl; /* device counters of the last forward (inside the workspace) */
    float *last_logits; /* [last_T][last_E] router logits of the last forward */
    int last_T, last_E;
    /* profiling */
    int prof_on;
    int prof_n_names;
    char prof_names[ORN_PROF_MAX_NAMES][32];
    double prof_total_ms[ORN_PROF_MAX_NAMES];
    long prof_calls[ORN_PROF_MAX_NAMES];
    orn_prof_rec *prof_pending;
    int prof_n_pending;
    hipEvent_t *prof_pool;
    int prof_pool_n, prof_pool_used;
};

/* error helpers (gpu_hip.c) */
int orn_set_err(gpu_context *ctx, int code, const char *fmt, ...);
int orn_hip_check(gpu_context *ctx, hipError_t e, const char *what);

/* profiling hooks (moe.c) */
int orn_prof_begin(gpu_context *ctx, const char *name);
void orn_prof_end(gpu_context *ctx, int slot);
int orn_prof_kernel(gpu_context *ctx, const char *name, hipEvent_t *start, hipEvent_t *stop);

/* the shape a store was created with (moe.c) */
const ornith_moe_shape *orn_store_shape(const ornith_moe_store *st);

/* fp16 bits -> float with the reference's rule, gguf.c:16-26 (prefill_pack.c) */
float orn_quirk_half(uint16_t h);

/* streamed experts (cache.c): a host tier and a pool of device slots */
typedef struct orn_cache orn_cache;
orn_cache *orn_cache_create(gpu_context *ctx, const ornith_moe_shape *sh);
void orn_cache_destroy(orn_cache *c);
size_t orn_cache_device_bytes(const orn_cache *c);
size_t orn_cache_host_bytes(const orn_cache *c);
/* base pointers of the host tier ([L][E+1] experts, the device layout) */
void orn_cache_host_tier(orn_cache *c, uint8_t **gate, uint8_t **up, uint8_t **body,
                         uint16_t **dv);
int orn_cache_quiesce(gpu_context *ctx, orn_cache *c);
void orn_cache_invalidate(orn_cache *c, int layer, int first, int n);
void orn_cache_slot_arrays(orn_cache *c, ornk_moe_args *a);
int orn_cache_prepare(gpu_context *ctx, orn_cache *c, int layer, ornk_moe_args *a);
int orn_cache_prefetch(gpu_context *ctx, orn_cache *c, int layer, const int *experts, int n);
int orn_cache_pin(gpu_context *ctx, orn_cache *c, int layer, const int *experts, int n, int pin);
void orn_cache_stats(orn_cache *c, ornith_moe_cache_stats *out, int reset);

/* workspace (moe.c) */
void *orn_ws_get(gpu_context *ctx, size_t bytes);
void orn_ws_release(gpu_context *ctx);

#endif /* ORNITH_HOST_INTERNAL_H */
