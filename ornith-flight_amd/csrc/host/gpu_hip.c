/* SPDX-License-Identifier: MIT
 *
 * gpu.h implemented on HIP for MI355X (gfx950).  C99.
 *
 * Contract followed (reference engine/src/gpu.c, the CPU backend):
 *   - gpu_init/gpu_destroy create/free a context (gpu.c:24-37);
 *   - gpu_alloc returns zero-filled buffers, NULL for size 0 or failure, and
 *     gpu_memory_used counts exactly the requested bytes (gpu.c:41-64);
 *   - copies clamp to the buffer sizes (gpu.c:76-100);
 *   - every call is synchronous at return and a silent no-op on NULL or
 *     out-of-range arguments (here: also when sizes exceed the buffers,
 *     because a device kernel must never read past an allocation).
 * GPU_BUF_SHARED buffers are pinned host allocations mapped into the device
 * address space, so host writes through gpu_get_cpu_ptr are visible to later
 * calls (t_gpu.c:46-66, inference.c:169-172).
 */
#include "internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int orn_set_err(gpu_context *ctx, int code, const char *fmt, ...)
{
    if (ctx) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(ctx->err, sizeof ctx->err, fmt, ap);
        va_end(ap);
    }
    return code;
}

int orn_hip_check(gpu_context *ctx, hipError_t e, const char *what)
{
    if (e == hipSuccess) return ORN_OK;
    return orn_set_err(ctx, ORN_EHIP, "%s: %s", what, hipGetErrorString(e));
}

const char *gpu_last_error(gpu_context *ctx) { return ctx ? ctx->err : "no context"; }

gpu_context *gpu_init(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return NULL;
    gpu_context *ctx = (gpu_context *)calloc(1, sizeof(gpu_context));
    if (!ctx) return NULL;
    if (hipGetDevice(&ctx->device) != hipSuccess) ctx->device = 0;
    if (hipSetDevice(ctx->device) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        free(ctx);
        return NULL;
    }
    if (hipHostMalloc((void **)&ctx->ctl_host, 64 * sizeof(int), hipHostMallocDefault) !=
        hipSuccess) {
        hipStreamDestroy(ctx->stream);
        free(ctx);
        return NULL;
    }
    memset(ctx->ctl_host, 0, 64 * sizeof(int));
    return ctx;
}

void gpu_destroy(gpu_context *ctx)
{
    if (!ctx) return;
    hipStreamSynchronize(ctx->stream);
    gpu_profile_enable(ctx, 0);
    orn_ws_release(ctx);
    if (ctx->sync) hipFree(ctx->sync);
    if (ctx->ctl_host) hipHostFree(ctx->ctl_host);
    hipStreamDestroy(ctx->stream);
    memset(ctx, 0, sizeof *ctx);
    free(ctx);
}

gpu_buffer *gpu_alloc(gpu_context *ctx, size_t size, gpu_buffer_flags flags)
{
    if (!ctx || size == 0) return NULL;
    gpu_buffer *b = (gpu_buffer *)calloc(1, sizeof(gpu_buffer));
    if (!b) return NULL;
    b->size = size;
    b->flags = flags;
    if (flags & GPU_BUF_SHARED) {
        if (hipHostMalloc(&b->host, size, hipHostMallocMapped) != hipSuccess) {
            free(b);
            return NULL;
        }
        memset(b->host, 0, size);
        if (hipHostGetDevicePointer(&b->dev, b->host, 0) != hipSuccess) {
            hipHostFree(b->host);
            free(b);
            return NULL;
        }
    } else {
        if (hipMalloc(&b->dev, size) != hipSuccess) {
            free(b);
            return NULL;
        }
        if (hipMemsetAsync(b->dev, 0, size, ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess) {
            hipFree(b->dev);
            free(b);
            return NULL;
        }
    }
    ctx->used_memory += size;
    return b;
}

void gpu_free(gpu_context *ctx, gpu_buffer *buf)
{
    if (!ctx || !buf) return;
    hipStreamSynchronize(ctx->stream);
    ctx->used_memory -= buf->size;
    if (buf->flags & GPU_BUF_SHARED) hipHostFree(buf->host);
    else hipFree(buf->dev);
    memset(buf, 0, sizeof *buf);
    free(buf);
}

void *gpu_get_cpu_ptr(gpu_context *ctx, gpu_buffer *buf)
{
    if (!buf) return NULL;
    if (ctx) hipStreamSynchronize(ctx->stream);
    return (buf->flags & GPU_BUF_SHARED) ? buf->host : NULL;
}

size_t gpu_buffer_size(gpu_context *ctx, const gpu_buffer *buf)
{
    (void)ctx;
    return buf ? buf->size : 0;
}

void *gpu_device_ptr(gpu_context *ctx, gpu_buffer *buf)
{
    (void)ctx;
    return buf ? buf->dev : NULL;
}

int gpu_device_info(gpu_context *ctx, char *name, size_t name_len, int *n_cus, size_t *hbm_bytes)
{
    if (!ctx) return ORN_EINVAL;
    hipDeviceProp_t p;
    int rc = orn_hip_check(ctx, hipGetDeviceProperties(&p, ctx->device), "hipGetDeviceProperties");
    if (rc) return rc;
    if (name && name_len) snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    if (n_cus) *n_cus = p.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
    return ORN_OK;
}

int gpu_probe_read_bandwidth(gpu_context *ctx, size_t bytes, int iters, double *gb_per_s)
{
    if (!ctx || !gb_per_s || bytes < 16 || iters < 1) return ORN_EINVAL;
    bytes &= ~(size_t)15;
    void *buf = NULL;
    uint32_t *out = NULL;
    hipEvent_t e0 = NULL, e1 = NULL;
    int rc = ORN_OK;
    if (hipMalloc(&buf, bytes) != hipSuccess ||
        hipMalloc((void **)&out, (size_t)ORNK_STREAM_GRID * 256 * sizeof(uint32_t)) != hipSuccess) {
        rc = orn_set_err(ctx, ORN_ENOMEM, "probe buffer of %zu bytes", bytes);
        goto done;
    }
    if ((rc = orn_hip_check(ctx, hipEventCreate(&e0), "hipEventCreate")) ||
        (rc = orn_hip_check(ctx, hipEventCreate(&e1), "hipEventCreate")) ||
        (rc = orn_hip_check(ctx, hipMemsetAsync(buf, 0x5a, bytes, ctx->stream), "hipMemsetAsync")) ||
        (rc = orn_hip_check(ctx, (hipError_t)ornk_stream_read(buf, bytes, out, ctx->stream),
                            "stream read")) ||
        (rc = orn_hip_check(ctx, hipEventRecord(e0, ctx->stream), "hipEventRecord")))
        goto done;
    for (int i = 0; i < iters; ++i)
        if ((rc = orn_hip_check(ctx, (hipError_t)ornk_stream_read(buf, bytes, out, ctx->stream),
                                "stream read")))
            goto done;
    float ms = 0.0f;
    if ((rc = orn_hip_check(ctx, hipEventRecord(e1, ctx->stream), "hipEventRecord")) ||
        (rc = orn_hip_check(ctx, hipEventSynchronize(e1), "hipEventSynchronize")) ||
        (rc = orn_hip_check(ctx, hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime")))
        goto done;
    *gb_per_s = ms > 0.0f ? (double)bytes * iters / ((double)ms * 1e-3) / 1e9 : 0.0;
done:
    hipStreamSynchronize(ctx->stream);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (out) hipFree(out);
    if (buf) hipFree(buf);
    return rc;
}

static void sync_ctx(gpu_context *ctx) { hipStreamSynchronize(ctx->stream); }

void gpu_copy_to_device(gpu_context *ctx, gpu_buffer *dst, const void *src, size_t size)
{
    if (!ctx || !dst || !src) return;
    size_t n = size < dst->size ? size : dst->size;
    if (n == 0) return;
    if (dst->flags & GPU_BUF_SHARED) {
        sync_ctx(ctx);
        memcpy(dst->host, src, n);
        return;
    }
    hipMemcpyAsync(dst->dev, src, n, hipMemcpyHostToDevice, ctx->stream);
    sync_ctx(ctx);
}

void gpu_copy_to_host(gpu_context *ctx, void *dst, const gpu_buffer *src, size_t size)
{
    if (!ctx || !dst || !src) return;
    size_t n = size < src->size ? size : src->size;
    if (n == 0) return;
    sync_ctx(ctx);
    if (src->flags & GPU_BUF_SHARED) {
        memcpy(dst, src->host, n);
        return;
    }
    hipMemcpyAsync(dst, src->dev, n, hipMemcpyDeviceToHost, ctx->stream);
    sync_ctx(ctx);
}

void gpu_copy_buffer(gpu_context *ctx, gpu_buffer *dst, const gpu_buffer *src, size_t size)
{
    if (!ctx || !dst || !src) return;
    size_t n = size;
    if (n > dst->size) n = dst->size;
    if (n > src->size) n = src->size;
    if (n == 0) return;
    hipMemcpyAsync(dst->dev, src->dev, n, hipMemcpyDefault, ctx->stream);
    sync_ctx(ctx);
}

static int fits(const gpu_buffer *b, size_t n_floats) { return b && n_floats <= b->size / 4; }

void gpu_matmul(gpu_context *ctx, gpu_buffer *C, const gpu_buffer *A, const gpu_buffer *B, int M,
                int N, int K, quant_mode a_quant, quant_mode b_quant)
{
    (void)a_quant;
    (void)b_quant;
    if (!ctx || !C || !A || !B || M <= 0 || N <= 0 || K < 0) return;
    if (!fits(A, (size_t)M * K) || !fits(B, (size_t)K * N) || !fits(C, (size_t)M * N)) return;
    orn_hip_check(ctx, (hipError_t)ornk_matmul_f32((float *)C->dev, (const float *)A->dev,
                                                   (const float *)B->dev, M, N, K, ctx->stream),
                  "gpu_matmul");
    sync_ctx(ctx);
}

void gpu_matmul_int4(gpu_context *ctx, gpu_buffer *C, const gpu_buffer *A_quant,
                     const gpu_buffer *A_scale, int M, int N, int K)
{
    /* The CPU backend zero-fills C (gpu.c:131-140); no int4 format is defined. */
    (void)A_quant;
    (void)A_scale;
    (void)K;
    if (!ctx || !C || M <= 0 || N <= 0) return;
    size_t n = (size_t)M * N;
    if (n > C->size / 4) n = C->size / 4;
    ornk_fill_f32((float *)C->dev, 0.0f, n, ctx->stream);
    sync_ctx(ctx);
}

void gpu_rmsnorm(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x, const gpu_buffer *weight,
                 int rows, int dim)
{
    (void)rows; /* one row, as gpu.c:144-156 */
    if (!ctx || !out || !x || !weight || dim <= 0) return;
    if (!fits(out, (size_t)dim) || !fits(x, (size_t)dim) || !fits(weight, (size_t)dim)) return;
    ornk_rmsnorm((float *)out->dev, (const float *)x->dev, (const float *)weight->dev, 1, dim,
                 ctx->stream);
    sync_ctx(ctx);
}

void gpu_silu(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x, int n)
{
    if (!ctx || !out || !x || n <= 0) return;
    if (!fits(out, (size_t)n) || !fits(x, (size_t)n)) return;
    ornk_silu((float *)out->dev, (const float *)x->dev, n, ctx->stream);
    sync_ctx(ctx);
}

void gpu_silu_mul(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *gate, const gpu_buffer *up,
                  int n)
{
    if (!ctx || !out || !gate || !up || n <= 0) return;
    if (!fits(out, (size_t)n) || !fits(gate, (size_t)n) || !fits(up, (size_t)n)) return;
    ornk_silu_mul((float *)out->dev, (const float *)gate->dev, (const float *)up->dev, n,
                  ctx->stream);
    sync_ctx(ctx);
}

/* RoPE, attention and the DeltaNet step are no-ops in the CPU backend
 * (gpu.c:188-206); the MoE hot path does not use them. */
/* gpu_metal.m:495-548 + ops.metal:113-139: rotate the first min(head_dim, 64)
 * dims of each of the n_heads Q heads and n_kv_heads K heads (one position,
 * pos_start; seq_len is unused, as there). */
void gpu_rope(gpu_context *ctx, gpu_buffer *Q, gpu_buffer *K, int seq_len, int head_dim,
              int n_heads, int n_kv_heads, float base, int pos_start)
{
    (void)seq_len;
    if (!ctx || !Q || !K || head_dim <= 0 || n_heads < 0 || n_kv_heads < 0) return;
    if (!fits(Q, (size_t)n_heads * head_dim) || !fits(K, (size_t)n_kv_heads * head_dim)) return;
    orn_hip_check(ctx, (hipError_t)ornk_rope((float *)Q->dev, (float *)K->dev, head_dim, n_heads,
                                             n_kv_heads, pos_start, base, ctx->stream),
                  "gpu_rope");
    sync_ctx(ctx);
}

/* gpu_metal.m:550-583 + attention.metal:17-68: one head, Q/K/V/out
 * [seq_len][head_dim], scale 1/sqrt(head_dim), every key for every query.
 * head_dim up to 256 (the kernel's register tile); larger is refused with an
 * error message. */
void gpu_attention(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *Q,
                   const gpu_buffer *K_cache, const gpu_buffer *V_cache, int seq_len, int head_dim)
{
    if (!ctx || !out || !Q || !K_cache || !V_cache || seq_len <= 0 || head_dim <= 0) return;
    const size_t n = (size_t)seq_len * head_dim;
    if (!fits(out, n) || !fits(Q, n) || !fits(K_cache, n) || !fits(V_cache, n)) return;
    if (head_dim > 256) {
        orn_set_err(ctx, ORN_EUNSUPPORTED, "gpu_attention: head_dim %d > 256", head_dim);
        return;
    }
    const float scale = 1.0f / sqrtf((float)head_dim);
    if (head_dim % 4 == 0) {
        /* matrix cores; the key splits' partials live in the context workspace */
        const size_t wsb = ornk_attention_mma_ws(seq_len, head_dim);
        void *ws = wsb ? orn_ws_get(ctx, wsb) : NULL;
        if (wsb && !ws) return;
        orn_hip_check(ctx, (hipError_t)ornk_attention_mma((float *)out->dev, (const float *)Q->dev,
                                                          (const float *)K_cache->dev,
                                                          (const float *)V_cache->dev, seq_len,
                                                          head_dim, scale, ws, ctx->stream),
                      "gpu_attention");
    } else {
        orn_hip_check(ctx, (hipError_t)ornk_attention((float *)out->dev, (const float *)Q->dev,
                                                      (const float *)K_cache->dev,
                                                      (const float *)V_cache->dev, seq_len,
                                                      head_dim, scale, ctx->stream),
                      "gpu_attention");
    }
    sync_ctx(ctx);
}

/* A no-op, as in both reference backends (gpu.c:202-206, gpu_metal.m:587-591):
 * the declaration has no output and no gate.  The Metal shader's step
 * (attention.metal:80-108) is gpu_deltanet_step_gated. */
void gpu_deltanet_step(gpu_context *ctx, gpu_buffer *state, const gpu_buffer *Q,
                       const gpu_buffer *K, const gpu_buffer *V, int dim)
{
    (void)ctx; (void)state; (void)Q; (void)K; (void)V; (void)dim;
}

int gpu_deltanet_step_gated(gpu_context *ctx, gpu_buffer *state, const gpu_buffer *Q,
                            const gpu_buffer *K, const gpu_buffer *V, gpu_buffer *out, int dim,
                            float gate)
{
    if (!ctx) return ORN_EINVAL;
    if (!state || !Q || !K || !V || !out || dim <= 0)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_deltanet_step_gated: bad arguments");
    if (!fits(state, (size_t)dim * dim) || !fits(Q, (size_t)dim) || !fits(K, (size_t)dim) ||
        !fits(V, (size_t)dim) || !fits(out, (size_t)dim))
        return orn_set_err(ctx, ORN_EINVAL, "gpu_deltanet_step_gated: buffer too small");
    int rc = orn_hip_check(ctx, (hipError_t)ornk_deltanet_step(
                                    (float *)state->dev, (const float *)Q->dev,
                                    (const float *)K->dev, (const float *)V->dev,
                                    (float *)out->dev, dim, gate, ctx->stream),
                           "gpu_deltanet_step_gated");
    sync_ctx(ctx);
    return rc;
}

int gpu_kv_cache_append(gpu_context *ctx, gpu_buffer *K_cache, gpu_buffer *V_cache,
                        const gpu_buffer *K_new, const gpu_buffer *V_new, int pos, int head_dim)
{
    if (!ctx) return ORN_EINVAL;
    if (!K_cache || !V_cache || !K_new || !V_new || pos < 0 || head_dim <= 0)
        return orn_set_err(ctx, ORN_EINVAL, "gpu_kv_cache_append: bad arguments");
    const size_t end = ((size_t)pos + 1) * (size_t)head_dim;
    if (!fits(K_cache, end) || !fits(V_cache, end) || !fits(K_new, (size_t)head_dim) ||
        !fits(V_new, (size_t)head_dim))
        return orn_set_err(ctx, ORN_EINVAL, "gpu_kv_cache_append: position %d past the cache",
                           pos);
    int rc = orn_hip_check(ctx, (hipError_t)ornk_kv_append((float *)K_cache->dev,
                                                           (float *)V_cache->dev,
                                                           (const float *)K_new->dev,
                                                           (const float *)V_new->dev, pos,
                                                           head_dim, ctx->stream),
                           "gpu_kv_cache_append");
    sync_ctx(ctx);
    return rc;
}

/* mlp.metal:49-87: out = (silu(x@gate) * (x@up)) @ down in fp32, no clamp. */
void gpu_expert_mlp(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x,
                    const gpu_buffer *gate_w, const gpu_buffer *up_w, const gpu_buffer *down_w,
                    int d_model, int hidden_dim, quant_mode quant)
{
    (void)quant;
    if (!ctx || !out || !x || !gate_w || !up_w || !down_w || d_model <= 0 || hidden_dim <= 0)
        return;
    const size_t D = (size_t)d_model, H = (size_t)hidden_dim;
    if (!fits(out, D) || !fits(x, D) || !fits(gate_w, D * H) || !fits(up_w, D * H) ||
        !fits(down_w, H * D))
        return;
    float *tmp = (float *)orn_ws_get(ctx, 3 * H * sizeof(float));
    if (!tmp) return;
    float *g = tmp, *u = tmp + H, *mid = tmp + 2 * H;
    hipStream_t s = ctx->stream;
    ornk_matmul_f32(g, (const float *)x->dev, (const float *)gate_w->dev, 1, hidden_dim, d_model, s);
    ornk_matmul_f32(u, (const float *)x->dev, (const float *)up_w->dev, 1, hidden_dim, d_model, s);
    ornk_silu_mul(mid, g, u, hidden_dim, s);
    ornk_matmul_f32((float *)out->dev, mid, (const float *)down_w->dev, 1, d_model, hidden_dim, s);
    sync_ctx(ctx);
}

/* mlp.metal:94-109 / model.c:1017-1025: sequential fp32 logits. */
void gpu_router(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x,
                const gpu_buffer *router_weight, int d_model, int n_experts)
{
    if (!ctx || !out || !x || !router_weight || d_model <= 0 || n_experts <= 0) return;
    if (!fits(out, (size_t)n_experts) || !fits(x, (size_t)d_model) ||
        !fits(router_weight, (size_t)d_model * n_experts))
        return;
    ornk_router_exact((const float *)x->dev, (const float *)router_weight->dev, NULL, 1, d_model,
                      n_experts, (float *)out->dev, ctx->stream);
    sync_ctx(ctx);
}

/* gpu_metal.m:663-685: exchange sort on the logits (n capped at 1024), softmax
 * over the first k; indices/weights are host arrays. */
void gpu_topk_softmax(gpu_context *ctx, uint32_t *indices, float *weights,
                      const gpu_buffer *logits, int n_experts, int top_k)
{
    if (!ctx || !indices || !weights || !logits) return;
    int n = n_experts < 1024 ? n_experts : 1024;
    int k = top_k < n ? top_k : n;
    if (n <= 0 || k <= 0 || !fits(logits, (size_t)n)) return;
    uint8_t *ws = (uint8_t *)orn_ws_get(ctx, 2 * 1024 * sizeof(float) + 256);
    if (!ws) return;
    uint32_t *d_idx = (uint32_t *)ws;
    float *d_w = (float *)(ws + 1024 * sizeof(float));
    if (ornk_topk((const float *)logits->dev, 1, n, k, 0, d_idx, d_w, NULL, ctx->stream) !=
        hipSuccess)
        return;
    hipMemcpyAsync(indices, d_idx, (size_t)k * sizeof(uint32_t), hipMemcpyDeviceToHost,
                   ctx->stream);
    hipMemcpyAsync(weights, d_w, (size_t)k * sizeof(float), hipMemcpyDeviceToHost, ctx->stream);
    sync_ctx(ctx);
}

void gpu_add(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *a, const gpu_buffer *b, int n)
{
    if (!ctx || !out || !a || !b || n <= 0) return;
    if (!fits(out, (size_t)n) || !fits(a, (size_t)n) || !fits(b, (size_t)n)) return;
    ornk_add((float *)out->dev, (const float *)a->dev, (const float *)b->dev, n, ctx->stream);
    sync_ctx(ctx);
}

void gpu_sync(gpu_context *ctx)
{
    if (ctx) sync_ctx(ctx);
}

size_t gpu_memory_used(gpu_context *ctx) { return ctx ? ctx->used_memory : 0; }

void gpu_print_info(gpu_context *ctx)
{
    if (!ctx) return;
    char name[128] = "";
    int cus = 0;
    size_t hbm = 0;
    gpu_device_info(ctx, name, sizeof name, &cus, &hbm);
    printf("=== GPU Info (HIP backend) ===\n");
    printf("Device:   %s, %d CUs, %.1f GiB HBM\n", name, cus, (double)hbm / (1024.0 * 1024 * 1024));
    printf("Memory:   %zu bytes\n", ctx->used_memory);
}
