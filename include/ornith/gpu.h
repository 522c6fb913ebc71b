/* SPDX-License-Identifier: MIT
 *
 * Backend abstraction — HIP (MI355X / gfx950) implementation.
 *
 * Drop-in for the reference engine's GPU abstraction: every declaration below
 * has the name, signature and meaning of engine/src/gpu.h:1-97, so the engine
 * links against libornith_hip.so instead of gpu.o (CPU fallback) or
 * gpu_metal.o (Metal) without touching model.c.  Per-symbol citations:
 *
 *   gpu_init / gpu_destroy            gpu.h:29-30   (CPU: gpu.c:24-37)
 *   gpu_alloc / gpu_free              gpu.h:33-34   (gpu.c:41-64; memory_used
 *                                                    counts requested bytes)
 *   gpu_get_cpu_ptr / gpu_buffer_size gpu.h:35-36   (gpu.c:66-74)
 *   gpu_copy_to_device/host/buffer    gpu.h:38-43   (gpu.c:76-100; sizes clamp)
 *   gpu_matmul                        gpu.h:46-49   (gpu.c:104-129, fp32 row-major)
 *   gpu_matmul_int4                   gpu.h:51-53   (gpu.c:131-140, zero-fills C)
 *   gpu_rmsnorm                       gpu.h:55-57   (gpu.c:144-156, eps 1e-6)
 *   gpu_silu / gpu_silu_mul           gpu.h:59-63   (gpu.c:158-186, no clamp)
 *   gpu_rope                          gpu.h:65-67   (gpu_metal.m:495-548,
 *                                                    ops.metal:113-139 semantics)
 *   gpu_attention                     gpu.h:69-71   (gpu_metal.m:550-583,
 *                                                    attention.metal:17-68; head_dim
 *                                                    <= 256)
 *   gpu_deltanet_step                 gpu.h:73-75   (a no-op in both reference
 *                                                    backends, gpu.c:202-206,
 *                                                    gpu_metal.m:587-591; same here)
 *   gpu_expert_mlp                    gpu.h:77-80   (mlp.metal:49-87 semantics)
 *   gpu_router                        gpu.h:82-84   (mlp.metal:94-109 semantics)
 *   gpu_topk_softmax                  gpu.h:86-87   (gpu_metal.m:663-685 semantics)
 *   gpu_add                           gpu.h:89-90   (gpu.c:229-238)
 *   gpu_sync / gpu_memory_used /
 *     gpu_print_info                  gpu.h:93-95   (gpu.c:242-256)
 *
 * Semantics shared with the reference backends: calls are synchronous at
 * return; void calls are silent no-ops on NULL arguments; constructors return
 * NULL on failure.  GPU_BUF_SHARED buffers live in pinned, device-mapped host
 * memory, so host writes through gpu_get_cpu_ptr are seen by later calls.
 */
#ifndef ORNITH_GPU_H
#define ORNITH_GPU_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpu_context gpu_context;
typedef struct gpu_buffer gpu_buffer;

typedef enum {
    QUANT_NONE = 0,
    QUANT_FP16,
    QUANT_INT8,
    QUANT_INT4
} quant_mode;

typedef enum {
    GPU_BUF_DEFAULT = 0,
    GPU_BUF_SHARED = 1 << 0,
    GPU_BUF_CONSTANT = 1 << 1
} gpu_buffer_flags;

/* Lifecycle */
gpu_context *gpu_init(void);
void gpu_destroy(gpu_context *ctx);

/* Buffers */
gpu_buffer *gpu_alloc(gpu_context *ctx, size_t size, gpu_buffer_flags flags);
void gpu_free(gpu_context *ctx, gpu_buffer *buf);
void *gpu_get_cpu_ptr(gpu_context *ctx, gpu_buffer *buf);
size_t gpu_buffer_size(gpu_context *ctx, const gpu_buffer *buf);

void gpu_copy_to_device(gpu_context *ctx, gpu_buffer *dst, const void *src, size_t size);
void gpu_copy_to_host(gpu_context *ctx, void *dst, const gpu_buffer *src, size_t size);
void gpu_copy_buffer(gpu_context *ctx, gpu_buffer *dst, const gpu_buffer *src, size_t size);

/* Compute */
void gpu_matmul(gpu_context *ctx, gpu_buffer *C, const gpu_buffer *A, const gpu_buffer *B,
                int M, int N, int K, quant_mode a_quant, quant_mode b_quant);

void gpu_matmul_int4(gpu_context *ctx, gpu_buffer *C, const gpu_buffer *A_quant,
                     const gpu_buffer *A_scale, int M, int N, int K);

void gpu_rmsnorm(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x,
                 const gpu_buffer *weight, int rows, int dim);

void gpu_silu(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x, int n);

void gpu_silu_mul(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *gate,
                  const gpu_buffer *up, int n);

void gpu_rope(gpu_context *ctx, gpu_buffer *Q, gpu_buffer *K, int seq_len, int head_dim,
              int n_heads, int n_kv_heads, float base, int pos_start);

void gpu_attention(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *Q,
                   const gpu_buffer *K_cache, const gpu_buffer *V_cache, int seq_len,
                   int head_dim);

void gpu_deltanet_step(gpu_context *ctx, gpu_buffer *state, const gpu_buffer *Q,
                       const gpu_buffer *K, const gpu_buffer *V, int dim);

void gpu_expert_mlp(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x,
                    const gpu_buffer *gate_w, const gpu_buffer *up_w, const gpu_buffer *down_w,
                    int d_model, int hidden_dim, quant_mode quant);

void gpu_router(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *x,
                const gpu_buffer *router_weight, int d_model, int n_experts);

void gpu_topk_softmax(gpu_context *ctx, uint32_t *indices, float *weights,
                      const gpu_buffer *logits, int n_experts, int top_k);

void gpu_add(gpu_context *ctx, gpu_buffer *out, const gpu_buffer *a, const gpu_buffer *b, int n);

/* Sync / info */
void gpu_sync(gpu_context *ctx);
size_t gpu_memory_used(gpu_context *ctx);
void gpu_print_info(gpu_context *ctx);

#ifdef __cplusplus
}
#endif

#endif /* ORNITH_GPU_H */
