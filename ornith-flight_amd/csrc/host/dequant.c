/* SPDX-License-Identifier: MIT
 *
 * Device dequantization API — the counterparts of gguf.h:111-137.
 * Validation and results follow gguf.c:605-638 / 652-711: false on NULL
 * arguments, unsupported types, expert_idx < 0, expert_idx >= E (E = the
 * last dim) or E == 0.  For K-quant types only whole super-blocks are
 * written (n_elems/256 of them), exactly like the reference.
 */
#include "internal.h"

#include <string.h>

static int supported(int type)
{
    return type == ORN_TYPE_F32 || type == ORN_TYPE_F16 || type == ORN_TYPE_Q4_K ||
           type == ORN_TYPE_Q6_K;
}

/* Floats the reference writes for a whole-tensor dequant. */
static uint64_t written_elems(int type, uint64_t n)
{
    if (type == ORN_TYPE_Q4_K || type == ORN_TYPE_Q6_K) return (n / ORN_QK_K) * ORN_QK_K;
    return n;
}

static int whole_blocks(int type, uint64_t n)
{
    return !(type == ORN_TYPE_Q4_K || type == ORN_TYPE_Q6_K) || n % ORN_QK_K == 0;
}

/* Element counts whose byte sizes (input and fp32 output, padded) cannot
 * wrap a size_t: a larger tensor could never be resident anyway. */
static int fits(uint64_t n) { return n <= (uint64_t)(SIZE_MAX / 16); }

static uint64_t slice_experts(const orn_tensor_info *t)
{
    if (t->n_dims == 0 || t->n_dims > 4) return 0;
    return t->dims[t->n_dims - 1];
}

bool gpu_dequantize_tensor_from_buf(gpu_context *ctx, const void *data,
                                    const orn_tensor_info *tensor, float *output)
{
    if (!ctx || !data || !tensor || !output) return false;
    if (!supported(tensor->type)) return false;
    const uint64_t n = tensor->n_elems;
    if (!fits(n)) return false;
    const size_t in_bytes = orn_row_size(tensor->type, n);
    const uint64_t n_out = written_elems(tensor->type, n);
    if (n_out == 0) return true;
    const size_t in_pad = (in_bytes + 255) & ~(size_t)255;
    uint8_t *ws = (uint8_t *)orn_ws_get(ctx, in_pad + n_out * sizeof(float));
    if (!ws) return false;
    float *dst = (float *)(ws + in_pad);
    hipStream_t s = ctx->stream;
    if (orn_hip_check(ctx, hipMemcpyAsync(ws, data, in_bytes, hipMemcpyHostToDevice, s), "upload"))
        return false;
    if (orn_hip_check(ctx, (hipError_t)ornk_dequant(ws, tensor->type, n, dst, s), "dequant"))
        return false;
    if (orn_hip_check(ctx, hipMemcpyAsync(output, dst, n_out * sizeof(float),
                                          hipMemcpyDeviceToHost, s), "download"))
        return false;
    return orn_hip_check(ctx, hipStreamSynchronize(s), "sync") == ORN_OK;
}

bool gpu_dequantize_expert_slice_from_buf(gpu_context *ctx, const void *data,
                                          const orn_tensor_info *tensor, int expert_idx,
                                          float *output)
{
    if (!ctx || !data || !tensor || !output) return false;
    if (expert_idx < 0) return false;
    const uint64_t E = slice_experts(tensor);
    if ((uint64_t)expert_idx >= E) return false;
    if (E == 0) return false;
    if (!supported(tensor->type)) return false;
    const uint64_t n = tensor->n_elems;
    if (!fits(n)) return false;
    /* A partial trailing super-block would be read past the tensor's bytes
     * (undefined in the reference); refuse instead of touching it. */
    if (!whole_blocks(tensor->type, n)) return false;
    const uint64_t per = n / E;
    if (per == 0) return true;
    const size_t in_bytes = orn_row_size(tensor->type, n);
    const size_t in_pad = (in_bytes + 255) & ~(size_t)255;
    uint8_t *ws = (uint8_t *)orn_ws_get(ctx, in_pad + per * sizeof(float));
    if (!ws) return false;
    float *dst = (float *)(ws + in_pad);
    hipStream_t s = ctx->stream;
    if (orn_hip_check(ctx, hipMemcpyAsync(ws, data, in_bytes, hipMemcpyHostToDevice, s), "upload"))
        return false;
    if (orn_hip_check(ctx, (hipError_t)ornk_dequant_slice(ws, tensor->type, n, E, expert_idx, dst,
                                                          s),
                      "slice"))
        return false;
    if (orn_hip_check(ctx, hipMemcpyAsync(output, dst, per * sizeof(float), hipMemcpyDeviceToHost,
                                          s), "download"))
        return false;
    return orn_hip_check(ctx, hipStreamSynchronize(s), "sync") == ORN_OK;
}

bool gpu_dequantize_tensor_buf(gpu_context *ctx, const gpu_buffer *data,
                               const orn_tensor_info *tensor, gpu_buffer *output)
{
    if (!ctx || !data || !tensor || !output) return false;
    if (!supported(tensor->type)) return false;
    const uint64_t n = tensor->n_elems;
    const uint64_t n_out = written_elems(tensor->type, n);
    if (orn_row_size(tensor->type, n) > data->size || n_out * sizeof(float) > output->size)
        return false;
    if (n_out == 0) return true;
    if (orn_hip_check(ctx, (hipError_t)ornk_dequant(data->dev, tensor->type, n,
                                                    (float *)output->dev, ctx->stream),
                      "dequant"))
        return false;
    return orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync") == ORN_OK;
}

bool gpu_dequantize_expert_slice_buf(gpu_context *ctx, const gpu_buffer *data,
                                     const orn_tensor_info *tensor, int expert_idx,
                                     gpu_buffer *output)
{
    if (!ctx || !data || !tensor || !output) return false;
    if (expert_idx < 0) return false;
    const uint64_t E = slice_experts(tensor);
    if ((uint64_t)expert_idx >= E) return false;
    if (E == 0) return false;
    if (!supported(tensor->type)) return false;
    const uint64_t n = tensor->n_elems;
    if (!whole_blocks(tensor->type, n)) return false;
    const uint64_t per = n / E;
    if (orn_row_size(tensor->type, n) > data->size || per * sizeof(float) > output->size)
        return false;
    if (per == 0) return true;
    if (orn_hip_check(ctx, (hipError_t)ornk_dequant_slice(data->dev, tensor->type, n, E, expert_idx,
                                                          (float *)output->dev, ctx->stream),
                      "slice"))
        return false;
    return orn_hip_check(ctx, hipStreamSynchronize(ctx->stream), "sync") == ORN_OK;
}
