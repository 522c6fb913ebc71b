/* SPDX-License-Identifier: MIT
 *
 * ORACLE — test infrastructure only.
 *
 * A C99 restatement of instax-dutta/ornith-flight's CPU arithmetic for the
 * routed-MoE hot path.  It is the checker for the HIP implementation: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and never as the thing that is measured or shipped.
 *
 * Every function states the reference file:line it follows.  Arithmetic is
 * plain fp32 in the reference's operation order; build with
 * -O2 -ffp-contract=off (no FMA contraction, no reassociation).
 *
 * Pinning (what checks each function against something independent):
 *   orc_fp16_to_fp32        golden vectors from the compiled reference dequant
 *                           (special patterns 0x0000/0x8000/subnormal/inf/nan)
 *                           + closed form over all 65536 inputs in tests
 *   orc_dequant_block_*     reference known-answer tests (1.0 / -31.0), golden
 *                           vectors from the compiled reference, closed form
 *   orc_q4k_one/q6k_one     equality with the block dequant at all 256 positions
 *   orc_dequant_tensor      golden vectors from the compiled reference
 *   orc_dequant_expert_slice golden vectors + the reference's slice identity
 *   orc_router_logits       golden routing from the compiled reference
 *                           (model_get_routing) + fp64 bound
 *   orc_topk_renorm         golden routing from the compiled reference incl.
 *                           constructed exact ties
 *   orc_topk_literal        golden layer outputs from the compiled reference
 *                           model_forward (selection changes the output)
 *   orc_moe_layer (both layouts, both modes) golden layer outputs from the
 *                           compiled reference model_forward (interleaved
 *                           layout) + fp64 brute force (contiguous layout)
 *   orc_moe_layer, file layout: equality with the contiguous layout on the
 *                           transposed matrices, for weights whose every
 *                           block shares one set of scales (the same matrix
 *                           is then exactly representable in both
 *                           orientations) + fp64 brute force
 *   orc_rope                fp64 complex rotation (same frequency formula),
 *                           pos 0 = identity, pair norms preserved
 *   orc_attention           fp64 softmax(QK^T/sqrt(d))V; seq 1 -> V; equal
 *                           keys -> mean of V
 *   orc_deltanet_step       fp64 recurrence; gate 1 -> state kept,
 *                           gate 0 -> state = outer(v, k)
 */
#ifndef ORNITH_ORACLE_H
#define ORNITH_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

float orc_fp16_to_fp32(uint16_t h);
void orc_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
void orc_dequant_block_q4k(const uint8_t *blk, float *y);
void orc_dequant_block_q6k(const uint8_t *blk, float *y);
float orc_q4k_one(const uint8_t *blk, int pos);
float orc_q6k_one(const uint8_t *blk, int pos);

/* Whole-tensor dequant. Returns 1 on success, 0 on NULL args / unsupported type. */
int orc_dequant_tensor(const void *data, int type, uint64_t n_elems, float *out);

/* Interleaved expert slice: slice[i] = full[i * n_experts + expert].
 * Returns 1 on success, 0 on NULL args, expert < 0, expert >= n_experts,
 * n_experts == 0 or unsupported type. */
int orc_dequant_expert_slice(const void *data, int type, uint64_t n_elems,
                             uint64_t n_experts, int expert, float *out);

/* Sequential fp32 router logits, logits[e] = sum_d x[d] * W[d*E + e]; an
 * optional bias is added after the sum (bias may be NULL). */
void orc_router_logits(const float *x, const float *W, int D, int E,
                       const float *bias, float *logits);

/* Exchange sort on logits + softmax over the top-k (model_get_routing). */
int orc_topk_renorm(const float *logits, int E, int k, uint32_t *idx, float *w);

/* Full softmax, then k passes of exchange selection on the probabilities
 * (model_forward inline routing). Weights are not renormalised. */
int orc_topk_literal(const float *logits, int E, int k, uint32_t *idx, float *w);

float orc_silu_clamped(float x);
float orc_silu_plain(float x);
void orc_matvec(float *out, const float *vec, const float *mat, int K, int M);
void orc_rmsnorm(float *out, const float *x, const float *w, int dim);

/* Routing modes. */
#define ORC_MODE_RENORM 0  /* exchange on logits, softmax over top-k */
#define ORC_MODE_LITERAL 1 /* full softmax, exchange on probabilities */

/* Weight layouts for the routed experts. */
#define ORC_LAYOUT_CONTIGUOUS 0  /* expert e's blocks at e * blocks_per_matrix */
#define ORC_LAYOUT_INTERLEAVED 1 /* fused tensor, element i of e at i*E + e */
/* GGUF file orientation (no reference counterpart: the reference reads every
 * matrix as vec@mat, model.c:351-357): expert e's blocks at
 * e * blocks_per_matrix, each matrix stored output-row-major with the input
 * index fastest (ggml ne = [K, M]), so W(k, i) is element i*K + k.  Applies
 * to the routed and the shared experts. */
#define ORC_LAYOUT_FILE 2

typedef struct {
    int D;       /* model dim (2048) */
    int H;       /* expert hidden dim (512) */
    int E;       /* routed experts (256) */
    int k;       /* experts per token (8) */
    int mode;    /* ORC_MODE_* */
    int layout;  /* ORC_LAYOUT_* */
    int gate_type, up_type, down_type;          /* routed tensors (Q4_K/Q4_K/Q6_K/F32/F16) */
    int sh_gate_type, sh_up_type, sh_down_type; /* shared expert tensors */
} orc_moe_cfg;

/* One MoE block for T tokens, following model.c:992-1144 per token:
 *   ffn_x = norm_w ? rmsnorm(x, norm_w) : x
 *   y     = (resid + shared(ffn_x)) + sum_a w_a * expert_a(ffn_x)
 * resid may be NULL (treated as all zeros, i.e. y = (0 + shared) + routed);
 * norm_w may be NULL (no normalisation); bias may be NULL.
 * Shared expert tensors may be NULL (no shared expert, as model.c:993).
 * idx_out / w_out (T*k each) may be NULL.
 * Returns 0 on success, negative on bad arguments / allocation failure. */
int orc_moe_layer(const orc_moe_cfg *cfg, int T, const float *x, const float *resid,
                  const float *norm_w, const float *router_W, const float *bias,
                  const void *gate, const void *up, const void *down,
                  const void *sh_gate, const void *sh_up, const void *sh_down,
                  float *out, uint32_t *idx_out, float *w_out);

/* orc_moe_layer with an optional shared-expert gate (no reference
 * counterpart: the reference loads no ffn_gate_inp_shexp and adds the shared
 * expert ungated, model.c:1003-1007).  shexp_gate [D] (NULL: none) scales the
 * shared expert's output by sigmoid(sum_i ffn_x[i] * shexp_gate[i]), the dot
 * a sequential fp32 sum, as Qwen-MoE models gate their shared expert. */
int orc_moe_layer_ex(const orc_moe_cfg *cfg, int T, const float *x, const float *resid,
                     const float *norm_w, const float *router_W, const float *bias,
                     const void *gate, const void *up, const void *down,
                     const void *sh_gate, const void *sh_up, const void *sh_down,
                     const float *shexp_gate, float *out, uint32_t *idx_out, float *w_out);

/* ops.metal:113-139 (= model.c:599-622 for one head): the pairs (i, i+1),
 * i < rot = min(head_dim, 64), of n_heads heads of x [n_heads][head_dim]
 * rotated by pos * inv_freq, inv_freq = 1/theta^(i/rot) rounded once from
 * double. */
void orc_rope(float *x, int n_heads, int head_dim, int pos, float theta);

/* attention.metal:17-68: out[r][c] = sum_t e^(s_rt) V[t][c] / sum_t e^(s_rt),
 * s_rt = (sum_d Q[r][d]*K[t][d]) * scale, t and d ascending, exp not
 * shifted, division only if the sum > 1e-10 (as the shader). */
void orc_attention(float *out, const float *Q, const float *K, const float *V, int seq, int hd,
                   float scale);

/* attention.metal:80-108 (the whole grid): state[j][i] = gate*state[j][i] +
 * (1-gate)*K[i]*V[j]; out[i] = sum_j Q[j]*state[j][i]. */
void orc_deltanet_step(float *state, const float *Q, const float *K, const float *V, float *out,
                       int dim, float gate);

/* Single (token, expert) FFN with the routed-expert SiLU clamp
 * (model.c:1085-1088) on already dequantized fp32 weights. */
void orc_expert_ffn(const float *x, const float *Wg, const float *Wu, const float *Wd,
                    int D, int H, int clamp, float *out);

#ifdef __cplusplus
}
#endif

#endif /* ORNITH_ORACLE_H */
