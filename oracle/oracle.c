/* SPDX-License-Identifier: MIT
 *
 * ORACLE — test infrastructure only (see oracle.h).  C99 restatement of the
 * reference CPU path for the routed-MoE layer.  Build: -O2 -ffp-contract=off.
 *
 * Loop order note: the reference's matvec is `for i { sum = 0; for k sum +=
 * v[k]*W[k*M+i]; }` (model.c:351-357).  orc_matvec keeps one running sum per
 * output and adds the products in the same k order, so every output sees the
 * identical sequence of fp32 roundings; only the loop nest is interchanged
 * (k outer) so the restatement runs at memory speed.  The router uses the
 * same interchange (model.c:1018-1025).
 */
#include "oracle.h"

#include "../include/ornith/kquant.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* gguf.c:16-26 — non-IEEE half->float: zero only for 0x0000; every other
 * pattern is treated as a normal number with exponent bias 112 (so 0x8000
 * becomes -2^-15, subnormals become 2^-15*(1+m/1024), exp=31 becomes
 * 2^16*(1+m/1024)). */
float orc_fp16_to_fp32(uint16_t h)
{
    if (h == 0) return 0.0f;
    uint32_t sign = ((uint32_t)(h & 0x8000u)) << 16;
    uint32_t expo = ((((uint32_t)(h & 0x7C00u)) >> 10) + 112u) << 23;
    uint32_t mant = ((uint32_t)(h & 0x03FFu)) << 13;
    uint32_t u = sign | expo | mant;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* gguf.c:31-40 — 6-bit scale/min of sub-block j from the 12 packed bytes. */
void orc_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = (uint8_t)(s[j] & 63);
        *m = (uint8_t)(s[j + 4] & 63);
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* gguf.c:43-61 — y[64c+l] = d*sc(2c)*(q&15) - dmin*m(2c);
 *                y[64c+32+l] = d*sc(2c+1)*(q>>4) - dmin*m(2c+1). */
void orc_dequant_block_q4k(const uint8_t *blk, float *y)
{
    const float d = orc_fp16_to_fp32(rd16(blk + ORN_Q4K_OFF_D));
    const float dmin = orc_fp16_to_fp32(rd16(blk + ORN_Q4K_OFF_DMIN));
    const uint8_t *scales = blk + ORN_Q4K_OFF_SCALES;
    const uint8_t *q = blk + ORN_Q4K_OFF_QS;
    for (int c = 0; c < 4; ++c) {
        uint8_t sc, m;
        orc_scale_min_k4(2 * c, scales, &sc, &m);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        orc_scale_min_k4(2 * c + 1, scales, &sc, &m);
        const float d2 = d * (float)sc;
        const float m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) y[64 * c + l] = d1 * (float)(q[32 * c + l] & 0x0F) - m1;
        for (int l = 0; l < 32; ++l) y[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
    }
}

/* gguf.c:64-86 — two 128-element halves; q in [-32,31]; y = d*sc*q. */
void orc_dequant_block_q6k(const uint8_t *blk, float *y)
{
    const float d = orc_fp16_to_fp32(rd16(blk + ORN_Q6K_OFF_D));
    const uint8_t *ql = blk + ORN_Q6K_OFF_QL;
    const uint8_t *qh = blk + ORN_Q6K_OFF_QH;
    const int8_t *sc = (const int8_t *)(blk + ORN_Q6K_OFF_SCALES);
    for (int n = 0; n < 2; ++n) {
        const uint8_t *L = ql + 64 * n;
        const uint8_t *Hh = qh + 32 * n;
        const int8_t *S = sc + 8 * n;
        float *Y = y + 128 * n;
        for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            int8_t q1 = (int8_t)((int8_t)((L[l] & 0x0F) | (((Hh[l] >> 0) & 3) << 4)) - 32);
            int8_t q2 = (int8_t)((int8_t)((L[l + 32] & 0x0F) | (((Hh[l] >> 2) & 3) << 4)) - 32);
            int8_t q3 = (int8_t)((int8_t)((L[l] >> 4) | (((Hh[l] >> 4) & 3) << 4)) - 32);
            int8_t q4 = (int8_t)((int8_t)((L[l + 32] >> 4) | (((Hh[l] >> 6) & 3) << 4)) - 32);
            Y[l + 0] = d * (float)S[is + 0] * (float)q1;
            Y[l + 32] = d * (float)S[is + 2] * (float)q2;
            Y[l + 64] = d * (float)S[is + 4] * (float)q3;
            Y[l + 96] = d * (float)S[is + 6] * (float)q4;
        }
    }
}

/* gguf.c:511-528 — one element of a Q4_K block. */
float orc_q4k_one(const uint8_t *blk, int pos)
{
    int sub = pos / 32, chunk = pos / 64, p = pos % 64, half = p / 32, sub_pos = p % 32;
    uint8_t sc, m;
    orc_scale_min_k4(sub, blk + ORN_Q4K_OFF_SCALES, &sc, &m);
    float d_val = orc_fp16_to_fp32(rd16(blk + ORN_Q4K_OFF_D)) * (float)sc;
    float min_val = orc_fp16_to_fp32(rd16(blk + ORN_Q4K_OFF_DMIN)) * (float)m;
    uint8_t b = blk[ORN_Q4K_OFF_QS + chunk * 32 + sub_pos];
    uint8_t q = (uint8_t)(half == 0 ? (b & 0x0F) : (b >> 4));
    return d_val * (float)q - min_val;
}

/* gguf.c:532-571 — one element of a Q6_K block. */
float orc_q6k_one(const uint8_t *blk, int pos)
{
    float d_out = orc_fp16_to_fp32(rd16(blk + ORN_Q6K_OFF_D));
    int pass = pos / 128, lane = (pos % 128) / 32, l = pos % 32, is = l / 16;
    int ql_off = (lane % 2 == 0) ? l : (32 + l);
    int ql_byte = (int)blk[ORN_Q6K_OFF_QL + pass * 64 + ql_off];
    int qh_byte = (int)blk[ORN_Q6K_OFF_QH + pass * 32 + l];
    int q_val;
    if (lane < 2)
        q_val = (ql_byte & 0x0F) | (((qh_byte >> (lane * 2)) & 3) << 4);
    else
        q_val = (ql_byte >> 4) | (((qh_byte >> (lane * 2)) & 3) << 4);
    q_val -= 32;
    int8_t sc_val = (int8_t)blk[ORN_Q6K_OFF_SCALES + pass * 8 + lane * 2 + is];
    return d_out * (float)sc_val * (float)q_val;
}

/* gguf.c:605-638 — whole tensor. */
int orc_dequant_tensor(const void *data, int type, uint64_t n_elems, float *out)
{
    if (!data || !out) return 0;
    const uint8_t *src = (const uint8_t *)data;
    uint64_t n_blocks = n_elems / ORN_QK_K;
    switch (type) {
    case ORN_TYPE_F32:
        memcpy(out, data, (size_t)orn_row_size(ORN_TYPE_F32, n_elems));
        return 1;
    case ORN_TYPE_F16:
        for (uint64_t i = 0; i < n_elems; ++i) out[i] = orc_fp16_to_fp32(rd16(src + 2 * i));
        return 1;
    case ORN_TYPE_Q4_K:
        for (uint64_t b = 0; b < n_blocks; ++b)
            orc_dequant_block_q4k(src + b * ORN_Q4K_BYTES, out + b * ORN_QK_K);
        return 1;
    case ORN_TYPE_Q6_K:
        for (uint64_t b = 0; b < n_blocks; ++b)
            orc_dequant_block_q6k(src + b * ORN_Q6K_BYTES, out + b * ORN_QK_K);
        return 1;
    default:
        return 0;
    }
}

/* gguf.c:652-711 — interleaved expert slice; validation order as the reference. */
int orc_dequant_expert_slice(const void *data, int type, uint64_t n_elems,
                             uint64_t n_experts, int expert, float *out)
{
    if (!data || !out) return 0;
    if (expert < 0) return 0;
    if ((uint64_t)expert >= n_experts) return 0;
    if (n_experts == 0) return 0;
    const uint8_t *src = (const uint8_t *)data;
    uint64_t per = n_elems / n_experts;
    switch (type) {
    case ORN_TYPE_F32: {
        const float *f = (const float *)data;
        for (uint64_t i = 0; i < per; ++i) out[i] = f[i * n_experts + (uint64_t)expert];
        return 1;
    }
    case ORN_TYPE_F16:
        for (uint64_t i = 0; i < per; ++i)
            out[i] = orc_fp16_to_fp32(rd16(src + 2 * (i * n_experts + (uint64_t)expert)));
        return 1;
    case ORN_TYPE_Q4_K:
        for (uint64_t i = 0; i < per; ++i) {
            uint64_t lin = i * n_experts + (uint64_t)expert;
            out[i] = orc_q4k_one(src + (lin / ORN_QK_K) * ORN_Q4K_BYTES, (int)(lin % ORN_QK_K));
        }
        return 1;
    case ORN_TYPE_Q6_K:
        for (uint64_t i = 0; i < per; ++i) {
            uint64_t lin = i * n_experts + (uint64_t)expert;
            out[i] = orc_q6k_one(src + (lin / ORN_QK_K) * ORN_Q6K_BYTES, (int)(lin % ORN_QK_K));
        }
        return 1;
    default:
        return 0;
    }
}

/* model.c:1017-1025 (router) — per expert a sequential fp32 sum from 0.0f of
 * x[d]*W[d*E+e] in d order.  A bias (used only by the skewed-routing
 * workload, not by the reference) is added once after the sum. */
void orc_router_logits(const float *x, const float *W, int D, int E,
                       const float *bias, float *logits)
{
    for (int e = 0; e < E; ++e) logits[e] = 0.0f;
    for (int d = 0; d < D; ++d) {
        const float xd = x[d];
        const float *row = W + (size_t)d * (size_t)E;
        for (int e = 0; e < E; ++e) {
            float p = xd * row[e];
            logits[e] = logits[e] + p;
        }
    }
    if (bias)
        for (int e = 0; e < E; ++e) logits[e] = logits[e] + bias[e];
}

/* Exchange selection: pass i swaps position i with every later j whose value
 * compares strictly greater (model.c:301-305, 1040-1048).  Running k passes
 * fixes positions 0..k-1 exactly as the reference's full sort does, because
 * pass i never writes a position below i. */
static void exchange_select(float *val, int *idx, int n, int k)
{
    for (int i = 0; i < k && i < n - 1; ++i)
        for (int j = i + 1; j < n; ++j)
            if (val[j] > val[i]) {
                float ft = val[i]; val[i] = val[j]; val[j] = ft;
                int it = idx[i]; idx[i] = idx[j]; idx[j] = it;
            }
}

/* model.c:291-318 (model_get_routing) / gpu_metal.m:663-685 — exchange sort on
 * logits, softmax over the top-k with the first (largest) score as max. */
int orc_topk_renorm(const float *logits, int E, int k, uint32_t *idx, float *w)
{
    if (!logits || !idx || !w || E <= 0 || k <= 0) return 0;
    if (k > E) k = E;
    float *val = (float *)malloc(sizeof(float) * (size_t)E);
    int *ix = (int *)malloc(sizeof(int) * (size_t)E);
    if (!val || !ix) { free(val); free(ix); return 0; }
    for (int i = 0; i < E; ++i) { val[i] = logits[i]; ix[i] = i; }
    exchange_select(val, ix, E, k);
    float max_score = val[0];
    float sum_exp = 0.0f;
    for (int i = 0; i < k; ++i) {
        float s = expf(val[i] - max_score);
        w[i] = s;
        sum_exp += s;
    }
    for (int i = 0; i < k; ++i) { w[i] /= sum_exp; idx[i] = (uint32_t)ix[i]; }
    free(val); free(ix);
    return k;
}

/* model.c:1027-1049 — full softmax over E (max by strict >, expf, sequential
 * sum, divide), then k passes of exchange selection on the probabilities;
 * the returned weights are the un-renormalised probabilities. */
int orc_topk_literal(const float *logits, int E, int k, uint32_t *idx, float *w)
{
    if (!logits || !idx || !w || E <= 0 || k <= 0) return 0;
    if (k > E) k = E;
    float *p = (float *)malloc(sizeof(float) * (size_t)E);
    int *ix = (int *)malloc(sizeof(int) * (size_t)E);
    if (!p || !ix) { free(p); free(ix); return 0; }
    float max_r = logits[0];
    for (int e = 1; e < E; ++e) if (logits[e] > max_r) max_r = logits[e];
    float sum_r = 0.0f;
    for (int e = 0; e < E; ++e) { p[e] = expf(logits[e] - max_r); sum_r += p[e]; }
    for (int e = 0; e < E; ++e) p[e] /= sum_r;
    for (int e = 0; e < E; ++e) ix[e] = e;
    exchange_select(p, ix, E, k);
    for (int i = 0; i < k; ++i) { idx[i] = (uint32_t)ix[i]; w[i] = p[i]; }
    free(p); free(ix);
    return k;
}

/* model.c:340-344 — routed-expert SiLU with clamp. */
float orc_silu_clamped(float x)
{
    if (x < -50.0f) return 0.0f;
    if (x > 50.0f) return x;
    return x / (1.0f + expf(-x));
}

/* gpu.c:176-186 — the shared expert's gpu_silu_mul has no clamp. */
float orc_silu_plain(float x) { return x / (1.0f + expf(-x)); }

/* model.c:351-357 (and gpu.c:104-115 with M=1): out[i] = sum_k v[k]*W[k*M+i]. */
void orc_matvec(float *out, const float *vec, const float *mat, int K, int M)
{
    for (int i = 0; i < M; ++i) out[i] = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float v = vec[k];
        const float *row = mat + (size_t)k * (size_t)M;
        for (int i = 0; i < M; ++i) {
            float p = v * row[i];
            out[i] = out[i] + p;
        }
    }
}

/* model.c:333-338 == gpu.c:144-156 (eps 1e-6). */
void orc_rmsnorm(float *out, const float *x, const float *w, int dim)
{
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) ss += x[i] * x[i];
    float inv_rms = 1.0f / sqrtf(ss / (float)dim + 1e-6f);
    for (int i = 0; i < dim; ++i) out[i] = w[i] * (x[i] * inv_rms);
}

/* model.c:1085-1088 (routed, clamp=1) / model.c:1003-1006 (shared, clamp=0). */
void orc_expert_ffn(const float *x, const float *Wg, const float *Wu, const float *Wd,
                    int D, int H, int clamp, float *out)
{
    float *g = (float *)malloc(sizeof(float) * (size_t)H * 3);
    if (!g) return;
    float *u = g + H, *mid = u + H;
    orc_matvec(g, x, Wg, D, H);
    orc_matvec(u, x, Wu, D, H);
    for (int i = 0; i < H; ++i)
        mid[i] = (clamp ? orc_silu_clamped(g[i]) : orc_silu_plain(g[i])) * u[i];
    orc_matvec(out, mid, Wd, H, D);
    free(g);
}

static size_t tensor_bytes(int type, uint64_t n) { return orn_row_size(type, n); }

/* Dequantize one K x M matrix stored in file orientation (element i*K + k
 * = W(k, i)) into the vec@mat order out[k*M + i]. */
static int fetch_file(const void *p, int type, int K, int M, float *out)
{
    const uint64_t n = (uint64_t)K * (uint64_t)M;
    float *t = (float *)malloc(sizeof(float) * (size_t)n);
    if (!t) return 0;
    const int ok = orc_dequant_tensor(p, type, n, t);
    if (ok)
        for (int i = 0; i < M; ++i)
            for (int k = 0; k < K; ++k) out[(size_t)k * M + i] = t[(size_t)i * K + k];
    free(t);
    return ok;
}

/* Dequantize routed expert e's K x M matrix (vec@mat: K input rows). */
static int fetch_expert(const orc_moe_cfg *c, const void *base, int type, int K, int M, int e,
                        float *out)
{
    const uint64_t per = (uint64_t)K * (uint64_t)M;
    if (c->layout == ORC_LAYOUT_INTERLEAVED)
        return orc_dequant_expert_slice(base, type, per * (uint64_t)c->E, (uint64_t)c->E, e, out);
    const uint8_t *p = (const uint8_t *)base + tensor_bytes(type, per) * (size_t)e;
    if (c->layout == ORC_LAYOUT_FILE) return fetch_file(p, type, K, M, out);
    return orc_dequant_tensor(p, type, per, out);
}

/* The shared expert's K x M matrix (one tensor). */
static int fetch_shared(const orc_moe_cfg *c, const void *p, int type, int K, int M, float *out)
{
    if (c->layout == ORC_LAYOUT_FILE) return fetch_file(p, type, K, M, out);
    return orc_dequant_tensor(p, type, (uint64_t)K * (uint64_t)M, out);
}

/* model.c:992-1144, for T tokens.  Experts are visited expert-major (each
 * selected expert is dequantized once and applied to all tokens that chose
 * it); every (token, expert) result is the same fp32 sequence the reference
 * computes, and the per-token combine runs in selection order afterwards. */
int orc_moe_layer_ex(const orc_moe_cfg *c, int T, const float *x, const float *resid,
                     const float *norm_w, const float *router_W, const float *bias,
                     const void *gate, const void *up, const void *down,
                     const void *sh_gate, const void *sh_up, const void *sh_down,
                     const float *shexp_gate, float *out, uint32_t *idx_out, float *w_out)
{
    if (!c || !x || !out || !router_W || !gate || !up || !down || T < 0) return -1;
    const int D = c->D, H = c->H, E = c->E, K = c->k;
    if (D <= 0 || H <= 0 || E <= 0 || K <= 0 || K > E) return -1;
    const uint64_t per = (uint64_t)D * (uint64_t)H;
    int rc = 0;

    float *ffn_x = (float *)malloc(sizeof(float) * (size_t)T * D);
    float *acc = (float *)malloc(sizeof(float) * (size_t)T * D);       /* x after shared add */
    float *ed = (float *)malloc(sizeof(float) * (size_t)T * K * D);   /* routed expert outputs */
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    uint32_t *idx = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)T * K);
    float *wt = (float *)malloc(sizeof(float) * (size_t)T * K);
    float *Wg = (float *)malloc(sizeof(float) * per);
    float *Wu = (float *)malloc(sizeof(float) * per);
    float *Wd = (float *)malloc(sizeof(float) * per);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)D);
    if (!ffn_x || !acc || !ed || !logits || !idx || !wt || !Wg || !Wu || !Wd || !tmp) {
        rc = -2;
        goto done;
    }

    for (int t = 0; t < T; ++t) {
        const float *xt = x + (size_t)t * D;
        if (norm_w) orc_rmsnorm(ffn_x + (size_t)t * D, xt, norm_w, D);
        else memcpy(ffn_x + (size_t)t * D, xt, sizeof(float) * (size_t)D);
        for (int i = 0; i < D; ++i) acc[(size_t)t * D + i] = resid ? resid[(size_t)t * D + i] : 0.0f;
    }

    /* Shared expert (model.c:1003-1007): fp32 weights from a whole-tensor
     * dequant, unclamped silu, then x = x + down. */
    if (sh_gate && sh_up && sh_down) {
        if (!fetch_shared(c, sh_gate, c->sh_gate_type, D, H, Wg) ||
            !fetch_shared(c, sh_up, c->sh_up_type, D, H, Wu) ||
            !fetch_shared(c, sh_down, c->sh_down_type, H, D, Wd)) { rc = -3; goto done; }
        for (int t = 0; t < T; ++t) {
            orc_expert_ffn(ffn_x + (size_t)t * D, Wg, Wu, Wd, D, H, 0, tmp);
            float *a = acc + (size_t)t * D;
            if (shexp_gate) {
                /* sigmoid(shexp_gate . ffn_x) times the shared output
                 * (no reference counterpart: model.c:1003-1007 adds the
                 * shared expert ungated) */
                float dot = 0.0f;
                for (int i = 0; i < D; ++i) dot += ffn_x[(size_t)t * D + i] * shexp_gate[i];
                const float g = 1.0f / (1.0f + expf(-dot));
                for (int i = 0; i < D; ++i) a[i] = a[i] + g * tmp[i];
            } else {
                for (int i = 0; i < D; ++i) a[i] = a[i] + tmp[i];
            }
        }
    }

    /* Router and selection per token. */
    for (int t = 0; t < T; ++t) {
        orc_router_logits(ffn_x + (size_t)t * D, router_W, D, E, bias, logits);
        int n = (c->mode == ORC_MODE_LITERAL)
                    ? orc_topk_literal(logits, E, K, idx + (size_t)t * K, wt + (size_t)t * K)
                    : orc_topk_renorm(logits, E, K, idx + (size_t)t * K, wt + (size_t)t * K);
        if (n != K) { rc = -4; goto done; }
    }

    /* Routed experts, expert-major. */
    for (int e = 0; e < E; ++e) {
        int used = 0;
        for (int p = 0; p < T * K && !used; ++p)
            if ((int)idx[p] == e && !(wt[p] < 1e-6f)) used = 1;
        if (!used) continue;
        if (!fetch_expert(c, gate, c->gate_type, D, H, e, Wg) ||
            !fetch_expert(c, up, c->up_type, D, H, e, Wu) ||
            !fetch_expert(c, down, c->down_type, H, D, e, Wd)) { rc = -5; goto done; }
        for (int p = 0; p < T * K; ++p) {
            if ((int)idx[p] != e || wt[p] < 1e-6f) continue;
            int t = p / K;
            orc_expert_ffn(ffn_x + (size_t)t * D, Wg, Wu, Wd, D, H, 1, ed + (size_t)p * D);
        }
    }

    /* Combine in selection order (model.c:1056-1090), then x = x + routed
     * (model.c:1142). */
    for (int t = 0; t < T; ++t) {
        for (int i = 0; i < D; ++i) tmp[i] = 0.0f;
        for (int a = 0; a < K; ++a) {
            size_t p = (size_t)t * K + a;
            float w = wt[p];
            if (w < 1e-6f) continue;
            const float *y = ed + p * D;
            for (int i = 0; i < D; ++i) tmp[i] += w * y[i];
        }
        const float *a0 = acc + (size_t)t * D;
        float *o = out + (size_t)t * D;
        for (int i = 0; i < D; ++i) o[i] = a0[i] + tmp[i];
    }
    if (idx_out) memcpy(idx_out, idx, sizeof(uint32_t) * (size_t)T * K);
    if (w_out) memcpy(w_out, wt, sizeof(float) * (size_t)T * K);

done:
    free(ffn_x); free(acc); free(ed); free(logits); free(idx); free(wt);
    free(Wg); free(Wu); free(Wd); free(tmp);
    return rc;
}

/* ops.metal:113-139 for every (head, pair); the CPU attention layer does the
 * same per head (model.c:599-622).  The frequency is rounded once from
 * double (the reference takes it from powf, within an ulp of this). */
void orc_rope(float *x, int n_heads, int head_dim, int pos, float theta)
{
    const int rot = head_dim < 64 ? head_dim : 64;
    for (int h = 0; h < n_heads; ++h) {
        float *v = x + (size_t)h * head_dim;
        for (int i = 0; i + 1 < rot; i += 2) {
            const float inv_freq = (float)(1.0 / pow((double)theta, (double)i / (double)rot));
            const float ang = (float)pos * inv_freq;
            const float c = cosf(ang), s = sinf(ang);
            const float a = v[i], b = v[i + 1];
            v[i] = a * c - b * s;
            v[i + 1] = a * s + b * c;
        }
    }
}

/* attention.metal:17-68.  The shader's thread (row, col) recomputes every
 * score; a score does not depend on col, so it is computed once per (row, t)
 * here with the same d order, and each col's sums run over t ascending as
 * the shader's: the same roundings, without the factor hd of work. */
void orc_attention(float *out, const float *Q, const float *K, const float *V, int seq, int hd,
                   float scale)
{
    float *w = (float *)malloc((size_t)seq * sizeof(float));
    if (!w) return;
    for (int r = 0; r < seq; ++r) {
        float sw = 0.0f;
        for (int t = 0; t < seq; ++t) {
            float score = 0.0f;
            for (int d = 0; d < hd; ++d) score += Q[(size_t)r * hd + d] * K[(size_t)t * hd + d];
            score *= scale;
            w[t] = expf(score);
            sw += w[t];
        }
        for (int c = 0; c < hd; ++c) {
            float ov = 0.0f;
            for (int t = 0; t < seq; ++t) ov += w[t] * V[(size_t)t * hd + c];
            if (sw > 1e-10f) ov /= sw;
            out[(size_t)r * hd + c] = ov;
        }
    }
    free(w);
}

/* attention.metal:80-108: thread i's two loops, for every i. */
void orc_deltanet_step(float *state, const float *Q, const float *K, const float *V, float *out,
                       int dim, float gate)
{
    for (int i = 0; i < dim; ++i) {
        for (int j = 0; j < dim; ++j) {
            const size_t idx = (size_t)j * dim + i;
            state[idx] = gate * state[idx] + (1.0f - gate) * K[i] * V[j];
        }
        float sum = 0.0f;
        for (int j = 0; j < dim; ++j) sum += Q[j] * state[(size_t)j * dim + i];
        out[i] = sum;
    }
}

int orc_moe_layer(const orc_moe_cfg *c, int T, const float *x, const float *resid,
                  const float *norm_w, const float *router_W, const float *bias,
                  const void *gate, const void *up, const void *down,
                  const void *sh_gate, const void *sh_up, const void *sh_down,
                  float *out, uint32_t *idx_out, float *w_out)
{
    return orc_moe_layer_ex(c, T, x, resid, norm_w, router_W, bias, gate, up, down, sh_gate,
                            sh_up, sh_down, NULL, out, idx_out, w_out);
}
