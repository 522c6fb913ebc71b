/* SPDX-License-Identifier: MIT
 *
 * The thin C ABI between the C99 host code (csrc/host/) and the hand-written
 * gfx950 kernels (csrc/kernels/ .hip files).  Plain pointers, sizes and a HIP
 * stream; every launcher returns a hipError_t value (0 = success) and only
 * enqueues work on the given stream.
 */
#ifndef ORNITH_KERNELS_LAUNCH_H
#define ORNITH_KERNELS_LAUNCH_H

#include <stddef.h>
#include <stdint.h>

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the down (Q6_K) MFMA layout ------------------------------------------
 * Per expert, [H/32][D/256] units of 6144 bytes, one per reduction step of
 * 32 and 256-column block: the 6-bit values q + 32 (0..63) of the unit's
 * 32 x 256 weights, in the lane order of the MFMA B operand (wave w, lane
 * l = 16g + c, column tile 4w + j, values k = 8g + e, e = 0..7):
 *   bytes 0..4095:    u32 [4][64][4] low nibbles, value e at bit
 *                     4*(e/2) + 16*(e%2) of word (w, l, j);
 *   bytes 4096..6143: u32 [4][64][2] high two bits, value e of tile j at bit
 *                     2*(e/2) + 16*(e%2) + 8*(j%2) of word (w, l, j/2).
 * 0.75 bytes per weight (the GGUF Q6_K body is 0.8125 with its scales). */
#define ORNK_DQ_UNIT 6144u
#define ORNK_DQ_BYTES(DH) ((size_t)(DH) / 4 * 3)

/* ---- generic fp32 ops behind gpu.h --------------------------------------- */
int ornk_fill_f32(float *p, float v, size_t n, hipStream_t s);
#define ORNK_STREAM_GRID 16384
int ornk_stream_read(const void *p, size_t bytes, uint32_t *out, hipStream_t s);
int ornk_matmul_f32(float *C, const float *A, const float *B, int M, int N, int K, hipStream_t s);
int ornk_rmsnorm(float *out, const float *x, const float *w, int rows, int dim, hipStream_t s);
int ornk_silu(float *out, const float *x, int n, hipStream_t s);
int ornk_silu_mul(float *out, const float *g, const float *u, int n, hipStream_t s);
int ornk_add(float *out, const float *a, const float *b, int n, hipStream_t s);

/* ---- attention-side ops behind gpu.h (attn.hip) --------------------------- */
/* RoPE on n_q heads of Q and n_k heads of K (first min(head_dim, 64) dims). */
int ornk_rope(float *Q, float *K, int head_dim, int n_q, int n_k, int pos, float theta,
              hipStream_t s);
/* Single-head attention, Q/K/V/out [seq][hd], hd <= 256. */
int ornk_attention(float *out, const float *Q, const float *K, const float *V, int seq, int hd,
                   float scale, hipStream_t s);
size_t ornk_attention_lds(int hd);
/* The same on the matrix cores (hd % 4 == 0, hd <= 256); ws holds
 * ornk_attention_mma_ws(seq, hd) bytes (0: none needed). */
size_t ornk_attention_mma_ws(int seq, int hd);
int ornk_attention_mma(float *out, const float *Q, const float *K, const float *V, int seq, int hd,
                       float scale, void *ws, hipStream_t s);
int ornk_deltanet_step(float *state, const float *Q, const float *K, const float *V, float *out,
                       int dim, float gate, hipStream_t s);
int ornk_kv_append(float *Kc, float *Vc, const float *Kn, const float *Vn, int pos, int hd,
                   hipStream_t s);

/* ---- fixed scratch of the forward that allocates nothing (scratch.hip) ---- */
/* Size of the per-device scratch array; equals ORN_NOALLOC_SCRATCH_BYTES of
 * ornith_hip.h. */
#define ORNK_SCRATCH_BYTES (32u << 20)
/* Device address of the scratch array on `device`, which must be the current
 * device; resolved once per device (hipGetSymbolAddress) and cached. */
int ornk_scratch_resolve(int device, void **addr);

/* ---- synthetic layers generated on the device (synth.hip) ------------------
 * The same bytes as the host generator (synth.c), written into one layer's
 * resident arrays: gate/up Q4_K blocks, down Q6_K bodies + d (store order:
 * vec@mat block-column-major, or file order when file = 1) and the router in
 * the [D/4][E][4] layout. */
typedef struct {
    uint64_t seed;
    int layer, D, H, n_experts, has_shared, file;
    uint8_t *gate, *up, *down_body;
    uint16_t *down_d;
    float *router;
} ornk_synth_args;
int ornk_synth_layer(const ornk_synth_args *a, hipStream_t s);

/* MFMA (prefill) layouts of n_e expert slots built from their resident
 * vec@mat blocks (prefill_pack.c arithmetic); dmax [n_e][3] and *scmax
 * (largest |Q6_K sub-scale|) are recomputed. */
typedef struct {
    int D, H, n_e;
    const uint8_t *gu[2], *down_body;
    const uint16_t *down_d;
    uint32_t *pq[2];
    uint16_t *psc[2], *pmn[2];
    float *pd[2], *pdm[2];
    uint8_t *dq;
    uint16_t *dsc;
    float *dd;
    float *dmax;
    int *scmax;
    /* NULL: slots [0, n_e) of the arrays above.  Else the n_e slot numbers
     * to pack (device-readable); the caller zeroes their dmax entries. */
    const int *slots;
} ornk_pack_args;
int ornk_pack_prefill(const ornk_pack_args *a, hipStream_t s);

/* Expert loads of a streamed store (cache.hip): for i < n, expert loads[2i]
 * of the host tier (device addresses of pinned host memory, [L*(E+1)]
 * experts) is copied into device slot loads[2i+1]; slots_out[i] receives
 * the slot and, with dmax, the slot's three dmax entries are zeroed. */
typedef struct {
    const int *loads;
    int n;
    const uint8_t *h_gate, *h_up, *h_body;
    const uint16_t *h_d;
    uint8_t *gate, *up, *body;
    uint16_t *d;
    int *slots_out;
    float *dmax;
    size_t nb;
} ornk_gather_args;
int ornk_cache_gather(const ornk_gather_args *a, hipStream_t s);

/* ---- GGUF dequant (gguf.c:605-711 semantics) ----------------------------- */
int ornk_dequant(const void *src, int type, uint64_t n_elems, float *dst, hipStream_t s);
int ornk_dequant_slice(const void *src, int type, uint64_t n_elems, uint64_t n_experts,
                       int expert, float *dst, hipStream_t s);

/* ---- routing -------------------------------------------------------------- */
/* Bit-exact sequential fp32 router logits for T tokens (model.c:1017-1025). */
int ornk_router_exact(const float *x, const float *W, const float *bias, int T, int D, int E,
                      float *logits, hipStream_t s);
/* Per-token top-k with the reference's exchange-selection semantics.
 * mode 0: exchange on logits + softmax over the top-k (model.c:301-317);
 * mode 1: full softmax + exchange on probabilities (model.c:1027-1049).
 * n_exact (device int, may be NULL) counts tokens whose selection ran the
 * literal exchange simulation (ties or NaN). */
int ornk_topk(const float *logits, int T, int E, int k, int mode, uint32_t *idx, float *w,
              int *n_exact, hipStream_t s);

/* ---- the routed-MoE layer -------------------------------------------------- */
/* Device layout of one layer's experts (expert index E is the shared expert):
 *   gate/up   : [E+1][H/256][D] Q4_K blocks of 144 B, block (row k, block
 *               column c) of expert e at ((e*(H/256) + c)*D + k)*144
 *   down_body : [E+1][D/256][H] Q6_K bodies of 208 B (ql|qh|scales)
 *   down_d    : [E+1][D/256][H] Q6_K super-scales (fp16 bits)
 *   router    : [D/4][E][4] fp32, W(d, e) at ((d/4)*E + e)*4 + d%4
 * Work buffers are owned by the host.
 *
 * Prefill (MFMA) layouts of one layer, per expert slot (prefill_pack.c): */
typedef struct {
    const uint32_t *pq[2];         /* gate, up nibbles [D/32][H/256][4][64][4] */
    const uint16_t *psc[2], *pmn[2]; /* [D/32][H/256][8][32] fp16 scales, mins */
    const float *pd[2], *pdm[2];   /* [H/256][D] d, dmin */
    const float *dmax;             /* [E+1][3] */
} ornk_gu_prefill;

typedef struct {
    const uint8_t *dq;   /* [H/32][D/256] units of ORNK_DQ_UNIT bytes: q + 32 in 6 bits */
    const uint16_t *dsc; /* [H/32][D/256][16][32] fp16 sub-block scales */
    const float *dd;     /* [D/256][H] d */
    const float *dmax;   /* [E+1][3] */
} ornk_dn_prefill;

/* File-orientation path (expert_file.hip): activations split into fp16
 * hi/lo (pairs in the order [0,2,1,3] within each group of 4 values), times
 * a power of two per row; inv = its inverse. */
typedef struct {
    uint32_t *xh, *xl;   /* [T][D/2] */
    uint16_t *xsh, *xsl; /* [T][D/32] sub-block sums / 32, hi and lo */
    float *xinv;         /* [T] */
    uint32_t *mh, *ml;   /* [rows_max][H/2] */
    float *minv;         /* [rows_max] */
} ornk_file_ws;

typedef struct {
    int T, D, H, E, k, has_shared, mode, apply_norm;
    int ep_lo, ep_n;  /* experts computed: [ep_lo, ep_lo + ep_n) (an expert-parallel share) */
    int ks_gu, ks_dn, rows_max, items_max, tchunk;
    const uint8_t *gate, *up, *down_body;
    const uint16_t *down_d;
    const float *router, *bias, *norm_w;
    const float *x, *resid;
    float *out;
    const float *shexp_gate; /* [D] or NULL: the shared expert scaled by sigmoid(gate . xin) */
    /* workspace */
    float *xn;        /* [T][D]  expert input (x or rmsnorm(x)) */
    float *logits;    /* [T][E] */
    uint32_t *idx;    /* [T][k] */
    float *w;         /* [T][k] */
    int *ctl;         /* [16] counters: 0 n_slots, 1 n_items, 2 n_rows, 3 n_literal;
                         zeroed by the routing step */
    int *slot_expert; /* [E+1] */
    int *slot_off;    /* [E+1] */
    int *slot_cnt;    /* [E+1] */
    int *row_token;   /* [rows_max] */
    int *pair_row;    /* [T*k] */
    int *items;       /* [items_max][4]: slot, row_begin, n_rows, expert (E = shared) */
    float *gu_part;   /* [ks_gu][rows_max][2H] */
    float *mid;       /* [rows_max][H] */
    float *dn_part;   /* [ks_dn][rows_max][D] */
    /* MFMA path (ks_gu = ks_dn = 1, tchunk <= 64) */
    int use_mfma;
    ornk_gu_prefill gu_pf;
    ornk_dn_prefill dn_pf;
    float *x_amax;    /* [T] max |xin| per token */
    int router_amax;  /* 1: the routing step writes x_amax (else the MFMA launchers do) */
    float *mid_amax;  /* [rows_max] max |mid| per row (written by the mid step) */
    int q6_wide;      /* 1: some Q6_K sub-scale of the layer exceeds 64 in magnitude (the
                         down kernels split sc * q in two exact fp16 operands) */
    /* File-orientation path: gate/up [E+1][H][D/256] Q4_K blocks, down body
     * and d [E+1][D][H/256] (the blocks in file order) */
    ornk_file_ws fw;
    /* Certified routing (router_cert.hip): T*E 64-bit handoff words, and a
     * 4 KB counter area that starts zeroed (the kernel keeps its counter at
     * zero between launches and advances a generation word in it). */
    double *route_est;
    int *sync;
    /* Profiling: if set, the expert-product launchers launch their main kernel
     * with hipExtLaunchKernel so that these events carry its start and end. */
    hipEvent_t ev_start, ev_stop;
} ornk_moe_args;

int ornk_moe_norm(const ornk_moe_args *a, hipStream_t s);
int ornk_moe_route(const ornk_moe_args *a, hipStream_t s);
/* Batches the one-wave-per-(token, 8 experts) router takes (and that can
 * produce x_amax on the side). */
#define ORN_ROUTER_PC_MAX_T 64
int ornk_router_pc_supported(int T, int D);
/* Whether the decode down kernel forms mid itself (the mid step is then
 * skipped): one token, 16 gate/up split-K slices, 8-step down slices. */
int ornk_down_dec_fuses_mid(int T, int H, int ks_gu, int ks_dn);
int ornk_moe_dispatch(const ornk_moe_args *a, hipStream_t s);
/* Certified routing of decode batches: logits, top-k and dispatch in one
 * launch (router_cert.hip); replaces ornk_moe_route + ornk_moe_dispatch
 * (and the norm step) for T <= ORN_CERT_MAX_T.  The logits it reports are
 * fp64 sums rounded to fp32 (the reference's exact chain for tokens whose
 * selection needed it); the selection equals the exact chain's. */
#define ORN_CERT_MAX_T 4
#define ORNK_SYNC_BYTES 4096u
int ornk_route_cert_supported(int T, int D, int E, int k);
int ornk_moe_route_cert(const ornk_moe_args *a, hipStream_t s);
/* items[i].w (i < min(ctl[1], items_max)) and slot_expert[s] (s < min(ctl[0],
 * slots_max)) replaced by remap[] of themselves: expert ids -> cache slots. */
int ornk_remap_items(int *items, int *slot_expert, const int *ctl, const int *remap,
                     int items_max, int slots_max, hipStream_t s);
int ornk_moe_gateup(const ornk_moe_args *a, hipStream_t s);
int ornk_moe_mid(const ornk_moe_args *a, hipStream_t s);
int ornk_moe_down(const ornk_moe_args *a, hipStream_t s);
/* MFMA expert products: prefill-shaped (items of <= 64 rows) and
 * decode-shaped (items of <= 16 rows, deeper load pipelining). */
int ornk_moe_gateup_mfma(const ornk_moe_args *a, hipStream_t s);
int ornk_moe_down_mfma(const ornk_moe_args *a, hipStream_t s);
int ornk_moe_gateup_dec(const ornk_moe_args *a, hipStream_t s);
/* 1 if the decode instances cover kt_gu (D/32/ks_gu) and kt_dn (H/32/ks_dn). */
int ornk_dec_supported(int kt_gu, int kt_dn);
int ornk_moe_down_dec(const ornk_moe_args *a, hipStream_t s);
/* out[r] = max_k |x[r][k]| (D a multiple of 4). */
int ornk_file_supported(int D, int H);
/* Output columns of one work group of the file-orientation down kernel. */
int ornk_file_down_cols(void);
int ornk_file_prep_x(const ornk_moe_args *a, hipStream_t s);
int ornk_file_gateup(const ornk_moe_args *a, hipStream_t s);
int ornk_file_down(const ornk_moe_args *a, hipStream_t s);
int ornk_rowmax(const float *x, int rows, int D, float *out, hipEvent_t start, hipStream_t s);
int ornk_moe_combine(const ornk_moe_args *a, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* ORNITH_KERNELS_LAUNCH_H */
