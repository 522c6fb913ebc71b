/* SPDX-License-Identifier: MIT
 *
 * libornith_hip — HIP/gfx950 backend extensions for the routed-MoE hot path.
 *
 * Plain C ABI: opaque handles, plain pointers and sizes, int status codes
 * (ORN_OK = 0, negative on error) with a per-context message from
 * gpu_last_error().  One HIP stream per context; single host thread per
 * context.  Unless ORN_MOE_ASYNC is given, calls are synchronous at return
 * like every gpu.h call.
 */
#ifndef ORNITH_HIP_H
#define ORNITH_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "gpu.h"
#include "kquant.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ORN_OK 0
#define ORN_EINVAL (-1)
#define ORN_ENOMEM (-2)
#define ORN_EHIP (-3)
#define ORN_EUNSUPPORTED (-4)

/* Last error message of a context ("" if none).  No reference counterpart:
 * the reference reports errors through err_buf strings (gguf.c:408-429). */
const char *gpu_last_error(gpu_context *ctx);

/* The Metal shader steps that gpu.h has no declaration for
 * (attention.metal:80-125): the gated DeltaNet step, state[j][i] =
 * gate*state[j][i] + (1-gate)*K[i]*V[j] over the dim x dim state, then
 * out[i] = sum_j Q[j]*state[j][i]; and the KV-cache append, K_cache[pos] =
 * K_new, V_cache[pos] = V_new (rows of head_dim floats).  Synchronous; 0 or
 * a negative status. */
int gpu_deltanet_step_gated(gpu_context *ctx, gpu_buffer *state, const gpu_buffer *Q,
                            const gpu_buffer *K, const gpu_buffer *V, gpu_buffer *out, int dim,
                            float gate);
int gpu_kv_cache_append(gpu_context *ctx, gpu_buffer *K_cache, gpu_buffer *V_cache,
                        const gpu_buffer *K_new, const gpu_buffer *V_new, int pos, int head_dim);

/* Device address of a buffer (for interop and tests). */
void *gpu_device_ptr(gpu_context *ctx, gpu_buffer *buf);

/* Name, compute-unit count and HBM size of the context's device. */
int gpu_device_info(gpu_context *ctx, char *name, size_t name_len, int *n_cus, size_t *hbm_bytes);

/* Measured read bandwidth of the context's device: a streaming-read kernel
 * (16-byte loads, grid-stride) over a fresh buffer of `bytes` (allocated and
 * freed by the call; use several times the 256 MB last-level cache), one
 * untimed launch, then `iters` launches between HIP events on the context's
 * stream.  Writes GB/s (1e9 B/s).  A measurement helper with no reference
 * counterpart: it gives the achievable figure next to the spec-sheet peak. */
int gpu_probe_read_bandwidth(gpu_context *ctx, size_t bytes, int iters, double *gb_per_s);

/* ---------------------------------------------------------------------------
 * Dequantization on the device — the expert-slice / dequant API of
 * engine/src/gguf.h:111-137 with the same validation and bool results.
 *
 * orn_tensor_info is layout-compatible with gguf_tensor_info (gguf.h:15-23),
 * so the engine can pass its descriptors directly.
 * ------------------------------------------------------------------------- */
typedef struct {
    const char *name;
    int type; /* orn_type / ggml_type */
    uint32_t n_dims;
    uint64_t dims[4];
    size_t offset;
    size_t size_bytes;
    size_t n_elems;
} orn_tensor_info;

/* gguf_dequantize_tensor_from_buf (gguf.h:115-117, gguf.c:605-638):
 * host bytes in, host floats out; the work runs on the GPU. */
bool gpu_dequantize_tensor_from_buf(gpu_context *ctx, const void *data,
                                    const orn_tensor_info *tensor, float *output);

/* gguf_dequantize_expert_slice_from_buf (gguf.h:119-127, gguf.c:652-711):
 * interleaved fused tensor, slice[i] = full[i*E + expert], E = last dim. */
bool gpu_dequantize_expert_slice_from_buf(gpu_context *ctx, const void *data,
                                          const orn_tensor_info *tensor, int expert_idx,
                                          float *output);

/* Device-resident variants of the two calls above (data and output are
 * buffers of this context; output must hold n_elems (or n_elems/E) floats). */
bool gpu_dequantize_tensor_buf(gpu_context *ctx, const gpu_buffer *data,
                               const orn_tensor_info *tensor, gpu_buffer *output);
bool gpu_dequantize_expert_slice_buf(gpu_context *ctx, const gpu_buffer *data,
                                     const orn_tensor_info *tensor, int expert_idx,
                                     gpu_buffer *output);

/* ---------------------------------------------------------------------------
 * GGUF container reader — the API of engine/src/gguf.h:67-108 (parse
 * gguf.c:289-404, open/close/accessors 408-487, tensor data 489-506, pread
 * reads 575-601) under orn_gguf_* names, so a model file goes to the device
 * without the engine's parser.  Same arguments, results and NULL/0/false
 * failures; gguf_open's err_buf gets the reason.  On files the reference
 * misparses (n_dims > 4, an alignment that is not a power of two, nested
 * arrays with elements, lengths past the end of the file) this reader
 * fails cleanly or, for nested arrays, skips them whole.
 * ------------------------------------------------------------------------- */
typedef struct orn_gguf orn_gguf;

/* Layout-compatible with gguf_metadata_value (gguf.h:44-66); `type` and
 * `elem_type` are gguf_value_type (0 uint8 .. 12 float64; 8 string, 9 array).
 * string.data is not NUL-terminated; array.data points at the raw elements
 * (for string arrays, at the first (u64 length, bytes) record).  Both stay
 * valid until orn_gguf_close. */
typedef struct {
    int type;
    union {
        uint8_t uint8;
        int8_t int8;
        uint16_t uint16;
        int16_t int16;
        uint32_t uint32;
        int32_t int32;
        uint64_t uint64;
        int64_t int64;
        float float32;
        double float64;
        bool boolean;
        struct {
            const char *data;
            size_t len;
        } string;
        struct {
            int elem_type;
            size_t count;
            const void *data;
        } array;
    } value;
} orn_gguf_value;

orn_gguf *orn_gguf_open(const char *path, char *err_buf, size_t err_buf_size); /* gguf.h:70 */
void orn_gguf_close(orn_gguf *g);                                                /* gguf.h:71 */
uint32_t orn_gguf_version(const orn_gguf *g);                                    /* gguf.h:73 */
uint64_t orn_gguf_tensor_count(const orn_gguf *g);                               /* gguf.h:74 */
uint64_t orn_gguf_metadata_count(const orn_gguf *g);                             /* gguf.h:75 */
const char *orn_gguf_architecture(const orn_gguf *g);                            /* gguf.h:77 */
size_t orn_gguf_alignment(const orn_gguf *g);                                    /* gguf.h:78 */
/* File offset of the data section (no reference accessor; gguf.c:375). */
size_t orn_gguf_data_offset(const orn_gguf *g);
bool orn_gguf_find_metadata(const orn_gguf *g, const char *key,
                            orn_gguf_value *out); /* gguf.h:80-81 */
const orn_tensor_info *orn_gguf_find_tensor(const orn_gguf *g, const char *name); /* gguf.h:83 */
uint64_t orn_gguf_list_tensors(const orn_gguf *g, const orn_tensor_info **tensors,
                               uint64_t max_count); /* gguf.h:84-86, sorted by name */
/* Address of a tensor's bytes in a read-only mapping of the file
 * (gguf.h:87-89); NULL if the mapping failed or the tensor runs past the
 * end of the file. */
const void *orn_gguf_tensor_data(const orn_gguf *g, const char *name);
const void *orn_gguf_tensor_data_from_info(const orn_gguf *g, const orn_tensor_info *info);
/* pread of a whole tensor (buffer_size >= size_bytes) or of the byte range
 * [byte_offset, byte_offset + n) of one; bytes read, 0 on failure
 * (gguf.h:96-108). */
size_t orn_gguf_read_tensor_data(const orn_gguf *g, const orn_tensor_info *tensor, void *buffer,
                                 size_t buffer_size);
size_t orn_gguf_read_tensor_bytes(const orn_gguf *g, const orn_tensor_info *tensor,
                                  size_t byte_offset, void *buffer, size_t n);
/* "<general.architecture>.<param>" as uint32 (gguf.h:137). */
bool orn_gguf_get_param_u32(const orn_gguf *g, const char *param, uint32_t *out);

/* gguf_dequantize_tensor / gguf_dequantize_expert_slice (gguf.h:129-135,
 * gguf.c:641-648, 714-722): the tensor's bytes are read from the file, the
 * dequantization runs on the GPU as in the _from_buf calls above. */
bool gpu_dequantize_tensor_gguf(gpu_context *ctx, const orn_gguf *g,
                                const orn_tensor_info *tensor, float *output);
bool gpu_dequantize_expert_slice_gguf(gpu_context *ctx, const orn_gguf *g,
                                      const orn_tensor_info *tensor, int expert_idx,
                                      float *output);

/* ---------------------------------------------------------------------------
 * Resident routed-MoE layers.  Replaces the per-token expert loop of
 * model.c:1009-1143 (router model.c:1017-1025, selection model.c:1027-1049 /
 * model_get_routing model.c:264-321, slice cache model.c:692-753, expert FFN
 * model.c:1080-1090, combine model.c:1056-1090) and the shared expert of
 * model.c:1003-1007 with one call per layer.
 * ------------------------------------------------------------------------- */
typedef struct ornith_moe_store ornith_moe_store;

typedef struct {
    int n_layers;   /* 40 for Ornith */
    int d_model;    /* D = 2048; 256 times a power of two, or a multiple of 2048 */
    int hidden;     /* H = 512 (expert_feed_forward_length); 256, 512 or 1024 */
    int n_experts;  /* E = 256 (<= 256) */
    int top_k;      /* k = 8 (<= 16) */
    int has_shared; /* 1: one always-on shared expert (model.c:1001-1007) */
    int prefill_layout; /* 1: also keep the MFMA layouts of every expert (about
                           1.13x the quantized bytes more) beside the GGUF
                           blocks; 0: GGUF blocks only (VALU path); 2: the MFMA
                           layouts only: blocks are packed as they are uploaded
                           or generated and not kept (1.13x the GGUF bytes in
                           all); gpu_moe_store_get_experts, the VALU path and
                           cache_slots are then unavailable */
    int file_layout;    /* 1: expert matrices and router in GGUF file orientation
                           (input index fastest: ggml ne = [K, M]; see
                           gpu_moe_store_set_experts); needs prefill_layout = 0.
                           No reference counterpart: the reference reads every
                           matrix as vec@mat (model.c:351-357). */
    int cache_slots;    /* 0: every expert resident in HBM.  N > 0: the experts
                           live in a host tier (pinned host memory) and stream
                           through N device slots, least recently used first
                           (the tiering of memory.c:79-421 over quantized
                           blocks); see gpu_moe_store_prefetch. */
} ornith_moe_shape;

enum { ORN_MAT_GATE = 0, ORN_MAT_UP = 1, ORN_MAT_DOWN = 2 };

ornith_moe_store *gpu_moe_store_create(gpu_context *ctx, const ornith_moe_shape *shape);
void gpu_moe_store_destroy(gpu_context *ctx, ornith_moe_store *store);
size_t gpu_moe_store_bytes(const ornith_moe_store *store);

/* Upload n consecutive experts of one matrix of one layer.  `blocks` holds,
 * for each expert, the GGUF block stream of its matrix in the reference's
 * vec@mat orientation (gate/up: K=D rows x M=H cols, Q4_K; down: K=H rows x
 * M=D cols, Q6_K), i.e. what gguf_dequantize_tensor_from_buf would read for
 * that expert.  expert_first == n_experts selects the shared expert.  The
 * store permutes whole blocks (never re-quantizes).
 * With shape.file_layout = 1 each expert's blocks are instead the GGUF file's
 * bytes for that expert (blk.N.ffn_{gate,up,down}_exps.weight, experts
 * slowest): gate/up H rows of D/256 Q4_K blocks along the input index, down
 * D rows of H/256 Q6_K blocks; they are kept in file order. */
int gpu_moe_store_set_experts(gpu_context *ctx, ornith_moe_store *store, int layer, int matrix,
                              int expert_first, int n, const void *blocks);

/* Router weights W[d*E + e] (model.c:1022 layout) and an optional additive
 * per-expert logit bias (NULL = none).  With shape.file_layout = 1, W is in
 * file orientation instead (ffn_gate_inp.weight: W[e*D + d]); the logits
 * are the same sequential sums over d either way.  */
int gpu_moe_store_set_router(gpu_context *ctx, ornith_moe_store *store, int layer,
                             const float *W, const float *bias);

/* RMSNorm weights applied when ORN_MOE_NORM is set (post_attention_norm,
 * model.c:996).  Default: all ones. */
int gpu_moe_store_set_norm(gpu_context *ctx, ornith_moe_store *store, int layer,
                           const float *w);

/* Shared-expert gate of one layer (no reference counterpart: model.c:
 * 1003-1007 adds the shared expert ungated and the reference loads no
 * ffn_gate_inp_shexp).  w [D] is the layer's blk.N.ffn_gate_inp_shexp.weight
 * (Qwen-MoE models gate their shared expert with it), or NULL to remove
 * it.  Applied only when ORN_MOE_SHEXP_GATE is set: the shared expert's
 * output is then scaled by sigmoid(w . xin) per token. */
int gpu_moe_store_set_shexp_gate(gpu_context *ctx, ornith_moe_store *store, int layer,
                                 const float *w);

/* Fill one layer from the deterministic synthetic generator (orn_synth_*),
 * with an optional Zipf(s) router bias when zipf_s > 0.  The blocks and the
 * router are generated on the device (the same bytes as the host
 * generator), so a 40-layer store fills in seconds. */
int gpu_moe_store_fill_synthetic(gpu_context *ctx, ornith_moe_store *store, int layer,
                                 uint64_t seed, float zipf_s);

/* Read back n experts of one matrix of one layer: the inverse of
 * gpu_moe_store_set_experts (same orientation and block streams).  No
 * reference counterpart: for checks and for saving a store. */
int gpu_moe_store_get_experts(gpu_context *ctx, ornith_moe_store *store, int layer, int matrix,
                              int expert_first, int n, void *blocks);

/* Upload n_layers MoE layers of a model file (file layers from
 * file_first_layer, store layers from store_first_layer) into a store
 * created with file_layout = 1: blk.N.ffn_{gate,up,down}_exps.weight
 * (Q4_K, Q4_K, Q6_K; ne = [D, H, E], [D, H, E], [H, D, E]), with a shared
 * expert blk.N.ffn_{gate,up,down}_shexp.weight (ne = [D, H], [D, H],
 * [H, D]), blk.N.ffn_gate_inp.weight (f32 or f16, ne = [D, E], W[e*D + d])
 * and blk.N.post_attention_norm.weight (f32 [D], when present).  Names as
 * model.c:707-711, 807, 847-852, 861; the bytes are read by range (32
 * experts at a time) and uploaded as they are, never re-quantized.
 * ORN_EUNSUPPORTED for a vec@mat store or a tensor of another type or
 * shape; ORN_EINVAL for a missing tensor or a failed read. */
int gpu_moe_store_load_gguf(gpu_context *ctx, ornith_moe_store *store, const orn_gguf *g,
                            int file_first_layer, int store_first_layer, int n_layers);

/* ---- streamed experts (shape.cache_slots > 0) ------------------------------
 * set_experts / fill_synthetic / load_gguf write the host tier; a forward
 * reads back the experts its dispatch chose (one device->host copy and a
 * stream synchronisation per layer), copies the missing ones into free or
 * least recently used slots (never a pinned one, never one it needs) and
 * runs on the slots.  A forward that needs more experts than there are
 * unpinned slots returns ORN_EINVAL.  ORN_MOE_GRAPH is refused.  Results are
 * those of a resident store, bit for bit. */

/* cache_stats (memory.h:40-55) for the device slots. */
typedef struct {
    uint64_t hits, misses, evictions; /* per (forward or pin, expert) */
    uint64_t prefetches;              /* experts loaded by gpu_moe_store_prefetch */
    uint64_t prefetch_hits;           /* of those, later used by a forward */
    uint64_t bytes_uploaded;          /* host -> device expert bytes */
    int slots, resident, pinned;
    size_t device_bytes, host_bytes;  /* slot pool and host tier */
} ornith_moe_cache_stats;

/* memory_prefetch_submit (memory.c:216-240) for experts: start loading
 * these experts of `layer` on the store's copy stream, into free or least
 * recently used slots that neither a pinned expert nor the last forward
 * holds; returns at once.  A hint: experts with no slot to go to are
 * skipped.  The next forward waits for the copies only if it reads or
 * replaces their slots. */
int gpu_moe_store_prefetch(gpu_context *ctx, ornith_moe_store *store, int layer,
                           const int *experts, int n);
/* memory_hot_promote (memory.c:196-212): load these experts (synchronously)
 * and exempt them from eviction (pin = 1), or make them evictable again
 * (pin = 0). */
int gpu_moe_store_pin(gpu_context *ctx, ornith_moe_store *store, int layer, const int *experts,
                      int n, int pin);
/* memory_get_stats / memory_reset_stats (memory.c:386-405); ORN_EINVAL for a
 * resident store. */
int gpu_moe_store_cache_stats(gpu_context *ctx, ornith_moe_store *store,
                              ornith_moe_cache_stats *out, int reset);

enum { ORN_ROUTE_RENORM = 0, ORN_ROUTE_LITERAL = 1 };
#define ORN_MOE_ASYNC 1u /* return without synchronising the stream */
#define ORN_MOE_NORM 2u  /* expert input = rmsnorm(x, layer norm weights) */
/* Expert-product kernels.  Default: the MFMA kernels (prefill layout, fp16
 * hi+lo activations, fp32 accumulate; decode-shaped instances up to 64
 * tokens, grouped GEMMs above) when the batch has at least
 * ORN_MOE_MFMA_MIN_TOKENS tokens and the store keeps the prefill layouts
 * (Q6_K sub-block scales of any magnitude: above 64 the down kernels split
 * sc * q in two exact fp16 operands); else the VALU matvec kernels (fp32
 * throughout). */
#define ORN_MOE_PATH_VALU 4u /* force the VALU kernels */
#define ORN_MOE_PATH_MFMA 8u /* force the MFMA kernels (EUNSUPPORTED if unavailable) */
#define ORN_MOE_MFMA_MIN_TOKENS 1
/* Replay as a HIP graph: the first call with a given (layer(s), token
 * count, route mode, flags, buffer addresses) runs normally and records its
 * kernel sequence; later identical calls launch the recorded graph (one
 * host call for the whole forward).  Buffer contents may change between
 * calls, their addresses may not.  Uploading to the store drops the
 * recordings.  Ignored while kernel profiling is on. */
#define ORN_MOE_GRAPH 16u
/* Scale the shared expert by its gate (gpu_moe_store_set_shexp_gate; a
 * layer without one is refused with ORN_EINVAL).  Not in the reference. */
#define ORN_MOE_SHEXP_GATE 32u
/* Routing of the smallest decode batches (up to 4 tokens, D a power-of-two
 * multiple of 256 up to 4096, E <= 256).  By default the router logits are fp64 sums
 * of the reference's fp32 products with a rigorous bound on their distance
 * from the reference's sequential fp32 chain (model.c:1017-1025); the top-k
 * selection equals the chain's exactly (where the bounds do not decide it,
 * the undecided experts run the chain itself), and logits, selection and
 * dispatch run in one launch.  The logits gpu_moe_last_logits reports are
 * then those sums rounded to fp32 (within a few ulp of the chain's), and the
 * weights follow from them.  With this flag every logit is the chain's,
 * bit for bit, on every batch size (a slower router at decode sizes).  Not
 * in the reference. */
#define ORN_MOE_EXACT_LOGITS 64u

typedef struct {
    int route_mode; /* ORN_ROUTE_RENORM (default, model_get_routing) or ORN_ROUTE_LITERAL */
    unsigned flags; /* ORN_MOE_* */
    /* Expert-parallel share (no reference counterpart; 0, 0 = every expert):
     * the forward routes every token over all experts, as each rank of an
     * expert-parallel deployment does, but computes only the selected
     * experts in [ep_first, ep_first + ep_count); the shared expert belongs
     * to the share with ep_first == 0.  Summing the outputs of the shares
     * that cover 0..E-1 (resid passed to one of them) gives the full
     * layer's output; idx_out / w_out are the full selection in every share. */
    int ep_first, ep_count;
} ornith_moe_opts;

/* One MoE block for n_tokens rows of x ([T][D] fp32):
 *   out = (resid + shared(xin)) + sum_a w_a * expert_a(xin),
 *   (shared(xin) scaled by sigmoid(gate . xin) with ORN_MOE_SHEXP_GATE),
 *   xin = (flags & ORN_MOE_NORM) ? rmsnorm(x) : x;  resid may be NULL (zeros).
 * idx_out ([T][k] uint32) and w_out ([T][k] fp32) may be NULL.  out may not
 * alias x or resid. */
int gpu_moe_forward(gpu_context *ctx, ornith_moe_store *store, int layer, const gpu_buffer *x,
                    int n_tokens, const gpu_buffer *resid, gpu_buffer *out, gpu_buffer *idx_out,
                    gpu_buffer *w_out, const ornith_moe_opts *opts);

/* gpu_moe_forward that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops or harnesses that forbid hipMalloc).  Same
 * arguments and results as gpu_moe_forward; the forward's work buffers
 * live in a fixed per-device scratch array of ORN_NOALLOC_SCRATCH_BYTES
 * (32 MiB: decode batches up to 64 tokens at the Ornith shape D=2048,
 * H=512, E=256, k=8), which each GPU the library runs on holds until the
 * process ends.  A call whose work buffers would not fit returns ORN_EINVAL
 * with the needed size in gpu_last_error(); ORN_MOE_GRAPH is refused
 * (instantiating a graph allocates).  Every call on one GPU shares that
 * GPU's scratch: calls that overlap on one GPU (two contexts, or
 * ORN_MOE_ASYNC calls on different streams) race.  After such a call,
 * gpu_moe_last_logits and gpu_moe_last_stats on this context read that
 * scratch: they report this call only until the next noalloc call on the
 * same GPU, from any context. */
#define ORN_NOALLOC_SCRATCH_BYTES (32u << 20)
int gpu_moe_forward_noalloc(gpu_context *ctx, ornith_moe_store *store, int layer,
                            const gpu_buffer *x, int n_tokens, const gpu_buffer *resid,
                            gpu_buffer *out, gpu_buffer *idx_out, gpu_buffer *w_out,
                            const ornith_moe_opts *opts);

/* Layer stack: for l in [first, first+n): x <- x + MoE_l(rmsnorm(x)) (the
 * per-layer MoE residual structure of model.c:992-1144).  tmp must hold
 * n_tokens*D floats.  Every expert is computed (opts' expert share is not
 * used: a share needs a reduction across ranks between layers). */
int gpu_moe_forward_stack(gpu_context *ctx, ornith_moe_store *store, int first_layer,
                          int n_layers, gpu_buffer *x, gpu_buffer *tmp, int n_tokens,
                          const ornith_moe_opts *opts);

/* Router logits of the last forward on this context (of the last layer,
 * after a stack call): T x E fp32, row-major, the values the top-k selection
 * ran on (the sums of model.c:1017-1025 plus the bias).  Copies
 * min(max_floats, T*E) floats to the host array `out` and stores T*E in
 * *n_floats (0 before any forward).  No reference counterpart: a test and
 * measurement helper like gpu_moe_last_stats.  After gpu_moe_forward_noalloc
 * the values live in the device's shared scratch and are valid only until
 * the next noalloc call on that GPU. */
int gpu_moe_last_logits(gpu_context *ctx, float *out, size_t max_floats, size_t *n_floats);

/* Counters of the last forward: number of active expert slots (incl. the
 * shared expert), token rows, and tokens whose top-k ran the literal
 * exchange selection (tied or non-finite logits among the top k+1).  After
 * gpu_moe_forward_noalloc: valid until the next noalloc call on that GPU. */
int gpu_moe_last_stats(gpu_context *ctx, int *n_slots, int *n_rows, int *n_literal);
/* Tokens of the last forward whose certified routing (see
 * ORN_MOE_EXACT_LOGITS) ran the reference's exact chain for some of their
 * logits because the bounds did not decide the selection (0 for the exact
 * routers).  No reference counterpart: a test and measurement helper. */
int gpu_moe_last_chained(gpu_context *ctx, int *n_chained);

/* ---------------------------------------------------------------------------
 * Kernel timing with HIP events recorded on the context's stream around every
 * launch of the MoE path (no reference counterpart; the reference times the
 * MoE block with clock_gettime, model.c:940-1148).
 * ------------------------------------------------------------------------- */
int gpu_profile_enable(gpu_context *ctx, int on);
void gpu_profile_reset(gpu_context *ctx);
int gpu_profile_count(gpu_context *ctx);
const char *gpu_profile_name(gpu_context *ctx, int i);
double gpu_profile_total_ms(gpu_context *ctx, int i);
long gpu_profile_calls(gpu_context *ctx, int i);

/* ---------------------------------------------------------------------------
 * Deterministic synthetic workload generator (host).  Counter-based
 * (SplitMix64 finaliser), so any block of any tensor can be produced
 * independently; quantized blocks use integer arithmetic only and halves are
 * rounded to nearest-even, so the bytes are identical on every host.
 * ------------------------------------------------------------------------- */
enum {
    ORN_SYN_GATE = 1,
    ORN_SYN_UP = 2,
    ORN_SYN_DOWN = 3,
    ORN_SYN_ROUTER = 4,
    ORN_SYN_ACT = 5,
    ORN_SYN_ZIPF = 6
};
uint64_t orn_synth_stream(int layer, int kind, int expert);
/* Q4_K: d, dmin ~ fp16(U(0.001, 0.01)); 12 random scale bytes; random qs. */
void orn_synth_q4k(uint64_t seed, uint64_t stream, uint64_t first_block, uint64_t n_blocks,
                   void *out);
/* Q6_K: random ql/qh; int8 scales uniform in [-32, 31]; d ~ fp16(U(0.001, 0.01)). */
void orn_synth_q6k(uint64_t seed, uint64_t stream, uint64_t first_block, uint64_t n_blocks,
                   void *out);
/* Approximately normal (Irwin-Hall sum of 12 16-bit uniforms, exact in
 * binary) scaled by sigma and rounded once to fp32. */
void orn_synth_normal(uint64_t seed, uint64_t stream, uint64_t n, float sigma, float *out);
/* Zipf(s) logit bias: b_e = -s * ln(rank_e), rank a seeded permutation of 1..E. */
void orn_synth_zipf_bias(uint64_t seed, uint64_t stream, int n_experts, float s, float *out);

#ifdef __cplusplus
}
#endif

#endif /* ORNITH_HIP_H */
