// SPDX-License-Identifier: MIT
//
// Expert products for weights in GGUF file orientation (store built with
// ornith_moe_shape.file_layout = 1).  In a GGUF file every matrix is stored
// output-row-major with the input index fastest (ggml ne = [K, M]): row i of
// gate/up (i < H) is D/256 Q4_K blocks along d, row n of down (n < D) is
// H/256 Q6_K blocks along the hidden index.  The reference reads its
// matrices as vec@mat (model.c:351-357) and has no path for this
// orientation; the arithmetic per element is its block dequant (gguf.c:43-61
// Q4_K, gguf.c:64-86 Q6_K) and the products accumulate in fp32.
//
// Here the block scales vary with the output column, so they cannot be
// folded into the activation tile as in the vec@mat kernels.  MFMA roles:
// rows = the item's token rows (16), columns = 16 output rows of the file
// matrix, k = the input index.
//   Q4_K (v_mfma_f32_16x16x32_f16): B = sc*q (sc the 6-bit sub-block scale
//     of this column, exact in fp16), P = sum over one super-block (8 steps
//     of 32), then acc += d(column) * P; the mins term is one more MFMA per
//     super-block over the rows' sub-block sums: acc -= dmin(column) *
//     sum_j m(column, j) * xsum(row, j).
//   Q6_K (v_mfma_f32_16x16x32_f16): sub-block scales are int8, so |sc * q|
//     reaches 4096, past fp16's exact integers; B = sc * (q - 32) goes in
//     as b1 = fp16(B) plus the exact remainder b2 = B - b1 (|b2| <= 1, one
//     fma), A_hi*b1 + A_lo*b1 + A_hi*b2 per step (the dropped A_lo*b2 is
//     below 2^-21 of |A*B|), P = sum over one super-block, acc += d(column)
//     * P.  (Steps of one 16-value sub-block on v_mfma_f32_16x16x16_f16
//     with the scale applied to each step's result ran 47.3 against 25.8
//     us at 16 tokens: twice the loads and four fp32 fmas per step.)
// Activations come from k_prep_rows (the expert inputs) and from the mid
// step (k_mid, expert_valu.hip, for the down kernel), which split each row
// (times a power of two s, |x*s| < 2^14) into fp16 hi + lo once per
// forward, and reach the waves through one LDS tile per super-block and
// work group; products of hi and lo with the exact B accumulate in fp32,
// and outputs are scaled back by 1/s.
//
// Any permutation of k applied to both A and B leaves a dot product
// unchanged; the loads use two: within each group of 8 consecutive values
// the prep stores the order [0,2,1,3,4,6,5,7], which is the order in which
// one v_bfi of a word of nibbles (or one v_perm of a word of bytes) yields
// fp16 pairs; and a Q4_K lane loads 16 consecutive bytes of nibbles (32
// values of two sub-blocks) that feed four steps.
#include "common.h"
#include "launch.h"
#include "mfma_ops.h"

using namespace orn_mfma;

namespace {

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// Activation tile of one super-block in LDS: [hi, lo][16 rows][256 values]
// (row stride padded to 264 halves), staged once per work group from the
// prepared rows src[r] (an LDS int[16]) and shared by its four waves.  Two
// tiles alternate, so one barrier per super-block suffices: a wave writes
// tile (s+1)&1 only after every wave has passed the barrier of super-block
// s, which each reaches after its reads of that tile for super-block s-1.
//
// Prefill-sized work items (up to 64 rows, RT = 4 row tiles of 16) stage one
// tile of 64 rows (68 KB) per work group instead of two alternating ones of
// 16: the tile is then rewritten only after a barrier that every wave
// reaches once done with the previous super-block, so that two work groups
// still fit in a CU's LDS.  Each converted weight operand then feeds RT row
// tiles, and each expert's weights stream once per 64 rows.
#define ORN_FAS 264
template <int RT>
struct FileTileT {
    _Float16 v[2][16 * RT][ORN_FAS];
};
typedef FileTileT<1> FileTile;

// With LIVE_ONLY (the down kernel's 16-row items) only the item's nr live
// rows are staged: an MFMA output row depends on its own A row alone, and
// rows at or past nr are never stored, so whatever the tile holds there (an
// earlier super-block's rows, or uninitialised LDS) cannot reach an output.
// Decode items hold a row or two.  Elsewhere every row is staged (clamped
// to the last live one): measured, predicated copies cost more there than
// the rows they skip.
template <int RT, bool LIVE_ONLY>
__device__ __forceinline__ void stage_tile(FileTileT<RT> &As, const uint32_t *__restrict__ xh,
                                           const uint32_t *__restrict__ xl, const int *src,
                                           int K, int s, int nr)
{
    if (RT > 1) __syncthreads();  // one tile: every wave is done with the last one
#pragma unroll
    for (int i = 0; i < 4 * RT; ++i) {  // 2 planes x 16RT rows x 32 chunks of 16 B
        const int idx = threadIdx.x + 256 * i;
        const int plane = idx / (512 * RT), row = (idx >> 5) % (16 * RT), ch = idx & 31;
        if (!LIVE_ONLY || RT > 1 || row < nr)
            *reinterpret_cast<uint4 *>(&As.v[plane][row][8 * ch]) =
                *reinterpret_cast<const uint4 *>((plane ? xl : xh) + (size_t)src[row] * (K >> 1) +
                                                 128 * s + 4 * ch);
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Row preparation: one work group per row of x ([n][K] fp32, K <= 2048,
// K % 256 == 0).  Writes hi/lo fp16 of x*s in the pair order above, inv[r]
// = 1/s, and with SUMS the sub-block sums sum_{32} x*s / 32 as fp16 hi/lo
// ([n][K/32], natural order; /32 keeps them below 2^14).  Rows at or past
// *live (when live is given) are skipped.
// ---------------------------------------------------------------------------
template <bool SUMS>
__global__ void __launch_bounds__(256)
    k_prep_rows(const float *__restrict__ x, int K, const int *__restrict__ live,
                uint32_t *__restrict__ hi, uint32_t *__restrict__ lo, float *__restrict__ inv,
                uint16_t *__restrict__ shi, uint16_t *__restrict__ slo)
{
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    if (live && r >= *live) return;
    const int ng = K >> 3;  // groups of 8 values
    const bool on = tid < ng;
    const float *xr = x + (size_t)r * K + 8 * tid;
    v4f a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (on) {
        a = *reinterpret_cast<const v4f *>(xr);
        b = *reinterpret_cast<const v4f *>(xr + 4);
    }
    float m = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                    fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = prep_scale(m);
    a *= s;
    b *= s;
    if (on) {
        uint32_t h[4], l[4];
        split2(a.x, a.z, h[0], l[0]);
        split2(a.y, a.w, h[1], l[1]);
        split2(b.x, b.z, h[2], l[2]);
        split2(b.y, b.w, h[3], l[3]);
        const size_t o = (size_t)r * (K >> 1) + 4 * tid;  // u32 words
        *reinterpret_cast<uint4 *>(hi + o) = make_uint4(h[0], h[1], h[2], h[3]);
        *reinterpret_cast<uint4 *>(lo + o) = make_uint4(l[0], l[1], l[2], l[3]);
    }
    if (tid == 0) inv[r] = 1.0f / s;
    if (SUMS) {
        // 4 consecutive threads hold one 32-value sub-block
        float t = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        t += __shfl_xor(t, 1, 64);
        t += __shfl_xor(t, 2, 64);
        if (on && (tid & 3) == 0) {
            t *= 0.03125f;
            const _Float16 th = (_Float16)t;
            const _Float16 tl = (_Float16)(t - (float)th);
            const size_t o = (size_t)r * (K >> 5) + (tid >> 2);
            shi[o] = __builtin_bit_cast(uint16_t, th);
            slo[o] = __builtin_bit_cast(uint16_t, tl);
        }
    }
}

// ---------------------------------------------------------------------------
// Gate/up, Q4_K.  Logical tile = (item * ks + kslice) * NCB + cb; wave w of
// the work group covers output columns cb*64F + 16Fw + 16ct + c (ct < F =
// ORN_FCT column tiles, c < 16) of the concatenated [gate | up] outputs,
// over super-blocks kslice*nsb .. +nsb; each activation operand feeds the
// ORN_FCT tiles.  Output gu[kslice][row][2H].
// ---------------------------------------------------------------------------
// Column tiles per wave: 4 for 16-row items; 2 for 64-row items, whose
// accumulators (4 row tiles) would otherwise leave one wave per SIMD.
template <int RT>
constexpr int gu_fct()
{
    return RT == 1 ? 4 : 2;
}

template <int RT>
__global__ void __launch_bounds__(256, 2)
    k_gu_file(const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up,
              const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl,
              const float *__restrict__ xinv, const uint16_t *__restrict__ sh,
              const uint16_t *__restrict__ sl, const int *__restrict__ ctl,
              const int4 *__restrict__ items, const int *__restrict__ row_token,
              float *__restrict__ gu, int D, int H, int ks, int rows_max)
{
    constexpr int ORN_FCT = gu_fct<RT>();
    const int NCB = (2 * H) / (64 * ORN_FCT);
    const int per_item = NCB * ks;
    const int n_live = ctl[1] * per_item;
    if ((int)blockIdx.x >= n_live) return;
    const int tile = xcd_remap(blockIdx.x, n_live);
    const int cb = tile % NCB;
    const int kslice = (tile / NCB) % ks;
    const int4 itm = items[tile / per_item];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
    // the wave's 16 * ORN_FCT columns lie in one matrix
    const int col0 = cb * (64 * ORN_FCT) + 16 * ORN_FCT * wave;
    const int m = col0 >= H, h0 = col0 - m * H + c;
    const int NSB = D >> 8, nsb = NSB / ks, s0 = kslice * nsb;
    const size_t rstride = (size_t)NSB * 144;  // bytes per file row
    const uint8_t *rowp = (m ? up : gate) + ((size_t)itm.w * H + h0) * rstride;  // tile ct: + 16ct rows
    const int nrows = itm.z;
    const int nrt = RT == 1 ? 1 : (nrows + 15) >> 4;  // live row tiles
    constexpr int NB = RT == 1 ? 2 : 1;                // activation tiles in LDS
    __shared__ __align__(16) FileTileT<RT> Ab[NB];
    __shared__ int src[16 * RT];
    if (threadIdx.x < 16 * RT)
        src[threadIdx.x] = row_token[itm.y + ((int)threadIdx.x < nrows ? (int)threadIdx.x : nrows - 1)];
    __syncthreads();
    const uint16_t *sah[RT], *sal[RT];  // A row 16rt + c of the mins operand
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int tok = src[16 * rt + c];
        sah[rt] = sh + (size_t)tok * (D >> 5);
        sal[rt] = sl + (size_t)tok * (D >> 5);
    }

    v4f acc[RT][ORN_FCT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < ORN_FCT; ++ct) acc[rt][ct] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = s0; s < s0 + nsb; ++s) {
        uint4 hd[ORN_FCT], w[ORN_FCT][2];
#pragma unroll
        for (int ct = 0; ct < ORN_FCT; ++ct) {
            const uint8_t *blk = rowp + (size_t)(16 * ct) * rstride + (size_t)s * 144;
            hd[ct] = *reinterpret_cast<const uint4 *>(blk);  // d, dmin, scales[12]
            w[ct][0] = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * g);
            w[ct][1] = *reinterpret_cast<const uint4 *>(blk + 80 + 16 * g);
        }
        FileTileT<RT> &As = Ab[NB == 2 ? (s & 1) : 0];
        stage_tile<RT, false>(As, xh, xl, src, D, s, nrows);
        v4f P[RT][ORN_FCT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < ORN_FCT; ++ct) P[rt][ct] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int L = 0; L < 2; ++L) {
            // this lane's 16 bytes: chunk p = 2L + g/2 (sub-blocks 2p low
            // nibbles, 2p+1 high), positions 16*(g&1) .. +16
            const int p = 2 * L + (g >> 1);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int j = 2 * p + (t >> 1);
                const int kl = 32 * j + 16 * (g & 1) + 8 * (t & 1);  // k - 256 s
                v8h xa[RT], xb[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    if (rt < nrt) {
                        xa[rt] = *reinterpret_cast<const v8h *>(&As.v[0][16 * rt + c][kl]);
                        xb[rt] = *reinterpret_cast<const v8h *>(&As.v[1][16 * rt + c][kl]);
                    }
                }
                const int sft = (t >> 1) ? 4 : 0;
#pragma unroll
                for (int ct = 0; ct < ORN_FCT; ++ct) {
                    uint32_t scj, mj;
                    orn_scale_min_k4(j, hd[ct].y, hd[ct].z, hd[ct].w, scj, mj);
                    const _Float16 sf = (_Float16)(float)scj;
                    const v2h sv = {sf, sf};
                    const v2h ns = sv * (v2h){(_Float16)-1024.0f, (_Float16)-1024.0f};
                    const uint32_t wa = (t & 1) ? w[ct][L].z : w[ct][L].x;
                    const uint32_t wb = (t & 1) ? w[ct][L].w : w[ct][L].y;
                    const uint32_t pr[4] = {magic_pair(wa >> sft), magic_pair(wa >> (sft + 8)),
                                            magic_pair(wb >> sft), magic_pair(wb >> (sft + 8))};
                    uint32_t o[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[i] = as_u32(__builtin_elementwise_fma(as_v2h(pr[i]), sv, ns));
                    const v8h bq = to_v8h(o[0], o[1], o[2], o[3]);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        if (rt < nrt) {
                            P[rt][ct] = mfma(xa[rt], bq, P[rt][ct]);
                            P[rt][ct] = mfma(xb[rt], bq, P[rt][ct]);
                        }
                    }
                }
            }
        }
        // mins: k = sub-block e of this super-block on the g == 0 lanes
        uint4 mh[RT], ml[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            mh[rt] = make_uint4(0u, 0u, 0u, 0u);
            ml[rt] = mh[rt];
            if (g == 0 && rt < nrt) {
                mh[rt] = *reinterpret_cast<const uint4 *>(sah[rt] + 8 * s);
                ml[rt] = *reinterpret_cast<const uint4 *>(sal[rt] + 8 * s);
            }
        }
#pragma unroll
        for (int ct = 0; ct < ORN_FCT; ++ct) {
            uint4 mb = make_uint4(0u, 0u, 0u, 0u);
            if (g == 0) {
                uint32_t mv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    uint32_t scj;
                    orn_scale_min_k4(e, hd[ct].y, hd[ct].z, hd[ct].w, scj, mv[e]);
                }
                // (1024 + m) as fp16 is 0x6400 | m; subtract 1024 (exact)
                const v2h off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
                uint32_t o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = as_u32(as_v2h(0x64006400u | mv[2 * i] | (mv[2 * i + 1] << 16)) + off);
                mb = make_uint4(o[0], o[1], o[2], o[3]);
            }
            const float d = orn_half_to_float(hd[ct].x & 0xFFFFu);
            const float dm32 = -32.0f * orn_half_to_float(hd[ct].x >> 16);  // sums stored / 32
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                if (rt < nrt) {
                    v4f Pm = {0.0f, 0.0f, 0.0f, 0.0f};
                    Pm = mfma(__builtin_bit_cast(v8h, mh[rt]), __builtin_bit_cast(v8h, mb), Pm);
                    Pm = mfma(__builtin_bit_cast(v8h, ml[rt]), __builtin_bit_cast(v8h, mb), Pm);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        acc[rt][ct][r] = fmaf(d, P[rt][ct][r], acc[rt][ct][r]);
                        acc[rt][ct][r] = fmaf(dm32, Pm[r], acc[rt][ct][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * rt + 4 * g + r;
            inv[r] = row < nrows ? xinv[src[row]] : 0.0f;
        }
        float *out = gu + ((size_t)kslice * rows_max + itm.y + 16 * rt) * (size_t)(2 * H) + col0 + c;
#pragma unroll
        for (int ct = 0; ct < ORN_FCT; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * rt + 4 * g + r;
                if (row < nrows) out[(size_t)(4 * g + r) * (2 * H) + 16 * ct] = acc[rt][ct][r] * inv[r];
            }
    }
}

// ---------------------------------------------------------------------------
// Down, Q6_K (gguf.c:64-86 value layout: within each 128-value half n, value
// 32Q + l (Q = 0..3, l < 32) takes ql[64n + 32(Q&1) + l] (low nibble for Q <
// 2, high for Q >= 2) and bits 2Q..2Q+1 of qh[32n + l], scale sc[8n + 2Q +
// l/16]).  Logical tile = (item * ks + kslice) * (D/(64*ORN_FDN)) + cb;
// wave w covers output columns cb*64*ORN_FDN + 16*ORN_FDN*w + 16ct + c (ct <
// ORN_FDN), each activation operand feeding the ORN_FDN tiles.  The store keeps each block's 208
// leading bytes and its d apart (body / dv, block order as in the file).
// Output dn[kslice][row][D].
// ---------------------------------------------------------------------------
#define ORN_FDN 2  // column tiles per wave in the down kernel

template <int RT>
__global__ void __launch_bounds__(256)
    k_dn_file(const uint8_t *__restrict__ body, const uint16_t *__restrict__ dv,
              const uint32_t *__restrict__ mh, const uint32_t *__restrict__ ml,
              const float *__restrict__ minv, const int *__restrict__ ctl,
              const int4 *__restrict__ items, float *__restrict__ dn, int D, int H, int ks,
              int rows_max)
{
    const int NCB = D / (64 * ORN_FDN);
    const int per_item = NCB * ks;
    const int n_live = ctl[1] * per_item;
    if ((int)blockIdx.x >= n_live) return;
    const int tile = xcd_remap(blockIdx.x, n_live);
    const int cb = tile % NCB;
    const int kslice = (tile / NCB) % ks;
    const int4 itm = items[tile / per_item];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
    const int n0 = cb * (64 * ORN_FDN) + 16 * ORN_FDN * wave + c;  // tile ct: column n0 + 16ct = file row
    const int NSB = H >> 8, nsb = NSB / ks, s0 = kslice * nsb;
    const size_t b0 = ((size_t)itm.w * D + n0) * NSB;  // first block of row n0
    const int nrows = itm.z;
    const int nrt = RT == 1 ? 1 : (nrows + 15) >> 4;
    constexpr int NB = RT == 1 ? 2 : 1;
    __shared__ __align__(16) FileTileT<RT> Ab[NB];  // A row = 16rt + c (mid rows)
    __shared__ int src[16 * RT];
    if (threadIdx.x < 16 * RT)
        src[threadIdx.x] = itm.y + ((int)threadIdx.x < nrows ? (int)threadIdx.x : nrows - 1);
    __syncthreads();

    v4f acc[RT][ORN_FDN];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < ORN_FDN; ++ct) acc[rt][ct] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = s0; s < s0 + nsb; ++s) {
        const uint8_t *blk[ORN_FDN];
        float d[ORN_FDN];
        uint32_t scs[ORN_FDN][4];
#pragma unroll
        for (int ct = 0; ct < ORN_FDN; ++ct) {
            const size_t bi = b0 + (size_t)(16 * ct) * NSB + s;
            blk[ct] = body + bi * 208;
            d[ct] = orn_half_to_float(dv[bi]);
            const uint4 scw = *reinterpret_cast<const uint4 *>(blk[ct] + 192);
            scs[ct][0] = scw.x;
            scs[ct][1] = scw.y;
            scs[ct][2] = scw.z;
            scs[ct][3] = scw.w;
        }
        // Lane group g takes l = 8g .. 8g+7 of every 32-value quarter: the
        // 8 bytes ql[64hn + 32(Q&1) + 8g ..] and qh[32hn + 8g ..] hold them
        // for all four Q; every word of the super-block is requested before
        // the first is used (one memory round trip per super-block).
        uint2 qa[2][2][ORN_FDN], qb[2][ORN_FDN];
#pragma unroll
        for (int hn = 0; hn < 2; ++hn)
#pragma unroll
            for (int ct = 0; ct < ORN_FDN; ++ct) {
                qa[hn][0][ct] = *reinterpret_cast<const uint2 *>(blk[ct] + 64 * hn + 8 * g);
                qa[hn][1][ct] = *reinterpret_cast<const uint2 *>(blk[ct] + 64 * hn + 32 + 8 * g);
                qb[hn][ct] = *reinterpret_cast<const uint2 *>(blk[ct] + 128 + 32 * hn + 8 * g);
            }
        FileTileT<RT> &As = Ab[NB == 2 ? (s & 1) : 0];
        stage_tile<RT, true>(As, mh, ml, src, H, s, nrows);
        v4f ps[RT][ORN_FDN];  // this super-block's sums, before d
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < ORN_FDN; ++ct) ps[rt][ct] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int hn = 0; hn < 2; ++hn) {
#pragma unroll
            for (int Q = 0; Q < 4; ++Q) {
                const int kl = 128 * hn + 32 * Q + 8 * g;  // this lane's 8 values, k - 256 s
                v8h xa[RT], xb[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    if (rt < nrt) {
                        xa[rt] = *reinterpret_cast<const v8h *>(&As.v[0][16 * rt + c][kl]);
                        xb[rt] = *reinterpret_cast<const v8h *>(&As.v[1][16 * rt + c][kl]);
                    }
                }
                const int sb = 8 * hn + 2 * Q + (g >> 1);  // the 16-value sub-block of l
#pragma unroll
                for (int ct = 0; ct < ORN_FDN; ++ct) {
                    const uint2 ql = qa[hn][Q & 1][ct], qh = qb[hn][ct];
                    // bytes q + 32 (0..63): low 4 bits from ql, high 2 from qh
                    const uint32_t w0 = ((ql.x >> (4 * (Q >> 1))) & 0x0F0F0F0Fu) |
                                        (((qh.x >> (2 * Q)) & 0x03030303u) << 4);
                    const uint32_t w1 = ((ql.y >> (4 * (Q >> 1))) & 0x0F0F0F0Fu) |
                                        (((qh.y >> (2 * Q)) & 0x03030303u) << 4);
                    // B = sc * (q - 32), |B| <= 4096, as b1 + b2 (q6_b2's
                    // remainder form) in the prep's pair order
                    const int scv = (int)(int8_t)((scs[ct][sb >> 2] >> (8 * (sb & 3))) & 0xFFu);
                    const v2h sv = {(_Float16)scv, (_Float16)scv};
                    const uint32_t p[4] = {__builtin_amdgcn_perm(0x64646464u, w0, 0x04020400u),
                                           __builtin_amdgcn_perm(0x64646464u, w0, 0x04030401u),
                                           __builtin_amdgcn_perm(0x64646464u, w1, 0x04020400u),
                                           __builtin_amdgcn_perm(0x64646464u, w1, 0x04030401u)};
                    uint32_t o1[4], o2[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const v2h qv = as_v2h(p[i]) + (v2h){(_Float16)-1056.0f, (_Float16)-1056.0f};
                        const v2h bh = qv * sv;
                        o1[i] = as_u32(bh);
                        o2[i] = as_u32(__builtin_elementwise_fma(qv, sv, -bh));
                    }
                    const v8h b1 = to_v8h(o1[0], o1[1], o1[2], o1[3]);
                    const v8h b2 = to_v8h(o2[0], o2[1], o2[2], o2[3]);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        if (rt < nrt) {
                            ps[rt][ct] = mfma(xa[rt], b1, ps[rt][ct]);
                            ps[rt][ct] = mfma(xb[rt], b1, ps[rt][ct]);
                            ps[rt][ct] = mfma(xa[rt], b2, ps[rt][ct]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < ORN_FDN; ++ct)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[rt][ct][r] = fmaf(d[ct], ps[rt][ct][r], acc[rt][ct][r]);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        float *out = dn + ((size_t)kslice * rows_max + itm.y + 16 * rt) * (size_t)D + n0;
#pragma unroll
        for (int ct = 0; ct < ORN_FDN; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * rt + 4 * g + r;
                if (row < nrows)
                    out[(size_t)(4 * g + r) * D + 16 * ct] = acc[rt][ct][r] * minv[itm.y + row];
            }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
extern "C" int ornk_file_down_cols(void) { return 64 * ORN_FDN; }

extern "C" int ornk_file_supported(int D, int H)
{
    return D % 256 == 0 && H % 256 == 0 && D <= 2048 && H <= 2048;
}

// x (or its rmsnorm) -> hi/lo + sums, one work group per token.
extern "C" int ornk_file_prep_x(const ornk_moe_args *a, hipStream_t s)
{
    if (!ornk_file_supported(a->D, a->H)) return hipErrorInvalidValue;
    const ornk_file_ws &f = a->fw;
    ORN_LAUNCH_EV(a, k_prep_rows<true>, dim3(a->T), dim3(256), 0, s, a->xn, a->D,
                  (const int *)nullptr, f.xh, f.xl, f.xinv, f.xsh, f.xsl);
    return hipGetLastError();
}

extern "C" int ornk_file_gateup(const ornk_moe_args *a, hipStream_t s)
{
    if (!ornk_file_supported(a->D, a->H) || (a->D / 256) % a->ks_gu) return hipErrorInvalidValue;
    const ornk_file_ws &f = a->fw;
    if (a->tchunk > 64) return hipErrorInvalidValue;
    const int RT = a->tchunk > 16 ? 4 : 1;
    const dim3 grid(a->items_max * ((2 * a->H) / (64 * (RT == 4 ? gu_fct<4>() : gu_fct<1>()))) *
                    a->ks_gu);
    if (RT == 4)
        ORN_LAUNCH_EV(a, k_gu_file<4>, grid, dim3(256), 0, s, a->gate, a->up, f.xh, f.xl, f.xinv,
                      f.xsh, f.xsl, a->ctl, reinterpret_cast<const int4 *>(a->items),
                      a->row_token, a->gu_part, a->D, a->H, a->ks_gu, a->rows_max);
    else
        ORN_LAUNCH_EV(a, k_gu_file<1>, grid, dim3(256), 0, s, a->gate, a->up, f.xh, f.xl, f.xinv,
                      f.xsh, f.xsl, a->ctl, reinterpret_cast<const int4 *>(a->items),
                      a->row_token, a->gu_part, a->D, a->H, a->ks_gu, a->rows_max);
    return hipGetLastError();
}

extern "C" int ornk_file_down(const ornk_moe_args *a, hipStream_t s)
{
    if (!ornk_file_supported(a->D, a->H) || (a->H / 256) % a->ks_dn) return hipErrorInvalidValue;
    const ornk_file_ws &f = a->fw;
    if (a->D % (64 * ORN_FDN)) return hipErrorInvalidValue;
    const dim3 grid(a->items_max * (a->D / (64 * ORN_FDN)) * a->ks_dn);
    if (a->tchunk > 64) return hipErrorInvalidValue;
    if (a->tchunk > 16)
        ORN_LAUNCH_EV(a, k_dn_file<4>, grid, dim3(256), 0, s, a->down_body, a->down_d, f.mh, f.ml,
                      f.minv, a->ctl, reinterpret_cast<const int4 *>(a->items), a->dn_part, a->D,
                      a->H, a->ks_dn, a->rows_max);
    else
        ORN_LAUNCH_EV(a, k_dn_file<1>, grid, dim3(256), 0, s, a->down_body, a->down_d, f.mh, f.ml,
                      f.minv, a->ctl, reinterpret_cast<const int4 *>(a->items), a->dn_part, a->D,
                      a->H, a->ks_dn, a->rows_max);
    return hipGetLastError();
}
