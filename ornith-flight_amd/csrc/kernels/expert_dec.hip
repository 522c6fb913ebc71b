// SPDX-License-Identifier: MIT
//
// Decode-shaped expert products on the matrix cores: work items of at most
// 16 token rows (one MFMA row tile) of one expert, split-K over the
// reduction dimension.  Operand preparation and its exactness argument:
// mfma_ops.h; memory layouts: prefill_pack.c.
//
// At decode sizes the weights are read once per launch and the step is
// bound by how many bytes are in flight, so each lane keeps NR reduction
// steps of weight loads in a register ring, refilled right after a step's
// registers are consumed.  The KT steps of a slice are a compile-time count
// and fully unrolled: a loop would carry the ring through the back edge as
// register copies, which wait for every load in flight.
//
// Work group: 4 waves over one 256-column block of one matrix.  Wave w owns
// column tiles 4w..4w+3 (one 16-byte weight load per lane and step for
// Q4_K, two for Q6_K).  The 16 x 32*KT activation tiles of the slice are
// prepared into LDS once (hi/lo split), so the waves never wait for each
// other after that; every step a wave runs 4 x (hi, lo) MFMAs and, for
// Q4_K, 2 more for the dmin term of its own two sub-blocks.
#include "common.h"
#include "launch.h"
#include "mfma_ops.h"


namespace {

using namespace orn_mfma;

typedef float v2f __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

#define ORN_DEC_NR 4  // reduction steps in flight per lane (scales in the ring)
// The down instances that form mid themselves (decode batches up to 64
// tokens) keep 2 steps in flight at 112 registers: four waves per SIMD (and
// four work groups per CU, 37 KB of LDS each) instead of three with 4 steps.
// Measured: 25.8 -> 23.7 us at 16 tokens, 6.9 -> 6.4 us at one token.  Their
// wide instances (real-range Q6_K scales) fit 128 registers the same way
// instead of 166: 28.2 -> 26.4 us at 16 tokens.
#define ORN_DEC_NR_MID 2
// Gate/up: 2 steps in flight and activation chunks of 2 steps.  One-tile
// instances (20 KB of LDS, 121 registers) run four waves per SIMD: 29.7 ->
// 29.1 us at 16 tokens (3 steps in flight spills; 5 waves with one step in
// flight: 45.9 us); two-tile ones (40 KB, 148 registers) three: 58.7 ->
// 52.5 us on the 256-token Zipf batch.
#define ORN_DEC_NR_GU 2

// Two-tile down instances keep the slice's scales in LDS and their ring holds
// only quant words: every step of a slice up to 16 in flight, 8 of the
// 32-step slices (whose scales take 32 more registers until stored).
constexpr int dec_nr_lds(int kt) { return kt <= 16 ? kt : 8; }

// Ring loads are raw buffer loads: a per-lane byte offset that stays fixed
// (one VGPR) plus the step's wave-uniform offset in an SGPR, so NR steps in
// flight cost no address registers.  0x00020000: 32-bit data format, the
// plain untyped-buffer setting.
__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ __forceinline__ uint4 bload16(rsrc_t r, uint32_t voff, uint32_t soff)
{
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 bload8(rsrc_t r, uint32_t voff, uint32_t soff)
{
    const v2u v = __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
    return make_uint2(v.x, v.y);
}


// ---------------------------------------------------------------------------
// Gate/up (Q4_K).  Logical tile = ((item * ks + kslice) * 2 + m) * (H/256) + b;
// output gu[kslice][row][m*H + n], the split-K partial over the reduction
// steps kslice*KT .. +KT-1.
//
// The slice's activation tiles (all KT steps) are prepared once into LDS:
// thread t prepares row t/16, a run of 2*KT consecutive reduction values
// (hi/lo of x*s*d and of x*s*dmin); after one barrier every wave streams its
// own weights with no further synchronisation.
// ---------------------------------------------------------------------------
// N = 4: one 16-byte LDS store of w[0..3]; N = 2: one 8-byte store of w[0..1]
template <int N>
__device__ __forceinline__ void st_words(uint32_t *p, const uint32_t *w)
{
    if constexpr (N == 4)
        *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    else
        *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
}

struct GuRing {
    uint4 q;       // nibble words of column tiles 4w..4w+3
    uint4 s0, s1;  // scales of sub-blocks 2w, 2w+1 at k = 8g..8g+7
    uint4 mn;      // mins of sub-block 2w + (c & 1) at k = 8g..8g+7
};

// LDS of one gate/up tile: activation tiles (hi/lo of A and Am) per chunk.
template <int KT, int KC, int RT>
struct GuLds {
    uint32_t As[KT / KC > 1 ? 2 : 1][KC][RT][4][16 * ORN_AST / 2];
    float s_inv[16 * RT];
};

// One gate/up tile (work group); returns false for a tile past the
// dispatched items.
template <int NR, int KT, int KC, int RT>
__device__ __forceinline__ bool gateup_dec_tile(GuLds<KT, KC, RT> &L, const ornk_gu_prefill &P,
                                                const float *__restrict__ xn,
                                                const float *__restrict__ x_amax, int n_items,
                                                const int4 *__restrict__ items,
                                                const int *__restrict__ row_token,
                                                float *__restrict__ gu, int D, int H, int ks,
                                                int rows_max, int tile)
{
    constexpr int NCHK = KT / KC, NBUF = NCHK > 1 ? 2 : 1;
    constexpr int LC = 2 * KC;  // activation values a thread prepares per chunk
    constexpr int GV = LC < 8 ? LC : 8;  // values per LDS store (8: 16 bytes, 4: 8 bytes)
    static_assert(LC % GV == 0 && (GV == 4 || GV == 8), "chunks of 2 or 4k steps");
    auto &As = L.As;
    auto &s_inv = L.s_inv;

    // The item and the live item count are read together; work groups past
    // the dispatched items then leave.
    const int NB = H >> 8;
    const int per_item = 2 * NB * ks;
    const int b = tile % NB;
    const int m = (tile / NB) & 1;
    const int kslice = (tile / (2 * NB)) % ks;
    const int item = tile / per_item;
    const int tid = threadIdx.x;
    if (item >= n_items) return false;
    const int4 itm = items[item];
    const int e = itm.w;
    const int nrows = itm.z;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int kt0 = kslice * KT;
    const size_t DH = (size_t)D * H;

    const uint32_t EQ = (uint32_t)(DH / 2), ES = (uint32_t)(DH / 16);
    const rsrc_t rq = make_rsrc(reinterpret_cast<const uint8_t *>(P.pq[m]) + (size_t)e * EQ, EQ);
    const rsrc_t rs = make_rsrc(reinterpret_cast<const uint8_t *>(P.psc[m]) + (size_t)e * ES, ES);
    const rsrc_t rm = make_rsrc(reinterpret_cast<const uint8_t *>(P.pmn[m]) + (size_t)e * ES, ES);
    const uint32_t qstep = (uint32_t)NB * 4096, sstep = (uint32_t)NB * 512;
    const uint32_t q_off = (uint32_t)(((size_t)kt0 * NB + b) * 4096) + (wave * 64 + lane) * 16;
    const uint32_t s_off = (uint32_t)((((size_t)kt0 * NB + b) * 8 + 2 * wave) * 64) + 16 * g;
    const uint32_t m_off = s_off + 64 * (c & 1);
    auto load_b = [&](GuRing &st, int kt) {
        st.q = bload16(rq, q_off, kt * qstep);
        st.s0 = bload16(rs, s_off, kt * sstep);
        st.s1 = bload16(rs, s_off + 64, kt * sstep);
        st.mn = bload16(rm, m_off, kt * sstep);
    };

    // Row tile rt holds the item's rows 16*rt .. 16*rt+15; thread (ar, seg)
    // prepares row ar of every tile.
    const int ar = tid >> 4, seg = tid & 15;
    int tok[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int row = 16 * rt + ar;
        tok[rt] = row_token[itm.y + (row < nrows ? row : 0)];  // rows past the item: a valid row, scaled by 0
    }
    GuRing st[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) load_b(st[i], i);
    __builtin_amdgcn_sched_barrier(0);

    // Activation tiles: A = x*s*d and Am = x*s*dmin, hi/lo, one chunk of KC
    // steps at a time (chunk ch in LDS buffer ch % 2).  Thread (ar, seg)
    // owns the LC values seg*LC.. of row ar in every chunk.
    const float dmx = P.dmax[e * 3 + m];
    const float *xr[RT];
    float amax[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        amax[rt] = x_amax[tok[rt]];
        xr[rt] = xn + (size_t)tok[rt] * D + 32 * kt0 + seg * LC;
    }
    const float *dr = P.pd[m] + (size_t)e * (DH / 256) + (size_t)b * D + 32 * kt0 + seg * LC;
    const float *dmr = P.pdm[m] + (size_t)e * (DH / 256) + (size_t)b * D + 32 * kt0 + seg * LC;
    // Wave w prepares rows 4w..4w+3 of each row tile.  A wave whose rows of
    // a tile all lie past the item (most waves at decode sizes, where items
    // hold one or a few rows) zeroes them in both buffers once and then
    // skips their loads and arithmetic (uniform per wave).  The d / dmin
    // values are the column block's, the same for every row.
    bool rows_live[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        rows_live[rt] = __builtin_amdgcn_readfirstlane(16 * rt + 4 * (tid >> 6)) < nrows;
    v4f xv[RT][LC / 4], dv[LC / 4], mv[LC / 4];
    auto a_load = [&](int ch) {
        if (!rows_live[0]) return;
#pragma unroll
        for (int i = 0; i < LC / 4; ++i) {
            dv[i] = *reinterpret_cast<const v4f *>(dr + 32 * KC * ch + 4 * i);
            mv[i] = *reinterpret_cast<const v4f *>(dmr + 32 * KC * ch + 4 * i);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            if (rows_live[rt])
#pragma unroll
                for (int i = 0; i < LC / 4; ++i)
                    xv[rt][i] = *reinterpret_cast<const v4f *>(xr[rt] + 32 * KC * ch + 4 * i);
    };
    float ascale[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        ascale[rt] = 0.0f;
        if (!rows_live[rt]) {
            const uint32_t z[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int buf = 0; buf < NBUF; ++buf)
#pragma unroll
                for (int o = 0; o < LC / GV; ++o) {
                    const int kk = seg * LC + GV * o, kl = kk >> 5, ko = kk & 31;
                    const int w0 = (ar * ORN_AST + ko) >> 1;
#pragma unroll
                    for (int a = 0; a < 4; ++a) st_words<GV / 2>(&As[buf][kl][rt][a][w0], z);
                }
        }
    }
    auto a_store = [&](int ch) {
        const int buf = ch % NBUF;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if (!rows_live[rt]) continue;
#pragma unroll
            for (int o = 0; o < LC / GV; ++o) {  // groups of GV values: one LDS store per array
                const int kk = seg * LC + GV * o;  // within the chunk
                const int kl = kk >> 5, ko = kk & 31;
                uint32_t hi[GV / 2], lo[GV / 2], mh[GV / 2], ml[GV / 2];
#pragma unroll
                for (int j = 0; j < GV / 2; ++j) {
                    const int v = GV * o + 2 * j;  // the pair's first value in the thread's run
                    const v4f x4 = xv[rt][v >> 2], d4 = dv[v >> 2], m4 = mv[v >> 2];
                    const int u = v & 3;
                    const float x0 = x4[u] * ascale[rt], x1 = x4[u + 1] * ascale[rt];
                    split2(x0 * d4[u], x1 * d4[u + 1], hi[j], lo[j]);
                    split2(x0 * m4[u], x1 * m4[u + 1], mh[j], ml[j]);
                }
                const int w0 = (ar * ORN_AST + ko) >> 1;
                st_words<GV / 2>(&As[buf][kl][rt][0][w0], hi);
                st_words<GV / 2>(&As[buf][kl][rt][1][w0], lo);
                st_words<GV / 2>(&As[buf][kl][rt][2][w0], mh);
                st_words<GV / 2>(&As[buf][kl][rt][3][w0], ml);
            }
        }
    };
    a_load(0);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        ascale[rt] = 16 * rt + ar < nrows ? row_scale(amax[rt], dmx) : 0.0f;
        if (seg == 0) s_inv[16 * rt + ar] = ascale[rt] != 0.0f ? 1.0f / ascale[rt] : 0.0f;
    }
    a_store(0);
    if (NCHK > 1) a_load(1);
    __syncthreads();

    // the second row tile's products only where the item reaches it
    // (uniform over the work group)
    const int rt_live = RT > 1 && nrows > 16 ? RT : 1;
    v4f acc[RT][4], accm[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rt][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
        accm[rt] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    }
    const int ro = c * ORN_AST + 8 * g;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int ch = kt / KC, kl = kt % KC;
        GuRing &r = st[kt % NR];
        v8h bq[4];
        bq[0] = q4_b(r.q.x, r.s0);
        bq[1] = q4_b(r.q.y, r.s0);
        bq[2] = q4_b(r.q.z, r.s1);
        bq[3] = q4_b(r.q.w, r.s1);
        const uint4 mz = c < 2 ? r.mn : make_uint4(0u, 0u, 0u, 0u);
        const v8h bm = __builtin_bit_cast(v8h, mz);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + NR < KT) load_b(r, kt + NR);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if (rt >= rt_live) break;
            const _Float16 *A = reinterpret_cast<const _Float16 *>(As[ch % NBUF][kl][rt][0]);
            const v8h ahi = *reinterpret_cast<const v8h *>(A + ro);
            const v8h alo = *reinterpret_cast<const v8h *>(A + 16 * ORN_AST + ro);
            const v8h mhi = *reinterpret_cast<const v8h *>(A + 32 * ORN_AST + ro);
            const v8h mlo = *reinterpret_cast<const v8h *>(A + 48 * ORN_AST + ro);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[rt][j] = mfma(ahi, bq[j], acc[rt][j]);
                acc[rt][j] = mfma(alo, bq[j], acc[rt][j]);
            }
            accm[rt] = mfma(mhi, bm, accm[rt]);
            accm[rt] = mfma(mlo, bm, accm[rt]);
        }
        if (kl == 0 && ch + 1 < NCHK) {
            // Next chunk's tiles into the other buffer (last read in chunk
            // ch-1, which every wave finished before the barrier below it),
            // then the loads for the chunk after it.
            a_store(ch + 1);
            if (ch + 2 < NCHK) a_load(ch + 2);
        }
        if (kl == KC - 1 && ch + 1 < NCHK) __syncthreads();
    }

    float *row0 = gu + ((size_t)kslice * rows_max + itm.y) * (2 * H);
    const int colb = m * H + 256 * b + 64 * wave + c;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int row = 16 * rt + 4 * g + rr;
            const float si = s_inv[row];
            const float m0 = __shfl(accm[rt][rr], 16 * g, 64);
            const float m1 = __shfl(accm[rt][rr], 16 * g + 1, 64);
            if (row < nrows) {
                float *o = row0 + (size_t)row * (2 * H) + colb;
                o[0] = (acc[rt][0][rr] - m0) * si;
                o[16] = (acc[rt][1][rr] - m0) * si;
                o[32] = (acc[rt][2][rr] - m1) * si;
                o[48] = (acc[rt][3][rr] - m1) * si;
            }
        }
    return true;
}

template <int NR, int KT, int KC, int RT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RT > 1 ? 3 : 4)))
    k_gateup_dec(ornk_gu_prefill P, const float *__restrict__ xn,
                 const float *__restrict__ x_amax, const int *__restrict__ ctl,
                 const int4 *__restrict__ items, const int *__restrict__ row_token,
                 float *__restrict__ gu, int T, int D, int H, int ks, int rows_max)
{
    __shared__ __align__(16) GuLds<KT, KC, RT> L;
    gateup_dec_tile<NR, KT, KC, RT>(L, P, xn, x_amax, ctl[1], items, row_token, gu, D, H,
                                           ks, rows_max, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Down (Q6_K).  Logical tile = (item * ks + kslice) * (D/256) + b; output
// dn[kslice][row][n].  Same structure (activation = mid row, hi/lo of
// mid*s*d).
//
// KSG > 0: the work group forms its rows' slice of mid itself from the KSG
// gate/up split-K partials, with the mid step's arithmetic (fixed-order sum
// from 0, clamped SiLU for routed rows, model.c:1087-1088, plain for the
// shared expert's, gpu.c:176-186), and scales each row's activation tile by
// that row's max |mid| over the slice (a power of two either way: only the
// hi/lo split point moves); the separate mid launch is skipped.
// ---------------------------------------------------------------------------
// One step of a lane's weights: the 6-bit values of its four column tiles
// (a word of low nibbles per tile, the high bits of tiles 2i and 2i+1 in one
// word; prefill_pack.c) and, unless they sit in LDS, their sub-block scales.
struct DnRing {
    uint4 qn, sc[4];
    uint2 qc;
};

// WIDE: Q6_K sub-scales up to |128| (q6_b2: three MFMAs per tile and step).
// LDS of one down tile.  SL: the slice's scales in LDS (two-tile instances,
// whose many rows per item make them bandwidth-bound: the deeper ring
// pays); one-tile instances carry them in the ring.
template <int KT, int KC, int KSG, int RT>
struct DnLds {
    static constexpr bool SL = RT > 1;
    uint32_t As[KT / KC > 1 ? 2 : 1][KC][RT][2][16 * ORN_AST / 2];
    uint4 Ss[SL ? KT : 1][64];  // per step: 16 tiles x 32 scales
    float s_inv[16 * RT];
    float Ms[KSG ? 16 : 1][KSG ? 32 * KT : 4];  // the rows' mid slices
    unsigned int s_amax[16];
};

// One down tile (logical tile number `tile`, after any XCD remapping).
template <int NR, int KT, int KC, int KSG, int RT, bool WIDE>
__device__ __forceinline__ void down_dec_tile(DnLds<KT, KC, KSG, RT> &L, const ornk_dn_prefill &P,
                                              const float *__restrict__ mid,
                                              const float *__restrict__ mid_amax,
                                              const int4 *__restrict__ items,
                                              float *__restrict__ dn, int D, int H, int ks,
                                              int rows_max, const float *__restrict__ gu,
                                              int shared_rows, int tile)
{
    constexpr int NCHK = KT / KC, NBUF = NCHK > 1 ? 2 : 1;
    constexpr int LC = 2 * KC;
    constexpr int KV = 32 * KT;  // reduction values of the slice
    static_assert(LC % 8 == 0 && KT % KC == 0, "a thread stores whole 8-value groups of a chunk");
    static_assert(KSG == 0 || RT == 1, "mid is formed in the kernel for one row tile only");
    static_assert(KSG == 0 || 32 * KT == 256, "mid is formed one value per thread");
    static_assert(KT % 4 == 0 && NR >= 1 && NR <= KT, "slices of 4k steps");
    constexpr bool SL = RT > 1;
    auto &As = L.As;
    auto &Ss = L.Ss;
    auto &s_inv = L.s_inv;
    auto &Ms = L.Ms;
    auto &s_amax = L.s_amax;

    const int NBD = D >> 8;
    const int per_item = NBD * ks;
    const int b = tile % NBD;
    const int kslice = (tile / NBD) % ks;
    const int item = tile / per_item;
    const int4 itm = items[item];
    const int e = itm.w;
    const int nrows = itm.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int kt0 = kslice * KT;
    const size_t DH = (size_t)D * H;

    const uint32_t EQ = (uint32_t)ORNK_DQ_BYTES(DH), ES = (uint32_t)(DH / 8);
    const rsrc_t rq = make_rsrc(P.dq + (size_t)e * EQ, EQ);
    const rsrc_t rs = make_rsrc(reinterpret_cast<const uint8_t *>(P.dsc) + (size_t)e * ES, ES);
    const uint32_t qstep = (uint32_t)NBD * ORNK_DQ_UNIT, sstep = (uint32_t)NBD * 1024;
    const uint32_t s_off = (uint32_t)((((size_t)kt0 * NBD + b) * 16 + 4 * wave) * 64) + 16 * g;
    const uint32_t q_off = (uint32_t)(((size_t)kt0 * NBD + b) * ORNK_DQ_UNIT) + (wave * 64 + lane) * 16;
    const uint32_t c_off = (uint32_t)(((size_t)kt0 * NBD + b) * ORNK_DQ_UNIT) + 4096 + (wave * 64 + lane) * 8;
    auto load_b = [&](DnRing &st, int kt) {
        st.qn = bload16(rq, q_off, kt * qstep);
        st.qc = bload8(rq, c_off, kt * qstep);
        if constexpr (!SL) {
#pragma unroll
            for (int j = 0; j < 4; ++j) st.sc[j] = bload16(rs, s_off + 64 * j, kt * sstep);
        }
    };

    const int ar = tid >> 4, seg = tid & 15;  // row ar of each row tile, as in k_gateup_dec
    int arow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) arow[rt] = 16 * rt + ar < nrows ? 16 * rt + ar : 0;
    // the slice's scales: KT x 64 16-byte pieces, KT/4 per thread, issued
    // before the ring so that their wait leaves the ring in flight
    uint4 sreg[SL ? KT / 4 : 1];
    if constexpr (SL) {
#pragma unroll
        for (int i = 0; i < KT / 4; ++i) {
            const int idx = 256 * i + tid;
            sreg[i] = bload16(rs, (uint32_t)(((size_t)(kt0 + (idx >> 6)) * NBD + b) * 1024) + 16 * (idx & 63), 0);
        }
    }
    DnRing st[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) load_b(st[i], i);
    __builtin_amdgcn_sched_barrier(0);

    float amax[RT];
    if (KSG) {
        // Thread t forms value h = t of each row (KV == 256 == threads).  The
        // partials of MG rows (MG * KSG = 16 per array) are loaded together,
        // so an item of 16 rows waits for 16 / MG memory latencies, not 16.
        constexpr int NS = KSG > 0 ? KSG : 1, MG = NS >= 16 ? 1 : 16 / NS;
        const size_t sstr = (size_t)rows_max * 2 * H;  // between gate/up slices
        if (tid < 16) s_amax[tid] = 0u;
        __syncthreads();
        for (int r0 = 0; r0 < nrows; r0 += MG) {  // uniform
            float gv[MG][NS], uv[MG][NS];
#pragma unroll
            for (int i = 0; i < MG; ++i) {
                if (r0 + i >= nrows) break;  // uniform
                const float *pg = gu + (size_t)(itm.y + r0 + i) * 2 * H + 32 * kt0 + tid;
#pragma unroll
                for (int sl = 0; sl < NS; ++sl) {
                    gv[i][sl] = pg[sl * sstr];
                    uv[i][sl] = pg[sl * sstr + H];
                }
            }
#pragma unroll
            for (int i = 0; i < MG; ++i) {
                const int r = r0 + i;
                if (r >= nrows) break;  // uniform
                float g = 0.0f, u = 0.0f;
#pragma unroll
                for (int sl = 0; sl < NS; ++sl) {
                    g = g + gv[i][sl];
                    u = u + uv[i][sl];
                }
                float act;
                if (itm.y + r < shared_rows) {
                    act = g / (1.0f + expf(-g));
                } else {
                    if (g < -50.0f) act = 0.0f;
                    else if (g > 50.0f) act = g;
                    else act = g / (1.0f + expf(-g));
                }
                const float v = act * u;
                Ms[r][tid] = v;
                float lmax = fabsf(v);
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, off, 64));
                // non-negative floats order like their bit patterns
                if (lane == 0) atomicMax(&s_amax[r], __float_as_uint(lmax));
            }
        }
        __syncthreads();
        amax[0] = __uint_as_float(s_amax[arow[0]]);
    } else {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) amax[rt] = mid_amax[itm.y + arow[rt]];
    }
    const float dmx = P.dmax[e * 3 + 2];
    const float *xr[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) xr[rt] = mid + (size_t)(itm.y + arow[rt]) * H + 32 * kt0 + seg * LC;
    const float *dr = P.dd + (size_t)e * (DH / 256) + (size_t)b * H + 32 * kt0 + seg * LC;
    // Waves whose rows of a tile all lie past the item zero them once and
    // skip their loads and arithmetic, as in the gate/up kernel.
    bool rows_live[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        rows_live[rt] = __builtin_amdgcn_readfirstlane(16 * rt + 4 * (tid >> 6)) < nrows;
    v4f xv[RT][LC / 4], dv[LC / 4];
    auto a_load = [&](int ch) {
        if (!rows_live[0]) return;
#pragma unroll
        for (int i = 0; i < LC / 4; ++i) dv[i] = *reinterpret_cast<const v4f *>(dr + 32 * KC * ch + 4 * i);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            if (rows_live[rt])
#pragma unroll
                for (int i = 0; i < LC / 4; ++i)
                    xv[rt][i] = KSG ? *reinterpret_cast<const v4f *>(
                                          &Ms[KSG ? arow[0] : 0][32 * KC * ch + seg * LC + 4 * i])
                                    : *reinterpret_cast<const v4f *>(xr[rt] + 32 * KC * ch + 4 * i);
    };
    float ascale[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        ascale[rt] = 0.0f;
        if (!rows_live[rt]) {
#pragma unroll
            for (int buf = 0; buf < NBUF; ++buf)
#pragma unroll
                for (int o = 0; o < LC / 8; ++o) {
                    const int kk = seg * LC + 8 * o, kl = kk >> 5, ko = kk & 31;
                    const int w0 = (ar * ORN_AST + ko) >> 1;
                    *reinterpret_cast<uint4 *>(&As[buf][kl][rt][0][w0]) = make_uint4(0u, 0u, 0u, 0u);
                    *reinterpret_cast<uint4 *>(&As[buf][kl][rt][1][w0]) = make_uint4(0u, 0u, 0u, 0u);
                }
        }
    }
    auto a_store = [&](int ch) {
        const int buf = ch % NBUF;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if (!rows_live[rt]) continue;
#pragma unroll
            for (int o = 0; o < LC / 8; ++o) {
                const int kk = seg * LC + 8 * o;
                const int kl = kk >> 5, ko = kk & 31;
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4f x4 = xv[rt][2 * o + (j >> 1)], d4 = dv[2 * o + (j >> 1)];
                    const int u = 2 * (j & 1);
                    split2(x4[u] * ascale[rt] * d4[u], x4[u + 1] * ascale[rt] * d4[u + 1], hi[j], lo[j]);
                }
                const int w0 = (ar * ORN_AST + ko) >> 1;
                *reinterpret_cast<uint4 *>(&As[buf][kl][rt][0][w0]) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                *reinterpret_cast<uint4 *>(&As[buf][kl][rt][1][w0]) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            }
        }
    };
    a_load(0);
    if constexpr (SL) {
#pragma unroll
        for (int i = 0; i < KT / 4; ++i) {
            const int idx = 256 * i + tid;
            Ss[idx >> 6][idx & 63] = sreg[i];
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        ascale[rt] = 16 * rt + ar < nrows ? row_scale(amax[rt], dmx) : 0.0f;
        if (seg == 0) s_inv[16 * rt + ar] = ascale[rt] != 0.0f ? 1.0f / ascale[rt] : 0.0f;
    }
    a_store(0);
    if (NCHK > 1) a_load(1);
    __syncthreads();

    const int rt_live = RT > 1 && nrows > 16 ? RT : 1;  // uniform, as in k_gateup_dec
    v4f acc[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rt][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    const int ro = c * ORN_AST + 8 * g;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int ch = kt / KC, kl = kt % KC;
        DnRing &r = st[kt % NR];
        v8h bq[4], bq2[WIDE ? 4 : 1];
        {
            const uint32_t nw[4] = {r.qn.x, r.qn.y, r.qn.z, r.qn.w};
            const uint32_t cw[4] = {r.qc.x, r.qc.x >> 8, r.qc.y, r.qc.y >> 8};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t p[4];
                q6_pairs(nw[j], cw[j], p);
                // tile 4w+j, k = 8g..8g+7
                const uint4 sc = SL ? Ss[SL ? kt : 0][4 * (4 * wave + j) + g] : r.sc[j];
                if (WIDE) q6_b2(p, sc, bq[j], bq2[WIDE ? j : 0]);
                else bq[j] = q6_b(p, sc);
            }
        }
        if (kt + NR < KT) {
            __builtin_amdgcn_sched_barrier(0);
            load_b(r, kt + NR);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if (rt >= rt_live) break;
            const _Float16 *A = reinterpret_cast<const _Float16 *>(As[ch % NBUF][kl][rt][0]);
            const v8h ahi = *reinterpret_cast<const v8h *>(A + ro);
            const v8h alo = *reinterpret_cast<const v8h *>(A + 16 * ORN_AST + ro);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[rt][j] = mfma(ahi, bq[j], acc[rt][j]);
                acc[rt][j] = mfma(alo, bq[j], acc[rt][j]);
                if (WIDE) acc[rt][j] = mfma(ahi, bq2[WIDE ? j : 0], acc[rt][j]);
            }
        }
        if (kl == 0 && ch + 1 < NCHK) {
            a_store(ch + 1);
            if (ch + 2 < NCHK) a_load(ch + 2);
        }
        if (kl == KC - 1 && ch + 1 < NCHK) __syncthreads();
    }

    float *row0 = dn + ((size_t)kslice * rows_max + itm.y) * D;
    const int colb = 256 * b + 64 * wave + c;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int row = 16 * rt + 4 * g + rr;
            const float si = s_inv[row];
            if (row < nrows) {
                float *o = row0 + (size_t)row * D + colb;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[16 * j] = acc[rt][j][rr] * si;
            }
        }
}

template <int NR, int KT, int KC, int KSG, int RT, bool WIDE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RT > 1 ? 2 : KSG ? (WIDE ? 3 : 4) : WIDE ? 2 : 3)))
    k_down_dec(ornk_dn_prefill P, const float *__restrict__ mid,
               const float *__restrict__ mid_amax, const int *__restrict__ ctl,
               const int4 *__restrict__ items, float *__restrict__ dn, int D, int H, int ks,
               int rows_max, const float *__restrict__ gu, int shared_rows)
{
    __shared__ __align__(16) DnLds<KT, KC, KSG, RT> L;
    // The D/256 work groups of one (item, slice) read the same gate/up
    // partials (KSG > 0) or mid rows: XCD-aware numbering puts them on one
    // XCD, so one L2 serves the rest.
    const int n_live = ctl[1] * (D >> 8) * ks;
    if ((int)blockIdx.x >= n_live) return;
    down_dec_tile<NR, KT, KC, KSG, RT, WIDE>(L, P, mid, mid_amax, items, dn, D, H, ks,
                                                    rows_max, gu, shared_rows,
                                                    xcd_remap(blockIdx.x, n_live));
}


}  // namespace

// Decode instances: work items of <= 16 rows (one row tile), or <= 32 (two,
// for batches above 64 tokens whose hot experts span several items); KT =
// D/32/ks (gate/up) or H/32/ks (down) reduction steps per slice, 4 to 32;
// activation tiles double-buffered in chunks of 2 steps for gate/up (LDS:
// 2 x 10 KB per row tile) and of 4 for down (2 x 10 KB).  Two-tile down
// instances also hold the slice's scales (1 KB per step, at most 32 KB), so
// that every instance keeps at most 73 KB (two work groups per CU, the
// occupancy their registers allow); one-tile instances keep at most 37 KB
// (four work groups per CU, four waves per SIMD where their registers
// allow).  Two-tile gate/up: 40 KB, three work groups and waves per SIMD.
extern "C" int ornk_dec_supported(int kt_gu, int kt_dn)
{
    auto ok = [](int kt) { return kt == 4 || kt == 8 || kt == 16 || kt == 32; };
    return ok(kt_gu) && ok(kt_dn);
}

extern "C" int ornk_moe_gateup_dec(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_gu;
    if (a->D % 32 || a->H % 256 || ks < 1 || (a->D / 32) % ks || a->tchunk > 32)
        return hipErrorInvalidValue;
    const int KT = a->D / 32 / ks;
    if (!ornk_dec_supported(KT, 4)) return hipErrorInvalidValue;
    const int RT = a->tchunk > 16 ? 2 : 1;
    const float *xin = a->apply_norm ? a->xn : a->x;
    hipEvent_t st = a->ev_start;  // the step's first kernel carries the start event
    if (!a->router_amax) {
        const int e = ornk_rowmax(xin, a->T, a->D, a->x_amax, st, s);
        if (e != hipSuccess) return e;
        st = nullptr;
    }
    const dim3 grid(a->items_max * 2 * (a->H / 256) * ks);
#define ORN_GU_DEC(K, R)                                                                       \
    ORN_LAUNCH_EV2(st, a->ev_stop, (k_gateup_dec<ORN_DEC_NR_GU, K, 2, R>), grid, dim3(256), 0, s, \
                   a->gu_pf, xin, a->x_amax, a->ctl, reinterpret_cast<const int4 *>(a->items), \
                   a->row_token, a->gu_part, a->T, a->D, a->H, ks, a->rows_max)
#define ORN_GU_DEC_RT(R)                \
    switch (KT) {                       \
    case 4: ORN_GU_DEC(4, R); break;    \
    case 8: ORN_GU_DEC(8, R); break;    \
    case 16: ORN_GU_DEC(16, R); break;  \
    default: ORN_GU_DEC(32, R); break;  \
    }
    if (RT == 2) {
        ORN_GU_DEC_RT(2)
    } else {
        ORN_GU_DEC_RT(1)
    }
#undef ORN_GU_DEC_RT
#undef ORN_GU_DEC
    return hipGetLastError();
}

// Decode plans of up to 64 tokens with 4, 8 or 16 gate/up slices and 8-step
// down slices: the down kernel forms mid itself (the instances compiled for
// those plans).  Larger batches, whose mid rows every column block of an
// item would form again, run the mid step.
extern "C" int ornk_down_dec_fuses_mid(int T, int H, int ks_gu, int ks_dn)
{
    return T >= 1 && T <= 64 && (ks_gu == 4 || ks_gu == 8 || ks_gu == 16) && ks_dn >= 1 &&
           H % (32 * ks_dn) == 0 && H / 32 / ks_dn == 8;
}

extern "C" int ornk_moe_down_dec(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_dn;
    if (a->H % 32 || a->D % 256 || ks < 1 || (a->H / 32) % ks || a->tchunk > 32)
        return hipErrorInvalidValue;
    const int KT = a->H / 32 / ks;
    if (!ornk_dec_supported(4, KT)) return hipErrorInvalidValue;
    const int RT = a->tchunk > 16 ? 2 : 1;
    const dim3 grid(a->items_max * (a->D / 256) * ks);
    const int shared_rows = a->has_shared ? a->T : 0;
    const bool wide = a->q6_wide != 0;
    if (RT == 1 && ornk_down_dec_fuses_mid(a->T, a->H, a->ks_gu, ks)) {
#define ORN_DN_MID(KSG, W)                                                                      \
    ORN_LAUNCH_EV(a, (k_down_dec<ORN_DEC_NR_MID, 8, 4, KSG, 1, W>), grid, dim3(256), 0, s, a->dn_pf, \
                  a->mid, a->mid_amax, a->ctl, reinterpret_cast<const int4 *>(a->items),         \
                  a->dn_part, a->D, a->H, ks, a->rows_max, a->gu_part, shared_rows)
#define ORN_DN_MID_W(KSG)         \
    if (wide) ORN_DN_MID(KSG, true); \
    else ORN_DN_MID(KSG, false)
        switch (a->ks_gu) {
        case 4: ORN_DN_MID_W(4); break;
        case 8: ORN_DN_MID_W(8); break;
        default: ORN_DN_MID_W(16); break;
        }
#undef ORN_DN_MID_W
#undef ORN_DN_MID
        return hipGetLastError();
    }
#define ORN_DN_DEC(K, R, W)                                                                       \
    ORN_LAUNCH_EV(a, (k_down_dec<R == 2 ? dec_nr_lds(K) : ORN_DEC_NR, K, 4, 0, R, W>), grid,        \
                  dim3(256), 0, s, a->dn_pf,                                                      \
                  a->mid, a->mid_amax, a->ctl, reinterpret_cast<const int4 *>(a->items),         \
                  a->dn_part, a->D, a->H, ks, a->rows_max, a->gu_part, shared_rows)
#define ORN_DN_DEC_RT(R, W)                \
    switch (KT) {                          \
    case 4: ORN_DN_DEC(4, R, W); break;    \
    case 8: ORN_DN_DEC(8, R, W); break;    \
    case 16: ORN_DN_DEC(16, R, W); break;  \
    default: ORN_DN_DEC(32, R, W); break;  \
    }
    if (RT == 2) {
        if (wide) {
            ORN_DN_DEC_RT(2, true)
        } else {
            ORN_DN_DEC_RT(2, false)
        }
    } else {
        if (wide) {
            ORN_DN_DEC_RT(1, true)
        } else {
            ORN_DN_DEC_RT(1, false)
        }
    }
#undef ORN_DN_DEC_RT
#undef ORN_DN_DEC
    return hipGetLastError();
}

