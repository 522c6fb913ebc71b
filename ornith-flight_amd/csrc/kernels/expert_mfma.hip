// SPDX-License-Identifier: MIT
//
// Prefill-shaped expert products on the matrix cores: grouped GEMMs over the
// dispatch's per-expert row groups with v_mfma_f32_16x16x32_f16 (operand
// preparation and its exactness argument: mfma_ops.h).
//
// Work group: 4 waves, up to 64 token rows x 256 outputs (one block column of
// one matrix), reduction in steps of 32.  Per step every thread prepares 8
// activation values of one row into LDS (double buffered); wave w builds the
// B operands of output tiles 4w..4w+3 in registers from the prefill layout
// (prefill_pack.c) and runs (live row tiles) x 4 x (hi, lo) MFMAs, plus
// (Q4_K) one 16-column tile holding the 8 sub-block mins for the dmin term of
// row tile w.  Each converted B operand feeds up to 8 MFMAs.
#include "common.h"
#include "launch.h"
#include "mfma_ops.h"


namespace {

using namespace orn_mfma;

#define ORN_MT 64   // token rows per work group (4 row tiles)
#define ORN_GU_KT_MAX 64  // reduction steps per gate/up slice (D <= 2048 at ks = 1)

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Weight streams are raw buffer loads: a fixed per-lane VGPR offset plus the
// step's wave-uniform offset in an SGPR (0x00020000: 32-bit data format).
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

// Empty asm that reads and writes a ring slot: the wait for the slot's loads
// lands here and no use of the slot moves above it.
__device__ __forceinline__ void pin4(uint4 &a) { asm volatile("" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w)); }
__device__ __forceinline__ void pinf(v4f &a) { asm volatile("" : "+v"(a)); }

// Activation tile rows: thread t prepares row t/4, reduction values
// 8*(t%4) .. +7 of the current step, for one or two scale vectors.  Rows
// past the item's end read a valid row and are zeroed by a zero row scale.
struct ARaw {
    v4f x0, x1, d0, d1, m0, m1;
};

template <bool MINS>
__device__ __forceinline__ void a_load(ARaw &r, const float *xrow, const float *dv,
                                       const float *dmv, int k)
{
    r.x0 = *reinterpret_cast<const v4f *>(xrow + k);
    r.x1 = *reinterpret_cast<const v4f *>(xrow + k + 4);
    r.d0 = *reinterpret_cast<const v4f *>(dv + k);
    r.d1 = *reinterpret_cast<const v4f *>(dv + k + 4);
    if (MINS) {
        r.m0 = *reinterpret_cast<const v4f *>(dmv + k);
        r.m1 = *reinterpret_cast<const v4f *>(dmv + k + 4);
    }
}

// Writes hi/lo of x*s*d (and of x*s*dmin) as 16 bytes each into t0, t1 (t2, t3).
template <bool MINS>
__device__ __forceinline__ void a_store(const ARaw &r, float s, _Float16 *t0, _Float16 *t1,
                                        _Float16 *t2, _Float16 *t3)
{
    const float x[8] = {r.x0.x * s, r.x0.y * s, r.x0.z * s, r.x0.w * s,
                        r.x1.x * s, r.x1.y * s, r.x1.z * s, r.x1.w * s};
    const float d[8] = {r.d0.x, r.d0.y, r.d0.z, r.d0.w, r.d1.x, r.d1.y, r.d1.z, r.d1.w};
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) split2(x[2 * i] * d[2 * i], x[2 * i + 1] * d[2 * i + 1], hi[i], lo[i]);
    *reinterpret_cast<uint4 *>(t0) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4 *>(t1) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    if (MINS) {
        const float m[8] = {r.m0.x, r.m0.y, r.m0.z, r.m0.w, r.m1.x, r.m1.y, r.m1.z, r.m1.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            split2(x[2 * i] * m[2 * i], x[2 * i + 1] * m[2 * i + 1], hi[i], lo[i]);
        *reinterpret_cast<uint4 *>(t2) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *reinterpret_cast<uint4 *>(t3) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
}

// LDS activation tiles of one reduction step: NARR arrays (hi, lo and, for
// Q4_K, mins hi, mins lo) of ROWS x ORN_AST halves, two steps (double buffer).
template <int ROWS, int NARR>
struct ATiles {
    _Float16 t[2][NARR][ROWS * ORN_AST];
};

// Row tiles 0..NTT-1 x this wave's 4 column tiles: acc[tt][j] += A[tt] * B[j]
// for the hi and lo halves of A; with WIDE, B[j] = bq[j] + bq2[j] (q6_b2:
// the correction bq2 takes A's hi half only).
template <int NTT, bool WIDE = false>
__device__ __forceinline__ void mma_step(const _Float16 *Ahi, const _Float16 *Alo,
                                         const v8h (&bq)[4], v4f (&acc)[NTT][4], int c, int g,
                                         const v8h *bq2 = nullptr)
{
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const int ro = (16 * tt + c) * ORN_AST + 8 * g;
        const v8h ahi = *reinterpret_cast<const v8h *>(Ahi + ro);
        const v8h alo = *reinterpret_cast<const v8h *>(Alo + ro);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[tt][j] = mfma(ahi, bq[j], acc[tt][j]);
            acc[tt][j] = mfma(alo, bq[j], acc[tt][j]);
            if (WIDE) acc[tt][j] = mfma(ahi, bq2[j], acc[tt][j]);
        }
    }
}

// ---------------------------------------------------------------------------
// Gate/up.  Logical tile = ((item * ks + kslice) * 2 + m) * (H/256) + b;
// output gu[kslice][row][m*H + n] (split-K partial over the reduction steps
// kslice*KT .. +KT-1).
// ---------------------------------------------------------------------------
struct GuBlock {
    rsrc_t rq, rs, rm;                // this expert's nibble words, scales, mins
    uint32_t q_off, s_off, m_off;     // this lane's byte offsets at the slice's first step
    uint32_t qstep, sstep;            // bytes per reduction step
    const float *xrow;                // already offset to this slice's first step
    const float *dsl;                 // LDS: d then dmin of the slice's KT*32 reduction rows
    float ascale;
    int aoff, ko, KT;                 // ko: this thread's first reduction value in a step
};

struct XRaw {
    v4f x0, x1;
};

// hi/lo of x*s*d and of x*s*dmin for this thread's 8 values of step kt into
// LDS (d, dmin from the slice's LDS copy).
__device__ __forceinline__ void a_store_l(const XRaw &r, const GuBlock &B, int kt, _Float16 *t0,
                                          _Float16 *t1, _Float16 *t2, _Float16 *t3)
{
    ARaw a;
    a.x0 = r.x0;
    a.x1 = r.x1;
    const float *dl = B.dsl + 32 * kt + B.ko;
    const float *ml = dl + 32 * B.KT;
    a.d0 = *reinterpret_cast<const v4f *>(dl);
    a.d1 = *reinterpret_cast<const v4f *>(dl + 4);
    a.m0 = *reinterpret_cast<const v4f *>(ml);
    a.m1 = *reinterpret_cast<const v4f *>(ml + 4);
    a_store<true>(a, B.ascale, t0, t1, t2, t3);
}

struct GuRingP {
    uint4 q, s0, s1, mn;
};

// Software pipeline over the slice's KT steps (KT a multiple of 4): weight
// loads 4 steps ahead in a register ring, activation loads 2 steps ahead;
// the activation tile of step kt+1 is prepared into LDS (double buffer)
// while step kt's MFMAs run, one barrier per step.  The loop is unrolled by
// 4 so ring slots are static; loads past the slice re-read its last step.
template <int NTT, int ROWS>
__device__ __forceinline__ void gateup_tile(const GuBlock &B, ATiles<ROWS, 4> &As,
                                            float (*Mt)[8], const float *s_inv, float *gu_row0,
                                            int H2, int col0, int nrows)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const bool a_live = wave < NTT;  // this wave's rows hold tokens (uniform)
    const int KT = B.KT;
    auto load_b = [&](GuRingP &st, int kt) {
        kt = kt < KT ? kt : KT - 1;
        st.q = bload16(B.rq, B.q_off, kt * B.qstep);
        st.s0 = bload16(B.rs, B.s_off, kt * B.sstep);
        st.s1 = bload16(B.rs, B.s_off + 64, kt * B.sstep);
        st.mn = bload16(B.rm, B.m_off, kt * B.sstep);
    };
    auto load_a = [&](XRaw &r, int kt) {
        kt = kt < KT ? kt : KT - 1;
        r.x0 = *reinterpret_cast<const v4f *>(B.xrow + 32 * kt);
        r.x1 = *reinterpret_cast<const v4f *>(B.xrow + 32 * kt + 4);
    };
    auto pin_a = [&](XRaw &r) {
        pinf(r.x0);
        pinf(r.x1);
    };

    v4f acc[NTT][4];
#pragma unroll
    for (int i = 0; i < NTT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    v4f accm = {0.0f, 0.0f, 0.0f, 0.0f};
    const int mro = (16 * wave + c) * ORN_AST + 8 * g;  // row tile `wave`, for the mins

    GuRingP r0, r1, r2, r3;
    XRaw a0, a1;
    load_b(r0, 0);
    load_b(r1, 1);
    load_b(r2, 2);
    load_b(r3, 3);
    load_a(a0, 0);
    load_a(a1, 1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();  // the slice's d/dmin are in LDS
    a_store_l(a0, B, 0, &As.t[0][0][B.aoff], &As.t[0][1][B.aoff], &As.t[0][2][B.aoff],
              &As.t[0][3][B.aoff]);
    __builtin_amdgcn_sched_barrier(0);
    load_a(a0, 2);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // Step k = kt + s: weights from ring slot s, activation tile from LDS
    // buffer k & 1; then the activation tile of step k+1 from raw slot
    // (k+1) % 2 into buffer (k+1) & 1, whose last reader was step k-1.
    auto sub = [&](GuRingP &rb, XRaw &ra, int k, int buf) {
        pin4(rb.q); pin4(rb.s0); pin4(rb.s1); pin4(rb.mn);
        v8h bq[4];
        bq[0] = q4_b(rb.q.x, rb.s0);
        bq[1] = q4_b(rb.q.y, rb.s0);
        bq[2] = q4_b(rb.q.z, rb.s1);
        bq[3] = q4_b(rb.q.w, rb.s1);
        const uint4 mz = c < 8 ? rb.mn : make_uint4(0u, 0u, 0u, 0u);  // mins tile: 8 columns
        const v8h bm = __builtin_bit_cast(v8h, mz);
        __builtin_amdgcn_sched_barrier(0);
        load_b(rb, k + 4);
        __builtin_amdgcn_sched_barrier(0);
        mma_step<NTT>(As.t[buf][0], As.t[buf][1], bq, acc, c, g);
        // the mins tile of row tile `wave` (every wave: a wave past the
        // item's row tiles reads prepared zero rows and its result is never
        // stored), branch-free so that the next step's activation
        // preparation below shares one scheduling region with the MFMAs
        accm = mfma(*reinterpret_cast<const v8h *>(&As.t[buf][2][mro]), bm, accm);
        accm = mfma(*reinterpret_cast<const v8h *>(&As.t[buf][3][mro]), bm, accm);
        pin_a(ra);
        const int nb = buf ^ 1;
        a_store_l(ra, B, k + 1 < KT ? k + 1 : KT - 1, &As.t[nb][0][B.aoff], &As.t[nb][1][B.aoff],
                  &As.t[nb][2][B.aoff], &As.t[nb][3][B.aoff]);
        __builtin_amdgcn_sched_barrier(0);
        load_a(ra, k + 3);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    for (int kt = 0; kt < KT; kt += 4) {
        sub(r0, a1, kt + 0, 0);
        sub(r1, a0, kt + 1, 1);
        sub(r2, a1, kt + 2, 0);
        sub(r3, a0, kt + 3, 1);
    }

    // dmin term of row tile `wave`: rows 16*wave + 4g + r, sub-block c.
    if (a_live && c < 8) {
#pragma unroll
        for (int r = 0; r < 4; ++r) Mt[16 * wave + 4 * g + r][c] = accm[r];
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int nt = 4 * wave + j, sb = nt >> 1;
            const int col = col0 + 16 * nt + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * tt + 4 * g + r;
                if (row < nrows)
                    gu_row0[(size_t)row * H2 + col] = (acc[tt][j][r] - Mt[row][sb]) * s_inv[row];
            }
        }
    }
}

// NTTMAX = 1: items of at most 16 rows (decode), one row tile, small LDS.
// NTTMAX = 4: items of at most 64 rows (prefill), 1..4 row tiles.
template <int NTTMAX>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
    k_gateup_mfma(ornk_gu_prefill P, const float *__restrict__ xn,
                  const float *__restrict__ x_amax, const int *__restrict__ ctl,
                  const int4 *__restrict__ items, const int *__restrict__ row_token,
                  float *__restrict__ gu, int D, int H, int ks, int rows_max)
{
    constexpr int ROWS = 16 * NTTMAX;
    __shared__ __align__(16) ATiles<ROWS, 4> As;
    __shared__ float Mt[ROWS][8];
    __shared__ float s_scale[ROWS], s_inv[ROWS];
    __shared__ int s_tok[ROWS];
    __shared__ __align__(16) float s_dd[2 * ORN_GU_KT_MAX * 32];  // d, then dmin, of the slice

    const int NB = H >> 8;
    const int per_item = 2 * NB * ks;
    const int n_live = ctl[1] * per_item;  // tiles of the items dispatch produced
    if ((int)blockIdx.x >= n_live) return;
    const int tile = xcd_remap(blockIdx.x, n_live);
    const int b = tile % NB;
    const int m = (tile / NB) & 1;
    const int kslice = (tile / (2 * NB)) % ks;
    const int item = tile / per_item;
    const int4 itm = items[item];
    const int e = itm.w;  // expert slot index (E = the shared expert)
    const int nrows = itm.z;  // 1..ROWS (plan)
    const size_t DH = (size_t)D * H;
    const int tid = threadIdx.x;

    if (tid < ROWS) {
        const int tok = row_token[itm.y + (tid < nrows ? tid : 0)];
        const float s = tid < nrows ? row_scale(x_amax[tok], P.dmax[e * 3 + m]) : 0.0f;
        s_tok[tid] = tok;
        s_scale[tid] = s;
        s_inv[tid] = s != 0.0f ? 1.0f / s : 0.0f;
    }
    __syncthreads();

    GuBlock B;
    B.KT = D / 32 / ks;
    const int kt0 = kslice * B.KT;
    const int k0 = 32 * kt0;
    const int lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const uint32_t EQ = (uint32_t)(DH / 2), ES = (uint32_t)(DH / 16);  // bytes per expert
    B.rq = make_rsrc(reinterpret_cast<const uint8_t *>(P.pq[m]) + (size_t)e * EQ, EQ);
    B.rs = make_rsrc(reinterpret_cast<const uint8_t *>(P.psc[m]) + (size_t)e * ES, ES);
    B.rm = make_rsrc(reinterpret_cast<const uint8_t *>(P.pmn[m]) + (size_t)e * ES, ES);
    B.qstep = (uint32_t)NB * 4096;
    B.sstep = (uint32_t)NB * 512;
    B.q_off = (uint32_t)(((size_t)kt0 * NB + b) * 4096) + (wave * 64 + lane) * 16;
    B.s_off = (uint32_t)((((size_t)kt0 * NB + b) * 8 + 2 * wave) * 64) + 16 * g;
    B.m_off = (uint32_t)((((size_t)kt0 * NB + b) * 8 + (c & 7)) * 64) + 16 * g;
    const int ar = (tid >> 2) & (ROWS - 1), ao = tid & 3;  // rows >= ROWS belong to dead waves
    B.xrow = xn + (size_t)s_tok[ar] * D + k0 + 8 * ao;
    {
        // d and dmin of the slice's 32*KT reduction rows into LDS (made
        // visible by the first barrier of the tile loop)
        const float *dg = P.pd[m] + (size_t)e * (DH / 256) + (size_t)b * D + k0;
        const float *mg = P.pdm[m] + (size_t)e * (DH / 256) + (size_t)b * D + k0;
        const int n4 = 8 * B.KT;  // v4f per array
        for (int i = tid; i < n4; i += 256) {
            reinterpret_cast<v4f *>(s_dd)[i] = reinterpret_cast<const v4f *>(dg)[i];
            reinterpret_cast<v4f *>(s_dd)[n4 + i] = reinterpret_cast<const v4f *>(mg)[i];
        }
    }
    B.dsl = s_dd;
    B.ko = 8 * ao;
    B.ascale = s_scale[ar];
    B.aoff = ar * ORN_AST + 8 * ao;
    float *row0 = gu + ((size_t)kslice * rows_max + itm.y) * (2 * H);
    const int col0 = m * H + 256 * b;
    if (NTTMAX == 1) {
        gateup_tile<1, ROWS>(B, As, Mt, s_inv, row0, 2 * H, col0, nrows);
    } else {
        switch ((nrows + 15) >> 4) {
        case 1: gateup_tile<1, ROWS>(B, As, Mt, s_inv, row0, 2 * H, col0, nrows); break;
        case 2: gateup_tile<2, ROWS>(B, As, Mt, s_inv, row0, 2 * H, col0, nrows); break;
        case 3: gateup_tile<3, ROWS>(B, As, Mt, s_inv, row0, 2 * H, col0, nrows); break;
        default: gateup_tile<4, ROWS>(B, As, Mt, s_inv, row0, 2 * H, col0, nrows); break;
        }
    }
}

// ---------------------------------------------------------------------------
// Down (Q6_K).  Logical tile = (item * ks + kslice) * (D/256) + b; output
// dn[kslice][row][n].
// ---------------------------------------------------------------------------
struct DnBlock {
    const uint8_t *qb;  // ORNK_DQ_UNIT-byte units, [H/32][D/256]
    const uint16_t *sc;
    const float *mrow, *dva;  // already offset to this slice's first step
    float ascale;
    int aoff, NBD, b, kt0, KT;
};

template <int NTT, int ROWS, bool WIDE>
__device__ __forceinline__ void down_tile(const DnBlock &B, ATiles<ROWS, 2> &As, const float *s_inv,
                                          float *dn_row0, int D, int col0, int nrows)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int NBD = B.NBD, b = B.b;
    const bool a_live = wave < NTT;
    auto b_load = [&](int kt, uint4 &qn, uint2 &qc, uint4 (&sv)[4]) {
        const size_t base = (size_t)(B.kt0 + kt) * NBD + b;
        const uint8_t *up = B.qb + base * ORNK_DQ_UNIT;
        qn = *reinterpret_cast<const uint4 *>(up + (wave * 64 + lane) * 16);
        qc = *reinterpret_cast<const uint2 *>(up + 4096 + (wave * 64 + lane) * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            sv[j] = *reinterpret_cast<const uint4 *>(B.sc + (base * 16 + 4 * wave + j) * 32 + 8 * g);
    };

    v4f acc[NTT][4];
#pragma unroll
    for (int i = 0; i < NTT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    ARaw ar;
    uint4 qn;
    uint2 qc;
    uint4 sv[4];
    v8h bq[4], bq2[WIDE ? 4 : 1];
    auto build_b = [&]() {
        const uint32_t nw[4] = {qn.x, qn.y, qn.z, qn.w};
        const uint32_t cw[4] = {qc.x, qc.x >> 8, qc.y, qc.y >> 8};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t p[4];
            q6_pairs(nw[j], cw[j], p);
            if (WIDE) q6_b2(p, sv[j], bq[j], bq2[WIDE ? j : 0]);
            else bq[j] = q6_b(p, sv[j]);
        }
    };
    if (a_live) {
        a_load<false>(ar, B.mrow, B.dva, nullptr, 0);
        a_store<false>(ar, B.ascale, &As.t[0][0][B.aoff], &As.t[0][1][B.aoff], nullptr, nullptr);
    }
    b_load(0, qn, qc, sv);
    build_b();
    __syncthreads();

    for (int kt = 0; kt < B.KT - 1; ++kt) {
        const int cur = kt & 1, nxt = cur ^ 1;
        if (a_live) a_load<false>(ar, B.mrow, B.dva, nullptr, 32 * (kt + 1));
        b_load(kt + 1, qn, qc, sv);
        mma_step<NTT, WIDE>(As.t[cur][0], As.t[cur][1], bq, acc, c, g, bq2);
        if (a_live)
            a_store<false>(ar, B.ascale, &As.t[nxt][0][B.aoff], &As.t[nxt][1][B.aoff], nullptr,
                           nullptr);
        build_b();
        __syncthreads();
    }
    {
        const int cur = (B.KT - 1) & 1;
        mma_step<NTT, WIDE>(As.t[cur][0], As.t[cur][1], bq, acc, c, g, bq2);
    }

#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = col0 + 16 * (4 * wave + j) + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * tt + 4 * g + r;
                if (row < nrows) dn_row0[(size_t)row * D + col] = acc[tt][j][r] * s_inv[row];
            }
        }
    }
}

// WIDE: Q6_K sub-scales up to |128| (q6_b2: three MFMAs per tile and step).
template <int NTTMAX, bool WIDE>
__global__ void __launch_bounds__(256)
    k_down_mfma(ornk_dn_prefill P, const float *__restrict__ mid,
                const float *__restrict__ mid_amax, const int *__restrict__ ctl,
                const int4 *__restrict__ items, float *__restrict__ dn, int D, int H, int ks,
                int rows_max)
{
    constexpr int ROWS = 16 * NTTMAX;
    __shared__ __align__(16) ATiles<ROWS, 2> As;
    __shared__ float s_scale[ROWS], s_inv[ROWS];

    const int NBD = D >> 8;
    const int per_item = NBD * ks;
    const int n_live = ctl[1] * per_item;
    if ((int)blockIdx.x >= n_live) return;
    const int tile = xcd_remap(blockIdx.x, n_live);
    const int b = tile % NBD;
    const int kslice = (tile / NBD) % ks;
    const int item = tile / per_item;
    const int4 itm = items[item];
    const int e = itm.w;
    const int nrows = itm.z;
    const size_t DH = (size_t)D * H;
    const int tid = threadIdx.x;

    if (tid < ROWS) {
        const float s = tid < nrows ? row_scale(mid_amax[itm.y + tid], P.dmax[e * 3 + 2]) : 0.0f;
        s_scale[tid] = s;
        s_inv[tid] = s != 0.0f ? 1.0f / s : 0.0f;
    }
    __syncthreads();

    DnBlock B;
    B.KT = H / 32 / ks;
    B.kt0 = kslice * B.KT;
    const int k0 = 32 * B.kt0;
    B.qb = P.dq + (size_t)e * ORNK_DQ_BYTES(DH);
    B.sc = P.dsc + (size_t)e * (DH / 16);
    const int ar = (tid >> 2) & (ROWS - 1), ao = tid & 3;
    B.mrow = mid + (size_t)(itm.y + (ar < nrows ? ar : 0)) * H + k0 + 8 * ao;
    B.dva = P.dd + (size_t)e * (DH / 256) + (size_t)b * H + k0 + 8 * ao;
    B.ascale = s_scale[ar];
    B.aoff = ar * ORN_AST + 8 * ao;
    B.NBD = NBD;
    B.b = b;
    float *row0 = dn + ((size_t)kslice * rows_max + itm.y) * D;
    const int col0 = 256 * b;
    if (NTTMAX == 1) {
        down_tile<1, ROWS, WIDE>(B, As, s_inv, row0, D, col0, nrows);
    } else {
        switch ((nrows + 15) >> 4) {
        case 1: down_tile<1, ROWS, WIDE>(B, As, s_inv, row0, D, col0, nrows); break;
        case 2: down_tile<2, ROWS, WIDE>(B, As, s_inv, row0, D, col0, nrows); break;
        case 3: down_tile<3, ROWS, WIDE>(B, As, s_inv, row0, D, col0, nrows); break;
        default: down_tile<4, ROWS, WIDE>(B, As, s_inv, row0, D, col0, nrows); break;
        }
    }
}

// max_k |x[r][k]| per row, one wave per row; every load of a lane is issued
// before the first use (D <= 64 * 4 * 16 per pass).
__global__ void __launch_bounds__(256)
    k_rowmax(const float *__restrict__ x, int rows, int D, float *__restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const v4f *p = reinterpret_cast<const v4f *>(x + (size_t)r * D);
    const int n4 = D >> 2;
    float mx = 0.0f;
    for (int i0 = 0; i0 < n4; i0 += 64 * 16) {
        v4f v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = i0 + lane + 64 * j;
            v[j] = i < n4 ? p[i] : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)),
                                 fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) out[r] = mx;
}

}  // namespace

extern "C" int ornk_rowmax(const float *x, int rows, int D, float *out, hipEvent_t start,
                           hipStream_t s)
{
    if (D % 4) return hipErrorInvalidValue;
    ORN_LAUNCH_EV2(start, nullptr, k_rowmax, dim3((rows + 3) / 4), dim3(256), 0, s, x, rows, D,
                   out);
    return hipGetLastError();
}

extern "C" int ornk_moe_gateup_mfma(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_gu;
    if (a->D % 32 || a->H % 256 || ks < 1 || (a->D / 32) % ks || a->tchunk > ORN_MT ||
        (a->D / 32 / ks) % 4 || a->D / 32 / ks > ORN_GU_KT_MAX)
        return hipErrorInvalidValue;
    const float *xin = a->apply_norm ? a->xn : a->x;
    hipEvent_t st = a->ev_start;  // the step's first kernel carries the start event
    if (!a->router_amax) {
        const int e = ornk_rowmax(xin, a->T, a->D, a->x_amax, st, s);
        if (e != hipSuccess) return e;
        st = nullptr;
    }
    const dim3 grid(a->items_max * 2 * (a->H / 256) * ks);
    if (a->tchunk <= 16)
        ORN_LAUNCH_EV2(st, a->ev_stop, k_gateup_mfma<1>, grid, dim3(256), 0, s, a->gu_pf, xin,
                       a->x_amax, a->ctl, reinterpret_cast<const int4 *>(a->items), a->row_token,
                       a->gu_part, a->D, a->H, ks, a->rows_max);
    else
        ORN_LAUNCH_EV2(st, a->ev_stop, k_gateup_mfma<4>, grid, dim3(256), 0, s, a->gu_pf, xin,
                       a->x_amax, a->ctl, reinterpret_cast<const int4 *>(a->items), a->row_token,
                       a->gu_part, a->D, a->H, ks, a->rows_max);
    return hipGetLastError();
}

extern "C" int ornk_moe_down_mfma(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_dn;
    if (a->H % 32 || a->D % 256 || ks < 1 || (a->H / 32) % ks || a->tchunk > ORN_MT)
        return hipErrorInvalidValue;
    const dim3 grid(a->items_max * (a->D / 256) * ks);
#define ORN_DNM(N, W)                                                                           \
    ORN_LAUNCH_EV(a, (k_down_mfma<N, W>), grid, dim3(256), 0, s, a->dn_pf, a->mid, a->mid_amax, \
                  a->ctl, reinterpret_cast<const int4 *>(a->items), a->dn_part, a->D, a->H, ks, \
                  a->rows_max)
    if (a->tchunk <= 16) {
        if (a->q6_wide) ORN_DNM(1, true);
        else ORN_DNM(1, false);
    } else {
        if (a->q6_wide) ORN_DNM(4, true);
        else ORN_DNM(4, false);
    }
#undef ORN_DNM
    return hipGetLastError();
}
