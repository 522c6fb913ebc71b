// SPDX-License-Identifier: MIT
//
// Prefill-shaped expert products on the matrix cores: grouped GEMMs over the
// dispatch's per-expert row groups with v_mfma_f32_16x16x32_f16.
//
// Arithmetic (all exact except the activation split and fp32 accumulation):
//   Q4_K (gguf.c:43-61):  W[k][n] = d(k,b) * (sc*q)[k][n] - dmin(k,b) * m[k][n]
//   Q6_K (gguf.c:64-86):  W[k][n] = d(k,b) * (sc*q)[k][n]
//   y[r][n] = sum_k x[r][k] * W[k][n]
//           = sum_k A[r][k] * B[k][n] - sum_k Am[r][k] * m[k][n]
// with B = sc*q (an integer, |B| <= 945 for Q4_K and <= 2048 for Q6_K when
// |sc| <= 64, so exact in fp16), A = x*d and Am = x*dmin.  A is scaled per
// row by a power of two s_r (|A| < 2^14, no fp16 overflow) and split into
// fp16 hi + lo (hi = A rounded toward zero, lo = the exact remainder rounded
// toward zero): A = hi + lo to about 2^-21 relative, so two MFMAs (hi, lo)
// per tile give fp32-class products; the sums accumulate in fp32 and the
// result is scaled back by 1/s_r (exact).
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

namespace {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

#define ORN_MT 64   // token rows per work group (4 row tiles)
#define ORN_AST 40  // LDS row stride of an activation tile, in halves (32 + 8 padding)

// Power of two s with amax*dmax*s in [2^13, 2^14); 1 when that product is 0,
// NaN or infinite.
__device__ __forceinline__ float row_scale(float amax, float dmax)
{
    const float t = amax * dmax;
    if (!(t > 0.0f) || !(t <= 3.0e38f)) return 1.0f;
    int e = 13 - ilogbf(t);
    e = e < -126 ? -126 : (e > 126 ? 126 : e);
    return ldexpf(1.0f, e);
}

__device__ __forceinline__ v2h as_v2h(uint32_t u) { return __builtin_bit_cast(v2h, u); }
__device__ __forceinline__ uint32_t as_u32(v2h v) { return __builtin_bit_cast(uint32_t, v); }

// (a0, a1) -> hi = rtz fp16, lo = rtz fp16 of the exact remainder a - hi
// (formed as fma(hi, -1, a), one mixed-precision fma per value).
__device__ __forceinline__ void split2(float a0, float a1, uint32_t &hi, uint32_t &lo)
{
    const v2h h = __builtin_bit_cast(v2h, __builtin_amdgcn_cvt_pkrtz(a0, a1));
    const float r0 = __builtin_fmaf((float)h[0], -1.0f, a0);
    const float r1 = __builtin_fmaf((float)h[1], -1.0f, a1);
    hi = as_u32(h);
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}

// Work-group id i < n -> logical tile index, a bijection on [0, n) such that
// each XCD (work groups are dealt to the 8 XCDs round-robin) runs one
// contiguous range of tiles: the tiles of one item, and the items of one
// expert, then share an L2.  n is the number of live tiles, so every XCD
// gets an equal share of them.
__device__ __forceinline__ int xcd_remap(int i, int n)
{
    const int q = n >> 3, r = n & 7, x = i & 7, pos = i >> 3;
    return x < r ? x * (q + 1) + pos : r * (q + 1) + (x - r) * q + pos;
}

__device__ __forceinline__ v8h to_v8h(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    const uint4 u = make_uint4(a, b, c, d);
    return __builtin_bit_cast(v8h, u);
}

// Q4_K B operand: word w holds q for k = 0..7 at bits 4*(e/2) + 16*(e%2);
// sc = the 8 sub-block scales (fp16, k order).  B = sc * q, exactly:
// fma(1024 + q, sc, -1024 sc).
__device__ __forceinline__ uint32_t magic_pair(uint32_t w)
{
    uint32_t r;  // (w & 0x000F000F) | 0x64006400 in one instruction
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(0x000F000Fu), "v"(w), "v"(0x64006400u));
    return r;
}

__device__ __forceinline__ v8h q4_b(uint32_t w, uint4 sc)
{
    const uint32_t s[4] = {sc.x, sc.y, sc.z, sc.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2h q = as_v2h(magic_pair(w >> (4 * i)));
        const v2h sv = as_v2h(s[i]);
        const v2h ns = sv * (v2h){(_Float16)-1024.0f, (_Float16)-1024.0f};
        o[i] = as_u32(__builtin_elementwise_fma(q, sv, ns));
    }
    return to_v8h(o[0], o[1], o[2], o[3]);
}

// Q6_K B operand: 8 bytes q + 32 (k order), sc as above.  B = sc * q with
// q = (1024 + (q + 32)) - 1056 exact and |sc * q| <= 2048.
__device__ __forceinline__ v8h q6_b(uint2 q, uint4 sc)
{
    const uint32_t s[4] = {sc.x, sc.y, sc.z, sc.w};
    const uint32_t p[4] = {__builtin_amdgcn_perm(0x64646464u, q.x, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, q.x, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, q.y, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, q.y, 0x04030402u)};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2h qv = as_v2h(p[i]) + (v2h){(_Float16)-1056.0f, (_Float16)-1056.0f};
        o[i] = as_u32(qv * as_v2h(s[i]));
    }
    return to_v8h(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ v4f mfma(v8h a, v8h b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

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
// for the hi and lo halves of A.
template <int NTT>
__device__ __forceinline__ void mma_step(const _Float16 *Ahi, const _Float16 *Alo,
                                         const v8h (&bq)[4], v4f (&acc)[NTT][4], int c, int g)
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
        }
    }
}

// ---------------------------------------------------------------------------
// Gate/up.  Logical tile = ((item * ks + kslice) * 2 + m) * (H/256) + b;
// output gu[kslice][row][m*H + n] (split-K partial over the reduction steps
// kslice*KT .. +KT-1).
// ---------------------------------------------------------------------------
struct GuBlock {
    const uint32_t *qn;
    const uint16_t *sc, *mn;
    const float *xrow, *dva, *dmva;  // already offset to this slice's first step
    float ascale;
    int aoff, NB, b, kt0, KT;
};

template <int NTT, int ROWS>
__device__ __forceinline__ void gateup_tile(const GuBlock &B, ATiles<ROWS, 4> &As,
                                            float (*Mt)[8], const float *s_inv, float *gu_row0,
                                            int H2, int col0, int nrows)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int NB = B.NB, b = B.b;
    const bool a_live = wave < NTT;  // this wave's rows hold tokens (uniform)
    auto b_load = [&](int kt, uint32_t (&qw)[4], uint4 (&sw)[2], uint4 &mw) {
        const size_t base = (size_t)(B.kt0 + kt) * NB + b;
#pragma unroll
        for (int j = 0; j < 4; ++j) qw[j] = B.qn[(base * 16 + 4 * wave + j) * 64 + lane];
#pragma unroll
        for (int h = 0; h < 2; ++h)
            sw[h] = *reinterpret_cast<const uint4 *>(B.sc + (base * 8 + 2 * wave + h) * 32 + 8 * g);
        const uint4 t = *reinterpret_cast<const uint4 *>(B.mn + (base * 8 + (c & 7)) * 32 + 8 * g);
        mw = c < 8 ? t : make_uint4(0, 0, 0, 0);  // columns 8..15 of the mins tile are zero
    };

    v4f acc[NTT][4];
#pragma unroll
    for (int i = 0; i < NTT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    v4f accm = {0.0f, 0.0f, 0.0f, 0.0f};

    ARaw ar;
    uint32_t qw[4];
    uint4 sw[2], mw;
    v8h bq[4], bm;
    if (a_live) {
        a_load<true>(ar, B.xrow, B.dva, B.dmva, 0);
        a_store<true>(ar, B.ascale, &As.t[0][0][B.aoff], &As.t[0][1][B.aoff], &As.t[0][2][B.aoff],
                      &As.t[0][3][B.aoff]);
    }
    b_load(0, qw, sw, mw);
#pragma unroll
    for (int j = 0; j < 4; ++j) bq[j] = q4_b(qw[j], sw[j >> 1]);
    bm = __builtin_bit_cast(v8h, mw);
    __syncthreads();

    const int mro = (16 * wave + c) * ORN_AST + 8 * g;  // row tile `wave`, for the mins
    for (int kt = 0; kt < B.KT - 1; ++kt) {
        const int cur = kt & 1, nxt = cur ^ 1;
        if (a_live) a_load<true>(ar, B.xrow, B.dva, B.dmva, 32 * (kt + 1));
        b_load(kt + 1, qw, sw, mw);
        mma_step<NTT>(As.t[cur][0], As.t[cur][1], bq, acc, c, g);
        if (a_live) {
            accm = mfma(*reinterpret_cast<const v8h *>(&As.t[cur][2][mro]), bm, accm);
            accm = mfma(*reinterpret_cast<const v8h *>(&As.t[cur][3][mro]), bm, accm);
            a_store<true>(ar, B.ascale, &As.t[nxt][0][B.aoff], &As.t[nxt][1][B.aoff],
                          &As.t[nxt][2][B.aoff], &As.t[nxt][3][B.aoff]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) bq[j] = q4_b(qw[j], sw[j >> 1]);
        bm = __builtin_bit_cast(v8h, mw);
        __syncthreads();
    }
    {
        const int cur = (B.KT - 1) & 1;
        mma_step<NTT>(As.t[cur][0], As.t[cur][1], bq, acc, c, g);
        if (a_live) {
            accm = mfma(*reinterpret_cast<const v8h *>(&As.t[cur][2][mro]), bm, accm);
            accm = mfma(*reinterpret_cast<const v8h *>(&As.t[cur][3][mro]), bm, accm);
        }
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
__global__ void __launch_bounds__(256)
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
    B.kt0 = kslice * B.KT;
    const int k0 = 32 * B.kt0;
    B.qn = P.pq[m] + (size_t)e * (DH / 8);
    B.sc = P.psc[m] + (size_t)e * (DH / 32);
    B.mn = P.pmn[m] + (size_t)e * (DH / 32);
    const int ar = (tid >> 2) & (ROWS - 1), ao = tid & 3;  // rows >= ROWS belong to dead waves
    B.xrow = xn + (size_t)s_tok[ar] * D + k0 + 8 * ao;
    B.dva = P.pd[m] + (size_t)e * (DH / 256) + (size_t)b * D + k0 + 8 * ao;
    B.dmva = P.pdm[m] + (size_t)e * (DH / 256) + (size_t)b * D + k0 + 8 * ao;
    B.ascale = s_scale[ar];
    B.aoff = ar * ORN_AST + 8 * ao;
    B.NB = NB;
    B.b = b;
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
    const uint2 *qb;
    const uint16_t *sc;
    const float *mrow, *dva;  // already offset to this slice's first step
    float ascale;
    int aoff, NBD, b, kt0, KT;
};

template <int NTT, int ROWS>
__device__ __forceinline__ void down_tile(const DnBlock &B, ATiles<ROWS, 2> &As, const float *s_inv,
                                          float *dn_row0, int D, int col0, int nrows)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int NBD = B.NBD, b = B.b;
    const bool a_live = wave < NTT;
    auto b_load = [&](int kt, uint2 (&qv)[4], uint4 (&sv)[4]) {
        const size_t base = (size_t)(B.kt0 + kt) * NBD + b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const size_t t = base * 16 + 4 * wave + j;
            qv[j] = B.qb[t * 64 + lane];
            sv[j] = *reinterpret_cast<const uint4 *>(B.sc + t * 32 + 8 * g);
        }
    };

    v4f acc[NTT][4];
#pragma unroll
    for (int i = 0; i < NTT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    ARaw ar;
    uint2 qv[4];
    uint4 sv[4];
    v8h bq[4];
    if (a_live) {
        a_load<false>(ar, B.mrow, B.dva, nullptr, 0);
        a_store<false>(ar, B.ascale, &As.t[0][0][B.aoff], &As.t[0][1][B.aoff], nullptr, nullptr);
    }
    b_load(0, qv, sv);
#pragma unroll
    for (int j = 0; j < 4; ++j) bq[j] = q6_b(qv[j], sv[j]);
    __syncthreads();

    for (int kt = 0; kt < B.KT - 1; ++kt) {
        const int cur = kt & 1, nxt = cur ^ 1;
        if (a_live) a_load<false>(ar, B.mrow, B.dva, nullptr, 32 * (kt + 1));
        b_load(kt + 1, qv, sv);
        mma_step<NTT>(As.t[cur][0], As.t[cur][1], bq, acc, c, g);
        if (a_live)
            a_store<false>(ar, B.ascale, &As.t[nxt][0][B.aoff], &As.t[nxt][1][B.aoff], nullptr,
                           nullptr);
#pragma unroll
        for (int j = 0; j < 4; ++j) bq[j] = q6_b(qv[j], sv[j]);
        __syncthreads();
    }
    {
        const int cur = (B.KT - 1) & 1;
        mma_step<NTT>(As.t[cur][0], As.t[cur][1], bq, acc, c, g);
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

template <int NTTMAX>
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
    B.qb = reinterpret_cast<const uint2 *>(P.dq + (size_t)e * DH);
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
        down_tile<1, ROWS>(B, As, s_inv, row0, D, col0, nrows);
    } else {
        switch ((nrows + 15) >> 4) {
        case 1: down_tile<1, ROWS>(B, As, s_inv, row0, D, col0, nrows); break;
        case 2: down_tile<2, ROWS>(B, As, s_inv, row0, D, col0, nrows); break;
        case 3: down_tile<3, ROWS>(B, As, s_inv, row0, D, col0, nrows); break;
        default: down_tile<4, ROWS>(B, As, s_inv, row0, D, col0, nrows); break;
        }
    }
}

// max_k |x[r][k]| per row, one wave per row.
__global__ void __launch_bounds__(256)
    k_rowmax(const float *__restrict__ x, int rows, int D, float *__restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float *p = x + (size_t)r * D;
    float mx = 0.0f;
    for (int i = lane; i < D; i += 64) mx = fmaxf(mx, fabsf(p[i]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) out[r] = mx;
}

}  // namespace

extern "C" int ornk_moe_gateup_mfma(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_gu;
    if (a->D % 32 || a->H % 256 || ks < 1 || (a->D / 32) % ks || a->tchunk > ORN_MT)
        return hipErrorInvalidValue;
    const float *xin = a->apply_norm ? a->xn : a->x;
    hipLaunchKernelGGL(k_rowmax, dim3((a->T + 3) / 4), dim3(256), 0, s, xin, a->T, a->D,
                       a->x_amax);
    const dim3 grid(a->items_max * 2 * (a->H / 256) * ks);
    if (a->tchunk <= 16)
        hipLaunchKernelGGL(k_gateup_mfma<1>, grid, dim3(256), 0, s, a->gu_pf, xin, a->x_amax,
                           a->ctl, reinterpret_cast<const int4 *>(a->items), a->row_token,
                           a->gu_part, a->D, a->H, ks, a->rows_max);
    else
        hipLaunchKernelGGL(k_gateup_mfma<4>, grid, dim3(256), 0, s, a->gu_pf, xin, a->x_amax,
                           a->ctl, reinterpret_cast<const int4 *>(a->items), a->row_token,
                           a->gu_part, a->D, a->H, ks, a->rows_max);
    return hipGetLastError();
}

extern "C" int ornk_moe_down_mfma(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_dn;
    if (a->H % 32 || a->D % 256 || ks < 1 || (a->H / 32) % ks || a->tchunk > ORN_MT)
        return hipErrorInvalidValue;
    const dim3 grid(a->items_max * (a->D / 256) * ks);
    if (a->tchunk <= 16)
        hipLaunchKernelGGL(k_down_mfma<1>, grid, dim3(256), 0, s, a->dn_pf, a->mid, a->mid_amax,
                           a->ctl, reinterpret_cast<const int4 *>(a->items), a->dn_part, a->D,
                           a->H, ks, a->rows_max);
    else
        hipLaunchKernelGGL(k_down_mfma<4>, grid, dim3(256), 0, s, a->dn_pf, a->mid, a->mid_amax,
                           a->ctl, reinterpret_cast<const int4 *>(a->items), a->dn_part, a->D,
                           a->H, ks, a->rows_max);
    return hipGetLastError();
}
