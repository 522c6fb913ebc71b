// SPDX-License-Identifier: MIT
//
// Decode-shaped expert products on the matrix cores: work items of at most
// 16 token rows (one MFMA row tile) of one expert, split-K over the
// reduction dimension.  Operand preparation and its exactness argument:
// mfma_ops.h; memory layouts: prefill_pack.c.
//
// At decode sizes the weights are read once per launch and the step is
// bound by how many bytes are in flight, so each lane keeps NR reduction
// steps of loads (weights, per-row scales and the activations they meet)
// in a register ring, refilled right after a step's registers are consumed.
// The KT steps of a slice are a compile-time count and fully unrolled: a
// loop would carry the ring through the back edge as register copies, which
// wait for every load in flight.
//
// Work group: 4 waves over one 256-column block of one matrix.  Wave w owns
// column tiles 4w..4w+3 (one 16-byte weight load per lane and step for
// Q4_K, two for Q6_K).  Each step all 256 threads prepare the 16 x 32
// activation tile (2 values per thread, hi/lo split) into LDS (double
// buffered, one barrier per step); every wave then runs 4 x (hi, lo) MFMAs
// and, for Q4_K, 2 more for the dmin term of its own two sub-blocks.
#include "common.h"
#include "launch.h"
#include "mfma_ops.h"

namespace {

using namespace orn_mfma;

typedef float v2f __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

#define ORN_DEC_NR 4  // reduction steps in flight per lane

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

__device__ __forceinline__ v2f bload8f(rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// LDS activation tiles: [buffer][hi, lo, mins hi, mins lo][16 rows x ORN_AST]
// as 32-bit words (two halves).
template <int NARR>
struct DecTiles {
    uint32_t w[2][NARR][16 * ORN_AST / 2];
};

// ---------------------------------------------------------------------------
// Gate/up (Q4_K).  Logical tile = ((item * ks + kslice) * 2 + m) * (H/256) + b;
// output gu[kslice][row][m*H + n], the split-K partial over the reduction
// steps kslice*KT .. +KT-1.
// ---------------------------------------------------------------------------
struct GuStage {
    uint4 q;         // nibble words of column tiles 4w..4w+3
    uint4 s0, s1;    // scales of sub-blocks 2w, 2w+1 at k = 8g..8g+7
    uint4 mn;        // mins of sub-block 2w + (c & 1) at k = 8g..8g+7
    v2f x, d, dm;    // activation row tid/16 at k pair 2*(tid%16), its d, dmin
};

template <int NR, int KT>
__global__ void __launch_bounds__(256)
    k_gateup_dec(ornk_gu_prefill P, const float *__restrict__ xn,
                 const float *__restrict__ x_amax, const int *__restrict__ ctl,
                 const int4 *__restrict__ items, const int *__restrict__ row_token,
                 float *__restrict__ gu, int T, int D, int H, int ks, int rows_max)
{
    __shared__ __align__(16) DecTiles<4> As;
    __shared__ float s_inv[16];

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
    const int e = itm.w;      // expert slot index (E = the shared expert)
    const int nrows = itm.z;  // 1..16 (plan)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int kt0 = kslice * KT;
    const size_t DH = (size_t)D * H;

    // Streams of this work group (buffer bases, wave-uniform) and this
    // lane's fixed byte offsets; step kt adds kt * (step bytes).
    const uint32_t EQ = (uint32_t)(DH / 2), ES = (uint32_t)(DH / 16);  // bytes per expert
    const rsrc_t rq = make_rsrc(reinterpret_cast<const uint8_t *>(P.pq[m]) + (size_t)e * EQ, EQ);
    const rsrc_t rs = make_rsrc(reinterpret_cast<const uint8_t *>(P.psc[m]) + (size_t)e * ES, ES);
    const rsrc_t rm = make_rsrc(reinterpret_cast<const uint8_t *>(P.pmn[m]) + (size_t)e * ES, ES);
    const uint32_t qstep = (uint32_t)NB * 4096, sstep = (uint32_t)NB * 512;
    const uint32_t q_off = (uint32_t)(((size_t)kt0 * NB + b) * 4096) + (wave * 64 + lane) * 16;
    const uint32_t s_off = (uint32_t)((((size_t)kt0 * NB + b) * 8 + 2 * wave) * 64) + 16 * g;
    const uint32_t m_off = s_off + 64 * (c & 1);
    // Activation prep: thread row ar, k pair kp of each step.
    const int ar = tid >> 4, kp = 2 * (tid & 15);
    const int arow = ar < nrows ? ar : 0;  // rows past the item read a valid row, scaled by 0
    const uint32_t ED = (uint32_t)(DH / 64);  // d (or dmin) bytes per expert
    const rsrc_t rd = make_rsrc(reinterpret_cast<const uint8_t *>(P.pd[m]) + (size_t)e * ED, ED);
    const rsrc_t rdm = make_rsrc(reinterpret_cast<const uint8_t *>(P.pdm[m]) + (size_t)e * ED, ED);
    const uint32_t d_off = (uint32_t)(((size_t)b * D + 32 * kt0 + kp) * 4);

    auto load_b = [&](GuStage &st, int kt) {
        st.q = bload16(rq, q_off, kt * qstep);
        st.s0 = bload16(rs, s_off, kt * sstep);
        st.s1 = bload16(rs, s_off + 64, kt * sstep);
        st.mn = bload16(rm, m_off, kt * sstep);
    };
    const rsrc_t rx = make_rsrc(xn, (uint32_t)((size_t)T * D * 4));
    uint32_t x_off = 0;
    auto load_a = [&](GuStage &st, int kt) {
        st.x = bload8f(rx, x_off, kt * 128);
        st.d = bload8f(rd, d_off, kt * 128);
        st.dm = bload8f(rdm, d_off, kt * 128);
    };

    // Prologue: the token index first, then the weight loads of the first NR
    // steps (independent of the tokens), then the token-dependent loads.
    const int tok = row_token[itm.y + arow];
    GuStage st[NR];
#pragma unroll
    for (int s = 0; s < NR; ++s) load_b(st[s], s);
    __builtin_amdgcn_sched_barrier(0);
    x_off = (uint32_t)(((size_t)tok * D + 32 * kt0 + kp) * 4);
    const float amax = x_amax[tok];
    const float dmx = P.dmax[e * 3 + m];
#pragma unroll
    for (int s = 0; s < NR; ++s) load_a(st[s], s);
    __builtin_amdgcn_sched_barrier(0);
    const float ascale = ar < nrows ? row_scale(amax, dmx) : 0.0f;
    if ((tid & 15) == 0) s_inv[ar] = ascale != 0.0f ? 1.0f / ascale : 0.0f;

    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    v4f accm = {0.0f, 0.0f, 0.0f, 0.0f};
    const int aw = (ar * ORN_AST + kp) >> 1;  // this thread's LDS word
    const int ro = c * ORN_AST + 8 * g;       // this lane's A operand (halves)

    auto step = [&](GuStage &st, int buf, bool refill, int ktn) {
        {
            const float x0 = st.x.x * ascale, x1 = st.x.y * ascale;
            uint32_t hi, lo, mhi, mlo;
            split2(x0 * st.d.x, x1 * st.d.y, hi, lo);
            split2(x0 * st.dm.x, x1 * st.dm.y, mhi, mlo);
            As.w[buf][0][aw] = hi;
            As.w[buf][1][aw] = lo;
            As.w[buf][2][aw] = mhi;
            As.w[buf][3][aw] = mlo;
        }
        v8h bq[4];
        bq[0] = q4_b(st.q.x, st.s0);
        bq[1] = q4_b(st.q.y, st.s0);
        bq[2] = q4_b(st.q.z, st.s1);
        bq[3] = q4_b(st.q.w, st.s1);
        const uint4 mz = c < 2 ? st.mn : make_uint4(0u, 0u, 0u, 0u);  // columns 2..15: zero
        const v8h bm = __builtin_bit_cast(v8h, mz);
        __builtin_amdgcn_sched_barrier(0);
        if (refill) {
            load_b(st, ktn);
            load_a(st, ktn);
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        const _Float16 *A0 = reinterpret_cast<const _Float16 *>(As.w[buf][0]);
        const _Float16 *A1 = reinterpret_cast<const _Float16 *>(As.w[buf][1]);
        const _Float16 *A2 = reinterpret_cast<const _Float16 *>(As.w[buf][2]);
        const _Float16 *A3 = reinterpret_cast<const _Float16 *>(As.w[buf][3]);
        const v8h ahi = *reinterpret_cast<const v8h *>(A0 + ro);
        const v8h alo = *reinterpret_cast<const v8h *>(A1 + ro);
        const v8h mhi = *reinterpret_cast<const v8h *>(A2 + ro);
        const v8h mlo = *reinterpret_cast<const v8h *>(A3 + ro);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[j] = mfma(ahi, bq[j], acc[j]);
            acc[j] = mfma(alo, bq[j], acc[j]);
        }
        accm = mfma(mhi, bm, accm);
        accm = mfma(mlo, bm, accm);
    };

#pragma unroll
    for (int kt = 0; kt < KT; ++kt) step(st[kt % NR], kt & 1, kt + NR < KT, kt + NR);

    // y = (acc - dmin term of the column's sub-block) / s_row.  accm of lane
    // (g, c < 2) holds rows 4g..4g+3 of sub-block 2w + c.
    float *row0 = gu + ((size_t)kslice * rows_max + itm.y) * (2 * H);
    const int colb = m * H + 256 * b + 64 * wave + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        const float si = s_inv[row];
        const float m0 = __shfl(accm[r], 16 * g, 64);
        const float m1 = __shfl(accm[r], 16 * g + 1, 64);
        if (row < nrows) {
            float *o = row0 + (size_t)row * (2 * H) + colb;
            o[0] = (acc[0][r] - m0) * si;
            o[16] = (acc[1][r] - m0) * si;
            o[32] = (acc[2][r] - m1) * si;
            o[48] = (acc[3][r] - m1) * si;
        }
    }
}

// ---------------------------------------------------------------------------
// Down (Q6_K).  Logical tile = (item * ks + kslice) * (D/256) + b; output
// dn[kslice][row][n].
// ---------------------------------------------------------------------------
struct DnStage {
    uint4 q0, q1;  // q + 32 of column tiles 4w..4w+3, 8 bytes per tile
    uint4 sc[4];   // scales of tiles 4w+j at k = 8g..8g+7
    v2f x, d;      // mid row tid/16 at k pair 2*(tid%16), its d
};

template <int NR, int KT>
__global__ void __launch_bounds__(256)
    k_down_dec(ornk_dn_prefill P, const float *__restrict__ mid,
               const float *__restrict__ mid_amax, const int *__restrict__ ctl,
               const int4 *__restrict__ items, float *__restrict__ dn, int D, int H, int ks,
               int rows_max)
{
    __shared__ __align__(16) DecTiles<2> As;
    __shared__ float s_inv[16];

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
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int kt0 = kslice * KT;
    const size_t DH = (size_t)D * H;

    const uint32_t EQ = (uint32_t)DH, ES = (uint32_t)(DH / 8), ED = (uint32_t)(DH / 64);
    const rsrc_t rq = make_rsrc(P.dq + (size_t)e * EQ, EQ);
    const rsrc_t rs = make_rsrc(reinterpret_cast<const uint8_t *>(P.dsc) + (size_t)e * ES, ES);
    const rsrc_t rd = make_rsrc(reinterpret_cast<const uint8_t *>(P.dd) + (size_t)e * ED, ED);
    const rsrc_t rx = make_rsrc(mid, (uint32_t)((size_t)rows_max * H * 4));
    const uint32_t qstep = (uint32_t)NBD * 8192, sstep = (uint32_t)NBD * 1024;
    const uint32_t q_off = (uint32_t)(((size_t)kt0 * NBD + b) * 8192) + (wave * 64 + lane) * 32;
    const uint32_t s_off = (uint32_t)((((size_t)kt0 * NBD + b) * 16 + 4 * wave) * 64) + 16 * g;
    const int ar = tid >> 4, kp = 2 * (tid & 15);
    const int arow = ar < nrows ? ar : 0;
    const uint32_t x_off = (uint32_t)(((size_t)(itm.y + arow) * H + 32 * kt0 + kp) * 4);
    const uint32_t d_off = (uint32_t)(((size_t)b * H + 32 * kt0 + kp) * 4);

    auto load = [&](DnStage &st, int kt) {
        st.q0 = bload16(rq, q_off, kt * qstep);
        st.q1 = bload16(rq, q_off + 16, kt * qstep);
#pragma unroll
        for (int j = 0; j < 4; ++j) st.sc[j] = bload16(rs, s_off + 64 * j, kt * sstep);
        st.x = bload8f(rx, x_off, kt * 128);
        st.d = bload8f(rd, d_off, kt * 128);
    };

    const float amax = mid_amax[itm.y + arow];
    const float dmx = P.dmax[e * 3 + 2];
    DnStage st[NR];
#pragma unroll
    for (int s = 0; s < NR; ++s) load(st[s], s);
    __builtin_amdgcn_sched_barrier(0);
    const float ascale = ar < nrows ? row_scale(amax, dmx) : 0.0f;
    if ((tid & 15) == 0) s_inv[ar] = ascale != 0.0f ? 1.0f / ascale : 0.0f;

    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    const int aw = (ar * ORN_AST + kp) >> 1;
    const int ro = c * ORN_AST + 8 * g;

    auto step = [&](DnStage &st, int buf, bool refill, int ktn) {
        {
            uint32_t hi, lo;
            split2(st.x.x * ascale * st.d.x, st.x.y * ascale * st.d.y, hi, lo);
            As.w[buf][0][aw] = hi;
            As.w[buf][1][aw] = lo;
        }
        v8h bq[4];
        bq[0] = q6_b(st.q0.x, st.q0.y, st.sc[0]);
        bq[1] = q6_b(st.q0.z, st.q0.w, st.sc[1]);
        bq[2] = q6_b(st.q1.x, st.q1.y, st.sc[2]);
        bq[3] = q6_b(st.q1.z, st.q1.w, st.sc[3]);
        __builtin_amdgcn_sched_barrier(0);
        if (refill) load(st, ktn);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        const v8h ahi = *reinterpret_cast<const v8h *>(
            reinterpret_cast<const _Float16 *>(As.w[buf][0]) + ro);
        const v8h alo = *reinterpret_cast<const v8h *>(
            reinterpret_cast<const _Float16 *>(As.w[buf][1]) + ro);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[j] = mfma(ahi, bq[j], acc[j]);
            acc[j] = mfma(alo, bq[j], acc[j]);
        }
    };

#pragma unroll
    for (int kt = 0; kt < KT; ++kt) step(st[kt % NR], kt & 1, kt + NR < KT, kt + NR);

    float *row0 = dn + ((size_t)kslice * rows_max + itm.y) * D;
    const int colb = 256 * b + 64 * wave + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        const float si = s_inv[row];
        if (row < nrows) {
            float *o = row0 + (size_t)row * D + colb;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[16 * j] = acc[j][r] * si;
        }
    }
}

}  // namespace

// Decode instances: work items of <= 16 rows; KT = D/32/ks (gate/up) or
// H/32/ks (down) reduction steps per slice, one of the instantiated counts.
extern "C" int ornk_dec_supported(int kt_gu, int kt_dn)
{
    auto ok = [](int kt) { return kt == 4 || kt == 8 || kt == 16 || kt == 32; };
    return ok(kt_gu) && ok(kt_dn);
}

extern "C" int ornk_moe_gateup_dec(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_gu;
    if (a->D % 32 || a->H % 256 || ks < 1 || (a->D / 32) % ks || a->tchunk > 16)
        return hipErrorInvalidValue;
    const int KT = a->D / 32 / ks;
    if (!ornk_dec_supported(KT, 4)) return hipErrorInvalidValue;
    const float *xin = a->apply_norm ? a->xn : a->x;
    if (!a->router_amax) {
        const int e = ornk_rowmax(xin, a->T, a->D, a->x_amax, s);
        if (e != hipSuccess) return e;
    }
    const dim3 grid(a->items_max * 2 * (a->H / 256) * ks);
#define ORN_GU_DEC(K)                                                                        \
    hipLaunchKernelGGL((k_gateup_dec<ORN_DEC_NR, K>), grid, dim3(256), 0, s, a->gu_pf, xin,   \
                       a->x_amax, a->ctl, reinterpret_cast<const int4 *>(a->items),           \
                       a->row_token, a->gu_part, a->T, a->D, a->H, ks, a->rows_max)
    switch (KT) {
    case 4: ORN_GU_DEC(4); break;
    case 8: ORN_GU_DEC(8); break;
    case 16: ORN_GU_DEC(16); break;
    default: ORN_GU_DEC(32); break;
    }
#undef ORN_GU_DEC
    return hipGetLastError();
}

extern "C" int ornk_moe_down_dec(const ornk_moe_args *a, hipStream_t s)
{
    const int ks = a->ks_dn;
    if (a->H % 32 || a->D % 256 || ks < 1 || (a->H / 32) % ks || a->tchunk > 16)
        return hipErrorInvalidValue;
    const int KT = a->H / 32 / ks;
    if (!ornk_dec_supported(4, KT)) return hipErrorInvalidValue;
    const dim3 grid(a->items_max * (a->D / 256) * ks);
#define ORN_DN_DEC(K)                                                                       \
    hipLaunchKernelGGL((k_down_dec<ORN_DEC_NR, K>), grid, dim3(256), 0, s, a->dn_pf, a->mid, \
                       a->mid_amax, a->ctl, reinterpret_cast<const int4 *>(a->items),        \
                       a->dn_part, a->D, a->H, ks, a->rows_max)
    switch (KT) {
    case 4: ORN_DN_DEC(4); break;
    case 8: ORN_DN_DEC(8); break;
    case 16: ORN_DN_DEC(16); break;
    default: ORN_DN_DEC(32); break;
    }
#undef ORN_DN_DEC
    return hipGetLastError();
}
