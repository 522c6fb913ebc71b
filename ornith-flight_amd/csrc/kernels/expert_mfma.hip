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
// Work group: 4 waves, 64 token rows x 256 outputs (one block column of one
// matrix), reduction in steps of 32.  Per step every thread prepares 8
// activation values of one row into LDS (double buffered); every wave builds
// the B operands of its 4 output tiles (64 columns) in registers from the
// prefill layout (prefill_pack.c) and runs 4 row tiles x 4 column tiles x
// (hi, lo) MFMAs, plus (Q4_K) one 16-column tile holding the 8 sub-block mins
// for the dmin term of its own row tile.
#include "common.h"
#include "launch.h"

namespace {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

#define ORN_MT 64   // token rows per work group
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

// (a0, a1) -> hi = rtz fp16, lo = rtz fp16 of the exact remainder.
__device__ __forceinline__ void split2(float a0, float a1, uint32_t &hi, uint32_t &lo)
{
    const v2h h = __builtin_bit_cast(v2h, __builtin_amdgcn_cvt_pkrtz(a0, a1));
    const float r0 = a0 - (float)h[0], r1 = a1 - (float)h[1];
    hi = as_u32(h);
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}

__device__ __forceinline__ v8h to_v8h(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    const uint4 u = make_uint4(a, b, c, d);
    return __builtin_bit_cast(v8h, u);
}

// Q4_K B operand: word w holds q for k = 0..7 at bits 4*(e/2) + 16*(e%2);
// sc = the 8 sub-block scales (fp16, k order).  B = sc * q, exactly:
// fma(1024 + q, sc, -1024 sc).
__device__ __forceinline__ v8h q4_b(uint32_t w, uint4 sc)
{
    const uint32_t s[4] = {sc.x, sc.y, sc.z, sc.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2h q = as_v2h(((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u);
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
// 8*(t%4) .. +7 of the current step, for one or two scale vectors.
struct ARaw {
    v4f x0, x1, d0, d1, m0, m1;
};

template <bool MINS>
__device__ __forceinline__ void a_load(ARaw &r, const float *xrow, bool live, const float *dv,
                                       const float *dmv, int k)
{
    const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
    r.x0 = live ? *reinterpret_cast<const v4f *>(xrow + k) : z;
    r.x1 = live ? *reinterpret_cast<const v4f *>(xrow + k + 4) : z;
    r.d0 = *reinterpret_cast<const v4f *>(dv + k);
    r.d1 = *reinterpret_cast<const v4f *>(dv + k + 4);
    if (MINS) {
        r.m0 = *reinterpret_cast<const v4f *>(dmv + k);
        r.m1 = *reinterpret_cast<const v4f *>(dmv + k + 4);
    }
}

// Writes hi/lo of x*s*d (and of x*s*dmin) as 16 bytes each at off in the
// tiles base[0], base[1] (and base[2], base[3]).
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

// ---------------------------------------------------------------------------
// Gate/up.  blockIdx.x = (item * 2 + m) * (H/256) + b; output gu[row][m*H + n].
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    k_gateup_mfma(ornk_gu_prefill P, const float *__restrict__ xn,
                  const float *__restrict__ x_amax, const int *__restrict__ ctl,
                  const int4 *__restrict__ items, const int *__restrict__ slot_expert,
                  const int *__restrict__ row_token, float *__restrict__ gu, int D, int H)
{
    __shared__ __align__(16) _Float16 As[2][4][ORN_MT * ORN_AST];
    __shared__ float Mt[ORN_MT][8];
    __shared__ float s_scale[ORN_MT], s_inv[ORN_MT];
    __shared__ int s_tok[ORN_MT];

    const int NB = H >> 8;
    const int b = blockIdx.x % NB;
    const int m = (blockIdx.x / NB) & 1;
    const int item = blockIdx.x / (2 * NB);
    if (item >= ctl[1]) return;
    const int4 itm = items[item];
    const int e = slot_expert[itm.x];
    const int nrows = itm.z;  // <= ORN_MT (plan)
    const size_t DH = (size_t)D * H;
    const uint32_t *qn = P.pq[m] + (size_t)e * (DH / 8);
    const uint16_t *sc = P.psc[m] + (size_t)e * (DH / 32);
    const uint16_t *mn = P.pmn[m] + (size_t)e * (DH / 32);
    const float *dv = P.pd[m] + (size_t)e * (DH / 256) + (size_t)b * D;
    const float *dmv = P.pdm[m] + (size_t)e * (DH / 256) + (size_t)b * D;
    const float dmx = P.dmax[e * 3 + m];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;

    if (tid < ORN_MT) {
        const int tok = tid < nrows ? row_token[itm.y + tid] : -1;
        const float s = tok >= 0 ? row_scale(x_amax[tok], dmx) : 1.0f;
        s_tok[tid] = tok;
        s_scale[tid] = s;
        s_inv[tid] = 1.0f / s;
    }
    __syncthreads();

    const int ar = tid >> 2, ao = tid & 3;
    const int atok = s_tok[ar];
    const float ascale = s_scale[ar];
    const float *xrow = xn + (size_t)(atok < 0 ? 0 : atok) * D + 8 * ao;
    const float *dva = dv + 8 * ao, *dmva = dmv + 8 * ao;
    const int aoff = ar * ORN_AST + 8 * ao;
    const int n_tt = (nrows + 15) >> 4;  // live row tiles

    auto b_load = [&](int kt, uint32_t (&qw)[4], uint4 (&sw)[2], uint4 &mw) {
        const size_t base = (size_t)kt * NB + b;
#pragma unroll
        for (int j = 0; j < 4; ++j) qw[j] = qn[(base * 16 + 4 * wave + j) * 64 + lane];
#pragma unroll
        for (int h = 0; h < 2; ++h)
            sw[h] = *reinterpret_cast<const uint4 *>(sc + (base * 8 + 2 * wave + h) * 32 + 8 * g);
        mw = c < 8 ? *reinterpret_cast<const uint4 *>(mn + (base * 8 + c) * 32 + 8 * g)
                   : make_uint4(0, 0, 0, 0);
    };

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    v4f accm = {0.0f, 0.0f, 0.0f, 0.0f};

    ARaw ar_raw;
    uint32_t qw[4];
    uint4 sw[2], mw;
    v8h bq[4], bm;
    a_load<true>(ar_raw, xrow, atok >= 0, dva, dmva, 0);
    b_load(0, qw, sw, mw);
    a_store<true>(ar_raw, ascale, &As[0][0][aoff], &As[0][1][aoff], &As[0][2][aoff],
                  &As[0][3][aoff]);
#pragma unroll
    for (int j = 0; j < 4; ++j) bq[j] = q4_b(qw[j], sw[j >> 1]);
    bm = __builtin_bit_cast(v8h, mw);
    __syncthreads();

    const int KT = D / 32;
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            a_load<true>(ar_raw, xrow, atok >= 0, dva, dmva, 32 * (kt + 1));
            b_load(kt + 1, qw, sw, mw);
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (tt < n_tt) {
                const int ro = (16 * tt + c) * ORN_AST + 8 * g;
                const v8h ahi = *reinterpret_cast<const v8h *>(&As[buf][0][ro]);
                const v8h alo = *reinterpret_cast<const v8h *>(&As[buf][1][ro]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[tt][j] = mfma(ahi, bq[j], acc[tt][j]);
                    acc[tt][j] = mfma(alo, bq[j], acc[tt][j]);
                }
            }
        }
        if (wave < n_tt) {
            const int ro = (16 * wave + c) * ORN_AST + 8 * g;
            const v8h mhi = *reinterpret_cast<const v8h *>(&As[buf][2][ro]);
            const v8h mlo = *reinterpret_cast<const v8h *>(&As[buf][3][ro]);
            accm = mfma(mhi, bm, accm);
            accm = mfma(mlo, bm, accm);
        }
        if (more) {
            const int nb = buf ^ 1;
            a_store<true>(ar_raw, ascale, &As[nb][0][aoff], &As[nb][1][aoff], &As[nb][2][aoff],
                          &As[nb][3][aoff]);
#pragma unroll
            for (int j = 0; j < 4; ++j) bq[j] = q4_b(qw[j], sw[j >> 1]);
            bm = __builtin_bit_cast(v8h, mw);
        }
        __syncthreads();
    }

    // dmin term of this wave's row tile: rows 16*wave + 4g + r, sub-block c.
    if (c < 8) {
#pragma unroll
        for (int r = 0; r < 4; ++r) Mt[16 * wave + 4 * g + r][c] = accm[r];
    }
    __syncthreads();
    const int H2 = 2 * H;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        if (tt >= n_tt) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int nt = 4 * wave + j, s = nt >> 1;
            const int col = m * H + 256 * b + 16 * nt + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * tt + 4 * g + r;
                if (row < nrows)
                    gu[(size_t)(itm.y + row) * H2 + col] = (acc[tt][j][r] - Mt[row][s]) * s_inv[row];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Down (Q6_K).  blockIdx.x = item * (D/256) + b; output dn[row][n].
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    k_down_mfma(ornk_dn_prefill P, const float *__restrict__ mid,
                const float *__restrict__ mid_amax, const int *__restrict__ ctl,
                const int4 *__restrict__ items, const int *__restrict__ slot_expert,
                float *__restrict__ dn, int D, int H)
{
    __shared__ __align__(16) _Float16 As[2][2][ORN_MT * ORN_AST];
    __shared__ float s_scale[ORN_MT], s_inv[ORN_MT];

    const int NBD = D >> 8;
    const int b = blockIdx.x % NBD;
    const int item = blockIdx.x / NBD;
    if (item >= ctl[1]) return;
    const int4 itm = items[item];
    const int e = slot_expert[itm.x];
    const int nrows = itm.z;
    const size_t DH = (size_t)D * H;
    const uint2 *qb = reinterpret_cast<const uint2 *>(P.dq + (size_t)e * DH);
    const uint16_t *sc = P.dsc + (size_t)e * (DH / 16);
    const float *dv = P.dd + (size_t)e * (DH / 256) + (size_t)b * H;
    const float dmx = P.dmax[e * 3 + 2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;

    if (tid < ORN_MT) {
        const float s = tid < nrows ? row_scale(mid_amax[itm.y + tid], dmx) : 1.0f;
        s_scale[tid] = s;
        s_inv[tid] = 1.0f / s;
    }
    __syncthreads();

    const int ar = tid >> 2, ao = tid & 3;
    const bool alive = ar < nrows;
    const float ascale = s_scale[ar];
    const float *mrow = mid + (size_t)(itm.y + (alive ? ar : 0)) * H + 8 * ao;
    const float *dva = dv + 8 * ao;
    const int aoff = ar * ORN_AST + 8 * ao;
    const int n_tt = (nrows + 15) >> 4;

    auto b_load = [&](int kt, uint2 (&qv)[4], uint4 (&sv)[4]) {
        const size_t base = (size_t)kt * NBD + b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const size_t t = base * 16 + 4 * wave + j;
            qv[j] = qb[t * 64 + lane];
            sv[j] = *reinterpret_cast<const uint4 *>(sc + t * 32 + 8 * g);
        }
    };

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    ARaw ar_raw;
    uint2 qv[4];
    uint4 sv[4];
    v8h bq[4];
    a_load<false>(ar_raw, mrow, alive, dva, nullptr, 0);
    b_load(0, qv, sv);
    a_store<false>(ar_raw, ascale, &As[0][0][aoff], &As[0][1][aoff], nullptr, nullptr);
#pragma unroll
    for (int j = 0; j < 4; ++j) bq[j] = q6_b(qv[j], sv[j]);
    __syncthreads();

    const int KT = H / 32;
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            a_load<false>(ar_raw, mrow, alive, dva, nullptr, 32 * (kt + 1));
            b_load(kt + 1, qv, sv);
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (tt < n_tt) {
                const int ro = (16 * tt + c) * ORN_AST + 8 * g;
                const v8h ahi = *reinterpret_cast<const v8h *>(&As[buf][0][ro]);
                const v8h alo = *reinterpret_cast<const v8h *>(&As[buf][1][ro]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[tt][j] = mfma(ahi, bq[j], acc[tt][j]);
                    acc[tt][j] = mfma(alo, bq[j], acc[tt][j]);
                }
            }
        }
        if (more) {
            const int nb = buf ^ 1;
            a_store<false>(ar_raw, ascale, &As[nb][0][aoff], &As[nb][1][aoff], nullptr, nullptr);
#pragma unroll
            for (int j = 0; j < 4; ++j) bq[j] = q6_b(qv[j], sv[j]);
        }
        __syncthreads();
    }

#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        if (tt >= n_tt) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = 256 * b + 16 * (4 * wave + j) + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * tt + 4 * g + r;
                if (row < nrows) dn[(size_t)(itm.y + row) * D + col] = acc[tt][j][r] * s_inv[row];
            }
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
    if (a->D % 32 || a->H % 256 || a->tchunk > ORN_MT) return hipErrorInvalidValue;
    const float *xin = a->apply_norm ? a->xn : a->x;
    hipLaunchKernelGGL(k_rowmax, dim3((a->T + 3) / 4), dim3(256), 0, s, xin, a->T, a->D,
                       a->x_amax);
    hipLaunchKernelGGL(k_gateup_mfma, dim3(a->items_max * 2 * (a->H / 256)), dim3(256), 0, s,
                       a->gu_pf, xin, a->x_amax, a->ctl, reinterpret_cast<const int4 *>(a->items),
                       a->slot_expert, a->row_token, a->gu_part, a->D, a->H);
    return hipGetLastError();
}

extern "C" int ornk_moe_down_mfma(const ornk_moe_args *a, hipStream_t s)
{
    if (a->H % 32 || a->D % 256 || a->tchunk > ORN_MT) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_down_mfma, dim3(a->items_max * (a->D / 256)), dim3(256), 0, s, a->dn_pf,
                       a->mid, a->mid_amax, a->ctl, reinterpret_cast<const int4 *>(a->items),
                       a->slot_expert, a->dn_part, a->D, a->H);
    return hipGetLastError();
}
