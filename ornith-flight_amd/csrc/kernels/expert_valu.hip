// SPDX-License-Identifier: MIT
//
// Routed-MoE expert path for decode-shaped work (few tokens per expert):
// dispatch -> fused Q4_K dequant-matvec for gate+up -> SiLU(gate)*up ->
// Q6_K dequant-matvec for down -> weighted combine.  fp32 VALU arithmetic
// (explicit fmaf), weights decoded in registers straight from the resident
// K-quant blocks with 128-bit loads; each output is reduced in a fixed order
// so results repeat bit for bit from run to run.
//
// Reference semantics (model.c:992-1144):
//   shared:  g = x@Wg, u = x@Wu, mid = silu(g)*u (no clamp, gpu.c:176-186),
//            y_sh = mid@Wd;  x = x + y_sh                (model.c:1003-1007)
//   routed:  for each selected expert with w >= 1e-6 (model.c:1066):
//            mid = silu_clamped(g)*u (model.c:340-344, 1087), y = mid@Wd,
//            routed += w*y in selection order; x = x + routed (model.c:1142)
//
// Matrix orientation is the reference's vec@mat (model.c:351-357):
// out[i] = sum_k v[k]*W[k*M + i]; K-quant super-blocks run along the output
// index, so one 144/210-byte block holds 256 consecutive outputs of one row.
#include "common.h"
#include "launch.h"

#define ORN_TCHUNK 8   // token rows per work item
#define ORN_TG_MAX 4   // token rows processed together in registers

namespace {

// ---------------------------------------------------------------------------
__global__ void k_reset_ctl(int *ctl)
{
    if (threadIdx.x < 16) ctl[threadIdx.x] = 0;
}

// ---------------------------------------------------------------------------
// Dispatch: one block.  List position j: 0 = shared expert (expert id E),
// j >= 1 = routed expert j-1.  Produces the active slots (shared first, then
// experts in ascending id), their row ranges, the work items (<= ORN_TCHUNK
// rows each) and the row <-> (token, selection slot) maps.
// ---------------------------------------------------------------------------
__device__ int block_excl_scan(int v, int *buf, int *total)
{
    const int tid = threadIdx.x, n = blockDim.x;
    buf[tid] = v;
    __syncthreads();
    for (int off = 1; off < n; off <<= 1) {
        int add = tid >= off ? buf[tid - off] : 0;
        __syncthreads();
        buf[tid] += add;
        __syncthreads();
    }
    int incl = buf[tid];
    if (total) *total = buf[n - 1];
    __syncthreads();
    return incl - v;
}

__global__ void __launch_bounds__(1024)
    k_dispatch(const uint32_t *__restrict__ idx, const float *__restrict__ w, int T, int k, int E,
               int has_shared, int *ctl, int *slot_expert, int *slot_off, int *slot_cnt,
               int *row_token, int *pair_row, int4 *items, int items_max)
{
    __shared__ int cnt[1024];
    __shared__ int cursor[1024];
    __shared__ int rowoff[1024];
    __shared__ int scanbuf[1024];
    const int tid = threadIdx.x;
    const int NJ = E + 1;
    cnt[tid] = 0;
    cursor[tid] = 0;
    __syncthreads();
    const int P = T * k;
    for (int p = tid; p < P; p += blockDim.x)
        if (!(w[p] < 1e-6f) && idx[p] < (uint32_t)E) atomicAdd(&cnt[idx[p] + 1], 1);
    if (tid == 0) cnt[0] = has_shared ? T : 0;
    __syncthreads();

    const int c = tid < NJ ? cnt[tid] : 0;
    const int flag = c > 0 ? 1 : 0;
    const int nit = (c + ORN_TCHUNK - 1) / ORN_TCHUNK;
    int n_slots, n_rows, n_items;
    const int slot = block_excl_scan(flag, scanbuf, &n_slots);
    const int roff = block_excl_scan(c, scanbuf, &n_rows);
    const int ioff = block_excl_scan(nit, scanbuf, &n_items);
    rowoff[tid] = roff;
    if (flag) {
        slot_expert[slot] = tid == 0 ? E : tid - 1;
        slot_off[slot] = roff;
        slot_cnt[slot] = c;
        for (int q = 0; q < nit && ioff + q < items_max; ++q) {
            const int r0 = q * ORN_TCHUNK;
            items[ioff + q] = make_int4(slot, roff + r0, min(ORN_TCHUNK, c - r0), tid == 0);
        }
    }
    if (tid == 0) {
        ctl[0] = n_slots;
        ctl[1] = n_items < items_max ? n_items : items_max;
        ctl[2] = n_rows;
    }
    __syncthreads();

    for (int p = tid; p < P; p += blockDim.x) {
        // Skip rule of model.c:1066; an index outside [0, E) cannot come out
        // of the router but is treated as skipped rather than trusted.
        if (w[p] < 1e-6f || idx[p] >= (uint32_t)E) {
            pair_row[p] = -1;
            continue;
        }
        const int j = (int)idx[p] + 1;
        const int r = rowoff[j] + atomicAdd(&cursor[j], 1);
        row_token[r] = p / k;
        pair_row[p] = r;
    }
    if (has_shared)
        for (int t = tid; t < T; t += blockDim.x) row_token[rowoff[0] + t] = t;
}

// ---------------------------------------------------------------------------
// Gate+up: split-K over the D input rows.  Block = 4 waves; item = up to
// ORN_TCHUNK rows (tokens) of one expert; blockIdx.x = item*ks + kslice.
// Lane layout inside a wave: ch = lane % CR picks (matrix m, block column
// bc, 16-byte qs chunk j) with CR = 16*(H/256) chunks per input row, and
// rr = lane / CR picks one of RW = 64/CR rows handled side by side.
//
// Q4_K chunk j of a block holds bytes 16j..16j+15 of qs: low nibbles are
// outputs 64*(j/2) + 16*(j%2) + u of sub-block 2*(j/2), high nibbles the same
// + 32 of sub-block 2*(j/2)+1 (gguf.c:43-61).  With D1 = d*sc, M1 = dmin*m
// the contribution of row k is x_k*(D1*q - M1); the M1 term is constant over
// the 16 outputs, so it is accumulated once per row and subtracted at the end.
// ---------------------------------------------------------------------------
template <int TG>
__device__ void gateup_group(const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up,
                             const float *__restrict__ xn, const int *__restrict__ row_token,
                             float *__restrict__ gu_part, int D, int H, int e, int row_g,
                             int kslice, int RK, int rows_max, float *xs, float *red)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NB = H >> 8;
    const int CR = 16 * NB;
    const int RW = 64 / CR;
    const int rr = lane / CR, ch = lane % CR;
    const int m = ch / (8 * NB), bc = (ch >> 3) % NB, j = ch & 7;
    const int c = j >> 1;
    const int k_start = kslice * RK;
    const int H2 = 2 * H;

    // Stage this group's activations for the K-slice.
    for (int i = tid; i < TG * RK; i += blockDim.x) {
        const int tt = i / RK, kk = i - tt * RK;
        xs[tt * RK + kk] = xn[(size_t)row_token[row_g + tt] * D + k_start + kk];
    }
    __syncthreads();

    float acc[TG][32];
    float macc[TG][2];
#pragma unroll
    for (int tt = 0; tt < TG; ++tt) {
#pragma unroll
        for (int u = 0; u < 32; ++u) acc[tt][u] = 0.0f;
        macc[tt][0] = 0.0f;
        macc[tt][1] = 0.0f;
    }
    const uint8_t *base = (m ? up : gate) + (size_t)(e * NB + bc) * (size_t)D * ORN_Q4K_BYTES;
    const int n_it = RK / (4 * RW);
#pragma unroll 2
    for (int it = 0; it < n_it; ++it) {
        const int rho = (it * 4 + wave) * RW + rr;
        const uint8_t *blk = base + (size_t)(k_start + rho) * ORN_Q4K_BYTES;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qv = *reinterpret_cast<const uint4 *>(blk + ORN_Q4K_OFF_QS + 16 * j);
        const float d = orn_half_to_float(hd.x & 0xFFFFu);
        const float dmin = orn_half_to_float(hd.x >> 16);
        uint32_t sc1, m1, sc2, m2;
        orn_scale_min_k4(2 * c, hd.y, hd.z, hd.w, sc1, m1);
        orn_scale_min_k4(2 * c + 1, hd.y, hd.z, hd.w, sc2, m2);
        const float D1 = d * (float)sc1, M1 = dmin * (float)m1;
        const float D2 = d * (float)sc2, M2 = dmin * (float)m2;
        const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
        float qlo[16], qhi[16];
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const uint32_t lo = qw[dw] & 0x0F0F0F0Fu;
            const uint32_t hi = (qw[dw] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                qlo[dw * 4 + b] = (float)((lo >> (8 * b)) & 0xFFu);
                qhi[dw * 4 + b] = (float)((hi >> (8 * b)) & 0xFFu);
            }
        }
#pragma unroll
        for (int tt = 0; tt < TG; ++tt) {
            const float xv = xs[tt * RK + rho];
            const float a1 = xv * D1, a2 = xv * D2;
            macc[tt][0] = fmaf(xv, M1, macc[tt][0]);
            macc[tt][1] = fmaf(xv, M2, macc[tt][1]);
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                acc[tt][u] = fmaf(a1, qlo[u], acc[tt][u]);
                acc[tt][16 + u] = fmaf(a2, qhi[u], acc[tt][16 + u]);
            }
        }
    }
    // Finish per lane, then reduce over the RW rows of the wave (butterfly)
    // and over the 4 waves in a fixed order through LDS.
#pragma unroll
    for (int tt = 0; tt < TG; ++tt) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            acc[tt][u] -= macc[tt][0];
            acc[tt][16 + u] -= macc[tt][1];
        }
    }
    for (int off = CR; off < 64; off <<= 1) {
#pragma unroll
        for (int tt = 0; tt < TG; ++tt)
#pragma unroll
            for (int u = 0; u < 32; ++u) acc[tt][u] += __shfl_xor(acc[tt][u], off, 64);
    }
    const int col0 = m * H + bc * 256 + 64 * c + 16 * (j & 1);
    for (int wv = 0; wv < 4; ++wv) {
        if (wave == wv && rr == 0) {
#pragma unroll
            for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    float *p0 = red + tt * H2 + col0 + u;
                    float *p1 = p0 + 32;
                    if (wv == 0) { *p0 = acc[tt][u]; *p1 = acc[tt][16 + u]; }
                    else { *p0 += acc[tt][u]; *p1 += acc[tt][16 + u]; }
                }
        }
        __syncthreads();
    }
    for (int i = tid; i < TG * H2; i += blockDim.x) {
        const int tt = i / H2, col = i - tt * H2;
        gu_part[((size_t)kslice * rows_max + row_g + tt) * H2 + col] = red[i];
    }
    __syncthreads();
}

__global__ void __launch_bounds__(256)
    k_gateup(const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up,
             const float *__restrict__ xn, const int *__restrict__ ctl,
             const int4 *__restrict__ items, const int *__restrict__ slot_expert,
             const int *__restrict__ row_token, float *__restrict__ gu_part, int D, int H, int ks,
             int rows_max)
{
    extern __shared__ float smem[];
    const int item = blockIdx.x / ks, kslice = blockIdx.x - item * ks;
    if (item >= ctl[1]) return;
    const int4 it = items[item];
    const int e = slot_expert[it.x];
    const int RK = D / ks;
    float *xs = smem;
    float *red = smem + ORN_TG_MAX * RK;
    int g = 0;
    while (g < it.z) {
        const int left = it.z - g;
        if (left >= 4) {
            gateup_group<4>(gate, up, xn, row_token, gu_part, D, H, e, it.y + g, kslice, RK,
                            rows_max, xs, red);
            g += 4;
        } else if (left >= 2) {
            gateup_group<2>(gate, up, xn, row_token, gu_part, D, H, e, it.y + g, kslice, RK,
                            rows_max, xs, red);
            g += 2;
        } else {
            gateup_group<1>(gate, up, xn, row_token, gu_part, D, H, e, it.y + g, kslice, RK,
                            rows_max, xs, red);
            g += 1;
        }
    }
}

// ---------------------------------------------------------------------------
// mid[row] = act(sum_ks gate) * sum_ks up.  Rows [0, T) are the shared
// expert's (unclamped silu); all others are routed (clamped silu).
// ---------------------------------------------------------------------------
__global__ void k_mid(const float *__restrict__ gu_part, const int *__restrict__ ctl,
                      float *__restrict__ mid, int H, int ks, int rows_max, int shared_rows)
{
    const int r = blockIdx.x;
    if (r >= ctl[2]) return;
    const int H2 = 2 * H;
    for (int h = threadIdx.x; h < H; h += blockDim.x) {
        float g = 0.0f, u = 0.0f;
        for (int s = 0; s < ks; ++s) {
            const float *p = gu_part + ((size_t)s * rows_max + r) * H2;
            g += p[h];
            u += p[H + h];
        }
        float act;
        if (r < shared_rows) {
            act = g / (1.0f + expf(-g));
        } else {
            if (g < -50.0f) act = 0.0f;
            else if (g > 50.0f) act = g;
            else act = g / (1.0f + expf(-g));
        }
        mid[(size_t)r * H + h] = act * u;
    }
}

// ---------------------------------------------------------------------------
// Down: split-K over the H rows, block = 4 waves, columns in groups of up to
// 8 block columns (2048 outputs).  Q6_K lane chunk lc = (n, jj, half of l):
// ql bytes 64n + 32jj + l0 .. +15 and qh bytes 32n + l0 .. +15 give outputs
// 128n + 32j + l0 + u for j = jj (low nibble, qh bits 2jj) and j = jj+2 (high
// nibble, qh bits 2jj+4), scales sc[8n + l0/16 + 2j] (gguf.c:64-86).  The
// "-32" offset is folded: sum a*(q-32) = sum a*q - 32*sum a.
// ---------------------------------------------------------------------------
template <int TG>
__device__ void down_group(const uint8_t *__restrict__ body, const uint16_t *__restrict__ dsc,
                           const float *__restrict__ mid, float *__restrict__ dn_part, int D, int H,
                           int e, int row_g, int kslice, int RH, int cg, int rows_max, float *ms,
                           float *red)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NBD = D >> 8;
    const int CR = 8 * NBD;
    const int CRg = CR < 64 ? CR : 64;
    const int RW = 64 / CRg;
    const int rr = lane / CRg, ch = lane % CRg;
    const int bc = cg * 8 + (ch >> 3), lc = ch & 7;
    const int n = lc >> 2, jj = (lc >> 1) & 1, l0 = (lc & 1) * 16;
    const int h_start = kslice * RH;
    const int ncols = CRg * 32;  // outputs of this column group

    for (int i = tid; i < TG * RH; i += blockDim.x) {
        const int tt = i / RH, hh = i - tt * RH;
        ms[tt * RH + hh] = mid[(size_t)(row_g + tt) * H + h_start + hh];
    }
    __syncthreads();

    float acc[TG][32];
    float csum[TG][2];
#pragma unroll
    for (int tt = 0; tt < TG; ++tt) {
#pragma unroll
        for (int u = 0; u < 32; ++u) acc[tt][u] = 0.0f;
        csum[tt][0] = 0.0f;
        csum[tt][1] = 0.0f;
    }
    const size_t bcol = (size_t)(e * NBD + bc) * (size_t)H;
    const int pos = (l0 >> 4) + 2 * jj;
    const int n_it = RH / (4 * RW);
#pragma unroll 2
    for (int it = 0; it < n_it; ++it) {
        const int rho = (it * 4 + wave) * RW + rr;
        const size_t bi = bcol + (size_t)(h_start + rho);
        const uint8_t *b = body + bi * 208;
        const uint4 qlv = *reinterpret_cast<const uint4 *>(b + 64 * n + 32 * jj + l0);
        const uint4 qhv = *reinterpret_cast<const uint4 *>(b + 128 + 32 * n + l0);
        const uint4 scv = *reinterpret_cast<const uint4 *>(b + 192);
        const float d = orn_half_to_float(dsc[bi]);
        const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
        const int sa = (int)(int8_t)orn_byte(scw[2 * n], pos);
        const int sb = (int)(int8_t)orn_byte(scw[2 * n + 1], pos);
        const float da = d * (float)sa, db = d * (float)sb;
        const uint32_t lw[4] = {qlv.x, qlv.y, qlv.z, qlv.w};
        const uint32_t hw[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
        float q0[16], q1[16];
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const uint32_t a0 = (lw[dw] & 0x0F0F0F0Fu) | (((hw[dw] >> (2 * jj)) & 0x03030303u) << 4);
            const uint32_t a1 =
                ((lw[dw] >> 4) & 0x0F0F0F0Fu) | (((hw[dw] >> (2 * jj + 4)) & 0x03030303u) << 4);
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                q0[dw * 4 + bb] = (float)((a0 >> (8 * bb)) & 0xFFu);
                q1[dw * 4 + bb] = (float)((a1 >> (8 * bb)) & 0xFFu);
            }
        }
#pragma unroll
        for (int tt = 0; tt < TG; ++tt) {
            const float xv = ms[tt * RH + rho];
            const float aa = xv * da, ab = xv * db;
            csum[tt][0] += aa;
            csum[tt][1] += ab;
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                acc[tt][u] = fmaf(aa, q0[u], acc[tt][u]);
                acc[tt][16 + u] = fmaf(ab, q1[u], acc[tt][16 + u]);
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < TG; ++tt) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            acc[tt][u] = fmaf(-32.0f, csum[tt][0], acc[tt][u]);
            acc[tt][16 + u] = fmaf(-32.0f, csum[tt][1], acc[tt][16 + u]);
        }
    }
    for (int off = CRg; off < 64; off <<= 1) {
#pragma unroll
        for (int tt = 0; tt < TG; ++tt)
#pragma unroll
            for (int u = 0; u < 32; ++u) acc[tt][u] += __shfl_xor(acc[tt][u], off, 64);
    }
    // Local column of output (n, j, l0+u) inside this column group.
    const int lcol0 = (bc - cg * 8) * 256 + 128 * n + 32 * jj + l0;
    for (int wv = 0; wv < 4; ++wv) {
        if (wave == wv && rr == 0) {
#pragma unroll
            for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    float *p0 = red + tt * ncols + lcol0 + u;
                    float *p1 = p0 + 64;
                    if (wv == 0) { *p0 = acc[tt][u]; *p1 = acc[tt][16 + u]; }
                    else { *p0 += acc[tt][u]; *p1 += acc[tt][16 + u]; }
                }
        }
        __syncthreads();
    }
    const int colbase = cg * 2048;
    for (int i = tid; i < TG * ncols; i += blockDim.x) {
        const int tt = i / ncols, col = i - tt * ncols;
        dn_part[((size_t)kslice * rows_max + row_g + tt) * D + colbase + col] = red[i];
    }
    __syncthreads();
}

__global__ void __launch_bounds__(256)
    k_down(const uint8_t *__restrict__ body, const uint16_t *__restrict__ dsc,
           const float *__restrict__ mid, const int *__restrict__ ctl,
           const int4 *__restrict__ items, const int *__restrict__ slot_expert,
           float *__restrict__ dn_part, int D, int H, int ks, int ncg, int rows_max)
{
    extern __shared__ float smem[];
    const int cg = blockIdx.x % ncg;
    const int rest = blockIdx.x / ncg;
    const int item = rest / ks, kslice = rest - item * ks;
    if (item >= ctl[1]) return;
    const int4 it = items[item];
    const int e = slot_expert[it.x];
    const int RH = H / ks;
    float *ms = smem;
    float *red = smem + ORN_TG_MAX * RH;
    int g = 0;
    while (g < it.z) {
        const int left = it.z - g;
        if (left >= 4) {
            down_group<4>(body, dsc, mid, dn_part, D, H, e, it.y + g, kslice, RH, cg, rows_max, ms,
                          red);
            g += 4;
        } else if (left >= 2) {
            down_group<2>(body, dsc, mid, dn_part, D, H, e, it.y + g, kslice, RH, cg, rows_max, ms,
                          red);
            g += 2;
        } else {
            down_group<1>(body, dsc, mid, dn_part, D, H, e, it.y + g, kslice, RH, cg, rows_max, ms,
                          red);
            g += 1;
        }
    }
}

// ---------------------------------------------------------------------------
// Combine (model.c:1003-1007, 1056-1090, 1142):
//   out = (resid + y_shared) + sum_a w_a * y_a   (selection order, skipped
//   pairs excluded), each y the fixed-order sum of its split-K partials.
// ---------------------------------------------------------------------------
__global__ void k_combine(const float *__restrict__ dn_part, const int *__restrict__ pair_row,
                          const float *__restrict__ w, const float *__restrict__ resid,
                          float *__restrict__ out, int T, int D, int k, int ks, int rows_max,
                          int has_shared)
{
    const int t = blockIdx.x;
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    if (t >= T || c >= D) return;
    float acc = resid ? resid[(size_t)t * D + c] : 0.0f;
    if (has_shared) {
        float y = 0.0f;
        for (int s = 0; s < ks; ++s) y += dn_part[((size_t)s * rows_max + t) * D + c];
        acc = acc + y;
    }
    float routed = 0.0f;
    for (int a = 0; a < k; ++a) {
        const int r = pair_row[t * k + a];
        if (r < 0) continue;
        float y = 0.0f;
        for (int s = 0; s < ks; ++s) y += dn_part[((size_t)s * rows_max + r) * D + c];
        routed += w[t * k + a] * y;
    }
    out[(size_t)t * D + c] = acc + routed;
}

}  // namespace

// ---------------------------------------------------------------------------
extern "C" int ornk_moe_norm(const ornk_moe_args *a, hipStream_t s)
{
    hipLaunchKernelGGL(k_reset_ctl, dim3(1), dim3(64), 0, s, a->ctl);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !a->apply_norm) return err;
    return ornk_rmsnorm(a->xn, a->x, a->norm_w, a->T, a->D, s);
}

extern "C" int ornk_moe_dispatch(const ornk_moe_args *a, hipStream_t s)
{
    if (a->E + 1 > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, a->idx, a->w, a->T, a->k, a->E,
                       a->has_shared, a->ctl, a->slot_expert, a->slot_off, a->slot_cnt,
                       a->row_token, a->pair_row, reinterpret_cast<int4 *>(a->items),
                       a->items_max);
    return hipGetLastError();
}

extern "C" int ornk_moe_gateup(const ornk_moe_args *a, hipStream_t s)
{
    const int NB = a->H / 256;
    if (a->H % 256 || NB < 1 || 16 * NB > 64) return hipErrorInvalidValue;
    const int RW = 64 / (16 * NB);
    const int RK = a->D / a->ks_gu;
    if (a->D % a->ks_gu || RK % (4 * RW)) return hipErrorInvalidValue;
    const size_t shmem = sizeof(float) * (size_t)ORN_TG_MAX * (RK + 2 * a->H);
    if (shmem > 160 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gateup, dim3(a->items_max * a->ks_gu), dim3(256), shmem, s, a->gate, a->up,
                       a->xn, a->ctl, reinterpret_cast<const int4 *>(a->items), a->slot_expert,
                       a->row_token, a->gu_part, a->D, a->H, a->ks_gu, a->rows_max);
    return hipGetLastError();
}

extern "C" int ornk_moe_mid(const ornk_moe_args *a, hipStream_t s)
{
    hipLaunchKernelGGL(k_mid, dim3(a->rows_max), dim3(256), 0, s, a->gu_part, a->ctl, a->mid, a->H,
                       a->ks_gu, a->rows_max, a->has_shared ? a->T : 0);
    return hipGetLastError();
}

extern "C" int ornk_moe_down(const ornk_moe_args *a, hipStream_t s)
{
    const int NBD = a->D / 256;
    if (a->D % 256 || NBD < 1) return hipErrorInvalidValue;
    const int CR = 8 * NBD;
    const int CRg = CR < 64 ? CR : 64;
    if (CR > 64 && CR % 64) return hipErrorInvalidValue;
    const int ncg = CR > 64 ? CR / 64 : 1;
    const int RW = 64 / CRg;
    const int RH = a->H / a->ks_dn;
    if (a->H % a->ks_dn || RH % (4 * RW)) return hipErrorInvalidValue;
    const size_t shmem = sizeof(float) * (size_t)ORN_TG_MAX * (RH + CRg * 32);
    if (shmem > 160 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_down, dim3(a->items_max * a->ks_dn * ncg), dim3(256), shmem, s,
                       a->down_body, a->down_d, a->mid, a->ctl,
                       reinterpret_cast<const int4 *>(a->items), a->slot_expert, a->dn_part, a->D,
                       a->H, a->ks_dn, ncg, a->rows_max);
    return hipGetLastError();
}

extern "C" int ornk_moe_combine(const ornk_moe_args *a, hipStream_t s)
{
    hipLaunchKernelGGL(k_combine, dim3(a->T, (a->D + 255) / 256), dim3(256), 0, s, a->dn_part,
                       a->pair_row, a->w, a->resid, a->out, a->T, a->D, a->k, a->ks_dn, a->rows_max,
                       a->has_shared);
    return hipGetLastError();
}
