// SPDX-License-Identifier: MIT
//
// Routed-MoE expert path on the vector ALUs (few tokens per expert):
// fused Q4_K dequant-matvec for gate+up -> SiLU(gate)*up ->
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
#include "mfma_ops.h"


namespace {

// ---------------------------------------------------------------------------
// Gate+up: split-K over the D input rows.  Block = 4 waves; work item = up
// to `tchunk` token rows of one expert; blockIdx.x = item*ks + kslice.  The
// item's tokens are processed one at a time (weights re-read from L1/L2 for
// the second token), which keeps the register budget near 100 VGPRs.
//
// Lane layout: ch = lane % CR picks (matrix m, block column bc, 32-byte qs
// chunk c) with CR = 8*(H/256) chunks per input row, and rr = lane / CR one
// of RW = 64/CR rows handled side by side.  Chunk c holds qs bytes
// 32c..32c+31: low nibbles are outputs 64c + l of sub-block 2c, high nibbles
// 64c + 32 + l of sub-block 2c+1 (gguf.c:43-61), so the per-row scale work is
// shared by 64 weights.
// With D = d*sc and M = dmin*m a row contributes x_k*(D*q - M); the M part is
// constant over a sub-block, so it is accumulated once per row and
// subtracted at the end.
//
// Memory pipelining: each lane keeps NPF rows of loads in flight in a ring
// of register sets that is fully unrolled (static register indices), and
// the prefetch row index is clamped at the slice end so the loop body has no
// branches.
// ---------------------------------------------------------------------------
#define ORN_NPF 4

__device__ __forceinline__ void q4_nibbles(uint32_t w, float *lo, float *hi)
{
    orn_bytes_to_float(w & 0x0F0F0F0Fu, lo);
    orn_bytes_to_float((w >> 4) & 0x0F0F0F0Fu, hi);
}

struct Q4Row {
    uint4 hd, q0, q1;  // header (d, dmin, scales) and the lane's 32 qs bytes
};

__device__ __forceinline__ void load_q4(const uint8_t *blk, int c, Q4Row &r)
{
    r.hd = *reinterpret_cast<const uint4 *>(blk);
    r.q0 = *reinterpret_cast<const uint4 *>(blk + ORN_Q4K_OFF_QS + 32 * c);
    r.q1 = *reinterpret_cast<const uint4 *>(blk + ORN_Q4K_OFF_QS + 32 * c + 16);
}

// One row of one lane chunk c: qs bytes 32c..32c+31, i.e. the 64 outputs
// 64c + l (low nibbles, sub-block 2c) and 64c + 32 + l (high nibbles,
// sub-block 2c+1), l = 0..31 (gguf.c:43-61).
__device__ __forceinline__ void q4_row(const Q4Row &r, int c, float xv, float *acc, float &macc0,
                                       float &macc1)
{
    const float d = orn_half_to_float(r.hd.x & 0xFFFFu);
    const float dmin = orn_half_to_float(r.hd.x >> 16);
    uint32_t sc1, m1, sc2, m2;
    orn_scale_min_k4(2 * c, r.hd.y, r.hd.z, r.hd.w, sc1, m1);
    orn_scale_min_k4(2 * c + 1, r.hd.y, r.hd.z, r.hd.w, sc2, m2);
    const float a1 = xv * (d * (float)sc1);
    const float a2 = xv * (d * (float)sc2);
    macc0 = fmaf(xv, dmin * (float)m1, macc0);
    macc1 = fmaf(xv, dmin * (float)m2, macc1);
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int dw = 0; dw < 8; ++dw) {
        float lo[4], hi[4];
        q4_nibbles(qw[dw], lo, hi);
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            acc[dw * 4 + bb] = fmaf(a1, lo[bb], acc[dw * 4 + bb]);
            acc[32 + dw * 4 + bb] = fmaf(a2, hi[bb], acc[32 + dw * 4 + bb]);
        }
    }
}

template <int NIT, int RWT>
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
    const int4 itm = items[item];
    const int e = itm.w;  // expert slot index (E = the shared expert)
    const int RK = D / ks;
    float *xs = smem;       // [RK]
    float *red = smem + RK; // [2H]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NB = H >> 8;
    const int CR = 8 * NB;
    const int RW = RWT > 0 ? RWT : 64 / CR;  // RWT == 64 / CR when given (launcher)
    const int rr = lane / CR, ch = lane % CR;
    const int c = ch & 3, bc = (ch >> 2) % NB, m = ch / (4 * NB);
    const int k_start = kslice * RK;
    const int H2 = 2 * H;
    const uint8_t *base =
        (m ? up : gate) + ((size_t)(e * NB + bc) * (size_t)D + (size_t)k_start) * ORN_Q4K_BYTES;
    // Rows per wave, a multiple of ORN_NPF (checked by the launcher).  With
    // compile-time NIT and RWT the ring loop unrolls into straight-line code
    // whose loads are one base address plus immediate offsets.
    const int n_it = NIT > 0 ? NIT : RK / (4 * RW);
    const int last = n_it - 1;
    const int col0 = m * H + bc * 256 + 64 * c;
    const int h0 = wave * RW + rr;      // this lane's first row; row i is h0 + 4*RW*i
    const size_t rstep = (size_t)4 * RW * ORN_Q4K_BYTES;

    for (int r = 0; r < itm.z; ++r) {
        // Opaque zero: keeps the ring's first loads inside this token's pass
        // instead of hoisted (and held in extra registers) across all passes.
        int z = 0;
        asm volatile("" : "+v"(z));
        const uint8_t *lb = base + (size_t)(h0 + z) * ORN_Q4K_BYTES;
        const float *xl = xs + h0;
        // The weights do not depend on the token: start their loads before
        // the activation slice is staged.
        Q4Row rs[ORN_NPF];
#pragma unroll
        for (int p = 0; p < ORN_NPF; ++p) {
            load_q4(lb + (size_t)min(p, last) * rstep, c, rs[p]);
            __builtin_amdgcn_sched_barrier(0);  // issue order = consumption order
        }

        const int row = itm.y + r;
        const float *xr = xn + (size_t)row_token[row] * D + k_start;
        for (int i = tid; i < RK; i += blockDim.x) xs[i] = xr[i];
        __syncthreads();

        float acc[64];
#pragma unroll
        for (int u = 0; u < 64; ++u) acc[u] = 0.0f;
        float macc0 = 0.0f, macc1 = 0.0f;
#pragma unroll
        for (int it = 0; it < n_it; it += ORN_NPF) {
            float xv[ORN_NPF];
#pragma unroll
            for (int p = 0; p < ORN_NPF; ++p) xv[p] = xl[(it + p) * 4 * RW];
#pragma unroll
            for (int p = 0; p < ORN_NPF; ++p) {
                // Use the slot, then refill it in place (the pins keep the
                // refill after the use), ORN_NPF rows ahead.
                orn_pin_u4(rs[p].hd);
                orn_pin_u4(rs[p].q0);
                orn_pin_u4(rs[p].q1);
                q4_row(rs[p], c, xv[p], acc, macc0, macc1);
#pragma unroll
                for (int u = 0; u < 64; u += 8) orn_pin8(acc + u);
                orn_pin2(macc0, macc1);
                load_q4(lb + (size_t)min(it + p + ORN_NPF, last) * rstep, c, rs[p]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            acc[u] -= macc0;
            acc[32 + u] -= macc1;
        }
        for (int off = CR; off < 64; off <<= 1) {
#pragma unroll
            for (int u = 0; u < 64; ++u) acc[u] += __shfl_xor(acc[u], off, 64);
        }
        for (int wv = 0; wv < 4; ++wv) {
            if (wave == wv && rr == 0) {
#pragma unroll
                for (int u = 0; u < 64; ++u) {
                    float *p0 = red + col0 + u;
                    *p0 = (wv == 0) ? acc[u] : *p0 + acc[u];
                }
            }
            __syncthreads();
        }
        float *dst = gu_part + ((size_t)kslice * rows_max + row) * H2;
        for (int i = tid; i < H2; i += blockDim.x) dst[i] = red[i];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// mid[row] = act(sum_ks gate) * sum_ks up.  Rows [0, shared_rows) belong to
// the shared expert (unclamped silu, gpu.c:176-186); all others are routed
// (clamped silu, model.c:340-344).
// ---------------------------------------------------------------------------
// Two kernels, bit-identical (each value sums its split-K partials from 0.0f
// in slice order, then the same activation), chosen by ks as measured:
//
// k_mid_wave: one wave per row (ks <= 2); lane l takes the NG groups of 4
// consecutive values 4*(l + 64i) .. +3 (H = 256*NG), so each load
// instruction of a wave reads 1 KB in one piece, and all of a row's partials
// are in flight together.
//
// With fh (file-orientation stores) the row goes out only as the down
// kernel's activations: hi/lo fp16 of mid * s (s = prep_scale(max |mid|)) in
// the pair order of k_prep_rows (expert_file.hip: the words of a 4-value
// group are the pairs (0, 2) and (1, 3)), and finv[r] = 1/s; the fp32 mid,
// which the file down kernel does not read, is not written.
template <int NG, int KS>
__global__ void __launch_bounds__(64)
    k_mid_wave(const float *__restrict__ gu_part, const int *__restrict__ ctl,
               float *__restrict__ mid, int H, int rows_max, int shared_rows,
               float *__restrict__ row_amax, uint32_t *__restrict__ fh, uint32_t *__restrict__ fl,
               float *__restrict__ finv)
{
    const int lane = threadIdx.x;
    const int r = blockIdx.x;
    if (r >= ctl[2]) return;
    const size_t kstride = (size_t)rows_max * 2 * H;
    const float *p = gu_part + (size_t)r * 2 * H + 4 * lane;
    v4f lg[KS][NG], lu[KS][NG];
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            lg[j][i] = *reinterpret_cast<const v4f *>(p + j * kstride + 256 * i);
            lu[j][i] = *reinterpret_cast<const v4f *>(p + j * kstride + H + 256 * i);
        }
    const bool shared_row = r < shared_rows;
    float amax = 0.0f;
    v4f m[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        v4f g = {0.0f, 0.0f, 0.0f, 0.0f}, u = g;
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            g = g + lg[j][i];
            u = u + lu[j][i];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float gv = g[e];
            float act;
            if (shared_row) {
                act = gv / (1.0f + expf(-gv));
            } else {
                if (gv < -50.0f) act = 0.0f;
                else if (gv > 50.0f) act = gv;
                else act = gv / (1.0f + expf(-gv));
            }
            m[i][e] = act * u[e];
            amax = fmaxf(amax, fabsf(m[i][e]));
        }
        if (!fh) *reinterpret_cast<v4f *>(mid + (size_t)r * H + 4 * lane + 256 * i) = m[i];
    }
    if (!row_amax && !fh) return;
    // max |mid| of the row, for the down step's scaling (order-free)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if (row_amax && lane == 0) row_amax[r] = amax;
    if (fh) {
        const float sc = orn_mfma::prep_scale(amax);
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const v4f a = m[i] * sc;
            uint32_t h0, h1, l0, l1;
            orn_mfma::split2(a.x, a.z, h0, l0);
            orn_mfma::split2(a.y, a.w, h1, l1);
            const size_t o = (size_t)r * (H >> 1) + 2 * lane + 128 * i;  // u32 words
            *reinterpret_cast<uint2 *>(fh + o) = make_uint2(h0, h1);
            *reinterpret_cast<uint2 *>(fl + o) = make_uint2(l0, l1);
        }
        if (lane == 0) finv[r] = 1.0f / sc;
    }
}

// k_mid_wg: one work group per row, a thread per value (ks >= 4).  KMAX > 0
// (= ks): the partials of a value are loaded together, one memory round trip
// per thread; KMAX = 0: any ks, four partials at a time.
template <int KMAX>
__global__ void __launch_bounds__(256)
    k_mid_wg(const float *__restrict__ gu_part, const int *__restrict__ ctl, float *__restrict__ mid,
          int H, int ks, int rows_max, int shared_rows, float *__restrict__ row_amax,
          uint32_t *__restrict__ fh, uint32_t *__restrict__ fl, float *__restrict__ finv)
{
    __shared__ float red[4];
    __shared__ __align__(16) float vrow[2048];  // the row, when fh (H <= 2048)
    const int r = blockIdx.x;
    if (r >= ctl[2]) return;
    float amax = 0.0f;
    const int H2 = 2 * H;
    const size_t kstride = (size_t)rows_max * H2;
    for (int h = threadIdx.x; h < H; h += blockDim.x) {
        const float *p = gu_part + (size_t)r * H2 + h;
        float g = 0.0f, u = 0.0f;
        if (KMAX > 0) {
            float gv[KMAX > 0 ? KMAX : 1], uv[KMAX > 0 ? KMAX : 1];
#pragma unroll
            for (int s = 0; s < KMAX; ++s) {
                const size_t o = (size_t)(s < ks ? s : 0) * kstride;
                gv[s] = p[o];
                uv[s] = p[o + H];
            }
#pragma unroll
            for (int s = 0; s < KMAX; ++s) {
                g = s < ks ? g + gv[s] : g;
                u = s < ks ? u + uv[s] : u;
            }
        } else {
            int s = 0;
            for (; s + 4 <= ks; s += 4) {
                const float g0 = p[(s + 0) * kstride], g1 = p[(s + 1) * kstride];
                const float g2 = p[(s + 2) * kstride], g3 = p[(s + 3) * kstride];
                const float u0 = p[(s + 0) * kstride + H], u1 = p[(s + 1) * kstride + H];
                const float u2 = p[(s + 2) * kstride + H], u3 = p[(s + 3) * kstride + H];
                g += g0; g += g1; g += g2; g += g3;
                u += u0; u += u1; u += u2; u += u3;
            }
            for (; s < ks; ++s) {
                g += p[s * kstride];
                u += p[s * kstride + H];
            }
        }
        float act;
        if (r < shared_rows) {
            act = g / (1.0f + expf(-g));
        } else {
            if (g < -50.0f) act = 0.0f;
            else if (g > 50.0f) act = g;
            else act = g / (1.0f + expf(-g));
        }
        const float v = act * u;
        if (fh) vrow[h] = v;
        else mid[(size_t)r * H + h] = v;
        amax = fmaxf(amax, fabsf(v));
    }
    if (row_amax || fh) {  // max |mid| of the row, for the down step's scaling
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        if (row_amax && threadIdx.x == 0) row_amax[r] = amax;
    }
    if (fh) {
        const int tid = threadIdx.x;
        const float s = orn_mfma::prep_scale(amax);
        if (tid < (H >> 3)) {  // 8 consecutive values a thread, as k_prep_rows
            const v4f a = *reinterpret_cast<const v4f *>(&vrow[8 * tid]) * s;
            const v4f b = *reinterpret_cast<const v4f *>(&vrow[8 * tid + 4]) * s;
            uint32_t hv[4], lv[4];
            orn_mfma::split2(a.x, a.z, hv[0], lv[0]);
            orn_mfma::split2(a.y, a.w, hv[1], lv[1]);
            orn_mfma::split2(b.x, b.z, hv[2], lv[2]);
            orn_mfma::split2(b.y, b.w, hv[3], lv[3]);
            const size_t o = (size_t)r * (H >> 1) + 4 * tid;  // u32 words
            *reinterpret_cast<uint4 *>(fh + o) = make_uint4(hv[0], hv[1], hv[2], hv[3]);
            *reinterpret_cast<uint4 *>(fl + o) = make_uint4(lv[0], lv[1], lv[2], lv[3]);
        }
        if (tid == 0) finv[r] = 1.0f / s;
    }
}

// ---------------------------------------------------------------------------
// Down: split-K over the H rows, block = 4 waves, one token per pass.  Lane
// chunk (block column bc, half n, l0 in {0,16}, jj in {0,1}) covers the 32
// outputs 128n + 32j + l0 + u for j in {jj, jj+2}, u = 0..15: low/high
// nibbles of ql[64n + 32jj + l0 + u] give j = jj / jj+2, qh[32n + l0 + u]
// bits 2j..2j+1 the top two bits, scale sc[8n + l0/16 + 2j] (gguf.c:64-86).
// The "-32" is folded: sum a*(q-32) = sum a*q - 32*sum a.  Loads are
// pipelined ORN_NPF rows deep as in k_gateup.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void q6_decode(uint32_t ql, uint32_t qh, int jj, float *q0, float *q1)
{
    const uint32_t a0 = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * jj)) & 0x03030303u) << 4);
    const uint32_t a1 = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * jj + 4)) & 0x03030303u) << 4);
    orn_bytes_to_float(a0, q0);
    orn_bytes_to_float(a1, q1);
}

template <int NIT, int RWT>
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
    const int4 itm = items[item];
    const int e = itm.w;  // expert slot index (E = the shared expert)
    const int RH = H / ks;
    const int NBD = D >> 8;
    const int CR = 8 * NBD;
    const int CRg = CR < 64 ? CR : 64;
    const int RW = RWT > 0 ? RWT : 64 / CRg;  // RWT == 64 / CRg when given (launcher)
    const int ncols = CRg * 32;   // outputs of this column group
    float *ms = smem;             // [RH]
    float *red = smem + RH;       // [ncols]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rr = lane / CRg, ch = lane % CRg;
    const int bc = cg * 8 + (ch >> 3), lc = ch & 7;
    const int n = lc >> 2, jj = (lc >> 1) & 1, l0 = (lc & 1) * 16;
    const int h_start = kslice * RH;
    const size_t bcol = (size_t)(e * NBD + bc) * (size_t)H + (size_t)h_start;
    const uint8_t *bbase = body + bcol * 208;
    const uint16_t *dbase = dsc + bcol;
    const int n_it = NIT > 0 ? NIT : RH / (4 * RW);  // as in k_gateup
    const int last = n_it - 1;
    const int pos = (l0 >> 4) + 2 * jj;  // byte of the scale dwords 2n (j=jj) and 2n+1 (j=jj+2)
    const int lcol0 = (bc - cg * 8) * 256 + 128 * n + 32 * jj + l0;

    const int h0 = wave * RW + rr;  // this lane's first row; row i is h0 + 4*RW*i
    const int hstep = 4 * RW;

    for (int r = 0; r < itm.z; ++r) {
        // Opaque zero, as in k_gateup: the ring's first loads stay in this pass.
        int z = 0;
        asm volatile("" : "+v"(z));
        const uint8_t *lb = bbase + (size_t)(h0 + z) * 208;
        const uint16_t *ld = dbase + h0 + z;
        const float *ml = ms + h0;
        uint4 qlr[ORN_NPF], qhr[ORN_NPF];
        uint2 scr[ORN_NPF];
        uint32_t dr[ORN_NPF];
#pragma unroll
        for (int p = 0; p < ORN_NPF; ++p) {  // weight loads before the activation staging
            const int hi = min(p, last) * hstep;
            const uint8_t *b = lb + (size_t)hi * 208;
            qlr[p] = *reinterpret_cast<const uint4 *>(b + 64 * n + 32 * jj + l0);
            qhr[p] = *reinterpret_cast<const uint4 *>(b + 128 + 32 * n + l0);
            scr[p] = *reinterpret_cast<const uint2 *>(b + 192 + 8 * n);
            dr[p] = ld[hi];
            __builtin_amdgcn_sched_barrier(0);  // issue order = consumption order
        }

        const int row = itm.y + r;
        const float *mr = mid + (size_t)row * H + h_start;
        for (int i = tid; i < RH; i += blockDim.x) ms[i] = mr[i];
        __syncthreads();

        float acc[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) acc[u] = 0.0f;
        float cs0 = 0.0f, cs1 = 0.0f;
#pragma unroll
        for (int it = 0; it < n_it; it += ORN_NPF) {
            float mv[ORN_NPF];
#pragma unroll
            for (int p = 0; p < ORN_NPF; ++p) mv[p] = ml[(it + p) * hstep];
#pragma unroll
            for (int p = 0; p < ORN_NPF; ++p) {
                orn_pin_u4(qlr[p]);
                orn_pin_u4(qhr[p]);
                asm volatile("" : "+v"(scr[p].x), "+v"(scr[p].y), "+v"(dr[p]));
                const float d = orn_half_to_float(dr[p]);
                const float xv = mv[p];
                const float a0 = xv * (d * (float)(int)(int8_t)orn_byte(scr[p].x, pos));
                const float a1 = xv * (d * (float)(int)(int8_t)orn_byte(scr[p].y, pos));
                cs0 += a0;
                cs1 += a1;
                const uint32_t qlw[4] = {qlr[p].x, qlr[p].y, qlr[p].z, qlr[p].w};
                const uint32_t qhw[4] = {qhr[p].x, qhr[p].y, qhr[p].z, qhr[p].w};
#pragma unroll
                for (int dw = 0; dw < 4; ++dw) {
                    float q0[4], q1[4];
                    q6_decode(qlw[dw], qhw[dw], jj, q0, q1);
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) {
                        acc[dw * 4 + bb] = fmaf(a0, q0[bb], acc[dw * 4 + bb]);
                        acc[16 + dw * 4 + bb] = fmaf(a1, q1[bb], acc[16 + dw * 4 + bb]);
                    }
                }
#pragma unroll
                for (int u = 0; u < 32; u += 8) orn_pin8(acc + u);
                orn_pin2(cs0, cs1);
                const int hi = min(it + p + ORN_NPF, last) * hstep;
                const uint8_t *b = lb + (size_t)hi * 208;
                qlr[p] = *reinterpret_cast<const uint4 *>(b + 64 * n + 32 * jj + l0);
                qhr[p] = *reinterpret_cast<const uint4 *>(b + 128 + 32 * n + l0);
                scr[p] = *reinterpret_cast<const uint2 *>(b + 192 + 8 * n);
                dr[p] = ld[hi];
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            acc[u] = fmaf(-32.0f, cs0, acc[u]);
            acc[16 + u] = fmaf(-32.0f, cs1, acc[16 + u]);
        }
        for (int off = CRg; off < 64; off <<= 1) {
#pragma unroll
            for (int u = 0; u < 32; ++u) acc[u] += __shfl_xor(acc[u], off, 64);
        }
        for (int wv = 0; wv < 4; ++wv) {
            if (wave == wv && rr == 0) {
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    float *p0 = red + lcol0 + u;
                    float *p1 = p0 + 64;
                    *p0 = (wv == 0) ? acc[u] : *p0 + acc[u];
                    *p1 = (wv == 0) ? acc[16 + u] : *p1 + acc[16 + u];
                }
            }
            __syncthreads();
        }
        float *dst = dn_part + ((size_t)kslice * rows_max + row) * D + cg * 2048;
        for (int i = tid; i < ncols; i += blockDim.x) dst[i] = red[i];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Combine (model.c:1003-1007, 1056-1090, 1142):
//   out = (resid + y_shared) + sum_a w_a * y_a   (selection order, skipped
//   pairs excluded), each y the fixed-order sum of its split-K partials.
// ---------------------------------------------------------------------------
// KS = ks (compile time, 1..16) and K = k (8, or 0: any k <= 16): every
// load of a thread is issued before the first add.
// sg (the shared-expert gate, NULL: none): the shared term is scaled by
// sigmoid(sg . xin[t]), the dot formed by every work group of the token in
// the same fixed order (8-strided per thread, then a butterfly per wave and
// the four waves in order).
template <int KS, int K>
__global__ void __launch_bounds__(256)
    k_combine(const float *__restrict__ dn_part, const int *__restrict__ pair_row,
              const float *__restrict__ w, const float *__restrict__ resid,
              float *__restrict__ out, int T, int D, int k, int rows_max, int has_shared,
              const float *__restrict__ sg, const float *__restrict__ xin)
{
    constexpr int KK = K > 0 ? K : 16;
    const int t = blockIdx.x;
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    float gsh = 1.0f;
    if (sg) {  // uniform over the work group
        __shared__ float red[4];
        float p = 0.0f;
        for (int i = threadIdx.x; i < D; i += blockDim.x) p += xin[(size_t)t * D + i] * sg[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) p += __shfl_xor(p, off, 64);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = p;
        __syncthreads();
        const float dot = ((red[0] + red[1]) + red[2]) + red[3];
        gsh = 1.0f / (1.0f + expf(-dot));
    }
    if (t >= T || c >= D) return;
    const int kk = K > 0 ? K : k;
    const size_t kstride = (size_t)rows_max * D;
    int rr[KK];
    float ww[KK];
#pragma unroll
    for (int a = 0; a < KK; ++a) {
        const int ai = a < kk ? a : 0;  // slots past k re-read slot 0, dropped below
        rr[a] = pair_row[t * k + ai];
        ww[a] = w[t * k + ai];
    }
    const float rv = resid ? resid[(size_t)t * D + c] : 0.0f;
    float ysh = 0.0f, y[KK];
#pragma unroll
    for (int a = 0; a < KK; ++a) y[a] = 0.0f;
    // Split-K partials in fixed order, up to four steps of loads at once.
    constexpr int CH = KS < 4 ? KS : 4;
#pragma unroll
    for (int s0 = 0; s0 < KS; s0 += CH) {
        float vs[CH], v[CH][KK];
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const float *base = dn_part + (size_t)(s0 + u) * kstride + c;
            vs[u] = has_shared ? base[(size_t)t * D] : 0.0f;
#pragma unroll
            for (int a = 0; a < KK; ++a) v[u][a] = base[(size_t)(rr[a] < 0 ? 0 : rr[a]) * D];
        }
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            ysh += vs[u];
#pragma unroll
            for (int a = 0; a < KK; ++a) y[a] += v[u][a];
        }
    }
    float acc = rv;
    if (has_shared) acc = acc + gsh * ysh;  // gsh = 1 without a gate: acc + ysh exactly
    float routed = 0.0f;
#pragma unroll
    for (int a = 0; a < KK; ++a)
        if (a < kk && rr[a] >= 0) routed += ww[a] * y[a];
    out[(size_t)t * D + c] = acc + routed;
}

}  // namespace

// ---------------------------------------------------------------------------
extern "C" int ornk_moe_norm(const ornk_moe_args *a, hipStream_t s)
{
    // the decode-sized router normalises its own input (ornk_moe_route)
    if (!a->apply_norm || ornk_router_pc_supported(a->T, a->D)) return hipSuccess;
    return ornk_rmsnorm(a->xn, a->x, a->norm_w, a->T, a->D, s);
}

extern "C" int ornk_moe_gateup(const ornk_moe_args *a, hipStream_t s)
{
    const int NB = a->H / 256;
    if (a->H % 256 || NB < 1 || 64 % (8 * NB)) return hipErrorInvalidValue;
    const int RW = 64 / (8 * NB);
    const int RK = a->D / a->ks_gu;
    if (a->D % a->ks_gu || RK % (4 * RW * ORN_NPF)) return hipErrorInvalidValue;
    const size_t shmem = sizeof(float) * (size_t)(RK + 2 * a->H);
    if (shmem > 64 * 1024) return hipErrorInvalidValue;
    const int n_it = RK / (4 * RW);
#define ORN_GU(N, R)                                                                            \
    ORN_LAUNCH_EV(a, (k_gateup<N, R>), dim3(a->items_max * a->ks_gu), dim3(256), shmem, s, a->gate, \
                       a->up, a->xn, a->ctl, reinterpret_cast<const int4 *>(a->items),          \
                       a->slot_expert, a->row_token, a->gu_part, a->D, a->H, a->ks_gu,          \
                       a->rows_max)
    // Straight-line instances for the Ornith shape (H = 512: RW = 4).
    if (RW == 4 && n_it == 4) ORN_GU(4, 4);
    else if (RW == 4 && n_it == 8) ORN_GU(8, 4);
    else if (RW == 4 && n_it == 16) ORN_GU(16, 4);
    else if (RW == 4 && n_it == 32) ORN_GU(32, 4);
    else ORN_GU(0, 0);
#undef ORN_GU
    return hipGetLastError();
}

extern "C" int ornk_moe_mid(const ornk_moe_args *a, hipStream_t s)
{
    const int H = a->H, ks = a->ks_gu;
    if (H % 256 || H > 1024 || ks < 1) return hipErrorInvalidValue;
    // measured: one wave per row wins at ks <= 2 (prefill: 20.6 against 27.7
    // us), four waves per row at ks >= 4 (7.9 against 9.3 us at 256 skewed
    // tokens, where a wave per row leaves 9 waves per CU)
    const int shared_rows = a->has_shared ? a->T : 0;
    float *amax = a->use_mfma ? a->mid_amax : nullptr;
    const ornk_file_ws &f = a->fw;
    if (ks <= 2) {
#define ORN_MIDW(NG, KS)                                                                      \
    ORN_LAUNCH_EV(a, (k_mid_wave<NG, KS>), dim3(a->rows_max), dim3(64), 0, s, a->gu_part,     \
                  a->ctl, a->mid, H, a->rows_max, shared_rows, amax, f.mh, f.ml, f.minv)
        switch ((H / 256) * 4 + ks) {
        case 4 + 1: ORN_MIDW(1, 1); break;
        case 4 + 2: ORN_MIDW(1, 2); break;
        case 8 + 1: ORN_MIDW(2, 1); break;
        case 8 + 2: ORN_MIDW(2, 2); break;
        case 16 + 1: ORN_MIDW(4, 1); break;
        case 16 + 2: ORN_MIDW(4, 2); break;
        default: return hipErrorInvalidValue;  // H = 768: refused by the store
        }
#undef ORN_MIDW
        return hipGetLastError();
    }
#define ORN_MID(K)                                                                             \
    ORN_LAUNCH_EV(a, k_mid_wg<K>, dim3(a->rows_max), dim3(256), 0, s, a->gu_part, a->ctl,      \
                  a->mid, H, ks, a->rows_max, shared_rows, amax, f.mh, f.ml, f.minv)
    switch (ks) {
    case 4: ORN_MID(4); break;
    case 8: ORN_MID(8); break;
    case 16: ORN_MID(16); break;
    default: ORN_MID(0); break;
    }
#undef ORN_MID
    return hipGetLastError();
}

extern "C" int ornk_moe_down(const ornk_moe_args *a, hipStream_t s)
{
    const int NBD = a->D / 256;
    if (a->D % 256 || NBD < 1) return hipErrorInvalidValue;
    const int CR = 8 * NBD;
    const int CRg = CR < 64 ? CR : 64;
    if (CR > 64 ? CR % 64 : 64 % CR) return hipErrorInvalidValue;
    const int ncg = CR > 64 ? CR / 64 : 1;
    const int RW = 64 / CRg;
    const int RH = a->H / a->ks_dn;
    if (a->H % a->ks_dn || RH % (4 * RW * ORN_NPF)) return hipErrorInvalidValue;
    const size_t shmem = sizeof(float) * (size_t)(RH + CRg * 32);
    if (shmem > 64 * 1024) return hipErrorInvalidValue;
    const int n_it = RH / (4 * RW);
#define ORN_DN(N, R)                                                                             \
    ORN_LAUNCH_EV(a, (k_down<N, R>), dim3(a->items_max * a->ks_dn * ncg), dim3(256), shmem, s,        \
                       a->down_body, a->down_d, a->mid, a->ctl,                                  \
                       reinterpret_cast<const int4 *>(a->items), a->slot_expert, a->dn_part,     \
                       a->D, a->H, a->ks_dn, ncg, a->rows_max)
    // Straight-line instances for the Ornith shape (D = 2048: RW = 1).
    if (RW == 1 && n_it == 4) ORN_DN(4, 1);
    else if (RW == 1 && n_it == 8) ORN_DN(8, 1);
    else if (RW == 1 && n_it == 16) ORN_DN(16, 1);
    else if (RW == 1 && n_it == 32) ORN_DN(32, 1);
    else ORN_DN(0, 0);
#undef ORN_DN
    return hipGetLastError();
}

extern "C" int ornk_moe_combine(const ornk_moe_args *a, hipStream_t s)
{
    const dim3 grid(a->T, (a->D + 255) / 256);
#define ORN_CMB(KS, K)                                                                          \
    ORN_LAUNCH_EV(a, (k_combine<KS, K>), grid, dim3(256), 0, s, a->dn_part, a->pair_row, a->w,  \
                       a->resid, a->out, a->T, a->D, a->k, a->rows_max, a->has_shared,        \
                       a->has_shared ? a->shexp_gate : nullptr, a->xn)
#define ORN_CMB_K(KS)                  \
    if (a->k == 8) ORN_CMB(KS, 8);     \
    else ORN_CMB(KS, 0)
    switch (a->ks_dn) {
    case 1: ORN_CMB_K(1); break;
    case 2: ORN_CMB_K(2); break;
    case 4: ORN_CMB_K(4); break;
    case 8: ORN_CMB_K(8); break;
    case 16: ORN_CMB_K(16); break;
    default: return hipErrorInvalidValue;
    }
#undef ORN_CMB_K
#undef ORN_CMB
    return hipGetLastError();
}
