// SPDX-License-Identifier: MIT
//
// Router logits and top-k selection with the reference's exact semantics.
//
// Reference arithmetic (model.c:1017-1025): logit[e] is a SEQUENTIAL fp32 sum,
// from 0.0f, of the fp32 products x[d]*W[d*E+e], d ascending.  Selection is
// exchange selection with strict '>' (model.c:301-305 / 1040-1048).
//
// A sequential 2048-long dependent chain per logit is too slow to be the
// default path, so the MoE path runs a CERTIFIED parallel computation:
//
//   * k_router_part: the same fp32 products, summed in fp64 over chunks of
//     ORN_RCHUNK rows, plus Q = sum over the chunk of |local prefix sum|.
//   * k_topk_cert:   combines chunks into P~ (~exact sum of the products) and
//     A' >= sum_k |P_k| (exact prefix sums, by the triangle inequality over
//     chunk carries).  The reference's sequential result differs from the
//     exact sum by at most u*sum_k|S_k| <= u*A/(1-n*u) (u = 2^-24), so every
//     reference logit lies in [P~ - B, P~ + B] with B = 1.01*u*A' (+ the bias
//     add's rounding).  If the top-k intervals are pairwise disjoint and lie
//     above every other interval, the reference's ordered top-k equals ours
//     and it has no ties, so exchange selection equals sorting.
//   * otherwise (near-ties, NaN/Inf) the block recomputes the token's logits
//     with the reference's sequential chain and selects on them exactly,
//     falling back to a literal exchange-selection simulation when ties are
//     present.
#include "common.h"
#include "launch.h"

#include <float.h>
#include <limits.h>

#define ORN_RCHUNK 128  // rows per certified chunk
#define ORN_TOPK_THREADS 256

namespace {

constexpr double kU = 5.9604644775390625e-08;  // 2^-24

// ---------------------------------------------------------------------------
// Exact sequential logits (reference arithmetic); W(d, e) = W[d*sd + e*se].
// ---------------------------------------------------------------------------
__global__ void k_router_exact(const float *x, const float *W, long long sd, long long se,
                               const float *bias, int T, int D, int E, float *logits)
{
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    const int t = blockIdx.y;
    if (e >= E || t >= T) return;
    const float *xr = x + (size_t)t * D;
    const float *w = W + (long long)e * se;
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc += xr[d] * w[(long long)d * sd];
    if (bias) acc += bias[e];
    logits[(size_t)t * E + e] = acc;
}

// ---------------------------------------------------------------------------
// Certified partial sums.  Wt is the router transposed, [E][D] (d fastest), so
// each lane streams its expert's column with 16-byte loads.  grid: (E/64,
// n_groups, ceil(T/TB)); block: 64*cpb threads, one wave per chunk of the
// group.  Output part[(t*E + e)*n_groups + g] = (sum, A_group) in fp64, where
// A_group bounds sum_{k in group} |prefix_k| with prefixes restarted at the
// group start.
// ---------------------------------------------------------------------------
template <int TB>
__global__ void k_router_part(const float *__restrict__ x, const float *__restrict__ Wt, int T,
                              int D, int E, int cpb, double2 *__restrict__ part, int *ctl)
{
    __shared__ double s_sum[4][TB][64];
    __shared__ double s_q[4][TB][64];
    __shared__ float xs[TB][4 * ORN_RCHUNK];
    const int lane = threadIdx.x & 63;
    const int c = threadIdx.x >> 6;           // chunk within group
    const int e = blockIdx.x * 64 + lane;
    const int g = blockIdx.y;
    const int n_groups = gridDim.y;
    const int t0 = blockIdx.z * TB;
    const int rows = cpb * ORN_RCHUNK;
    const int dg = g * rows;
    const bool live = e < E;

    // The first block clears the per-forward counters (routing is the
    // first step of every forward).
    if (ctl && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x < 16)
        ctl[threadIdx.x] = 0;
    for (int i = threadIdx.x; i < TB * rows; i += blockDim.x) {
        const int tt = i / rows, r = i - tt * rows;
        xs[tt][r] = (t0 + tt < T) ? x[(size_t)(t0 + tt) * D + dg + r] : 0.0f;
    }
    __syncthreads();

    double S[TB], Q[TB];
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) { S[tt] = 0.0; Q[tt] = 0.0; }

    if (live) {
        const float4 *wp = reinterpret_cast<const float4 *>(Wt + (size_t)e * D + dg + c * ORN_RCHUNK);
        const float *xc = &xs[0][c * ORN_RCHUNK];
        for (int i0 = 0; i0 < ORN_RCHUNK / 4; i0 += 8) {
            float4 wv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) wv[u] = wp[i0 + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float wr[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int d = (i0 + u) * 4 + r;
#pragma unroll
                    for (int tt = 0; tt < TB; ++tt) {
                        const float p = xc[tt * 4 * ORN_RCHUNK + d] * wr[r];
                        S[tt] += (double)p;
                        Q[tt] += fabs(S[tt]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) { s_sum[c][tt][lane] = S[tt]; s_q[c][tt][lane] = Q[tt]; }
    __syncthreads();
    if (c == 0 && live) {
#pragma unroll
        for (int tt = 0; tt < TB; ++tt) {
            if (t0 + tt >= T) continue;
            double carry = 0.0, A = 0.0;
            for (int cc = 0; cc < cpb; ++cc) {
                A += (double)ORN_RCHUNK * fabs(carry) + s_q[cc][tt][lane];
                carry += s_sum[cc][tt][lane];
            }
            part[((size_t)(t0 + tt) * E + e) * n_groups + g] = make_double2(carry, A);
        }
    }
}

// ---------------------------------------------------------------------------
// Block-wide argmax over (value desc, index asc).  Invalid entries carry
// index INT_MAX so that any valid entry wins ties against them.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(double va, int ia, double vb, int ib)
{
    return va > vb || (va == vb && ia < ib);
}

template <int NW>
__device__ void block_argmax(double v, int i, double *sv, int *si, double &ov, int &oi)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        double v2 = __shfl_xor(v, off, 64);
        int i2 = __shfl_xor(i, off, 64);
        if (better(v2, i2, v, i)) { v = v2; i = i2; }
    }
    if (lane == 0) { sv[wave] = v; si[wave] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        double bv = sv[0];
        int bi = si[0];
        for (int w = 1; w < NW; ++w)
            if (better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
        sv[NW] = bv;
        si[NW] = bi;
    }
    __syncthreads();
    ov = sv[NW];
    oi = si[NW];
    __syncthreads();
}

__device__ __forceinline__ float block_sum_f(float v, float *red)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = orn_wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < nw; ++w) s += red[w];
    __syncthreads();
    return s;
}

// Exact selection on fp32 values held one per thread (thread e <-> entry e,
// e < n), with the reference's exchange semantics.  Returns the first k
// entries in sel_i/sel_v (shared).  Uses the fast sorted path when the top
// k+1 values are pairwise distinct and no NaN exists anywhere; otherwise runs
// the literal exchange selection on a single lane.
template <int NW>
__device__ void exact_select(float val, int n, int k, float *vals_s, int *idx_s, double *sv, int *si,
                             int *sel_i, float *sel_v, int *flag_s)
{
    const int e = threadIdx.x;
    const bool valid = e < n;
    if (threadIdx.x == 0) *flag_s = 0;
    __syncthreads();
    if (valid && isnan(val)) *flag_s = 1;
    if (valid) { vals_s[e] = val; idx_s[e] = e; }
    __syncthreads();
    bool slow = *flag_s != 0;
    if (!slow) {
        bool taken = false;
        double prev = 0.0;
        int kk = k < n ? k + 1 : k;  // also look at the (k+1)-th value
        for (int r = 0; r < kk; ++r) {
            double bv;
            int bi;
            block_argmax<NW>((valid && !taken) ? (double)val : -HUGE_VAL,
                             (valid && !taken) ? e : INT_MAX, sv, si, bv, bi);
            if (e == bi) taken = true;
            if (r > 0 && bv == prev) slow = true;  // tie among the top k+1
            if (r < k && threadIdx.x == 0) { sel_i[r] = bi; sel_v[r] = (float)bv; }
            prev = bv;
        }
        __syncthreads();
    }
    if (slow) {
        if (threadIdx.x == 0) {
            // k passes of exchange selection (model.c:1040-1048).
            for (int i = 0; i < k && i < n - 1; ++i)
                for (int j = i + 1; j < n; ++j)
                    if (vals_s[j] > vals_s[i]) {
                        float ft = vals_s[i]; vals_s[i] = vals_s[j]; vals_s[j] = ft;
                        int it = idx_s[i]; idx_s[i] = idx_s[j]; idx_s[j] = it;
                    }
            for (int i = 0; i < k; ++i) { sel_i[i] = idx_s[i]; sel_v[i] = vals_s[i]; }
        }
        __syncthreads();
    }
}

// Renormalised weights over the selected logits (model.c:307-317).
__device__ void renorm_weights(const float *sel_v, int k, float *w)
{
    const float mx = sel_v[0];
    float s[64];
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) { s[i] = expf(sel_v[i] - mx); sum += s[i]; }
    for (int i = 0; i < k; ++i) w[i] = s[i] / sum;
}

// ---------------------------------------------------------------------------
// The reference's sequential logits (model.c:1017-1025) for the experts in
// list[0..n): products rounded to fp32, added in d order from 0.0f, then the
// optional bias; results in lf[e].  The weight rows of up to `cb` experts at
// a time are first copied into LDS by the whole block (every load in
// flight at once), then one thread per expert runs its dependent chain out
// of LDS.  xs holds x (D floats); rows has room for cb*D floats.
// ---------------------------------------------------------------------------
__device__ void exact_logits(const int *list, int n, const float *xs, float *rows, int cb,
                             const float *__restrict__ Wt, const float *bias, int D, float *lf)
{
    const int q = D / 4;
    for (int b0 = 0; b0 < n; b0 += cb) {
        const int nb = min(cb, n - b0);
        float4 *r4 = reinterpret_cast<float4 *>(rows);
        for (int i = threadIdx.x; i < nb * q; i += blockDim.x) {
            const int r = i / q, c = i - r * q;
            r4[i] = reinterpret_cast<const float4 *>(Wt + (size_t)list[b0 + r] * D)[c];
        }
        __syncthreads();
        if ((int)threadIdx.x < nb) {
            const int e = list[b0 + threadIdx.x];
            const float4 *w = r4 + (size_t)threadIdx.x * q;
            const float4 *x4 = reinterpret_cast<const float4 *>(xs);
            float acc = 0.0f;
            for (int i = 0; i < q; ++i) {
                const float4 wv = w[i], xv = x4[i];
                acc += xv.x * wv.x;
                acc += xv.y * wv.y;
                acc += xv.z * wv.z;
                acc += xv.w * wv.w;
            }
            if (bias) acc += bias[e];
            lf[e] = acc;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Certified top-k, one block per token (E <= 256).
//
//  1. Every reference logit lies in [v - B, v + B] (v = P~ + bias).
//  2. If the k best intervals are disjoint from each other and from all
//     other intervals, the reference's ordered top-k is ours: done.
//  3. Otherwise only experts whose interval reaches tau = min over our top-k
//     of (v - B) can be in the reference's top-k (k experts provably have
//     reference values >= tau).  Their exact sequential logits are computed;
//     if the best k+1 of those are pairwise distinct, the reference's top-k
//     is their order by value (exchange selection sorts when there are no
//     ties), since every other expert is strictly below tau.
//  4. Exact ties (or NaN/Inf) are resolved by computing every expert's exact
//     logit and running the literal exchange selection.
// In the literal mode (selection on softmax probabilities) step 3 also
// requires the candidates' logits to be at least 1e-5 apart: probabilities
// then differ by a relative 1e-5, far more than the few ulps by which expf
// and the division can move them, so they cannot round to equal values;
// otherwise step 4 runs, with this device's expf.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(ORN_TOPK_THREADS)
    k_topk_cert(const double2 *__restrict__ part, int n_groups, int rows_per_group,
                const float *__restrict__ x, const float *__restrict__ Wt,
                const float *__restrict__ bias, int D, int E, int k, int mode, uint32_t *idx_out,
                float *w_out, int *n_exact, int cb)
{
    constexpr int NW = ORN_TOPK_THREADS / 64;
    __shared__ double sv[NW + 1];
    __shared__ int si[NW + 1];
    __shared__ double top_v[17], top_b[17];
    __shared__ int sel_i[16];
    __shared__ float sel_v[16];
    __shared__ float vals_s[ORN_TOPK_THREADS];
    __shared__ int idx_s[ORN_TOPK_THREADS];
    __shared__ float red[NW];
    __shared__ int flag_s, cert_s;
    __shared__ float w_s[16];
    __shared__ float lg_s[ORN_TOPK_THREADS];
    __shared__ float lf_s[ORN_TOPK_THREADS];
    __shared__ int list_s[ORN_TOPK_THREADS];
    __shared__ int n_list_s;
    __shared__ float sum_s;
    extern __shared__ float dyn[];  // x (D floats) then cb weight rows

    const int t = blockIdx.x;
    const int e = threadIdx.x;
    const bool valid = e < E;

    // 1. Combine chunk groups: value v = P~ (+bias), bound B.
    double v = -HUGE_VAL, B = 0.0;
    bool finite = true;
    if (valid) {
        double carry = 0.0, A = 0.0;
        const double2 *pp = part + ((size_t)t * E + e) * n_groups;
        for (int g = 0; g < n_groups; ++g) {
            const double2 q = pp[g];
            A += (double)rows_per_group * fabs(carry) + q.y;
            carry += q.x;
        }
        B = 1.01 * kU * A + 1e-37;
        v = carry;
        if (bias) {
            v = carry + (double)bias[e];
            B = B * (1.0 + kU) + 1.01 * kU * (fabs(v) + B);
        }
        finite = isfinite(v) && isfinite(B);
    }
    if (threadIdx.x == 0) { flag_s = 0; cert_s = 1; }
    __syncthreads();
    if (!finite) flag_s = 1;
    __syncthreads();
    const bool all_finite = (flag_s == 0);

    double wv = v;         // value used for the literal-mode weights
    bool cand_s = false;   // this expert's exact logit was computed (step 3)

    // 2. top-k by (v desc, e asc) and the certification test.
    bool taken = false;
    bool certified = all_finite;
    if (all_finite) {
        for (int r = 0; r < k; ++r) {
            double bv;
            int bi;
            block_argmax<NW>((valid && !taken) ? v : -HUGE_VAL, (valid && !taken) ? e : INT_MAX, sv,
                             si, bv, bi);
            if (e == bi) { taken = true; top_v[r] = v; top_b[r] = B; sel_i[r] = e; }
        }
        __syncthreads();
        double hi_rest;
        int who;
        block_argmax<NW>((valid && !taken) ? v + B : -HUGE_VAL, (valid && !taken) ? e : INT_MAX, sv,
                         si, hi_rest, who);
        if (threadIdx.x == 0) {
            bool ok = true;
            double m = (who == INT_MAX) ? -HUGE_VAL : hi_rest;
            for (int r = k - 1; r >= 0 && ok; --r) {
                if (!(top_v[r] - top_b[r] > m)) ok = false;
                m = fmax(m, top_v[r] + top_b[r]);
            }
            cert_s = ok ? 1 : 0;
        }
        __syncthreads();
        certified = cert_s != 0;
    }

    if (certified) {
        if (threadIdx.x < k) sel_v[threadIdx.x] = (float)top_v[threadIdx.x];
        __syncthreads();
    } else {
        if (threadIdx.x == 0 && n_exact) atomicAdd(n_exact, 1);
        float *xs = dyn;
        float *rows = dyn + D;
        for (int i = threadIdx.x; i < D; i += blockDim.x) xs[i] = x[(size_t)t * D + i];
        if (threadIdx.x == 0) { flag_s = all_finite ? 0 : 1; n_list_s = 0; }
        __syncthreads();
        bool resolved = false;
        if (all_finite) {
            // 3. Exact logits for the candidate set only.
            double tau = HUGE_VAL;
            for (int r = 0; r < k; ++r) tau = fmin(tau, top_v[r] - top_b[r]);
            const bool cand = valid && (v + B >= tau);
            cand_s = cand;
            if (cand) list_s[atomicAdd(&n_list_s, 1)] = e;
            __syncthreads();
            exact_logits(list_s, n_list_s, xs, rows, cb, Wt, bias, D, lf_s);
            const float lf = cand ? lf_s[e] : 0.0f;
            if (cand && !isfinite(lf)) flag_s = 1;
            __syncthreads();
            if (flag_s == 0) {
                bool tk = false, tie = false;
                double prev = 0.0;
                for (int r = 0; r <= k; ++r) {
                    double bv;
                    int bi;
                    block_argmax<NW>((cand && !tk) ? (double)lf : -HUGE_VAL,
                                     (cand && !tk) ? e : INT_MAX, sv, si, bv, bi);
                    if (bi == INT_MAX) break;  // fewer than k+1 candidates
                    if (e == bi) tk = true;
                    if (r > 0) {
                        const double gap = prev - bv;
                        if (!(gap > 0.0)) tie = true;
                        if (mode == 1 && !(gap > 1e-5)) tie = true;
                    }
                    if (r < k && threadIdx.x == 0) { sel_i[r] = bi; sel_v[r] = (float)bv; }
                    prev = bv;
                }
                resolved = !tie;
            }
            __syncthreads();
            if (resolved && cand) wv = (double)lf;
        }
        if (!resolved) {
            // 4. Every expert's exact logit, literal exchange selection.
            if (threadIdx.x == 0) n_list_s = E;
            if (valid) list_s[e] = e;
            __syncthreads();
            exact_logits(list_s, E, xs, rows, cb, Wt, bias, D, lf_s);
            const float lf = valid ? lf_s[e] : 0.0f;
            wv = (double)lf;
            float sel_val = lf;
            if (mode == 1) {
                if (threadIdx.x == 0) {
                    float mx = lf_s[0];
                    for (int j = 1; j < E; ++j) if (lf_s[j] > mx) mx = lf_s[j];
                    float sacc = 0.0f;
                    for (int j = 0; j < E; ++j) { lg_s[j] = expf(lf_s[j] - mx); sacc += lg_s[j]; }
                    sum_s = sacc;
                }
                __syncthreads();
                if (valid) sel_val = lg_s[e] / sum_s;
                __syncthreads();
            }
            exact_select<NW>(sel_val, E, k, vals_s, idx_s, sv, si, sel_i, sel_v, &flag_s);
            if (mode == 1) {
                // Selection ran on the probabilities, which are the weights.
                if (threadIdx.x < k) {
                    idx_out[(size_t)t * k + threadIdx.x] = (uint32_t)sel_i[threadIdx.x];
                    w_out[(size_t)t * k + threadIdx.x] = sel_v[threadIdx.x];
                }
                return;
            }
        }
    }

    // Weights.  Renormalised mode: softmax over the k selected logits
    // (model.c:307-317).  Literal mode: full softmax probabilities.
    if (mode == 0) {
        if (threadIdx.x == 0) renorm_weights(sel_v, k, w_s);
        __syncthreads();
    } else {
        const float mx = sel_v[0];
        float ex = valid ? expf((float)wv - mx) : 0.0f;
        float sum = block_sum_f(ex, red);
        if (valid) vals_s[e] = ex / sum;
        __syncthreads();
        if (threadIdx.x < k) w_s[threadIdx.x] = vals_s[sel_i[threadIdx.x]];
        __syncthreads();
    }
    if (threadIdx.x < k) {
        idx_out[(size_t)t * k + threadIdx.x] = (uint32_t)sel_i[threadIdx.x];
        w_out[(size_t)t * k + threadIdx.x] = w_s[threadIdx.x];
    }
}

// ---------------------------------------------------------------------------
// Exact top-k from given fp32 logits (gpu_topk_softmax and E > 256), one
// block of 1024 threads per token, n <= 1024.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
    k_topk_exact(const float *logits, int n, int k, int mode, uint32_t *idx_out, float *w_out,
                 int *n_exact)
{
    constexpr int NW = 16;
    __shared__ double sv[NW + 1];
    __shared__ int si[NW + 1];
    __shared__ int sel_i[1024];
    __shared__ float sel_v[1024];
    __shared__ float vals_s[1024];
    __shared__ int idx_s[1024];
    __shared__ float red[NW];
    __shared__ int flag_s;
    __shared__ float lg_s[1024];
    const int t = blockIdx.x;
    const int e = threadIdx.x;
    const bool valid = e < n;
    float val = valid ? logits[(size_t)t * n + e] : 0.0f;
    if (mode == 1) {
        __shared__ float sum_s;
        if (valid) lg_s[e] = val;
        __syncthreads();
        if (threadIdx.x == 0) {
            float mx = lg_s[0];
            for (int j = 1; j < n; ++j) if (lg_s[j] > mx) mx = lg_s[j];
            float s = 0.0f;
            for (int j = 0; j < n; ++j) { lg_s[j] = expf(lg_s[j] - mx); s += lg_s[j]; }
            sum_s = s;
        }
        __syncthreads();
        if (valid) val = lg_s[e] / sum_s;
        __syncthreads();
    }
    (void)red;
    exact_select<NW>(val, n, k, vals_s, idx_s, sv, si, sel_i, sel_v, &flag_s);
    if (threadIdx.x == 0) {
        if (n_exact && flag_s) atomicAdd(n_exact, 1);
        if (mode == 0) {
            const float mx = sel_v[0];
            float sum = 0.0f;
            for (int i = 0; i < k; ++i) { lg_s[i] = expf(sel_v[i] - mx); sum += lg_s[i]; }
            for (int i = 0; i < k; ++i) sel_v[i] = lg_s[i] / sum;
        }
    }
    __syncthreads();
    if (threadIdx.x < k) {
        idx_out[(size_t)t * k + threadIdx.x] = (uint32_t)sel_i[threadIdx.x];
        w_out[(size_t)t * k + threadIdx.x] = sel_v[threadIdx.x];
    }
}

}  // namespace

extern "C" int ornk_router_exact(const float *x, const float *W, const float *bias, int T, int D,
                                 int E, float *logits, hipStream_t s)
{
    if (T <= 0 || E <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_router_exact, dim3((E + 63) / 64, T), dim3(64), 0, s, x, W, (long long)E,
                       1LL, bias, T, D, E, logits);
    return hipGetLastError();
}

extern "C" int ornk_topk(const float *logits, int T, int E, int k, int mode, uint32_t *idx,
                         float *w, int *n_exact, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    if (E <= 0 || E > 1024 || k <= 0 || k > E) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_topk_exact, dim3(T), dim3(1024), 0, s, logits, E, k, mode, idx, w,
                       n_exact);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// MoE routing step: certified logits + top-k into a->idx / a->w.
// ---------------------------------------------------------------------------
extern "C" int ornk_moe_route(const ornk_moe_args *a, hipStream_t s)
{
    const int T = a->T, D = a->D, E = a->E;
    if (T <= 0) return hipSuccess;
    if (E > ORN_TOPK_THREADS || a->k > 16 || D % 64 != 0 || D % ORN_RCHUNK != 0)
        return hipErrorInvalidValue;
    const int n_chunks = D / ORN_RCHUNK;
    int cpb = (T <= 32 || n_chunks % 4 != 0) ? 1 : 4;
    const int n_groups = n_chunks / cpb;
    double2 *part = reinterpret_cast<double2 *>(a->rpart);
    const float *xin = a->apply_norm ? a->xn : a->x;
    if (T <= 2) {
        hipLaunchKernelGGL(k_router_part<1>, dim3((E + 63) / 64, n_groups, T), dim3(64 * cpb), 0, s,
                           xin, a->router, T, D, E, cpb, part, a->ctl);
    } else if (T <= 16) {
        hipLaunchKernelGGL(k_router_part<2>, dim3((E + 63) / 64, n_groups, (T + 1) / 2),
                           dim3(64 * cpb), 0, s, xin, a->router, T, D, E, cpb, part, a->ctl);
    } else {
        hipLaunchKernelGGL(k_router_part<4>, dim3((E + 63) / 64, n_groups, (T + 3) / 4),
                           dim3(64 * cpb), 0, s, xin, a->router, T, D, E, cpb, part, a->ctl);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    // Dynamic LDS: x plus cb weight rows for the exact fallback, within 56 KB.
    int cb = (56 * 1024) / (4 * D) - 1;
    if (cb > 8) cb = 8;
    if (cb < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_topk_cert, dim3(T), dim3(ORN_TOPK_THREADS),
                       sizeof(float) * (size_t)D * (size_t)(cb + 1), s, part, n_groups,
                       cpb * ORN_RCHUNK, xin, a->router, a->bias, D, E, a->k, a->mode, a->idx, a->w,
                       a->ctl + 3, cb);
    return hipGetLastError();
}
