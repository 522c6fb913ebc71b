// SPDX-License-Identifier: MIT
//
// Router logits and top-k selection with the reference's exact semantics.
//
// Reference arithmetic (model.c:1017-1025): logit[e] is a SEQUENTIAL fp32 sum,
// from 0.0f, of the fp32 products x[d]*W[d*E+e], d ascending.  Selection is
// exchange selection with strict '>' (model.c:301-305 / 1040-1048).
//
// The MoE path computes every logit with exactly that arithmetic, one chain
// per (token, expert), all chains in parallel (k_router_pc for decode-sized
// batches, k_router_dec / k_router_seq above), so the logits are
// bit-identical to the reference's by construction.  Top-k selection and
// the dispatch that follows it: dispatch.hip.
#include "common.h"
#include "launch.h"
#include "mfma_ops.h"

#include <float.h>
#include <limits.h>


namespace {

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

// ---------------------------------------------------------------------------
// MoE router logits, many tokens (prefill).  Lane = expert e0 + lane; wave w
// = tokens t0 + w*TPW .. t0 + w*TPW + TPW-1 (TPW independent chains per
// lane).  The block's 64 weight columns and its tokens' activations stream
// through LDS in chunks of ORN_RDC values of d, so every weight byte read
// from L2 serves 4*TPW tokens: each thread keeps its share of the next
// ORN_RPF chunks in flight in registers, copies chunk c into one of two LDS
// slots, and every chain then consumes the chunk in d order.
// ---------------------------------------------------------------------------
#define ORN_RDC 64                 // d values per chunk (half the barriers of 32:
                                   // 76.0 -> 72.8 us at 2048 tokens)
#define ORN_RPF 4                  // chunks in flight
#define ORN_RWS4 (ORN_RDC / 4 + 1) // LDS row stride of a weight row, in float4 (padded)

template <int TPW>
__global__ void __launch_bounds__(256)
    k_router_seq(const float *__restrict__ x, const float *__restrict__ Wq,
                 const float *__restrict__ bias, int T, int D, int E,
                 float *__restrict__ logits, int *ctl, float *__restrict__ amax)
{
    constexpr int TB = 4 * TPW;               // tokens per block
    constexpr int XF4 = TB * ORN_RDC / 4;     // activation float4 per chunk
    constexpr int XPT = (XF4 + 255) / 256;    // ... per thread
    constexpr int WF4 = 64 * ORN_RDC / 4;     // weight float4 per chunk
    constexpr int WPT = WF4 / 256;            // ... per thread
    static_assert(WF4 % 256 == 0, "chunk must split evenly over the block");
    __shared__ v4f wl[2][64 * ORN_RWS4];
    __shared__ v4f xl[2][XF4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int e0 = blockIdx.x * 64, t0 = blockIdx.y * TB;
    // The routing step is the first of every forward: clear its counters.
    if (ctl && blockIdx.x == 0 && blockIdx.y == 0 && tid < 16) ctl[tid] = 0;
    const int nc = D / ORN_RDC;

    // Weights in the d-quad layout Wq[D/4][E][4]: the 64 experts of one
    // quad are 1 KB contiguous.  Chunk c holds quads 8c..8c+7.
    const float *wsrc[WPT];
    int wdst[WPT];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
        const int q = tid + 256 * i, d4 = q / 64, r = q % 64;
        const int e = min(e0 + r, E - 1);  // rows past E load a valid row, never used
        wsrc[i] = Wq + ((size_t)d4 * E + e) * 4;
        wdst[i] = r * ORN_RWS4 + d4;
    }
    const size_t wstep = (size_t)(ORN_RDC / 4) * E * 4;  // floats per chunk
    const float *xsrc[XPT];
    bool xon[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const int q = tid + 256 * i, tt = q / (ORN_RDC / 4), d4 = q % (ORN_RDC / 4);
        xon[i] = q < XF4;
        const int t = min(t0 + min(tt, TB - 1), T - 1);
        xsrc[i] = x + (size_t)t * D + 4 * d4;
    }

    v4f rw[ORN_RPF * WPT], rx[ORN_RPF * XPT];
#pragma unroll
    for (int p = 0; p < ORN_RPF; ++p) {
        const int c = min(p, nc - 1);
#pragma unroll
        for (int i = 0; i < WPT; ++i)
            rw[p * WPT + i] = *reinterpret_cast<const v4f *>(wsrc[i] + (size_t)c * wstep);
#pragma unroll
        for (int i = 0; i < XPT; ++i)
            rx[p * XPT + i] = *reinterpret_cast<const v4f *>(xsrc[i] + (size_t)c * ORN_RDC);
    }

    float acc[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) acc[j] = 0.0f;
    // amax (block column 0): the staging threads' running max |x| over
    // their token's quads, folded over the token's ORN_RDC/4 threads below
    const bool want_amax = amax && blockIdx.x == 0;
    float xmax = 0.0f;

    for (int c0 = 0; c0 < nc; c0 += ORN_RPF) {
#pragma unroll
        for (int p = 0; p < ORN_RPF; ++p) {
            const int c = c0 + p;
            if (c < nc) {  // uniform over the block
                const int sl = c & 1;
#pragma unroll
                for (int i = 0; i < WPT; ++i) wl[sl][wdst[i]] = rw[p * WPT + i];
#pragma unroll
                for (int i = 0; i < XPT; ++i)
                    if (xon[i]) {
                        const v4f v = rx[p * XPT + i];
                        xl[sl][tid + 256 * i] = v;
                        if (want_amax)
                            xmax = fmaxf(xmax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)),
                                                     fmaxf(fabsf(v.z), fabsf(v.w))));
                    }
                const int cn = min(c + ORN_RPF, nc - 1);
#pragma unroll
                for (int i = 0; i < WPT; ++i)
                    rw[p * WPT + i] = *reinterpret_cast<const v4f *>(wsrc[i] + (size_t)cn * wstep);
#pragma unroll
                for (int i = 0; i < XPT; ++i)
                    rx[p * XPT + i] = *reinterpret_cast<const v4f *>(xsrc[i] + (size_t)cn * ORN_RDC);
                __syncthreads();
                const v4f *wr = &wl[sl][lane * ORN_RWS4];
                const v4f *xr = &xl[sl][wave * TPW * (ORN_RDC / 4)];
                // Each quad's LDS reads are issued before the previous
                // quad's arithmetic (two register sets; the empty asm keeps
                // the reads above it and the arithmetic below it): 78 ->
                // 71-74 us at 2048 tokens.  Groups of two quads ran 74-77,
                // and of four took a wave per SIMD in registers.
                constexpr int RG = 1, NG = ORN_RDC / 4 / RG;
                v4f wA[RG], wB[RG], xA[TPW][RG], xB[TPW][RG];
                auto rd = [&](v4f (&w)[RG], v4f (&xv)[TPW][RG], int g) {
#pragma unroll
                    for (int q = 0; q < RG; ++q) {
                        w[q] = wr[RG * g + q];
#pragma unroll
                        for (int j = 0; j < TPW; ++j) xv[j][q] = xr[j * (ORN_RDC / 4) + RG * g + q];
                    }
                };
                rd(wA, xA, 0);
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    v4f(&wc)[RG] = (g & 1) ? wB : wA;
                    v4f(&wn)[RG] = (g & 1) ? wA : wB;
                    v4f(&xc)[TPW][RG] = (g & 1) ? xB : xA;
                    v4f(&xn)[TPW][RG] = (g & 1) ? xA : xB;
                    if (g + 1 < NG) rd(wn, xn, g + 1);
#pragma unroll
                    for (int j = 0; j < TPW; ++j) asm volatile("" : "+v"(acc[j])::"memory");
#pragma unroll
                    for (int q = 0; q < RG; ++q)
#pragma unroll
                        for (int j = 0; j < TPW; ++j) {
                            const v4f xv = xc[j][q], wv = wc[q];
                            acc[j] = acc[j] + xv.x * wv.x;
                            acc[j] = acc[j] + xv.y * wv.y;
                            acc[j] = acc[j] + xv.z * wv.z;
                            acc[j] = acc[j] + xv.w * wv.w;
                        }
                }
            }
        }
    }
    const int e = e0 + lane;
    if (e < E) {
        const float b = bias ? bias[e] : 0.0f;
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const int t = t0 + wave * TPW + j;
            if (t < T) logits[(size_t)t * E + e] = bias ? acc[j] + b : acc[j];
        }
    }
    if (want_amax) {
        // thread q = tt * (ORN_RDC/4) + d4 staged token tt's quads d4, d4 +
        // ORN_RDC/4, ... (XPT = 1: TB * ORN_RDC/4 <= 256 threads)
        static_assert(XPT == 1, "one staged quad per thread and chunk");
#pragma unroll
        for (int off = 1; off < ORN_RDC / 4; off <<= 1) xmax = fmaxf(xmax, __shfl_xor(xmax, off, 64));
        const int tt = tid / (ORN_RDC / 4), t = t0 + tt;
        if (xon[0] && tid % (ORN_RDC / 4) == 0 && t < T) amax[t] = xmax;
    }
}

// ---------------------------------------------------------------------------
// MoE router logits, few tokens (decode).  Block = one wave = one token over
// 64 experts (lane = expert), so the 2 MiB router streams through 4*T CUs.
// A lane's weights for quad d4 are the 16 bytes at Wq[d4][e][0..3], so one
// wave load instruction reads 1 KB contiguous.  The loads run ORN_DPF quads
// ahead in a register ring (branch-free, fully unrolled); the token's
// activation row sits in LDS and is read as a broadcast.
// ---------------------------------------------------------------------------
#define ORN_DPF 8  // weight quads in flight per lane

// Orders LDS accesses of the lanes of one wave across this point (the wave's
// LDS operations execute in issue order; this keeps the compiler from
// moving them).
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ void __launch_bounds__(64)
    k_router_dec(const float *__restrict__ x, const float *__restrict__ Wq,
                 const float *__restrict__ bias, int T, int D, int E,
                 float *__restrict__ logits, int *ctl, float *__restrict__ amax)
{
    extern __shared__ v4f xsh[];  // [D/4]
    const int lane = threadIdx.x;
    const int e0 = blockIdx.x * 64;
    const int t = blockIdx.y;
    // The routing step is the first of every forward: clear its counters.
    if (ctl && blockIdx.x == 0 && blockIdx.y == 0 && lane < 16) ctl[lane] = 0;
    const int nd4 = D / 4;  // a multiple of ORN_DPF (checked by the launcher)
    v4f *xw = xsh;
    const v4f *xg = reinterpret_cast<const v4f *>(x + (size_t)t * D);
    {
        // All loads first, then the LDS writes (D <= 4096: at most 16 per lane).
        v4f tmp[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (lane + 64 * j < nd4) tmp[j] = xg[lane + 64 * j];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (lane + 64 * j < nd4) xw[lane + 64 * j] = tmp[j];
        // max |x| of the row for the MFMA activation scaling (block column 0)
        if (amax && blockIdx.x == 0) {
            float mx = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (lane + 64 * j < nd4)
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(tmp[j].x), fabsf(tmp[j].y)),
                                         fmaxf(fabsf(tmp[j].z), fabsf(tmp[j].w))));
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            if (lane == 0) amax[t] = mx;
        }
    }
    wave_sync();

    const int e = min(e0 + lane, E - 1);  // lanes past E compute a copy, never stored
    const v4f *wp = reinterpret_cast<const v4f *>(Wq) + e;  // quad d4 at wp[d4*E]
    v4f r[ORN_DPF];
#pragma unroll
    for (int p = 0; p < ORN_DPF; ++p) r[p] = wp[(size_t)p * E];
    float acc = 0.0f;
    for (int i0 = 0; i0 < nd4; i0 += ORN_DPF) {
        v4f xv4[ORN_DPF];  // this iteration's activations, read up front
#pragma unroll
        for (int p = 0; p < ORN_DPF; ++p) xv4[p] = xw[i0 + p];
#pragma unroll
        for (int p = 0; p < ORN_DPF; ++p) {
            // Use the slot, then refill it: the refill reuses its registers.
            const v4f xv = xv4[p];
            acc = acc + xv.x * r[p].x;
            acc = acc + xv.y * r[p].y;
            acc = acc + xv.z * r[p].z;
            acc = acc + xv.w * r[p].w;
            r[p] = wp[(size_t)min(i0 + p + ORN_DPF, nd4 - 1) * E];
            __builtin_amdgcn_sched_barrier(0);  // keep the refill here, ORN_DPF quads ahead
        }
    }
    if (e0 + lane < E) logits[(size_t)t * E + e0 + lane] = bias ? acc + bias[e0 + lane] : acc;
}

// ---------------------------------------------------------------------------
// Decode-sized batches: one work group of two waves per (token, 8 experts).
// Wave 1 (the producer) streams W and forms the products; wave 0 (the
// consumer) only adds them, so its instruction stream is the chain itself.
//
// Lane l = 8*es + q (es: expert e0+es, q = 0..7) of the producer multiplies
// the k quad 8*it + q of x and W(., e0+es), i.e. k = 32*it + 4q + j (j =
// 0..3), so a wave load covers 8 experts x 32 k (W's [D/4][E][4] layout: 8
// runs of 128 contiguous bytes), and writes its four products to pb[it %
// (3C)][l].  The consumer lanes of expert es (every lane of the group keeps
// the same chain) read the 32 products of a step back in k order as 8
// consecutive quads and add them.  Each logit is therefore acc = acc +
// fl(x[k]*W[k]) for k ascending, one add per element, bit-identical to
// model.c:1017-1025.
//
// The ND = D/32 steps form chunks of C steps in a three-chunk LDS ring.  The
// producer runs two chunks ahead: chunks 0 and 1 before barrier B_0, chunk
// c+1 between B_{c-1} and B_c.  The consumer adds chunk c between B_c and
// B_{c+1} and reads the next step a step ahead, across chunk edges too
// (that chunk is complete since the previous barrier), so it never waits on
// LDS.  Both waves pass the same ND/C barriers; the producer, ~4x shorter
// per step, is the one that waits.
//
// Before that the group stages x[t] in LDS and, when amax != NULL (block
// column 0), writes max_k |x[t][k]| for the MFMA activation scaling.  With
// norm_w the input is first replaced by its rmsnorm (one thread runs the
// norm's sequential sum while the producer's first weight loads are in
// flight; block column 0 writes the normalised rows to xn_out).  With fxh
// (file-orientation stores) block column 0's producer wave, done before the
// consumer's chain is, also writes the row as the file kernels' activations
// (the outputs of k_prep_rows<true>, expert_file.hip, with its arithmetic).
// ---------------------------------------------------------------------------
// Steps per chunk of the product ring (three chunks).  With the x*x buffer
// folded into the ring a group holds 20 KB of LDS at D = 2048 (40 KB with
// chunks of 8 and a separate buffer): measured route step 9.5 -> 9.2 us at
// 16 tokens, 18.6 -> 13.4 at 32, 28.5 -> 26.7 at 64.
#define ORN_PC_CHUNK 4

template <int ND>
__global__ void __launch_bounds__(128)
    k_router_pc(const float *__restrict__ x, const float *__restrict__ Wq,
                const float *__restrict__ bias, int T, int E, float *__restrict__ logits,
                int *ctl, float *__restrict__ amax, const float *__restrict__ norm_w,
                float *__restrict__ xn_out, uint32_t *__restrict__ fxh, uint32_t *__restrict__ fxl,
                float *__restrict__ fxinv, uint16_t *__restrict__ fxsh, uint16_t *__restrict__ fxsl)
{
    constexpr int D = 32 * ND, NR = ND < 16 ? ND : 16;
    constexpr int C = ND < ORN_PC_CHUNK ? ND : ORN_PC_CHUNK, NC = ND / C;
    constexpr int NPB = 3 * C * 64 > D / 4 ? 3 * C * 64 : D / 4;
    __shared__ v4f xs[D / 4];
    // the product ring; before the chain starts, x*x for the rmsnorm (with
    // norm_w), so that a CU holds more groups
    __shared__ v4f pbuf[NPB];
    v4f *const ps = pbuf;
    v4f(*const pb)[64] = reinterpret_cast<v4f(*)[64]>(pbuf);
    __shared__ float inv_s, mx_s[2];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the roles branch per wave
    const int es = lane >> 3, q = lane & 7;
    const int e0 = blockIdx.x * 8;
    const int t = blockIdx.y;
    const bool producer = wave == 1;
    // The routing step is the first of every forward: clear its counters.
    if (ctl && blockIdx.x == 0 && blockIdx.y == 0 && tid < 16) ctl[tid] = 0;
    const int e = min(e0 + es, E - 1);  // lanes past E compute a copy, never stored
    const v4f *wp = reinterpret_cast<const v4f *>(Wq) + (size_t)q * E + e;  // step it: + 8*it*E
    v4f ring[NR];
    if (producer) {
#pragma unroll
        for (int i = 0; i < NR; ++i) ring[i] = wp[(size_t)8 * i * E];
    }
    {
        const v4f *xg = reinterpret_cast<const v4f *>(x + (size_t)t * D);
        constexpr int NX = (D / 4 + 127) / 128;  // v4f per thread
        v4f tmp[NX], wn[NX];
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int j = tid + 128 * i;
            tmp[i] = j < D / 4 ? xg[j] : v4f{};
        }
        if (norm_w) {
            // The layer's rmsnorm (gpu.c:144-156) on the fly: x*x into LDS,
            // one thread sums the products in order (the reference's
            // roundings), then x <- w * (x * inv_rms).  Block column 0 also
            // writes the normalised row out for the expert steps.
            const v4f *wg = reinterpret_cast<const v4f *>(norm_w);
#pragma unroll
            for (int i = 0; i < NX; ++i) {
                const int j = tid + 128 * i;
                if (j < D / 4) {
                    wn[i] = wg[j];
                    ps[j] = tmp[i] * tmp[i];
                }
            }
            __syncthreads();
            if (tid == 0) {
                const float ss = orn_lds_seq_sum32_n<ND>(ps);
                inv_s = 1.0f / sqrtf(ss / (float)D + 1e-6f);
            }
            __syncthreads();
            const float inv = inv_s;
#pragma unroll
            for (int i = 0; i < NX; ++i) tmp[i] = wn[i] * (tmp[i] * inv);
            if (blockIdx.x == 0) {
                v4f *xo = reinterpret_cast<v4f *>(xn_out + (size_t)t * D);
#pragma unroll
                for (int i = 0; i < NX; ++i)
                    if (tid + 128 * i < D / 4) xo[tid + 128 * i] = tmp[i];
            }
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int j = tid + 128 * i;
            if (j < D / 4) {
                xs[j] = tmp[i];
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(tmp[i].x), fabsf(tmp[i].y)),
                                     fmaxf(fabsf(tmp[i].z), fabsf(tmp[i].w))));
            }
        }
        if ((amax || fxh) && blockIdx.x == 0) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            if (lane == 0) mx_s[wave] = mx;
        }
    }
    __syncthreads();
    if (amax && blockIdx.x == 0 && tid == 0) amax[t] = fmaxf(mx_s[0], mx_s[1]);

    if (producer) {
        auto prod = [&](int it, const v4f xv) {  // products of step it into pb[it % 3C]
            const v4f w = ring[it % NR];
            if (it + NR < ND) ring[it % NR] = wp[(size_t)8 * (it + NR) * E];
            pb[it % (3 * C)][lane] = xv * w;
        };
        // x of step it+1 is read from LDS during step it.
        v4f xnext = xs[q];
        auto step = [&](int it) {
            const v4f xv = xnext;
            if (it + 1 < ND) xnext = xs[8 * (it + 1) + q];
            prod(it, xv);
        };
#pragma unroll
        for (int it = 0; it < (2 * C < ND ? 2 * C : ND); ++it) step(it);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            __syncthreads();  // B_c
            if (c + 2 < NC) {
#pragma unroll
                for (int s = 0; s < C; ++s) step((c + 2) * C + s);
            }
        }
        if (fxh && blockIdx.x == 0) {
            // hi/lo of x*s in groups of 8 (pair order [0,2,1,3,4,6,5,7]) and
            // the 32-value sub-block sums / 32, lane l taking groups l + 64i
            const float sc = orn_mfma::prep_scale(fmaxf(mx_s[0], mx_s[1]));
            constexpr int NG = D / 8;
#pragma unroll
            for (int i = 0; i < (NG + 63) / 64; ++i) {
                const int g = lane + 64 * i;
                const bool on = g < NG;
                const v4f a = xs[on ? 2 * g : 0] * sc, b = xs[on ? 2 * g + 1 : 0] * sc;
                if (on) {
                    uint32_t h[4], l[4];
                    orn_mfma::split2(a.x, a.z, h[0], l[0]);
                    orn_mfma::split2(a.y, a.w, h[1], l[1]);
                    orn_mfma::split2(b.x, b.z, h[2], l[2]);
                    orn_mfma::split2(b.y, b.w, h[3], l[3]);
                    const size_t o = (size_t)t * (D >> 1) + 4 * g;
                    *reinterpret_cast<uint4 *>(fxh + o) = make_uint4(h[0], h[1], h[2], h[3]);
                    *reinterpret_cast<uint4 *>(fxl + o) = make_uint4(l[0], l[1], l[2], l[3]);
                }
                float sm = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
                sm += __shfl_xor(sm, 1, 64);
                sm += __shfl_xor(sm, 2, 64);
                if (on && (g & 3) == 0) {
                    sm *= 0.03125f;
                    const _Float16 th = (_Float16)sm;
                    const _Float16 tl = (_Float16)(sm - (float)th);
                    const size_t o = (size_t)t * (D >> 5) + (g >> 2);
                    fxsh[o] = __builtin_bit_cast(uint16_t, th);
                    fxsl[o] = __builtin_bit_cast(uint16_t, tl);
                }
            }
            if (lane == 0) fxinv[t] = 1.0f / sc;
        }
        return;
    }

    auto rd = [&](v4f(&r)[8], int it) {
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = pb[it % (3 * C)][8 * es + i];
    };
    float acc = 0.0f;
    v4f ca[8], cb[8];
#pragma unroll
    for (int it = 0; it < ND; ++it) {
        if (it % C == 0) {
            __syncthreads();  // B_{it/C}: chunk it/C + 1 is complete
            if (it == 0) rd(ca, 0);
        }
        v4f(&cur)[8] = (it & 1) ? cb : ca;
        v4f(&nxt)[8] = (it & 1) ? ca : cb;
        if (it + 1 < ND) rd(nxt, it + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc = acc + cur[i].x;
            acc = acc + cur[i].y;
            acc = acc + cur[i].z;
            acc = acc + cur[i].w;
        }
        // Keeps each step's adds in its step (they would otherwise sink into
        // the conditional store below, holding every product in registers).
        asm volatile("" : "+v"(acc));
    }
    if (q == 0 && e0 + es < E) logits[(size_t)t * E + e0 + es] = bias ? acc + bias[e0 + es] : acc;
}

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
// MoE routing step: exact logits into a->logits (selection: dispatch.hip).
// ---------------------------------------------------------------------------
extern "C" int ornk_router_pc_supported(int T, int D)
{
    return T >= 1 && T <= ORN_ROUTER_PC_MAX_T &&
           (D == 256 || D == 512 || D == 1024 || D == 2048 || D == 4096);
}

extern "C" int ornk_moe_route(const ornk_moe_args *a, hipStream_t s)
{
    const int T = a->T, D = a->D, E = a->E;
    if (T <= 0) return hipSuccess;
    if (E < 1 || E > 256 || a->k < 1 || a->k > 16 || a->k > E || D % (4 * ORN_DPF) ||
        D % (ORN_RDC * ORN_RPF) || D > 4096)
        return hipErrorInvalidValue;
    const float *xin = a->apply_norm ? a->xn : a->x;
    float *amax = a->router_amax ? a->x_amax : nullptr;  // every routing kernel can write it
    const dim3 gd((E + 7) / 8, T);
    if (ornk_router_pc_supported(T, D)) {
        // the norm runs inside the router here (ornk_moe_norm launches nothing)
        const float *xr = a->apply_norm ? a->x : xin;
        const float *nw = a->apply_norm ? a->norm_w : nullptr;
        float *xo = a->apply_norm ? a->xn : nullptr;
#define ORN_RPC(N)                                                                              \
    ORN_LAUNCH_EV(a, k_router_pc<N>, gd, dim3(128), 0, s, xr, a->router, a->bias, T, E,         \
                       a->logits, a->ctl, amax, nw, xo, a->fw.xh, a->fw.xl, a->fw.xinv,         \
                       a->fw.xsh, a->fw.xsl)
        switch (D) {
        case 256: ORN_RPC(8); break;
        case 512: ORN_RPC(16); break;
        case 1024: ORN_RPC(32); break;
        case 2048: ORN_RPC(64); break;
        default: ORN_RPC(128); break;
        }
#undef ORN_RPC
    } else if (T >= 1024) {
        ORN_LAUNCH_EV(a, k_router_seq<4>, dim3((E + 63) / 64, (T + 15) / 16), dim3(256), 0, s,
                           xin, a->router, a->bias, T, D, E, a->logits, a->ctl, amax);
    } else if (T >= 384) {
        // 4 tokens per block: enough blocks for every CU (measured at 512
        // tokens: 36.5 us against 49.5 us for k_router_dec; at 256, 31 us
        // against 25-34 us)
        ORN_LAUNCH_EV(a, k_router_seq<1>, dim3((E + 63) / 64, (T + 3) / 4), dim3(256), 0, s,
                           xin, a->router, a->bias, T, D, E, a->logits, a->ctl, amax);
    } else {
        ORN_LAUNCH_EV(a, k_router_dec, dim3((E + 63) / 64, T), dim3(64), sizeof(float) * (size_t)D,
                           s, xin, a->router, a->bias, T, D, E, a->logits, a->ctl, amax);
    }
    return hipGetLastError();
}
