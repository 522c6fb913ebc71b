// SPDX-License-Identifier: MIT
//
// The attention-side ops of the gpu.h backend: RoPE, single-head scaled
// dot-product attention, the gated DeltaNet step and the KV-cache append,
// with the semantics of the reference's Metal kernels (ops.metal:113-139,
// attention.metal:17-125) as dispatched by gpu_metal.m:495-583.  fp32
// throughout, compiled with -ffp-contract=off.
#include "common.h"
#include "launch.h"

namespace {

// ops.metal:113-139 on Q (heads [0, n_q)) and K (heads [0, n_k)) in one
// launch: the pair (x[i], x[i+1]), i = 2p < rot, of every head is rotated by
// pos * theta^(-i/rot).  The frequency is computed in double and rounded
// once, so it is the correctly rounded value of the formula (the Metal and
// CPU builds take it from a float pow, within an ulp of that).
__global__ void k_rope(float *Q, float *K, int head_dim, int n_q, int n_k, int rot, int pos,
                       float theta)
{
    const int half = rot / 2;
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (half <= 0 || g >= (n_q + n_k) * half) return;
    int head = g / half;
    const int i = 2 * (g % half);
    float *x = Q;
    if (head >= n_q) {
        head -= n_q;
        x = K;
    }
    const float inv_freq = (float)(1.0 / pow((double)theta, (double)i / (double)rot));
    const float ang = (float)pos * inv_freq;
    const float c = cosf(ang), s = sinf(ang);
    float *h = x + (size_t)head * head_dim;
    const float a = h[i], b = h[i + 1];
    h[i] = a * c - b * s;
    h[i + 1] = a * s + b * c;
}

// attention.metal:17-68: out[r][c] = sum_t e^(s_rt) V[t][c] / sum_t e^(s_rt),
// s_rt = (Q[r] . K[t]) * scale, every key for every query (no mask), where
// the shader divides only when the sum exceeds 1e-10 and otherwise returns
// the unnormalised sum; so does this kernel.  The exponent is taken relative
// to the running row maximum m (online softmax): the unshifted sums are
// e^m times the shifted ones.  Where the shader's unshifted e^s overflows
// (scores above ~88, which make its output Inf or NaN) this kernel still
// returns the softmax.
//
// Work group: 256 threads, ATT_R = 16 query rows; keys in tiles of ATT_T =
// 16 staged in LDS (K with a padded row stride, so the 16 keys a row group
// reads at one time sit in different banks); 50 KB of LDS at hd = 256.
// Thread (r = tid/16, j = tid%16) scores key j of the tile for row r and
// owns output columns j, j+16, ... of row r.
constexpr int ATT_R = 16, ATT_T = 16, ATT_MAXD = 256;

__global__ __launch_bounds__(256) void k_attention(float *out, const float *Q, const float *K,
                                                   const float *V, int seq, int hd, float scale)
{
    extern __shared__ float lds[];
    const int ks = hd + 1;                 // padded K row stride
    float *Qs = lds;                       // [ATT_R][ks]
    float *Ks = Qs + ATT_R * ks;           // [ATT_T][ks]
    float *Vs = Ks + ATT_T * ks;           // [ATT_T][hd]
    float *Ps = Vs + ATT_T * hd;           // [ATT_R][ATT_T]
    const int tid = threadIdx.x, r = tid >> 4, j = tid & 15;
    const int row0 = blockIdx.x * ATT_R;
    for (int e = tid; e < ATT_R * hd; e += 256) {
        const int rr = e / hd, d = e - rr * hd;
        Qs[rr * ks + d] = row0 + rr < seq ? Q[(size_t)(row0 + rr) * hd + d] : 0.0f;
    }
    float acc[ATT_MAXD / 16];
#pragma unroll
    for (int c = 0; c < ATT_MAXD / 16; ++c) acc[c] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (int t0 = 0; t0 < seq; t0 += ATT_T) {
        __syncthreads();  // the previous tile's Ks/Vs/Ps are consumed
        for (int e = tid; e < ATT_T * hd; e += 256) {
            const int tt = e / hd, d = e - tt * hd;
            const bool in = t0 + tt < seq;
            Ks[tt * ks + d] = in ? K[(size_t)(t0 + tt) * hd + d] : 0.0f;
            Vs[tt * hd + d] = in ? V[(size_t)(t0 + tt) * hd + d] : 0.0f;
        }
        __syncthreads();
        float s0 = 0.0f;
        const float *q = Qs + r * ks, *k0 = Ks + j * ks;
        for (int d = 0; d < hd; ++d) s0 += q[d] * k0[d];
        s0 = t0 + j < seq ? s0 * scale : -INFINITY;
        float tm = s0;
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) tm = fmaxf(tm, __shfl_xor(tm, o, 16));
        const float mn = fmaxf(m, tm);  // finite: key t0 is always in range
        const float corr = expf(m - mn);
        const float p0 = expf(s0 - mn);
        float ps = p0;
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) ps += __shfl_xor(ps, o, 16);
        l = l * corr + ps;
        m = mn;
        Ps[r * ATT_T + j] = p0;
        __syncthreads();
        const float *pr = Ps + r * ATT_T;
#pragma unroll
        for (int c = 0; c < ATT_MAXD / 16; ++c) {
            const int col = j + 16 * c;
            if (col < hd) {
                float a = acc[c] * corr;
                for (int t = 0; t < ATT_T; ++t) a += pr[t] * Vs[t * hd + col];
                acc[c] = a;
            }
        }
    }
    if (row0 + r >= seq) return;
    // attention.metal:60-62: normalise only when the unshifted sum e^m * l
    // exceeds 1e-10; else the unnormalised sum e^m * acc
    const float em = expf(m);
    const float f = em * l > 1e-10f ? 1.0f / l : em;
#pragma unroll
    for (int c = 0; c < ATT_MAXD / 16; ++c) {
        const int col = j + 16 * c;
        if (col < hd) out[(size_t)(row0 + r) * hd + col] = acc[c] * f;
    }
}

// ---------------------------------------------------------------------------
// The same attention on the matrix cores (v_mfma_f32_16x16x4f32: fp32 operands,
// fp32 accumulation), for head dims that are a multiple of 4 (HD = 64, 128 or
// 256: the smallest instance that holds hd; dims past hd are zero in Q, K and
// V and never stored).
//
// Work group: 4 waves over 64 query rows (wave w: rows 16w..16w+15 of the
// group's tile) and one split of the keys (grid.y splits, whole tiles of 16
// keys each).  Per tile of 16 keys, staged in LDS once for the four waves
// (double buffered, the next tile's loads in flight during this one's math):
//   S = Q K^T     HD/4 MFMAs; the wave's Q rows sit in registers as A
//                 operands, K rows are read from LDS as B operands;
//   p = e^(S*scale - m) with the running row maximum m and sum l (online
//                 softmax; m = -inf until a key is seen);
//   O = O*corr + P V   4 * HD/16 MFMAs; P goes from the C to the A layout
//                 through a 1 KB LDS slice per wave, V is staged transposed.
// The reduction index of every MFMA is permuted identically in both
// operands (k = 16*(s/4) + 4*g + s%4 for lane group g at step s, keys 4g + q
// at PV step q), so a lane's four consecutive steps read one 16-byte LDS
// word.  With one split the group writes out; else it writes O, m, l of its
// split and k_attn_merge combines the splits:
//   M = max m_i, L = sum l_i e^(m_i - M), O = sum O_i e^(m_i - M),
//   out = O / L where the unshifted sum e^M L exceeds 1e-10, else O e^M
// (attention.metal:60-62).
// ---------------------------------------------------------------------------
constexpr int AM_TK = 16;  // keys per tile

template <int HD>
struct AttnLds {
    float k[2][AM_TK][HD + 4];      // key rows (padded: conflict-free B reads)
    float vt[2][HD][AM_TK + 4];     // value tile transposed: vt[col][key]
    float p[4][16][AM_TK + 4];      // per wave: P in row-major, for the A layout
};

template <int HD>
__global__ void __launch_bounds__(256) k_attn_mma(float *out, float *Op, float *mlp,
                                                  const float *Q, const float *K, const float *V,
                                                  int seq, int hd, float scale, int tiles_per_split)
{
    __shared__ __align__(16) AttnLds<HD> L;  // 79 KB at HD = 256
    constexpr int NS = HD / 4, NC = HD / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const int q0 = blockIdx.x * 64 + 16 * wave;
    const int n_tiles = (seq + AM_TK - 1) / AM_TK;
    const int t_lo = blockIdx.y * tiles_per_split;
    const int t_hi = min(n_tiles, t_lo + tiles_per_split);

    // Q rows (A operands): lane row q0 + c, steps s = 4j + i hold k = 16j + 4g + i
    float qa[NS];
    {
        const int r = q0 + c;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int k = 16 * j + 4 * g;
            v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (r < seq && k < hd) v = *reinterpret_cast<const v4f *>(Q + (size_t)r * hd + k);
#pragma unroll
            for (int i = 0; i < 4; ++i) qa[4 * j + i] = v[i];
        }
    }
    // staging: thread tid loads float4 number tid + 256i of each tile
    constexpr int F4 = AM_TK * HD / 4, F4T = F4 / 256;
    static_assert(F4 % 256 == 0, "whole float4s per thread");
    v4f rk[F4T], rv[F4T];
    auto load_tile = [&](int t) {
#pragma unroll
        for (int i = 0; i < F4T; ++i) {
            const int f = tid + 256 * i, key = f / (HD / 4), col = 4 * (f % (HD / 4));
            const int kk = t * AM_TK + key;
            const bool on = kk < seq && col < hd;
            rk[i] = on ? *reinterpret_cast<const v4f *>(K + (size_t)kk * hd + col)
                       : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
            rv[i] = on ? *reinterpret_cast<const v4f *>(V + (size_t)kk * hd + col)
                       : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < F4T; ++i) {
            const int f = tid + 256 * i, key = f / (HD / 4), col = 4 * (f % (HD / 4));
            *reinterpret_cast<v4f *>(&L.k[buf][key][col]) = rk[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) L.vt[buf][col + e][key] = rv[i][e];
        }
    };

    v4f o[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) o[j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    float m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
    }

    if (t_lo < t_hi) {
        load_tile(t_lo);
        store_tile(0);
        if (t_lo + 1 < t_hi) load_tile(t_lo + 1);
    }
    __syncthreads();
    for (int t = t_lo; t < t_hi; ++t) {
        const int buf = (t - t_lo) & 1;
        // S = Q K^T for this wave's 16 rows and the tile's 16 keys
        v4f sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const v4f kb = *reinterpret_cast<const v4f *>(&L.k[buf][c][16 * j + 4 * g]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * j + i], kb[i], sacc, 0, 0, 0);
        }
        // C layout: this lane holds key c, rows 4g + r
        const bool key_on = t * AM_TK + c < seq;
        float p[4], corr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float sc = key_on ? sacc[r] * scale : -INFINITY;
            float tm = sc;
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) tm = fmaxf(tm, __shfl_xor(tm, off, 16));
            const float mn = fmaxf(m[r], tm);
            const bool none = mn == -INFINITY;  // no key of this row seen yet
            corr[r] = none ? 1.0f : expf(m[r] - mn);
            p[r] = none ? 0.0f : expf(sc - mn);
            float ps = p[r];
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) ps += __shfl_xor(ps, off, 16);
            l[r] = l[r] * corr[r] + ps;
            m[r] = mn;
        }
        // P to the A layout through this wave's LDS slice
#pragma unroll
        for (int r = 0; r < 4; ++r) L.p[wave][4 * g + r][c] = p[r];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const v4f pa = *reinterpret_cast<const v4f *>(&L.p[wave][c][4 * g]);
        // O rows 4g + r scale by their corr; then O += P V
#pragma unroll
        for (int j = 0; j < NC; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j][r] *= corr[r];
            const v4f vb = *reinterpret_cast<const v4f *>(&L.vt[buf][16 * j + c][4 * g]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[q], vb[q], o[j], 0, 0, 0);
        }
        // the next tile: written into the other buffer (last read two tiles
        // ago, before the previous barrier), then loads for the one after
        if (t + 1 < t_hi) {
            store_tile(buf ^ 1);
            if (t + 2 < t_hi) load_tile(t + 2);
        }
        __syncthreads();
    }

    // rows 4g + r of the wave's tile, columns 16j + c
    const int nsplit = gridDim.y;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = q0 + 4 * g + r;
        if (row >= seq) continue;
        if (nsplit == 1) {
            const float em = expf(m[r]);
            const float f = em * l[r] > 1e-10f ? 1.0f / l[r] : em;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int col = 16 * j + c;
                if (col < hd) out[(size_t)row * hd + col] = o[j][r] * f;
            }
        } else {
            float *po = Op + ((size_t)blockIdx.y * seq + row) * hd;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int col = 16 * j + c;
                if (col < hd) po[col] = o[j][r];
            }
            if (c == 0) {
                mlp[((size_t)blockIdx.y * seq + row) * 2] = m[r];
                mlp[((size_t)blockIdx.y * seq + row) * 2 + 1] = l[r];
            }
        }
    }
}

// Combines the key splits of k_attn_mma: one thread per output element.
__global__ void k_attn_merge(float *out, const float *Op, const float *mlp, int seq, int hd,
                             int nsplit)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)seq * hd) return;
    const size_t row = i / hd, col = i - row * hd;
    float M = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, mlp[((size_t)sp * seq + row) * 2]);
    float Ls = 0.0f, O = 0.0f;
    for (int sp = 0; sp < nsplit; ++sp) {
        const float mi = mlp[((size_t)sp * seq + row) * 2];
        const float w = mi == -INFINITY ? 0.0f : expf(mi - M);
        Ls += mlp[((size_t)sp * seq + row) * 2 + 1] * w;
        O += Op[((size_t)sp * seq + row) * hd + col] * w;
    }
    const float em = expf(M);
    out[i] = em * Ls > 1e-10f ? O / Ls : O * em;
}

// attention.metal:80-108: thread i updates column i of the dim x dim state,
// state[j][i] = gate*state[j][i] + (1-gate)*K[i]*V[j], then
// out[i] = sum_j Q[j]*state[j][i] (j ascending), in the kernel's own order
// of operations.  Loads and stores are coalesced over i.
__global__ void k_deltanet_step(float *state, const float *Q, const float *K, const float *V,
                                float *out, int dim, float gate)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const float ki = K[i], omg = 1.0f - gate;
    for (int j = 0; j < dim; ++j) {
        float *p = state + (size_t)j * dim + i;
        *p = gate * *p + omg * ki * V[j];
    }
    float sum = 0.0f;
    for (int j = 0; j < dim; ++j) sum += Q[j] * state[(size_t)j * dim + i];
    out[i] = sum;
}

// attention.metal:113-125.
__global__ void k_kv_append(float *Kc, float *Vc, const float *Kn, const float *Vn, int pos,
                            int hd)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= hd) return;
    Kc[(size_t)pos * hd + t] = Kn[t];
    Vc[(size_t)pos * hd + t] = Vn[t];
}

}  // namespace

extern "C" int ornk_rope(float *Q, float *K, int head_dim, int n_q, int n_k, int pos, float theta,
                         hipStream_t s)
{
    const int rot = head_dim < 64 ? head_dim : 64;
    const int n = (n_q + n_k) * (rot / 2);
    if (head_dim <= 0 || n_q < 0 || n_k < 0 || n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope, dim3((n + 255) / 256), dim3(256), 0, s, Q, K, head_dim, n_q, n_k,
                       rot, pos, theta);
    return hipGetLastError();
}

extern "C" size_t ornk_attention_lds(int hd)
{
    return ((size_t)ATT_R * (hd + 1) + (size_t)ATT_T * (hd + 1) + (size_t)ATT_T * hd +
            (size_t)ATT_R * ATT_T) * sizeof(float);
}

extern "C" int ornk_attention(float *out, const float *Q, const float *K, const float *V, int seq,
                              int hd, float scale, hipStream_t s)
{
    if (seq <= 0 || hd <= 0) return hipSuccess;
    if (hd > ATT_MAXD) return hipErrorInvalidValue;
    const size_t lds = ornk_attention_lds(hd);  // <= 50,304 B
    hipLaunchKernelGGL(k_attention, dim3((seq + ATT_R - 1) / ATT_R), dim3(256), lds, s, out, Q, K,
                       V, seq, hd, scale);
    return hipGetLastError();
}

// The matrix-core attention: hd % 4 == 0 and hd <= 256.  ws: workspace of
// ornk_attention_mma_ws(seq, hd) bytes (the key splits' partial results).
static int attn_splits(int seq)
{
    const int nq = (seq + 63) / 64, nt = (seq + AM_TK - 1) / AM_TK;
    int ns = 512 / nq;
    ns = ns < 1 ? 1 : ns;
    return ns > nt ? nt : ns;
}

extern "C" size_t ornk_attention_mma_ws(int seq, int hd)
{
    const int ns = attn_splits(seq);
    return ns > 1 ? (size_t)ns * seq * (hd + 2) * sizeof(float) : 0;
}

extern "C" int ornk_attention_mma(float *out, const float *Q, const float *K, const float *V,
                                  int seq, int hd, float scale, void *ws, hipStream_t s)
{
    if (seq <= 0 || hd <= 0) return hipSuccess;
    if (hd % 4 || hd > 256) return hipErrorInvalidValue;
    const int nt = (seq + AM_TK - 1) / AM_TK;
    int ns = attn_splits(seq);
    const int per = (nt + ns - 1) / ns;
    ns = (nt + per - 1) / per;  // every split holds at least one tile
    if (ns > 1 && !ws) return hipErrorInvalidValue;
    float *Op = static_cast<float *>(ws);
    float *mlp = Op ? Op + (size_t)ns * seq * hd : nullptr;
    const dim3 grid((seq + 63) / 64, ns);
#define ORN_ATT(HD_)                                                                          \
    hipLaunchKernelGGL(k_attn_mma<HD_>, grid, dim3(256), 0, s, out, Op, mlp,                  \
                       Q, K, V, seq, hd, scale, per)
    if (hd <= 64) ORN_ATT(64);
    else if (hd <= 128) ORN_ATT(128);
    else ORN_ATT(256);
#undef ORN_ATT
    if (ns > 1) {
        const size_t n = (size_t)seq * hd;
        hipLaunchKernelGGL(k_attn_merge, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out,
                           Op, mlp, seq, hd, ns);
    }
    return hipGetLastError();
}

extern "C" int ornk_deltanet_step(float *state, const float *Q, const float *K, const float *V,
                                  float *out, int dim, float gate, hipStream_t s)
{
    if (dim <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_deltanet_step, dim3((dim + 255) / 256), dim3(256), 0, s, state, Q, K, V,
                       out, dim, gate);
    return hipGetLastError();
}

extern "C" int ornk_kv_append(float *Kc, float *Vc, const float *Kn, const float *Vn, int pos,
                              int hd, hipStream_t s)
{
    if (hd <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_kv_append, dim3((hd + 255) / 256), dim3(256), 0, s, Kc, Vc, Kn, Vn, pos,
                       hd);
    return hipGetLastError();
}
