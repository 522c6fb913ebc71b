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
