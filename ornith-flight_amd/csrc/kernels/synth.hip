// SPDX-License-Identifier: MIT
//
// Device-side synthetic layer generation: the same bytes as the host
// generator (csrc/host/synth.c), written straight into a store's resident
// layouts, plus the MFMA (prefill) layouts built from those blocks on the
// device (the arithmetic of csrc/host/prefill_pack.c).  A 40-layer
// Ornith-shape store (47 GB with both layouts) fills in seconds this way
// instead of minutes of host generation and PCIe copies.
//
// Generator: word(key, i) = fmix(key + (i+1)*G), the i-th SplitMix64 output
// of the stream keyed by (seed, stream id).  Block b of a quantized tensor is
// words 32b..32b+25 laid out as bytes (little-endian), with the fp16 scales
// from words 32b+30 and 32b+31: U(0.001, 0.01) computed in double (one
// multiply, one add; this file is compiled with -ffp-contract=off) and
// rounded to nearest-even half by integer code.  Normals are Irwin-Hall sums
// of 12 16-bit uniforms (exact binary fractions) scaled by sigma with one
// double multiply and one double->float rounding.  Every step is exact or a
// single IEEE rounding, so the device bytes equal the host's.
#include "common.h"
#include "launch.h"
#include "../../../include/ornith/ornith_hip.h"

namespace {

#define ORN_G 0x9E3779B97F4A7C15ull

__device__ __forceinline__ uint64_t fmix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t key_of(uint64_t seed, uint64_t stream)
{
    return fmix(fmix(seed + ORN_G) ^ (stream * ORN_G + ORN_G));
}

__device__ __forceinline__ uint64_t word(uint64_t key, uint64_t i)
{
    return fmix(key + (i + 1) * ORN_G);
}

__device__ __forceinline__ uint64_t stream_of(int layer, int kind, int expert)
{
    return ((uint64_t)(uint32_t)layer << 32) | ((uint64_t)(kind & 0xFF) << 24) |
           (uint64_t)(expert & 0xFFFFFF);
}

// Nearest-even half of a positive double in the normal fp16 range.
__device__ __forceinline__ uint32_t half_rne(double v)
{
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    int ex = (int)((b >> 52) & 0x7FF) - 1023;
    const uint64_t m = (b & ((1ull << 52) - 1)) | (1ull << 52);
    uint64_t keep = m >> 42;
    const uint64_t rem = m & ((1ull << 42) - 1);
    const uint64_t halfway = 1ull << 41;
    if (rem > halfway || (rem == halfway && (keep & 1))) ++keep;
    if (keep == (1ull << 11)) {
        keep >>= 1;
        ++ex;
    }
    return (((uint32_t)(ex + 15)) << 10) | (uint32_t)(keep & 0x3FF);
}

__device__ __forceinline__ uint32_t scale_half(uint64_t w)
{
    const double u = (double)(uint32_t)w * (1.0 / 4294967296.0);
    double v = 0.009 * u;
    v = 0.001 + v;
    return half_rne(v);
}

// ---------------------------------------------------------------------------
// Q4_K blocks of one matrix of one layer: thread = one 16-byte chunk (9 per
// block) of block q of expert e in the store's order.  Block q holds the
// generator's block b: vec@mat stores keep block (row k, block column c) at
// q = c*K + k with b = k*NBc + c; file-orientation stores keep b = q.
// ---------------------------------------------------------------------------
__global__ void k_synth_q4k(uint8_t *__restrict__ dst, uint64_t seed, int layer, int kind, int n_e,
                            int nb, int K, int NBc, int file)
{
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_e = (size_t)nb * 9;
    if (t >= per_e * (size_t)n_e) return;
    const int e = (int)(t / per_e);
    const size_t r = t % per_e;
    const int q = (int)(r / 9), j = (int)(r % 9);
    const int b = file ? q : (q % K) * NBc + q / K;
    const uint64_t key = key_of(seed, stream_of(layer, kind, e));
    uint64_t w0 = word(key, (uint64_t)b * 32 + 2 * j), w1 = word(key, (uint64_t)b * 32 + 2 * j + 1);
    if (j == 0) {
        const uint32_t d = scale_half(word(key, (uint64_t)b * 32 + 30));
        const uint32_t dm = scale_half(word(key, (uint64_t)b * 32 + 31));
        w0 = (w0 & ~0xFFFFFFFFull) | (uint64_t)(d | (dm << 16));
    }
    uint4 v = make_uint4((uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1, (uint32_t)(w1 >> 32));
    *reinterpret_cast<uint4 *>(dst + ((size_t)e * nb + q) * ORN_Q4K_BYTES + 16 * j) = v;
}

// Q6_K: 13 chunks of the 208-byte body per block, plus the fp16 d (chunk
// 13 writes it).  Scale bytes (192..207, chunk 12) become (byte & 63) - 32.
__global__ void k_synth_q6k(uint8_t *__restrict__ body, uint16_t *__restrict__ dd, uint64_t seed,
                            int layer, int n_e, int nb, int K, int NBc, int file)
{
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_e = (size_t)nb * 14;
    if (t >= per_e * (size_t)n_e) return;
    const int e = (int)(t / per_e);
    const size_t r = t % per_e;
    const int q = (int)(r / 14), j = (int)(r % 14);
    const int b = file ? q : (q % K) * NBc + q / K;
    const uint64_t key = key_of(seed, stream_of(layer, ORN_SYN_DOWN, e));
    if (j == 13) {
        dd[(size_t)e * nb + q] = (uint16_t)scale_half(word(key, (uint64_t)b * 32 + 30));
        return;
    }
    uint64_t w0 = word(key, (uint64_t)b * 32 + 2 * j), w1 = word(key, (uint64_t)b * 32 + 2 * j + 1);
    if (j == 12) {
        auto fix = [](uint64_t w) {
            uint64_t o = 0;
            for (int i = 0; i < 8; ++i) {
                const int v = (int)((w >> (8 * i)) & 63) - 32;
                o |= (uint64_t)(uint8_t)(int8_t)v << (8 * i);
            }
            return o;
        };
        w0 = fix(w0);
        w1 = fix(w1);
    }
    uint4 v = make_uint4((uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1, (uint32_t)(w1 >> 32));
    *reinterpret_cast<uint4 *>(body + ((size_t)e * nb + q) * 208 + 16 * j) = v;
}

// Router: W(d, e) = sigma * normal(i), i = d*E + e (vec@mat order) or
// e*D + d (file orientation), written into the store's [D/4][E][4] layout;
// thread = one (d/4, e) quad.
__device__ __forceinline__ float normal_at(uint64_t key, uint64_t i, double sd)
{
    int64_t s = 0;
    for (int w = 0; w < 3; ++w) {
        const uint64_t x = word(key, 3 * i + (uint64_t)w);
        s += (int64_t)(x & 0xFFFF) + (int64_t)((x >> 16) & 0xFFFF) +
             (int64_t)((x >> 32) & 0xFFFF) + (int64_t)(x >> 48);
    }
    const double z = (double)(s - 393210) * (1.0 / 65536.0);
    return (float)(sd * z);
}

__global__ void k_synth_router(float *__restrict__ wq, uint64_t seed, int layer, int D, int E,
                               float sigma, int file)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (D / 4) * E) return;
    const int d4 = t / E, e = t % E;
    const uint64_t key = key_of(seed, stream_of(layer, ORN_SYN_ROUTER, 0));
    v4f v;
    for (int j = 0; j < 4; ++j) {
        const int d = 4 * d4 + j;
        const uint64_t i = file ? (uint64_t)e * D + d : (uint64_t)d * E + e;
        v[j] = normal_at(key, i, (double)sigma);
    }
    *reinterpret_cast<v4f *>(wq + (size_t)t * 4) = v;
}

// ---------------------------------------------------------------------------
// MFMA layouts from the resident blocks (prefill_pack.c arithmetic).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint16_t int_half(int v)
{
    if (v == 0) return 0;
    uint32_t s = 0;
    if (v < 0) {
        s = 0x8000u;
        v = -v;
    }
    const int e = 31 - __clz(v);
    const uint32_t mant = ((uint32_t)v << (10 - e)) & 0x3FFu;
    return (uint16_t)(s | ((uint32_t)(e + 15) << 10) | mant);
}

__device__ __forceinline__ int q4_at(const uint8_t *qs, int p)
{
    const int c = p / 64, r = p % 64;
    return r < 32 ? (qs[32 * c + r] & 15) : (qs[32 * c + r - 32] >> 4);
}

__device__ __forceinline__ int q6_at(const uint8_t *ql, const uint8_t *qh, int p)
{
    const int n = p / 128, r = p % 128, j = r / 32, l = r % 32;
    const int lo = (j & 1) ? ql[64 * n + l + 32] : ql[64 * n + l];
    const int nib = (j < 2) ? (lo & 15) : (lo >> 4);
    const int hi = (qh[32 * n + l] >> (2 * j)) & 3;
    return (nib | (hi << 4)) - 32;
}

// Non-negative floats order like their bit patterns: max by integer atomics.
// One atomic per wave: every wave of the packers below lies inside one expert
// (its K * NB threads are a multiple of 64), so lane 0 adds the wave's max.
__device__ __forceinline__ void atomic_max_abs(float *p, float v)
{
    unsigned u = __float_as_uint(fabsf(v));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) u = max(u, (unsigned)__shfl_xor((int)u, o, 64));
    if ((threadIdx.x & 63) == 0) atomicMax(reinterpret_cast<unsigned int *>(p), u);
}

__device__ __forceinline__ void atomic_max_wave(int *p, int v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) atomicMax(p, v);
}

// Q4_K nibble words: thread = one 32-bit word (8 values of one column).
// Blocks: [n_e][NB][K] in vec@mat store order (block (k, b) at b*K + k).
__global__ void k_pack_q4k_words(const uint8_t *__restrict__ blocks, uint32_t *__restrict__ qn,
                                 int n_e, int K, int NB, const int *__restrict__ slots)
{
    const size_t per_e = (size_t)K * NB * 32;  // words per expert: K/32 * NB * 4 * 64 * 4
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_e * (size_t)n_e) return;
    const int e = slots ? slots[t / per_e] : (int)(t / per_e);
    size_t w = t % per_e;
    const int ntl = (int)(w % 4);
    w /= 4;
    const int lane = (int)(w % 64);
    w /= 64;
    const int wv = (int)(w % 4);
    w /= 4;
    const int b = (int)(w % NB);
    const int kt = (int)(w / NB);
    const int g = lane / 16, col = lane % 16, nt = 4 * wv + ntl, p = 16 * nt + col;
    const uint8_t *eb = blocks + (size_t)e * K * NB * ORN_Q4K_BYTES;
    uint32_t out = 0;
    for (int ei = 0; ei < 8; ++ei) {
        const int k = 32 * kt + 8 * g + ei;
        const uint8_t *blk = eb + ((size_t)b * K + k) * ORN_Q4K_BYTES;
        out |= (uint32_t)q4_at(blk + ORN_Q4K_OFF_QS, p) << (4 * (ei / 2) + 16 * (ei % 2));
    }
    qn[(size_t)e * (per_e) + (t % per_e)] = out;
}

// Q4_K scales, mins, d, dmin and the per-expert max |d|, |dmin|: thread =
// one block (k, b).
__global__ void k_pack_q4k_scales(const uint8_t *__restrict__ blocks, uint16_t *__restrict__ sc,
                                  uint16_t *__restrict__ mn, float *__restrict__ d,
                                  float *__restrict__ dm, float *__restrict__ dmax, int dmax_col,
                                  int n_e, int K, int NB, const int *__restrict__ slots)
{
    const size_t per_e = (size_t)K * NB;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_e * (size_t)n_e) return;
    const int e = slots ? slots[t / per_e] : (int)(t / per_e);
    const int q = (int)(t % per_e);
    const int b = q / K, k = q % K;
    const uint8_t *blk = blocks + ((size_t)e * per_e + q) * ORN_Q4K_BYTES;
    const float dv = orn_half_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const float dmv = orn_half_to_float((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
    d[(size_t)e * per_e + (size_t)b * K + k] = dv;
    dm[(size_t)e * per_e + (size_t)b * K + k] = dmv;
    atomic_max_abs(&dmax[e * 3 + dmax_col], fmaxf(fabsf(dv), fabsf(dmv)));
    const uint8_t *s = blk + ORN_Q4K_OFF_SCALES;
    const int kt = k / 32, kk = k % 32;
    const size_t base = (size_t)e * (per_e * 8);
    for (int j = 0; j < 8; ++j) {
        int scv, mv;
        if (j < 4) {
            scv = s[j] & 63;
            mv = s[j + 4] & 63;
        } else {
            scv = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            mv = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const size_t o = base + (((size_t)kt * NB + b) * 8 + j) * 32 + kk;
        sc[o] = int_half(scv);
        mn[o] = int_half(mv);
    }
}

// Q6_K q + 32 in the packed 6-bit down layout (ORNK_DQ_UNIT units): thread
// = one lane's pair of column tiles (2jp, 2jp + 1) in one unit, writing the
// two nibble words and the high-bit word they share.
// Bodies: [n_e][NB][K] x 208 B in store order, d separately.
__global__ void k_pack_q6k_bytes(const uint8_t *__restrict__ body, uint8_t *__restrict__ qb,
                                 int n_e, int K, int NB, const int *__restrict__ slots)
{
    const size_t per_e = (size_t)K * NB * 16;  // lane x tile pairs per expert
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_e * (size_t)n_e) return;
    const int e = slots ? slots[t / per_e] : (int)(t / per_e);
    size_t w = t % per_e;
    const int jp = (int)(w % 2);
    w /= 2;
    const int lane = (int)(w % 64);
    w /= 64;
    const int wv = (int)(w % 4);
    w /= 4;
    const int b = (int)(w % NB);
    const int kt = (int)(w / NB);
    const int g = lane / 16, col = lane % 16;
    const uint8_t *eb = body + (size_t)e * K * NB * 208;
    uint32_t nib[2] = {0u, 0u}, hi = 0u;
    for (int h = 0; h < 2; ++h) {
        const int p = 16 * (4 * wv + 2 * jp + h) + col;
        for (int ei = 0; ei < 8; ++ei) {
            const int k = 32 * kt + 8 * g + ei;
            const uint8_t *blk = eb + ((size_t)b * K + k) * 208;
            const uint32_t v = (uint32_t)(q6_at(blk + ORN_Q6K_OFF_QL, blk + ORN_Q6K_OFF_QH, p) + 32);
            nib[h] |= (v & 15u) << (4 * (ei / 2) + 16 * (ei % 2));
            hi |= (v >> 4) << (2 * (ei / 2) + 16 * (ei % 2) + 8 * h);
        }
    }
    uint8_t *unit = qb + (size_t)e * ORNK_DQ_BYTES((size_t)K * NB * 256) +
                    ((size_t)kt * NB + b) * ORNK_DQ_UNIT;
    const int wl = wv * 64 + lane;
    *reinterpret_cast<uint2 *>(unit + wl * 16 + 8 * jp) = make_uint2(nib[0], nib[1]);
    *reinterpret_cast<uint32_t *>(unit + 4096 + wl * 8 + 4 * jp) = hi;
}

// Q6_K scales, d, the per-expert max |d| and the largest |scale|: thread =
// one block.
__global__ void k_pack_q6k_scales(const uint8_t *__restrict__ body, const uint16_t *__restrict__ dd,
                                  uint16_t *__restrict__ sc, float *__restrict__ d,
                                  float *__restrict__ dmax, int *__restrict__ scmax, int n_e,
                                  int K, int NB, const int *__restrict__ slots)
{
    const size_t per_e = (size_t)K * NB;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_e * (size_t)n_e) return;
    const int e = slots ? slots[t / per_e] : (int)(t / per_e);
    const int q = (int)(t % per_e);
    const int b = q / K, k = q % K;
    const uint8_t *blk = body + ((size_t)e * per_e + q) * 208;
    const float dv = orn_half_to_float(dd[(size_t)e * per_e + q]);
    d[(size_t)e * per_e + (size_t)b * K + k] = dv;
    atomic_max_abs(&dmax[e * 3 + 2], dv);
    const int8_t *scs = reinterpret_cast<const int8_t *>(blk + ORN_Q6K_OFF_SCALES);
    const int kt = k / 32, kk = k % 32;
    int mx = 0;
    for (int nt = 0; nt < 16; ++nt) {
        const int v = scs[nt];
        mx = max(mx, v < 0 ? -v : v);
        sc[(size_t)e * (per_e * 16) + (((size_t)kt * NB + b) * 16 + nt) * 32 + kk] = int_half(v);
    }
    atomic_max_wave(scmax, mx);
}

inline dim3 grid_for(size_t n) { return dim3((unsigned)((n + 255) / 256)); }

}  // namespace

extern "C" int ornk_synth_layer(const ornk_synth_args *a, hipStream_t s)
{
    const int E1 = a->n_experts + a->has_shared;
    const int D = a->D, H = a->H;
    const int nb = D * H / 256;
    if (D % 256 || H % 256 || E1 < 1) return hipErrorInvalidValue;
    // gate/up: K = D rows of M = H outputs; down: K = H rows of M = D outputs
    hipLaunchKernelGGL(k_synth_q4k, grid_for((size_t)E1 * nb * 9), dim3(256), 0, s, a->gate,
                       a->seed, a->layer, (int)ORN_SYN_GATE, E1, nb, D, H / 256, a->file);
    hipLaunchKernelGGL(k_synth_q4k, grid_for((size_t)E1 * nb * 9), dim3(256), 0, s, a->up,
                       a->seed, a->layer, (int)ORN_SYN_UP, E1, nb, D, H / 256, a->file);
    hipLaunchKernelGGL(k_synth_q6k, grid_for((size_t)E1 * nb * 14), dim3(256), 0, s, a->down_body,
                       a->down_d, a->seed, a->layer, E1, nb, H, D / 256, a->file);
    hipLaunchKernelGGL(k_synth_router, grid_for((size_t)(D / 4) * a->n_experts), dim3(256), 0, s,
                       a->router, a->seed, a->layer, D, a->n_experts, 0.02f, a->file);
    return hipGetLastError();
}

extern "C" int ornk_pack_prefill(const ornk_pack_args *a, hipStream_t s)
{
    const int D = a->D, H = a->H, n = a->n_e;
    const size_t DH = (size_t)D * H;
    if (D % 256 || H % 256 || n < 1) return hipErrorInvalidValue;
    // with a slot list the caller has zeroed the slots' dmax entries
    if (!a->slots) hipMemsetAsync(a->dmax, 0, (size_t)n * 3 * sizeof(float), s);
    hipMemsetAsync(a->scmax, 0, sizeof(int), s);
    for (int m = 0; m < 2; ++m) {
        hipLaunchKernelGGL(k_pack_q4k_words, grid_for((size_t)n * DH / 8), dim3(256), 0, s,
                           a->gu[m], a->pq[m], n, D, H / 256, a->slots);
        hipLaunchKernelGGL(k_pack_q4k_scales, grid_for((size_t)n * DH / 256), dim3(256), 0, s,
                           a->gu[m], a->psc[m], a->pmn[m], a->pd[m], a->pdm[m], a->dmax, m, n, D,
                           H / 256, a->slots);
    }
    hipLaunchKernelGGL(k_pack_q6k_bytes, grid_for((size_t)n * DH / 16), dim3(256), 0, s,
                       a->down_body, a->dq, n, H, D / 256, a->slots);
    hipLaunchKernelGGL(k_pack_q6k_scales, grid_for((size_t)n * DH / 256), dim3(256), 0, s,
                       a->down_body, a->down_d, a->dsc, a->dd, a->dmax, a->scmax, n, H, D / 256,
                       a->slots);
    return hipGetLastError();
}
