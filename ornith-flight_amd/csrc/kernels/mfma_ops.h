// SPDX-License-Identifier: MIT
//
// Operand preparation for the expert products on the matrix cores
// (v_mfma_f32_16x16x32_f16), shared by the prefill- and decode-shaped
// kernels.
//
// Arithmetic (all exact except the activation split and fp32 accumulation):
//   Q4_K (gguf.c:43-61):  W[k][n] = d(k,b) * (sc*q)[k][n] - dmin(k,b) * m[k][n]
//   Q6_K (gguf.c:64-86):  W[k][n] = d(k,b) * (sc*q)[k][n]
//   y[r][n] = sum_k x[r][k] * W[k][n]
//           = sum_k A[r][k] * B[k][n] - sum_k Am[r][k] * m[k][n]
// with B = sc*q (an integer, |B| <= 945 for Q4_K and <= 2048 for Q6_K when
// |sc| <= 64, so exact in fp16; larger Q6_K scales add an exact correction
// operand, q6_b2), A = x*d and Am = x*dmin.  A is scaled per
// row by a power of two s_r (|A| < 2^14, no fp16 overflow) and split into
// fp16 hi + lo (hi = A rounded toward zero, lo = the exact remainder rounded
// toward zero): A = hi + lo to about 2^-21 relative, so two MFMAs (hi, lo)
// per tile give fp32-class products; the sums accumulate in fp32 and the
// result is scaled back by 1/s_r (exact).
//
// Operand lane layout of v_mfma_f32_16x16x32_f16 (lane l, e = 0..7):
//   A: row l % 16, k = 8*(l/16) + e;   B: column l % 16, k = 8*(l/16) + e;
//   C: column l % 16, rows 4*(l/16) + r (r = 0..3).
#pragma once

#include "common.h"

namespace orn_mfma {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

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

// (a0, a1) -> hi = rtz fp16, lo = rtz fp16 of the remainder a - hi, which is
// exact in fp32 (hi is a truncation of a).  The remainder is one
// v_fma_mix_f32 per value: hi's fp16 half times -1 plus a (the compiler
// would otherwise turn fma(hi, -1, a) into a convert and a subtract).
__device__ __forceinline__ void split2(float a0, float a1, uint32_t &hi, uint32_t &lo)
{
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a0, a1));
    float r0, r1;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r0) : "v"(h), "v"(a0));
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r1) : "v"(h), "v"(a1));
    hi = h;
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

// (w & 0x000F000F) | 0x64006400 in one instruction: the fp16 pair
// (1024 + low nibble of the low half, 1024 + low nibble of the high half).
__device__ __forceinline__ uint32_t magic_pair(uint32_t w)
{
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(0x000F000Fu), "v"(w), "v"(0x64006400u));
    return r;
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
        const v2h q = as_v2h(magic_pair(w >> (4 * i)));
        const v2h sv = as_v2h(s[i]);
        const v2h ns = sv * (v2h){(_Float16)-1024.0f, (_Float16)-1024.0f};
        o[i] = as_u32(__builtin_elementwise_fma(q, sv, ns));
    }
    return to_v8h(o[0], o[1], o[2], o[3]);
}

// Packed 6-bit Q6_K values of one lane and column tile (the down layout of
// prefill_pack.c): nw holds the low four bits of the 8 values (value e at
// bit 4*(e/2) + 16*(e%2), the v_bfi pair order of magic_pair), cw the high
// two bits (value e at bit 2*(e/2) + 16*(e%2)).  Pair i = values (2i, 2i+1)
// as the fp16 pair (1024 + (q + 32)): the nibbles through one v_bfi, the
// high bits into bits 4-5 of each half.
__device__ __forceinline__ void q6_pairs(uint32_t nw, uint32_t cw, uint32_t (&p)[4])
{
#pragma unroll
    for (int i = 0; i < 4; ++i)
        p[i] = magic_pair(nw >> (4 * i)) | (((cw >> (2 * i)) & 0x00030003u) << 4);
}

// Q6_K B operand from the pairs p (k order) and sc as above.  B = sc * q
// with q = (1024 + (q + 32)) - 1056 exact and |sc * q| <= 2048.
__device__ __forceinline__ v8h q6_b(const uint32_t (&p)[4], uint4 sc)
{
    const uint32_t s[4] = {sc.x, sc.y, sc.z, sc.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2h qv = as_v2h(p[i]) + (v2h){(_Float16)-1056.0f, (_Float16)-1056.0f};
        o[i] = as_u32(qv * as_v2h(s[i]));
    }
    return to_v8h(o[0], o[1], o[2], o[3]);
}

// Q6_K B operand for any sub-scale (|sc| <= 128, as real quantizers emit):
// B = sc * q (|B| <= 4096) as b1 + b2 with b1 = fp16(sc * q) rounded to
// nearest and b2 = sc * q - b1 from one fma, exact (an integer of magnitude
// <= 1: fp16 holds every integer up to 2048 and every even one up to 4096).
// The kernels add A_hi*b1 + A_lo*b1 + A_hi*b2; the dropped A_lo*b2 is below
// 2^-21 of |A*B|, the order of the activation split itself.
__device__ __forceinline__ void q6_b2(const uint32_t (&p)[4], uint4 sc, v8h &b1, v8h &b2)
{
    const uint32_t s[4] = {sc.x, sc.y, sc.z, sc.w};
    uint32_t o1[4], o2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2h qv = as_v2h(p[i]) + (v2h){(_Float16)-1056.0f, (_Float16)-1056.0f};
        const v2h sv = as_v2h(s[i]);
        const v2h bh = qv * sv;
        o1[i] = as_u32(bh);
        o2[i] = as_u32(__builtin_elementwise_fma(qv, sv, -bh));
    }
    b1 = to_v8h(o1[0], o1[1], o1[2], o1[3]);
    b2 = to_v8h(o2[0], o2[1], o2[2], o2[3]);
}

__device__ __forceinline__ v4f mfma(v8h a, v8h b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Row scale of the file-orientation activations: the power of two s with
// amax * s in [2^13, 2^14); 1 for 0 or non-finite.
__device__ __forceinline__ float prep_scale(float amax)
{
    if (!(amax > 0.0f) || !(amax <= 3.0e38f)) return 1.0f;
    int e = 13 - ilogbf(amax);
    e = e < -126 ? -126 : (e > 126 ? 126 : e);
    return ldexpf(1.0f, e);
}

}  // namespace orn_mfma
