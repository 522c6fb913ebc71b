/* SPDX-License-Identifier: MIT
 *
 * Prefill (MFMA) layouts of the expert matrices, built on the host when an
 * expert is uploaded.  They hold the same quantized values as the GGUF
 * blocks, rearranged so that one 32-bit (Q4_K) or 64-bit (Q6_K) load gives a
 * lane the eight reduction-dimension values of one output column that a
 * v_mfma_f32_16x16x32_f16 B operand needs, plus the per-row scales in a form
 * the kernels use directly:
 *
 *   B[k][n] = sc(k, n) * q(k, n)   exact in fp16 (|B| <= 945 for Q4_K,
 *                                   <= 2048 for Q6_K when |sc| <= 64; the
 *                                   down kernels split larger ones in two)
 *   W[k][n] = d(k, b) * B[k][n] - dmin(k, b) * m(k, n)     (Q4_K, gguf.c:43-61)
 *   W[k][n] = d(k, b) * B[k][n]                            (Q6_K, gguf.c:64-86)
 *
 * with b = n / 256 the block column, d and dmin decoded with the reference's
 * fp16 rule (gguf.c:16-26).
 *
 * Lane l of a 16x16x32 B operand holds k = 8*(l/16) + e (e = 0..7) of
 * column l % 16.  Q4_K words place value e at bit 4*(e/2) + 16*(e%2), so
 * ((w >> 4i) & 0x000F000F) | 0x64006400 is the fp16 pair (1024 + q_{2i},
 * 1024 + q_{2i+1}).  Q6_K stores the 6-bit q + 32 split the same way: its
 * low four bits in a word of that order, its high two bits in a second word
 * (value e at bit 2*(e/2) + 16*(e%2), one byte per half-word per tile, two
 * tiles per word), so one v_bfi and an OR give the pair.
 *
 * A kernel wave covers the four 16-column tiles 4w..4w+3 of a 256-column
 * block, so the words of those four tiles sit side by side per lane:
 * [K/32][M/256][4 w][64 lanes][4 tiles] -- one 16-byte load per lane and
 * reduction step for Q4_K; for Q6_K one 16-byte load of nibble words and one
 * 8-byte load of high-bit words from the step's 6144-byte unit
 * (ORNK_DQ_UNIT: 4096 bytes of nibbles, then 2048 of high bits).
 */
#include "internal.h"

#include <stdlib.h>
#include <string.h>

/* gguf.c:16-26: 0 -> 0, otherwise exponent bias 112 for every pattern. */
float orn_quirk_half(uint16_t h)
{
    if (h == 0) return 0.0f;
    uint32_t u = ((uint32_t)(h & 0x8000u) << 16) | ((((h & 0x7C00u) >> 10) + 112u) << 23) |
                 ((uint32_t)(h & 0x03FFu) << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* IEEE binary16 bits of an integer |v| <= 2048 (exact). */
static uint16_t int_half(int v)
{
    if (v == 0) return 0;
    uint16_t s = 0;
    if (v < 0) {
        s = 0x8000u;
        v = -v;
    }
    int e = 0;
    while ((v >> (e + 1)) != 0) ++e;           /* e = floor(log2 v) */
    const uint32_t mant = ((uint32_t)v << (10 - e)) & 0x3FFu;
    return (uint16_t)(s | ((uint32_t)(e + 15) << 10) | mant);
}

/* gguf.c:31-40 */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Quant of output position p (0..255) of a Q4_K block (gguf.c:43-61). */
static int q4_at(const uint8_t *qs, int p)
{
    const int c = p / 64, r = p % 64;
    return r < 32 ? (qs[32 * c + r] & 15) : (qs[32 * c + r - 32] >> 4);
}

/* Quant (-32..31) of output position p of a Q6_K block (gguf.c:64-86). */
static int q6_at(const uint8_t *ql, const uint8_t *qh, int p)
{
    const int n = p / 128, r = p % 128, j = r / 32, l = r % 32;
    const int lo = (j & 1) ? ql[64 * n + l + 32] : ql[64 * n + l];
    const int nib = (j < 2) ? (lo & 15) : (lo >> 4);
    const int hi = (qh[32 * n + l] >> (2 * j)) & 3;
    return (nib | (hi << 4)) - 32;
}

void orn_pack_q4k_prefill(const uint8_t *blocks, int K, int M, uint32_t *qn, uint16_t *sc,
                          uint16_t *mn, float *d, float *dm, float *dmax)
{
    const int NB = M / 256, KT = K / 32;
    float mx = 0.0f;
    memset(qn, 0, (size_t)KT * NB * 16 * 64 * 4);
    for (int k = 0; k < K; ++k) {
        const int kt = k / 32, kk = k % 32, g = kk / 8, e = kk % 8;
        const int shift = 4 * (e / 2) + 16 * (e % 2);
        for (int b = 0; b < NB; ++b) {
            const uint8_t *blk = blocks + ((size_t)k * NB + b) * ORN_Q4K_BYTES;
            const float dv = orn_quirk_half((uint16_t)(blk[0] | (blk[1] << 8)));
            const float dmv = orn_quirk_half((uint16_t)(blk[2] | (blk[3] << 8)));
            d[(size_t)b * K + k] = dv;
            dm[(size_t)b * K + k] = dmv;
            if (dv == dv && dv > mx) mx = dv;
            if (dv == dv && -dv > mx) mx = -dv;
            if (dmv == dmv && dmv > mx) mx = dmv;
            if (dmv == dmv && -dmv > mx) mx = -dmv;
            for (int s = 0; s < 8; ++s) {
                int scv, mv;
                scale_min_k4(s, blk + ORN_Q4K_OFF_SCALES, &scv, &mv);
                const size_t o = (((size_t)kt * NB + b) * 8 + s) * 32 + kk;
                sc[o] = int_half(scv);
                mn[o] = int_half(mv);
            }
            const uint8_t *qs = blk + ORN_Q4K_OFF_QS;
            for (int p = 0; p < 256; ++p) {
                const int nt = p / 16, col = p % 16;
                const size_t w =
                    ((((size_t)kt * NB + b) * 4 + nt / 4) * 64 + 16 * g + col) * 4 + nt % 4;
                qn[w] |= (uint32_t)q4_at(qs, p) << shift;
            }
        }
    }
    *dmax = mx;
}

int orn_pack_q6k_prefill(const uint8_t *blocks, int K, int M, uint8_t *qb, uint16_t *sc, float *d,
                         float *dmax)
{
    const int NB = M / 256;
    int scmax = 0;
    float mx = 0.0f;
    memset(qb, 0, ORNK_DQ_BYTES((size_t)K * M));
    for (int k = 0; k < K; ++k) {
        const int kt = k / 32, kk = k % 32, g = kk / 8, e = kk % 8;
        for (int b = 0; b < NB; ++b) {
            const uint8_t *blk = blocks + ((size_t)k * NB + b) * ORN_Q6K_BYTES;
            const uint8_t *ql = blk + ORN_Q6K_OFF_QL, *qh = blk + ORN_Q6K_OFF_QH;
            const int8_t *scs = (const int8_t *)(blk + ORN_Q6K_OFF_SCALES);
            const float dv =
                orn_quirk_half((uint16_t)(blk[ORN_Q6K_OFF_D] | (blk[ORN_Q6K_OFF_D + 1] << 8)));
            d[(size_t)b * K + k] = dv;
            if (dv == dv && dv > mx) mx = dv;
            if (dv == dv && -dv > mx) mx = -dv;
            for (int nt = 0; nt < 16; ++nt) {
                const int v = scs[nt];
                if (v > scmax) scmax = v;
                if (-v > scmax) scmax = -v;
                sc[(((size_t)kt * NB + b) * 16 + nt) * 32 + kk] = int_half(v);
            }
            uint8_t *unit = qb + ((size_t)kt * NB + b) * ORNK_DQ_UNIT;
            for (int p = 0; p < 256; ++p) {
                const int nt = p / 16, col = p % 16, wl = (nt / 4) * 64 + 16 * g + col;
                const uint32_t v = (uint32_t)(q6_at(ql, qh, p) + 32);
                uint32_t *nw = (uint32_t *)(unit + (size_t)wl * 16) + nt % 4;
                uint32_t *hw = (uint32_t *)(unit + 4096 + (size_t)wl * 8) + (nt % 4) / 2;
                *nw |= (v & 15u) << (4 * (e / 2) + 16 * (e % 2));
                *hw |= (v >> 4) << (2 * (e / 2) + 16 * (e % 2) + 8 * (nt % 2));
            }
        }
    }
    *dmax = mx;
    return scmax;
}
