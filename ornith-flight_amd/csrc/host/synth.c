/* SPDX-License-Identifier: MIT
 *
 * Deterministic synthetic workload generator (host).
 *
 * word(key, i) = fmix(key + (i+1)*G): the i-th SplitMix64 output of a
 * stream keyed by (seed, stream id), so every block of every tensor is an
 * independent pure function of its coordinates.  Quantized blocks are built
 * from integers only; the two fp16 super-scales are U(0.001, 0.01) computed
 * in double (one multiply, one add) and rounded to nearest-even half.
 * Normals are Irwin-Hall sums of 12 16-bit uniforms, which are exact binary
 * fractions, scaled by sigma with one double->float rounding.
 * Build with -ffp-contract=off so the double arithmetic is never fused.
 */
#include "../../../include/ornith/ornith_hip.h"

#include <math.h>
#include <string.h>

#define ORN_G 0x9E3779B97F4A7C15ull

static uint64_t fmix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t key_of(uint64_t seed, uint64_t stream)
{
    return fmix(fmix(seed + ORN_G) ^ (stream * ORN_G + ORN_G));
}

static uint64_t word(uint64_t key, uint64_t i) { return fmix(key + (i + 1) * ORN_G); }

uint64_t orn_synth_stream(int layer, int kind, int expert)
{
    return ((uint64_t)(uint32_t)layer << 32) | ((uint64_t)(kind & 0xFF) << 24) |
           (uint64_t)(expert & 0xFFFFFF);
}

/* Round a positive double in the normal fp16 range to the nearest-even half. */
static uint16_t half_rne(double v)
{
    uint64_t b;
    memcpy(&b, &v, sizeof b);
    int ex = (int)((b >> 52) & 0x7FF) - 1023;
    uint64_t m = (b & ((1ull << 52) - 1)) | (1ull << 52); /* 53-bit significand */
    uint64_t keep = m >> 42;                              /* 11 bits */
    uint64_t rem = m & ((1ull << 42) - 1);
    const uint64_t halfway = 1ull << 41;
    if (rem > halfway || (rem == halfway && (keep & 1))) ++keep;
    if (keep == (1ull << 11)) {
        keep >>= 1;
        ++ex;
    }
    return (uint16_t)((((unsigned)(ex + 15)) << 10) | (unsigned)(keep & 0x3FF));
}

static uint16_t scale_half(uint64_t w)
{
    double u = (double)(uint32_t)w * (1.0 / 4294967296.0);
    double v = 0.009 * u;
    v = 0.001 + v;
    return half_rne(v);
}

static void put_words(uint8_t *dst, uint64_t key, uint64_t base, int n_bytes)
{
    for (int i = 0; i < n_bytes; i += 8) {
        uint64_t w = word(key, base + (uint64_t)(i / 8));
        for (int b = 0; b < 8 && i + b < n_bytes; ++b) dst[i + b] = (uint8_t)(w >> (8 * b));
    }
}

void orn_synth_q4k(uint64_t seed, uint64_t stream, uint64_t first_block, uint64_t n_blocks,
                   void *out)
{
    const uint64_t key = key_of(seed, stream);
    uint8_t *o = (uint8_t *)out;
    for (uint64_t i = 0; i < n_blocks; ++i) {
        const uint64_t b = first_block + i;
        uint8_t *blk = o + i * ORN_Q4K_BYTES;
        put_words(blk, key, b * 32, ORN_Q4K_BYTES);
        uint16_t d = scale_half(word(key, b * 32 + 30));
        uint16_t dm = scale_half(word(key, b * 32 + 31));
        blk[0] = (uint8_t)d;
        blk[1] = (uint8_t)(d >> 8);
        blk[2] = (uint8_t)dm;
        blk[3] = (uint8_t)(dm >> 8);
    }
}

void orn_synth_q6k(uint64_t seed, uint64_t stream, uint64_t first_block, uint64_t n_blocks,
                   void *out)
{
    const uint64_t key = key_of(seed, stream);
    uint8_t *o = (uint8_t *)out;
    for (uint64_t i = 0; i < n_blocks; ++i) {
        const uint64_t b = first_block + i;
        uint8_t *blk = o + i * ORN_Q6K_BYTES;
        put_words(blk, key, b * 32, 208);
        for (int s = 0; s < 16; ++s) {
            int v = (int)(blk[ORN_Q6K_OFF_SCALES + s] & 63) - 32;
            blk[ORN_Q6K_OFF_SCALES + s] = (uint8_t)(int8_t)v;
        }
        uint16_t d = scale_half(word(key, b * 32 + 30));
        blk[ORN_Q6K_OFF_D] = (uint8_t)d;
        blk[ORN_Q6K_OFF_D + 1] = (uint8_t)(d >> 8);
    }
}

void orn_synth_normal(uint64_t seed, uint64_t stream, uint64_t n, float sigma, float *out)
{
    const uint64_t key = key_of(seed, stream);
    const double sd = (double)sigma;
    for (uint64_t i = 0; i < n; ++i) {
        int64_t s = 0;
        for (int w = 0; w < 3; ++w) {
            uint64_t x = word(key, 3 * i + (uint64_t)w);
            s += (int64_t)(x & 0xFFFF) + (int64_t)((x >> 16) & 0xFFFF) +
                 (int64_t)((x >> 32) & 0xFFFF) + (int64_t)(x >> 48);
        }
        double z = (double)(s - 393210) * (1.0 / 65536.0);
        out[i] = (float)(sd * z);
    }
}

void orn_synth_zipf_bias(uint64_t seed, uint64_t stream, int n_experts, float s, float *out)
{
    if (n_experts <= 0) return;
    const uint64_t key = key_of(seed, stream);
    int rank[1024];
    int n = n_experts < 1024 ? n_experts : 1024;
    for (int i = 0; i < n; ++i) rank[i] = i + 1;
    for (int i = n - 1; i > 0; --i) {
        int j = (int)(word(key, (uint64_t)i) % (uint64_t)(i + 1));
        int t = rank[i];
        rank[i] = rank[j];
        rank[j] = t;
    }
    for (int e = 0; e < n; ++e) out[e] = (float)(-(double)s * log((double)rank[e]));
}
