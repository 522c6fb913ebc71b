"""Vectorised numpy decoders of Q4_K / Q6_K super-blocks into their integer
and scale components (test infrastructure).

The components are what the reference's dequantization multiplies together
(engine/src/gguf.c:43-61 for Q4_K, gguf.c:64-86 for Q6_K, with the fp16
rule of gguf.c:16-26 and the 6-bit scale unpacking of gguf.c:31-40).  Each
decoder also rebuilds the fp32 weights from its components in the
reference's operation order, and tests/test_mfma_emulation.py checks those
against the oracle bit for bit, so the components are pinned by the same
goldens that pin the oracle's dequantization.

Element p of a block (0..255) is flat element 256*block + p.
"""
import numpy as np


def quirk_half(bits):
    """gguf.c:16-26 on an array of uint16 patterns: 0 -> 0, every other
    pattern as a normal number with exponent bias 112."""
    h = np.asarray(bits).astype(np.uint32) & 0xFFFF
    u = ((h & 0x8000) << 16) | ((((h & 0x7C00) >> 10) + 112) << 23) | ((h & 0x03FF) << 13)
    u = np.where(h == 0, 0, u).astype(np.uint32)
    return u.view(np.float32)


def _half_at(b, off):
    return quirk_half(b[:, off].astype(np.uint32) | (b[:, off + 1].astype(np.uint32) << 8))


def q4k_components(blocks):
    """blocks: uint8 [n*144] -> (d [n], dmin [n], sc [n,256], m [n,256], q [n,256]).

    sc, m and q are per element (sc and m repeat over each 32-value sub-block)."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 144)
    n = b.shape[0]
    d, dmin = _half_at(b, 0), _half_at(b, 2)
    s = b[:, 4:16].astype(np.int64)
    sc8 = np.empty((n, 8), np.int64)
    m8 = np.empty((n, 8), np.int64)
    for j in range(8):  # gguf.c:31-40
        if j < 4:
            sc8[:, j] = s[:, j] & 63
            m8[:, j] = s[:, j + 4] & 63
        else:
            sc8[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            m8[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = b[:, 16:].astype(np.int64)
    q = np.empty((n, 256), np.int64)
    for c in range(4):  # 64 values per 32 bytes: low nibbles, then high nibbles
        q[:, 64 * c:64 * c + 32] = qs[:, 32 * c:32 * c + 32] & 15
        q[:, 64 * c + 32:64 * c + 64] = qs[:, 32 * c:32 * c + 32] >> 4
    sub = np.arange(256) // 32
    return d, dmin, sc8[:, sub], m8[:, sub], q


def q4k_weights(comp):
    """fp32 weights in the reference's order: (d*sc)*q - dmin*m, one rounding."""
    d, dmin, sc, m, q = comp
    d1 = d[:, None] * sc.astype(np.float32)
    m1 = dmin[:, None] * m.astype(np.float32)
    return (d1 * q.astype(np.float32) - m1).astype(np.float32)


def q6k_components(blocks):
    """blocks: uint8 [n*210] -> (d [n], sc [n,256] int8 values, q [n,256] in -32..31)."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 210)
    n = b.shape[0]
    ql = b[:, 0:128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    scs = b[:, 192:208].view(np.int8).astype(np.int64)
    d = _half_at(b, 208)
    q = np.empty((n, 256), np.int64)
    sc = np.empty((n, 256), np.int64)
    l = np.arange(32)
    for h in range(2):  # two halves of 128 values
        L, Q, S = ql[:, 64 * h:64 * h + 64], qh[:, 32 * h:32 * h + 32], scs[:, 8 * h:8 * h + 8]
        parts = ((L[:, l] & 15), (L[:, l + 32] & 15), (L[:, l] >> 4), (L[:, l + 32] >> 4))
        for j in range(4):
            q[:, 128 * h + 32 * j + l] = (parts[j] | (((Q[:, l] >> (2 * j)) & 3) << 4)) - 32
            sc[:, 128 * h + 32 * j + l] = S[:, (l // 16) + 2 * j]
    return d, sc, q


def q6k_weights(comp):
    """fp32 weights in the reference's order: (d*sc)*q (exact)."""
    d, sc, q = comp
    return ((d[:, None] * sc.astype(np.float32)) * q.astype(np.float32)).astype(np.float32)


def vecmat(flat, K, M):
    """Flat element k*M + i of a [K x M] matrix (the reference's vec@mat
    reading, engine/src/model.c:351-357) -> array [K, M]."""
    return np.asarray(flat).reshape(K, M)
