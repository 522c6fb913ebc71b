"""CPU checks of the prefill (MFMA) layouts built by prefill_pack.c.

Every weight W[k][n] of an expert matrix is rebuilt from the packed arrays
exactly as the MFMA kernels use them (d * (sc*q) - dmin * m for Q4_K,
d * (sc*q) for Q6_K, with q taken from the lane-ordered words) and compared
bit for bit with the oracle's dequantization of the original GGUF blocks
(gguf.c:43-86).  The packers are internal symbols of libornith_hip (not part
of the C API); no GPU is needed.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

Q4, Q6 = 12, 14  # ggml type ids


@pytest.fixture(scope="module")
def L():
    import ornith_moe
    lib = ornith_moe.lib()
    f = lib.orn_pack_q4k_prefill
    f.restype = None
    f.argtypes = [C.c_void_p, C.c_int, C.c_int] + [C.c_void_p] * 6
    g = lib.orn_pack_q6k_prefill
    g.restype = C.c_int
    g.argtypes = [C.c_void_p, C.c_int, C.c_int] + [C.c_void_p] * 4
    return lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def f16(u16):
    return u16.view(np.float16).astype(np.float64)


def test_q4k_prefill_layout_rebuilds_weights(L):
    import ornith_moe as om
    K, M = 64, 512
    nb = K * M // 256
    blocks = om.synth_q4k(5, om.synth_stream(0, om.SYN_GATE, 3), nb)
    # exercise the fp16 quirk and zero scales too
    blocks = blocks.reshape(nb, 144).copy()
    blocks[0, 0:2] = [0x00, 0x00]          # d = 0
    blocks[1, 2:4] = [0x01, 0x00]          # dmin: a subnormal pattern (quirk: 2^-15*(1+1/1024))
    blocks[2, 4:16] = 0                    # all sub-block scales and mins 0
    blocks = blocks.reshape(-1)
    KT, NB = K // 32, M // 256
    qn = np.zeros(KT * NB * 16 * 64, np.uint32)
    sc = np.zeros(KT * NB * 8 * 32, np.uint16)
    mn = np.zeros_like(sc)
    d = np.zeros(NB * K, np.float32)
    dm = np.zeros_like(d)
    dmax = np.zeros(1, np.float32)
    L.orn_pack_q4k_prefill(_p(blocks), K, M, _p(qn), _p(sc), _p(mn), _p(d), _p(dm), _p(dmax))

    ok, ref = O.dequant_tensor(blocks, Q4, K * M)
    assert ok
    ref = ref.reshape(K, M)
    W = np.zeros((K, M), np.float64)
    qn5 = qn.reshape(KT, NB, 4, 64, 4)  # [step][block column][wave][lane][tile]
    sc4 = f16(sc).reshape(KT, NB, 8, 32)
    mn4 = f16(mn).reshape(KT, NB, 8, 32)
    d2, dm2 = d.reshape(NB, K).astype(np.float64), dm.reshape(NB, K).astype(np.float64)
    for k in range(K):
        kt, kk = divmod(k, 32)
        g, e = divmod(kk, 8)
        shift = 4 * (e // 2) + 16 * (e % 2)
        for n in range(M):
            b, p = divmod(n, 256)
            nt, c = divmod(p, 16)
            q = (int(qn5[kt, b, nt // 4, 16 * g + c, nt % 4]) >> shift) & 15
            s = p // 32
            W[k, n] = d2[b, k] * (sc4[kt, b, s, kk] * q) - dm2[b, k] * mn4[kt, b, s, kk]
    assert np.array_equal(W.astype(np.float32).view(np.uint32), ref.view(np.uint32))
    assert dmax[0] == max(np.abs(d).max(), np.abs(dm).max())
    # the B operand values sc*q are integers <= 945 (exact in fp16)
    assert sc4.max() <= 63 and mn4.max() <= 63


def test_q6k_prefill_layout_rebuilds_weights(L):
    import ornith_moe as om
    K, M = 64, 512
    nb = K * M // 256
    blocks = om.synth_q6k(6, om.synth_stream(0, om.SYN_DOWN, 2), nb).reshape(nb, 210).copy()
    blocks[3, 192 + 5] = np.uint8(100)       # one sub-scale above 64 -> reported
    blocks[4, 208:210] = [0x00, 0x00]        # d = 0
    blocks = blocks.reshape(-1)
    KT, NB = K // 32, M // 256
    qb = np.full(KT * NB * 6144, 0xFF, np.uint8)  # the packer clears what it ORs into
    sc = np.zeros(KT * NB * 16 * 32, np.uint16)
    d = np.zeros(NB * K, np.float32)
    dmax = np.zeros(1, np.float32)
    scmax = L.orn_pack_q6k_prefill(_p(blocks), K, M, _p(qb), _p(sc), _p(d), _p(dmax))
    assert scmax == 100

    ok, ref = O.dequant_tensor(blocks, Q6, K * M)
    assert ok
    ref = ref.reshape(K, M)
    # 6144-byte unit per [step][block column]: nibble words [wave][lane][tile],
    # then high-bit words [wave][lane][tile pair]
    unit = qb.reshape(KT, NB, 6144)
    nib = unit[..., :4096].copy().view(np.uint32).reshape(KT, NB, 4, 64, 4)
    hib = unit[..., 4096:].copy().view(np.uint32).reshape(KT, NB, 4, 64, 2)

    def q6(kt, b, w, l, j, e):
        sh = 4 * (e // 2) + 16 * (e % 2)
        hs = 2 * (e // 2) + 16 * (e % 2) + 8 * (j % 2)
        return int((nib[kt, b, w, l, j] >> sh) & 15) | (int((hib[kt, b, w, l, j // 2] >> hs) & 3) << 4)

    sc4 = f16(sc).reshape(KT, NB, 16, 32)
    d2 = d.reshape(NB, K).astype(np.float64)
    W = np.zeros((K, M), np.float64)
    for k in range(K):
        kt, kk = divmod(k, 32)
        g, e = divmod(kk, 8)
        for n in range(M):
            b, p = divmod(n, 256)
            nt, c = divmod(p, 16)
            q = q6(kt, b, nt // 4, 16 * g + c, nt % 4, e) - 32
            W[k, n] = d2[b, k] * (sc4[kt, b, nt, kk] * q)
    assert np.array_equal(W.astype(np.float32).view(np.uint32), ref.view(np.uint32))


def test_q6_wide_operand_split_is_exact():
    """The down kernels' operand for Q6_K sub-scales above 64 (mfma_ops.h
    q6_b2, expert_file.hip k_dn_file): b1 = fp16(sc * q) rounded to nearest
    even, b2 = sc * q - b1 from one fma.  Over every int8 scale and every
    q - 32 in [-32, 31]: b2 is an integer of magnitude <= 1 (exact in fp16),
    b1 + b2 == sc * q, and b2 == 0 exactly where |sc * q| <= 2048 or the
    product is even; the products that need b2 occur (so a kernel that
    dropped it would be wrong on real scales)."""
    sc = np.arange(-128, 128, dtype=np.int64)[:, None]
    q = np.arange(-32, 32, dtype=np.int64)[None, :]
    exact = sc * q
    # fp16 products of two fp16 integers: one rounding of the exact value
    b1 = (sc.astype(np.float16) * q.astype(np.float16)).astype(np.float64)
    assert np.all(np.isfinite(b1))
    b2 = exact - b1
    assert np.all(b2 == np.round(b2)) and np.abs(b2).max() <= 1
    assert np.all(b2.astype(np.float16).astype(np.float64) == b2)
    assert np.all(b1 + b2 == exact)
    small = (np.abs(exact) <= 2048) | (exact % 2 == 0)
    assert np.all(b2[small] == 0) and np.all(b2[~small] != 0)
    assert (~small).sum() > 0 and np.abs(sc).max() == 128
