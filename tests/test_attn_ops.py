"""The attention-side gpu.h ops: gpu_rope, gpu_attention, and the Metal
shader steps with no gpu.h declaration (gpu_deltanet_step_gated,
gpu_kv_cache_append).  Semantics: ops.metal:113-139 and attention.metal:17-125
as dispatched by gpu_metal.m:495-583; gpu_deltanet_step stays a no-op, as in
both reference backends.

CPU: the oracle's restatements (orc_rope, orc_attention, orc_deltanet_step)
against fp64 mathematics -- a complex rotation with the same frequency and
angle, softmax(QK^T/sqrt(d))V, the recurrence -- and special cases (pos 0 is
the identity, dims past 64 untouched, one key returns V, equal keys return
the mean of V, gate 1 keeps the state, gate 0 makes it outer(v, k)).

GPU: each op against the oracle.  RoPE within a few ulp (the device's and
glibc's cos/sin), attention within 2e-6 relative (the device sums in another
order and shifts the exponent by the running maximum), the DeltaNet step and
the append bit for bit.  Where the shader's unshifted exp overflows (scores
above 88) the device still returns the softmax; that case is checked against
fp64.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def rope64(x, pos, theta):
    """fp64 complex rotation with the float32 angle the ops compute."""
    x = np.asarray(x, np.float64)
    hd = x.shape[1]
    rot = min(hd, 64)
    y = x.copy()
    for i in range(0, rot - 1, 2):
        inv = np.float32(1.0 / (float(theta) ** (i / rot)))
        ang = np.float32(np.float32(pos) * inv)
        z = (x[:, i] + 1j * x[:, i + 1]) * np.exp(1j * np.float64(ang))
        y[:, i], y[:, i + 1] = z.real, z.imag
    return y


def attention64(Q, K, V):
    s = (Q.astype(np.float64) @ K.astype(np.float64).T) / np.sqrt(Q.shape[1])
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(axis=1, keepdims=True)) @ V.astype(np.float64)


# ------------------------------------------------------------ oracle pins
@pytest.mark.parametrize("hd,pos,theta", [(256, 0, 1e7), (256, 7, 1e7), (256, 4095, 1e7),
                                          (32, 123, 1e4), (64, 100000, 1e7)])
def test_oracle_rope(hd, pos, theta):
    x = f32(np.random.default_rng(hd + pos).standard_normal((6, hd)))
    y = O.rope(x, pos, theta)
    if pos == 0:
        assert np.array_equal(y, x)
    rot = min(hd, 64)
    assert np.array_equal(y[:, rot:], x[:, rot:])
    ref = rope64(x, pos, theta)
    err = np.abs(y - ref) / (np.abs(x[:, :rot]).max() + 1e-30)
    assert err.max() < 4e-7, err.max()
    n0 = x[:, 0:rot:2] ** 2 + x[:, 1:rot:2] ** 2
    n1 = y[:, 0:rot:2].astype(np.float64) ** 2 + y[:, 1:rot:2].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5)


@pytest.mark.parametrize("seq,hd", [(1, 64), (5, 32), (37, 80)])
def test_oracle_attention(seq, hd):
    rng = np.random.default_rng(seq * 1000 + hd)
    Q, K, V = (f32(rng.standard_normal((seq, hd))) for _ in range(3))
    out = O.attention(Q, K, V)
    assert np.allclose(out, attention64(Q, K, V), rtol=1e-5, atol=1e-6)
    if seq == 1:
        assert np.allclose(out, V, rtol=2e-7, atol=0)
    Ke = np.repeat(K[:1], seq, axis=0)
    assert np.allclose(O.attention(Q, Ke, V), V.mean(axis=0, keepdims=True).repeat(seq, 0),
                       rtol=1e-5, atol=1e-6)


def test_oracle_deltanet():
    rng = np.random.default_rng(9)
    dim = 48
    S, q, k, v = (f32(rng.standard_normal(s)) for s in ((dim, dim), dim, dim, dim))
    st, out = O.deltanet_step(S, q, k, v, 0.9)
    ref = 0.9 * S.astype(np.float64) + 0.1 * np.outer(v, k)
    assert np.allclose(st, ref, rtol=1e-6, atol=1e-6)
    assert np.allclose(out, q.astype(np.float64) @ ref, rtol=1e-5, atol=1e-5)
    st1, out1 = O.deltanet_step(S, q, k, v, 1.0)
    assert np.array_equal(st1, S)
    st0, _ = O.deltanet_step(S, q, k, v, 0.0)
    assert np.array_equal(st0, f32(np.outer(v, k)))


# ------------------------------------------------------------ GPU
@pytest.fixture(scope="module")
def om():
    import ornith_moe
    ornith_moe.lib()
    return ornith_moe


@pytest.fixture(scope="module")
def ctx(om):
    c = om.Context()
    yield c
    c.close()


@pytest.mark.gpu
@pytest.mark.parametrize("hd,nq,nk,pos,theta", [(256, 16, 2, 0, 1e7), (256, 16, 2, 17, 1e7),
                                                (256, 16, 2, 262143, 1e7), (32, 4, 4, 99, 1e4),
                                                (63, 3, 1, 5, 1e6)])
def test_gpu_rope(om, ctx, hd, nq, nk, pos, theta):
    rng = np.random.default_rng(pos + hd)
    q = f32(rng.standard_normal((nq, hd)))
    k = f32(rng.standard_normal((nk, hd)))
    qb, kb = ctx.upload(q), ctx.upload(k)
    om.lib().gpu_rope(ctx.ptr, qb.ptr, kb.ptr, 1, hd, nq, nk, C.c_float(theta), pos)
    gq = ctx.download(qb, np.float32, q.shape)
    gk = ctx.download(kb, np.float32, k.shape)
    rot = min(hd, 64)
    for got, x in ((gq, q), (gk, k)):
        ref = O.rope(x, pos, theta)
        assert np.array_equal(got[:, rot:], x[:, rot:])
        assert np.array_equal(got[:, rot - rot % 2:rot], x[:, rot - rot % 2:rot])
        err = np.abs(got - ref).max() / np.abs(x).max()
        assert err < 6e-7, err
    for b in (qb, kb):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("seq,hd", [(1, 64), (7, 256), (16, 128), (33, 80), (300, 256),
                                    (1000, 64), (1500, 256), (513, 96), (65, 4), (5, 30),
                                    (41, 18)])
def test_gpu_attention(om, ctx, seq, hd):
    """Head dims that are a multiple of 4 run on the matrix cores (fp32
    MFMA; dims padded to 64/128/256, keys split over work groups and merged
    from 17 positions on); others (30, 18) on the VALU kernel.  Within 2e-6
    of the oracle (fp32, the shader's order) relative to the largest
    output."""
    rng = np.random.default_rng(seq + 7 * hd)
    Q, K, V = (f32(rng.standard_normal((seq, hd))) for _ in range(3))
    bufs = [ctx.upload(a) for a in (Q, K, V)]
    ob = ctx.alloc(Q.nbytes)
    om.lib().gpu_attention(ctx.ptr, ob.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, seq, hd)
    got = ctx.download(ob, np.float32, Q.shape)
    ref = O.attention(Q, K, V)
    scale = np.abs(ref).max()
    err = np.abs(got - ref).max() / scale
    assert err < 2e-6, err
    for b in bufs + [ob]:
        b.free()


@pytest.mark.gpu
def test_gpu_attention_large_scores(om, ctx):
    """Scores above 88: the shader's unshifted e^s overflows (the oracle
    gives NaN); the device returns the softmax."""
    rng = np.random.default_rng(5)
    seq, hd = 40, 64
    Q = f32(rng.standard_normal((seq, hd)) * 6)
    K = f32(rng.standard_normal((seq, hd)) * 6)
    V = f32(rng.standard_normal((seq, hd)))
    assert np.isnan(O.attention(Q, K, V)).any()
    bufs = [ctx.upload(a) for a in (Q, K, V)]
    ob = ctx.alloc(Q.nbytes)
    om.lib().gpu_attention(ctx.ptr, ob.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, seq, hd)
    got = ctx.download(ob, np.float32, Q.shape)
    assert np.isfinite(got).all()
    # scores of a few hundred carry fp32 rounding of ~3e-5 each, which
    # e^s turns into a relative change of the weights of that size
    assert np.allclose(got, attention64(Q, K, V), rtol=1e-4, atol=5e-5)
    for b in bufs + [ob]:
        b.free()


@pytest.mark.gpu
def test_gpu_attention_tiny_sums_unnormalised(om, ctx):
    """Every score of a row near -35: the shader's sum of e^s stays below
    1e-10, so it skips the division and returns the weighted sum itself
    (attention.metal:60-62); rows with ordinary scores are normalised."""
    rng = np.random.default_rng(9)
    seq, hd = 40, 64
    u = rng.standard_normal(hd)
    u /= np.linalg.norm(u)
    Q = f32(rng.standard_normal((seq, hd)) * 0.05)
    Q[:20] += f32(u * 14.0)  # rows 0..19: scores ~ -35
    K = f32(-u * 20.0 + rng.standard_normal((seq, hd)) * 0.02)
    V = f32(rng.standard_normal((seq, hd)))
    ref = O.attention(Q, K, V)
    assert np.abs(ref[:20]).max() < 1e-12 < np.abs(ref[20:]).max()
    bufs = [ctx.upload(a) for a in (Q, K, V)]
    ob = ctx.alloc(Q.nbytes)
    om.lib().gpu_attention(ctx.ptr, ob.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, seq, hd)
    got = ctx.download(ob, np.float32, Q.shape)
    for rows in (slice(0, 20), slice(20, seq)):
        err = np.abs(got[rows] - ref[rows]).max() / np.abs(ref[rows]).max()
        assert err < 1e-5, (rows, err)
    for b in bufs + [ob]:
        b.free()


@pytest.mark.gpu
def test_gpu_attention_refuses_wide_heads(om, ctx):
    seq, hd = 4, 320
    bufs = [ctx.upload(np.ones((seq, hd), np.float32)) for _ in range(4)]
    om.lib().gpu_attention(ctx.ptr, bufs[3].ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, seq, hd)
    assert "head_dim 320" in ctx.last_error()
    assert np.array_equal(ctx.download(bufs[3], np.float32, (seq, hd)), np.ones((seq, hd)))
    for b in bufs:
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("dim,gate", [(100, 0.9), (256, 0.5), (512, 0.0), (64, 1.0)])
def test_gpu_deltanet_step_gated(om, ctx, dim, gate):
    rng = np.random.default_rng(dim)
    S = f32(rng.standard_normal((dim, dim)))
    sb, ob = ctx.upload(S), ctx.alloc(dim * 4)
    st = S
    for step in range(3):
        q, k, v = (f32(rng.standard_normal(dim)) for _ in range(3))
        bq, bk, bv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
        assert om.lib().gpu_deltanet_step_gated(ctx.ptr, sb.ptr, bq.ptr, bk.ptr, bv.ptr, ob.ptr,
                                                dim, C.c_float(gate)) == 0
        st, out = O.deltanet_step(st, q, k, v, gate)
        assert np.array_equal(ctx.download(sb, np.float32, S.shape).view(np.uint32),
                              st.view(np.uint32)), step
        assert np.array_equal(ctx.download(ob, np.float32, (dim,)).view(np.uint32),
                              out.view(np.uint32)), step
        for b in (bq, bk, bv):
            b.free()
    # the gpu.h declaration stays a no-op (gpu.c:202-206, gpu_metal.m:587-591)
    before = ctx.download(sb, np.float32, S.shape)
    om.lib().gpu_deltanet_step(ctx.ptr, sb.ptr, ob.ptr, ob.ptr, ob.ptr, dim)
    assert np.array_equal(ctx.download(sb, np.float32, S.shape), before)
    small = ctx.alloc(4)
    assert om.lib().gpu_deltanet_step_gated(ctx.ptr, small.ptr, ob.ptr, ob.ptr, ob.ptr, ob.ptr,
                                            dim, C.c_float(gate)) != 0
    for b in (sb, ob, small):
        b.free()


@pytest.mark.gpu
def test_gpu_kv_cache_append(om, ctx):
    hd, L = 256, 8
    Kc, Vc = ctx.upload(np.zeros((L, hd), np.float32)), ctx.upload(np.zeros((L, hd), np.float32))
    rng = np.random.default_rng(3)
    ref_k, ref_v = np.zeros((L, hd), np.float32), np.zeros((L, hd), np.float32)
    for pos in (0, 3, 7):
        k, v = f32(rng.standard_normal(hd)), f32(rng.standard_normal(hd))
        kb, vb = ctx.upload(k), ctx.upload(v)
        assert om.lib().gpu_kv_cache_append(ctx.ptr, Kc.ptr, Vc.ptr, kb.ptr, vb.ptr, pos, hd) == 0
        ref_k[pos], ref_v[pos] = k, v
        kb.free()
        vb.free()
    assert np.array_equal(ctx.download(Kc, np.float32, (L, hd)), ref_k)
    assert np.array_equal(ctx.download(Vc, np.float32, (L, hd)), ref_v)
    kb = ctx.upload(np.zeros(hd, np.float32))
    assert om.lib().gpu_kv_cache_append(ctx.ptr, Kc.ptr, Vc.ptr, kb.ptr, kb.ptr, L, hd) != 0
    assert "past the cache" in ctx.last_error()
    for b in (Kc, Vc, kb):
        b.free()
