"""GGUF file-orientation experts (ornith_moe_shape.file_layout = 1).

Real GGUF files store every matrix with the input index fastest (ggml ne =
[K, M]); the reference reads matrices as vec@mat (model.c:351-357) and has no
path for that orientation, so parity here is pinned by:
  * CPU: the oracle's file layout equals its contiguous (vec@mat) layout
    bit for bit on weights whose every block shares one set of scales (the
    same dense matrix is then exactly representable in both orientations,
    packed from one integer matrix), and matches an fp64 brute force built
    from the pinned block dequant on random blocks;
  * GPU: the file-layout kernels against the oracle (random blocks, Q6_K
    sub-scales up to +-128), and against the already pinned vec@mat MFMA
    path on the same matrices in the other orientation.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

# The file kernels keep fp32-class activations (fp16 hi + lo planes): the
# measured error is ~1e-6.  A lost lo plane moves the output by 1e-4 to 1e-3
# at the Ornith shape (tests/test_mfma_emulation.py measures each term of the
# vec@mat kernels' arithmetic; tests/precision_study.py gives 1.5e-3 for a
# hi-only activation rounded toward zero and 4.4e-4 rounded to nearest over
# three tokens, 2.3e-3 and 1.3e-3 worst over 2048), so the bar here is 1e-5
# rather than the north-star 1e-3.
TOL = 1e-5
Q4K, Q6K = 144, 210


def file_plan(D, H, E, k, T):
    """The reduction split of the file-orientation plan (moe.c
    make_plan_file): returns (super-blocks per gate/up wave, per down wave)
    and the super-block counts D/256, H/256."""
    def pow2_floor(v):
        p = 1
        while p * 2 <= v:
            p *= 2
        return p
    rows = T * k + T
    slots = min(T * k, E) + 1
    tchunk = 64 if T * k >= 16 * E else 16
    est = max(slots + rows // tchunk, 1)
    kg = pow2_floor(max(8192 // (est * (2 * H // 256)), 1))
    kd = pow2_floor(max(8192 // (est * (D // 128)), 1))
    while kg > 1 and (D // 256) % kg:
        kg //= 2
    while kd > 1 and (H // 256) % kd:
        kd //= 2
    return (D // 256) // kg, (H // 256) // kd, D // 256, H // 256


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------- packers
def fp16_bits(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint16)[0]


def pack_q4k(q, d, dmin, sc, m):
    """q [nblk][256] ints 0..15; one (sc, m) < 16 for all 8 sub-blocks
    (gguf.c:31-61 layout: d, dmin, scales[12], qs[128])."""
    nb = q.shape[0]
    out = np.zeros((nb, Q4K), np.uint8)
    out[:, 0:2] = np.frombuffer(np.uint16(fp16_bits(d)).tobytes(), np.uint8)
    out[:, 2:4] = np.frombuffer(np.uint16(fp16_bits(dmin)).tobytes(), np.uint8)
    out[:, 4:8] = sc
    out[:, 8:12] = m
    out[:, 12:16] = sc | (m << 4)
    for p in range(4):
        lo = q[:, 64 * p: 64 * p + 32]
        hi = q[:, 64 * p + 32: 64 * p + 64]
        out[:, 16 + 32 * p: 48 + 32 * p] = (lo | (hi << 4)).astype(np.uint8)
    return out


def pack_q6k(q, d, sc):
    """q [nblk][256] ints 0..63; one int8 sc for all 16 sub-blocks
    (gguf.c:64-86 layout: ql[128], qh[64], scales[16], d)."""
    nb = q.shape[0]
    out = np.zeros((nb, Q6K), np.uint8)
    for n in range(2):
        b = q[:, 128 * n: 128 * n + 128]
        y0, y1, y2, y3 = b[:, 0:32], b[:, 32:64], b[:, 64:96], b[:, 96:128]
        out[:, 64 * n: 64 * n + 32] = ((y0 & 15) | ((y2 & 15) << 4)).astype(np.uint8)
        out[:, 64 * n + 32: 64 * n + 64] = ((y1 & 15) | ((y3 & 15) << 4)).astype(np.uint8)
        out[:, 128 + 32 * n: 160 + 32 * n] = ((y0 >> 4) | ((y1 >> 4) << 2) | ((y2 >> 4) << 4)
                                              | ((y3 >> 4) << 6)).astype(np.uint8)
    out[:, 192:208] = np.uint8(np.int8(sc).view(np.uint8))
    out[:, 208:210] = np.frombuffer(np.uint16(fp16_bits(d)).tobytes(), np.uint8)
    return out


def both_orientations(qmat, packer, *args):
    """qmat [K][M] integers -> (vec@mat blocks, file blocks) of one matrix."""
    K, M = qmat.shape
    ref = packer(qmat.reshape(K * M // 256, 256), *args)       # row k, blocks along i
    fil = packer(qmat.T.reshape(M * K // 256, 256), *args)     # row i, blocks along k
    return ref.reshape(-1), fil.reshape(-1)


class TwoWay:
    """One layer given in both orientations (E routed experts + shared)."""

    def __init__(self, D, H, E, seed):
        rng = np.random.default_rng(seed)
        self.D, self.H, self.E = D, H, E
        mats = {"gate": [], "up": [], "down": []}
        for _ in range(E + 1):
            for nm in ("gate", "up"):
                mats[nm].append(both_orientations(rng.integers(0, 16, (D, H)), pack_q4k,
                                                  0.0123, 0.0071, 5, 3))
            mats["down"].append(both_orientations(rng.integers(0, 64, (H, D)), pack_q6k,
                                                  0.0019, -7))
        self.ref = {nm: np.concatenate([a for a, _ in v]) for nm, v in mats.items()}
        self.fil = {nm: np.concatenate([b for _, b in v]) for nm, v in mats.items()}
        self.router = (rng.standard_normal((D, E)) * 0.05).astype(np.float32)

    def per(self, nm):
        return self.D * self.H // 256 * (Q6K if nm == "down" else Q4K)

    def oracle(self, x, file):
        src = self.fil if file else self.ref
        E, p = self.E, {nm: self.per(nm) for nm in src}
        return O.moe_layer(D=self.D, H=self.H, E=E, k=8, x=x, router_W=self.router,
                           gate=src["gate"][:E * p["gate"]], up=src["up"][:E * p["up"]],
                           down=src["down"][:E * p["down"]],
                           sh_gate=src["gate"][E * p["gate"]:], sh_up=src["up"][E * p["up"]:],
                           sh_down=src["down"][E * p["down"]:],
                           layout=O.LAYOUT_FILE if file else O.LAYOUT_CONTIGUOUS)


# ---------------------------------------------------------------- CPU (oracle)
def test_oracle_file_layout_equals_vecmat_on_shared_scales():
    L = TwoWay(256, 256, 16, seed=5)
    x = np.random.default_rng(1).standard_normal((3, 256)).astype(np.float32)
    a = L.oracle(x, file=False)
    b = L.oracle(x, file=True)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def test_oracle_file_layout_fp64_brute_force():
    """Random synthetic blocks read in file orientation: the oracle against
    float64 products of the dequantized (pinned) and transposed matrices."""
    import ornith_moe as om
    D = H = 256
    E, k = 16, 8
    syn = om.SyntheticLayer(23, 0, D, H, E, True, 0.0)
    x = np.random.default_rng(2).standard_normal((2, D)).astype(np.float32)
    out, idx, w = O.moe_layer(D=D, H=H, E=E, k=k, x=x, router_W=syn.router,
                              gate=syn.routed("gate"), up=syn.routed("up"),
                              down=syn.routed("down"), sh_gate=syn.shared("gate"),
                              sh_up=syn.shared("up"), sh_down=syn.shared("down"),
                              layout=O.LAYOUT_FILE)

    def mat(which, e, K, M, typ):
        data = syn.routed(which) if e < E else syn.shared(which)
        per = D * H // 256 * (Q6K if typ == O.TYPE_Q6_K else Q4K)
        blk = data[(e % E) * per:(e % E + 1) * per] if e < E else data
        ok, v = O.dequant_tensor(blk, typ, K * M)
        assert ok
        return v.astype(np.float64).reshape(M, K)  # [out][in]

    def ffn(xv, e, clamp):
        g = mat("gate", e, D, H, O.TYPE_Q4_K) @ xv
        u = mat("up", e, D, H, O.TYPE_Q4_K) @ xv
        silu = g / (1.0 + np.exp(-np.clip(g, -80.0, 80.0)))
        if clamp:  # model.c:1087-1088: 0 below -50, identity above 50
            silu = np.where(g < -50.0, 0.0, np.where(g > 50.0, g, silu))
        mid = silu * u
        return mat("down", e, H, D, O.TYPE_Q6_K) @ mid

    for t in range(x.shape[0]):
        xv = x[t].astype(np.float64)
        ref = ffn(xv, E, False)
        for j in range(k):
            ref = ref + float(w[t, j]) * ffn(xv, int(idx[t, j]), True)
        err = np.abs(out[t] - ref).max() / np.abs(ref).max()
        assert err < 1e-5, err


# ---------------------------------------------------------------- GPU
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


def row_err(out, ref):
    scale = np.abs(ref).max(axis=1)
    assert np.all(scale > 0) and np.all(np.isfinite(out)), "degenerate or non-finite output"
    return np.abs(out.astype(np.float64) - ref).max(axis=1) / scale


def forward(ctx, store, x, k):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * k * 4), ctx.alloc(T * k * 4)
    store.forward(0, xb, T, ob, idx=ib, w=wb)
    out = ctx.download(ob, np.float32, x.shape)
    idx = ctx.download(ib, np.uint32, (T, k))
    w = ctx.download(wb, np.float32, (T, k))
    for b in (xb, ob, ib, wb):
        b.free()
    return out, idx, w


def file_store(om, ctx, D, H, E, k, gate, up, down, router_de):
    st = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=False, file_layout=True)
    st.set_experts(0, om.MAT_GATE, 0, gate, E + 1)
    st.set_experts(0, om.MAT_UP, 0, up, E + 1)
    st.set_experts(0, om.MAT_DOWN, 0, down, E + 1)
    st.set_router(0, np.ascontiguousarray(router_de.T))  # file orientation: [E][D]
    return st


def forward_full(ctx, store, x, k, flags=0, mode=0, resid=None):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * k * 4), ctx.alloc(T * k * 4)
    rb = ctx.upload(resid) if resid is not None else None
    store.forward(0, xb, T, ob, resid=rb, idx=ib, w=wb, flags=flags, mode=mode)
    res = (ctx.download(ob, np.float32, x.shape), ctx.download(ib, np.uint32, (T, k)),
           ctx.download(wb, np.float32, (T, k)))
    for b in (xb, ob, ib, wb, rb):
        if b is not None:
            b.free()
    return res


@pytest.fixture(scope="module")
def ornith_file(om, ctx):
    """One Ornith-shape file-orientation layer (random blocks), shared by
    the Ornith-shape cases."""
    D, H, E, k = 2048, 512, 256, 8
    syn = om.SyntheticLayer(31, 0, D, H, E, True, 0.0)
    st = file_store(om, ctx, D, H, E, k, syn.gate, syn.up, syn.down, syn.router)
    yield syn, st
    st.close()


def oracle_file(syn, D, H, E, k, x, **kw):
    return O.moe_layer(D=D, H=H, E=E, k=k, x=x, router_W=syn.router,
                       gate=syn.routed("gate"), up=syn.routed("up"),
                       down=syn.routed("down"), sh_gate=syn.shared("gate"),
                       sh_up=syn.shared("up"), sh_down=syn.shared("down"),
                       layout=O.LAYOUT_FILE, **kw)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,T", [((256, 256, 16), 1), ((256, 256, 16), 3),
                                     ((256, 256, 16), 37), ((256, 1024, 16), 1),
                                     ((256, 1024, 16), 100)])
def test_file_layout_parity(om, ctx, shape, T):
    D, H, E = shape
    k = 8
    say("file layout parity", shape, T)
    syn = om.SyntheticLayer(31, 0, D, H, E, True, 0.0)
    st = file_store(om, ctx, D, H, E, k, syn.gate, syn.up, syn.down, syn.router)
    try:
        x = np.random.default_rng(T).standard_normal((T, D)).astype(np.float32)
        out, idx, w = forward(ctx, st, x, k)
        ref, ridx, rw = oracle_file(syn, D, H, E, k, x)
        assert np.array_equal(idx, ridx)
        # the device's expf may differ from the host's by an ulp
        assert np.allclose(w, rw, rtol=1e-5, atol=1e-7)
        e = row_err(out, ref)
        say("  max row err", e.max())
        assert e.max() <= TOL
    finally:
        st.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 16, 64, 256, 2048])
def test_file_layout_parity_ornith(om, ctx, ornith_file, T):
    """Ornith shape.  From T = 64 on, the plan gives each wave more than one
    super-block, so the loop over super-blocks (double-buffered tiles with
    one barrier per super-block for 16-row items; one 64-row tile with a
    barrier before each rewrite for the 64-row items of T = 2048) runs
    several iterations.  At T = 2048 items hold up to 64 rows, so the
    partially filled row tiles of the four-tile kernels are exercised.  The
    oracle runs a stated subset of the tokens (every token's routing is
    checked)."""
    D, H, E, k = 2048, 512, 256, 8
    syn, st = ornith_file
    nsb_gu, nsb_dn, NSB_GU, NSB_DN = file_plan(D, H, E, k, T)
    say(f"file layout Ornith T={T}: super-blocks per wave gate/up {nsb_gu}, down {nsb_dn}")
    if T >= 64:
        assert nsb_gu > 1 and nsb_dn > 1
    x = np.random.default_rng(T).standard_normal((T, D)).astype(np.float32)
    out, idx, w = forward(ctx, st, x, k)
    lg = O.router_logits_rows(x, syn.router)
    for t in range(T):
        assert np.array_equal(idx[t], O.topk(lg[t], k)[0]), t
    sub = np.arange(T) if T <= 64 else np.unique(np.linspace(0, T - 1, 40).astype(int))
    ref, ridx, rw = oracle_file(syn, D, H, E, k, x[sub])
    assert np.array_equal(idx[sub], ridx)
    assert np.allclose(w[sub], rw, rtol=1e-5, atol=1e-7)
    e = row_err(out[sub], ref)
    say(f"  max row err {e.max():.2e} over {len(sub)} tokens")
    assert e.max() <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("T", [16, 100])
def test_file_layout_shexp_gate(om, ctx, ornith_file, T):
    """The optional shared-expert gate (ORN_MOE_SHEXP_GATE) on the file
    path, with NORM and resid = x, against the oracle's gated layer."""
    D, H, E, k = 2048, 512, 256, 8
    syn, st = ornith_file
    rng = np.random.default_rng(70 + T)
    nw = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    gv = (0.02 * rng.standard_normal(D)).astype(np.float32)
    st.set_norm(0, nw)
    st.set_shexp_gate(0, gv)
    try:
        x = rng.standard_normal((T, D)).astype(np.float32)
        out, idx, w = forward_full(ctx, st, x, k, flags=om.MOE_NORM | om.MOE_SHEXP_GATE, resid=x)
        sub = np.arange(T) if T <= 16 else np.unique(np.linspace(0, T - 1, 24).astype(int))
        ref, ridx, _ = oracle_file(syn, D, H, E, k, x[sub], norm_w=nw, resid=x[sub],
                                   shexp_gate=gv)
        assert np.array_equal(idx[sub], ridx)
        e = row_err(out[sub], ref)
        say(f"  gated T={T}: max row err {e.max():.2e}")
        assert e.max() <= TOL
    finally:
        st.set_shexp_gate(0, None)
        st.set_norm(0, np.ones(D, np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("T,flags,mode", [(16, "norm", 0), (100, "norm", 0), (16, "", 1),
                                          (100, "norm", 1)])
def test_file_layout_norm_resid_literal(om, ctx, ornith_file, T, flags, mode):
    """The call the engine integration makes (ORN_MOE_NORM with resid = x):
    at T <= 64 the router's fused norm writes the normalised rows the
    expert steps read, above that the separate norm kernel does; and the
    literal routing mode (model.c:1027-1049)."""
    D, H, E, k = 2048, 512, 256, 8
    syn, st = ornith_file
    rng = np.random.default_rng(50 + T + mode)
    nw = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    st.set_norm(0, nw)
    try:
        x = rng.standard_normal((T, D)).astype(np.float32)
        norm = flags == "norm"
        out, idx, w = forward_full(ctx, st, x, k, flags=om.MOE_NORM if norm else 0, mode=mode,
                                   resid=x if norm else None)
        sub = np.arange(T) if T <= 16 else np.unique(np.linspace(0, T - 1, 24).astype(int))
        ref, ridx, rw = oracle_file(syn, D, H, E, k, x[sub], mode=mode,
                                    norm_w=nw if norm else None, resid=x[sub] if norm else None)
        assert np.array_equal(idx[sub], ridx)
        assert np.allclose(w[sub], rw, rtol=1e-5, atol=1e-7)
        e = row_err(out[sub], ref)
        say(f"  T={T} flags={flags} mode={mode}: max row err {e.max():.2e}")
        assert e.max() <= TOL
    finally:
        st.set_norm(0, np.ones(D, np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("T", [9, 40, 100])
def test_file_layout_large_q6_scales(om, ctx, T):
    """Q6_K sub-scales across the whole int8 range (real files reach +-128):
    items of 16 rows (T = 9) and of 64 rows, the four-row-tile down instance
    that prefill from a real file runs (T * k >= 16 E: T = 40, 100)."""
    D, H, E, k = 256, 256, 16, 8
    syn = om.SyntheticLayer(37, 0, D, H, E, True, 0.0)
    down = syn.down.copy().reshape(-1, Q6K)
    rng = np.random.default_rng(3)
    down[:, 192:208] = rng.integers(-128, 128, (down.shape[0], 16)).astype(np.int8).view(np.uint8)
    down = down.reshape(-1)
    st = file_store(om, ctx, D, H, E, k, syn.gate, syn.up, down, syn.router)
    try:
        x = rng.standard_normal((T, D)).astype(np.float32)
        out, idx, w = forward(ctx, st, x, k)
        per = D * H // 256 * Q6K
        ref, ridx, _ = O.moe_layer(D=D, H=H, E=E, k=k, x=x, router_W=syn.router,
                                   gate=syn.routed("gate"), up=syn.routed("up"),
                                   down=down[:E * per], sh_gate=syn.shared("gate"),
                                   sh_up=syn.shared("up"), sh_down=down[E * per:],
                                   layout=O.LAYOUT_FILE)
        assert np.array_equal(idx, ridx)
        assert row_err(out, ref).max() <= TOL
    finally:
        st.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 16, 100])
def test_file_layout_matches_vecmat_path(om, ctx, T):
    """The same matrices in both orientations: the file kernels against the
    vec@mat MFMA kernels (and both against the oracle)."""
    D, H, E, k = 256, 256, 16, 8
    L = TwoWay(D, H, E, seed=9)
    ref_st = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=True)
    ref_st.set_experts(0, om.MAT_GATE, 0, L.ref["gate"], E + 1)
    ref_st.set_experts(0, om.MAT_UP, 0, L.ref["up"], E + 1)
    ref_st.set_experts(0, om.MAT_DOWN, 0, L.ref["down"], E + 1)
    ref_st.set_router(0, L.router)
    fil_st = file_store(om, ctx, D, H, E, k, L.fil["gate"], L.fil["up"], L.fil["down"], L.router)
    try:
        x = np.random.default_rng(100 + T).standard_normal((T, D)).astype(np.float32)
        a = forward(ctx, ref_st, x, k)
        b = forward(ctx, fil_st, x, k)
        assert np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2])
        assert row_err(b[0], a[0].astype(np.float64)).max() <= 1e-4
        ref = L.oracle(x, file=True)[0]
        assert row_err(b[0], ref).max() <= TOL
    finally:
        ref_st.close()
        fil_st.close()


@pytest.mark.gpu
def test_file_layout_refuses_forced_path_and_prefill_layout(om, ctx):
    with pytest.raises(RuntimeError):
        om.Store(ctx, 1, 256, 256, 16, 8, True, prefill_layout=True, file_layout=True)
    syn = om.SyntheticLayer(31, 0, 256, 256, 16, True, 0.0)
    st = file_store(om, ctx, 256, 256, 16, 8, syn.gate, syn.up, syn.down, syn.router)
    try:
        x = np.ones((1, 256), np.float32)
        xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
        with pytest.raises(RuntimeError):
            st.forward(0, xb, 1, ob, flags=om.MOE_PATH_MFMA)
        xb.free()
        ob.free()
    finally:
        st.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 16])
def test_file_layout_graph_replay_matches_eager(om, ctx, T):
    """ORN_MOE_GRAPH on a file-layout store: each replay sees new input
    contents, with eager forwards and synchronisations in between, and must
    equal an eager forward of the same input bit for bit."""
    D, H, E, k = 256, 256, 16, 8
    syn = om.SyntheticLayer(31, 0, D, H, E, True, 0.0)
    st = file_store(om, ctx, D, H, E, k, syn.gate, syn.up, syn.down, syn.router)
    xb, ob = ctx.alloc(T * D * 4), ctx.alloc(T * D * 4)
    ib, wb = ctx.alloc(T * k * 4), ctx.alloc(T * k * 4)
    try:
        for i in range(4):
            x = np.random.default_rng(700 + 10 * T + i).standard_normal((T, D)).astype(np.float32)
            om.lib().gpu_copy_to_device(ctx.ptr, xb.ptr, x.ctypes.data, x.nbytes)
            st.forward(0, xb, T, ob, idx=ib, w=wb, flags=om.MOE_GRAPH)
            g = ctx.download(ob, np.float32, (T, D))
            gi = ctx.download(ib, np.uint32, (T, k))
            e, ei, _ = forward(ctx, st, x, k)
            assert np.array_equal(gi, ei)
            assert np.array_equal(g.view(np.uint32), e.view(np.uint32))
    finally:
        for b in (xb, ob, ib, wb):
            b.free()
        st.close()
