"""Streamed experts (ornith_moe_shape.cache_slots > 0, csrc/host/cache.c):
the experts live in a pinned host tier and stream through a fixed pool of
device slots with the reference's tiering policy (memory.c:79-421: hot-store
pins, LRU eviction, prefetch).

Pinned by:
  * the oracle: every streamed forward against orc_moe_layer (the
    reference's MoE block restated, engine/src/model.c:992-1144) on the same
    bytes -- indices exact, outputs within 1e-5 per row -- including the
    Ornith shape and the file orientation;
  * equality: every forward of a streamed store equals the same forward of a
    resident store holding the same bytes, bit for bit (outputs, indices,
    weights, logits) -- decode, MFMA and file-orientation paths, layers
    interleaved so that experts are evicted and reloaded;
  * the policy: a host model of the cache (free slots first, then the least
    recently used key that is neither pinned nor needed by the forward;
    a forward's keys are touched in its slot order, the shared expert first,
    then ascending expert id) predicts hits, misses and evictions exactly
    from the resident store's routing;
  * prefetch and pin semantics (prefetched experts are hits, pinned ones are
    never evicted) and the refusals (too few slots, ORN_MOE_GRAPH);
  * a prefetch issued while an asynchronous forward that joined the previous
    prefetch is still in flight (the load list must not be rewritten before
    the earlier gather has read it).
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-5  # the parity bar of the resident forwards (tests/test_gpu_moe.py)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


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
    assert np.all(scale > 0) and np.all(np.isfinite(out))
    return np.abs(out.astype(np.float64) - ref).max(axis=1) / scale


def check_oracle(syn, x, k, got, norm_w=None, layout=None):
    """A streamed forward's (out, idx, w, ...) against the oracle."""
    D, E = x.shape[1], syn.E
    H = syn.nb * 256 // D
    kw = {} if layout is None else {"layout": layout}
    ref, ridx, rw = O.moe_layer(D=D, H=H, E=E, k=k, x=x, router_W=syn.router, bias=syn.bias,
                                norm_w=norm_w, gate=syn.routed("gate"), up=syn.routed("up"),
                                down=syn.routed("down"), sh_gate=syn.shared("gate"),
                                sh_up=syn.shared("up"), sh_down=syn.shared("down"), **kw)
    assert np.array_equal(got[1], ridx)
    assert np.allclose(got[2], rw, rtol=1e-5, atol=1e-7)
    err = row_err(got[0], ref).max()
    assert err <= TOL, err
    return err


def fwd(ctx, st, layer, x, k, flags=0):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * k * 4), ctx.alloc(T * k * 4)
    st.forward(layer, xb, T, ob, idx=ib, w=wb, flags=flags)
    res = (ctx.download(ob, np.float32, x.shape), ctx.download(ib, np.uint32, (T, k)),
           ctx.download(wb, np.float32, (T, k)), st.last_logits(T))
    for b in (xb, ob, ib, wb):
        b.free()
    return res


class CacheModel:
    """The slot policy of cache.c restated over keys (layer, expert)."""

    def __init__(self, slots):
        self.slots, self.tick = slots, 0
        self.last = {}      # key -> tick of last use
        self.pinned = set()
        self.hits = self.misses = self.evictions = 0

    def forward(self, layer, experts):
        need = [(layer, e) for e in experts]
        assert len(need) <= self.slots
        missing = []
        for key in need:
            if key in self.last:
                self.hits += 1
                self.tick += 1
                self.last[key] = self.tick
            else:
                missing.append(key)
        for key in missing:
            self.misses += 1
            if len(self.last) >= self.slots:
                cand = [kk for kk in self.last if kk not in self.pinned and kk not in need]
                victim = min(cand, key=lambda kk: self.last[kk])
                del self.last[victim]
                self.evictions += 1
            self.tick += 1
            self.last[key] = self.tick


def needed(idx, w, E, has_shared=True):
    """The dispatch's slot order: the shared expert, then every expert with a
    kept pair (w >= 1e-6, model.c:1066) in ascending id."""
    kept = sorted({int(e) for e, ww in zip(idx.reshape(-1), w.reshape(-1)) if not ww < 1e-6})
    return ([E] if has_shared else []) + kept


def make_pair(om, ctx, L, D, H, E, k, slots, seed=5, prefill=True):
    """A resident and a streamed store of the same L layers, plus the host
    copies (syns, norm weights) for the oracle."""
    res = om.Store(ctx, L, D, H, E, k, True, prefill_layout=prefill)
    stm = om.Store(ctx, L, D, H, E, k, True, prefill_layout=prefill, cache_slots=slots)
    syns, norms = [], []
    for l in range(L):
        syn = om.SyntheticLayer(seed, l, D, H, E, True, 1.1 if l == 1 else 0.0)
        res.load_layer(l, syn)
        stm.load_layer(l, syn)
        nw = np.random.default_rng(l).uniform(0.5, 1.5, D).astype(np.float32)
        res.set_norm(l, nw)
        stm.set_norm(l, nw)
        syns.append(syn)
        norms.append(nw)
    return res, stm, syns, norms


def test_streamed_equals_resident_and_policy(om, ctx):
    L, D, H, E, k, C = 3, 256, 256, 16, 8, 20
    res, stm, syns, norms = make_pair(om, ctx, L, D, H, E, k, C)
    model = CacheModel(C)
    worst = 0.0
    try:
        st0 = stm.cache_stats()
        assert st0["slots"] == C and st0["resident"] == 0 and st0["host_bytes"] > 0
        rng = np.random.default_rng(1)
        steps = [(l, T, f) for T, f in ((1, 0), (3, 0), (16, om.MOE_NORM), (100, 0),
                                        (5, om.MOE_PATH_VALU)) for l in (0, 2, 1, 0)]
        for i, (l, T, flags) in enumerate(steps):
            x = rng.standard_normal((T, D)).astype(np.float32)
            a = fwd(ctx, stm, l, x, k, flags)
            b = fwd(ctx, res, l, x, k, flags)
            worst = max(worst, check_oracle(syns[l], x, k, a,
                                            norm_w=norms[l] if flags & om.MOE_NORM else None))
            for u, v in zip(a, b):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), (i, l, T)
            model.forward(l, needed(b[1], b[2], E))
            s = stm.cache_stats()
            assert (s["hits"], s["misses"], s["evictions"]) == \
                (model.hits, model.misses, model.evictions), (i, s, vars(model))
        s = stm.cache_stats()
        say(f"  {len(steps)} forwards bit-identical, max row err vs oracle {worst:.2e}; hits "
            f"{s['hits']} misses {s['misses']} evictions {s['evictions']} uploaded "
            f"{s['bytes_uploaded'] / 1e6:.1f} MB")
        assert s["evictions"] > 0 and s["hits"] > 0
        # the host tier holds exactly what was uploaded
        syn = om.SyntheticLayer(5, 2, D, H, E, True)
        assert np.array_equal(stm.get_experts(2, om.MAT_DOWN, 0, E + 1), syn.down)
    finally:
        res.close()
        stm.close()


def test_prefetch_and_pin(om, ctx):
    L, D, H, E, k, C = 3, 256, 256, 16, 8, 12
    res, stm, syns, _ = make_pair(om, ctx, L, D, H, E, k, C, prefill=False)
    try:
        rng = np.random.default_rng(2)
        x = rng.standard_normal((1, D)).astype(np.float32)
        b = fwd(ctx, res, 1, x, k)
        want = needed(b[1], b[2], E)
        stm.prefetch(1, want)
        s = stm.cache_stats()
        assert s["prefetches"] == len(want) and s["resident"] == len(want)
        a = fwd(ctx, stm, 1, x, k)
        check_oracle(syns[1], x, k, a)
        for u, v in zip(a, b):
            assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
        s = stm.cache_stats(reset=True)
        assert s["misses"] == 0 and s["hits"] == len(want) and s["prefetch_hits"] == len(want)
        # pin two experts of layer 0; forwards over layers 1 and 2 never evict them
        stm.pin(0, [3, 7])
        assert stm.cache_stats()["pinned"] == 2
        for i in range(12):
            l = 1 + i % 2
            x = rng.standard_normal((1, D)).astype(np.float32)
            a, b = fwd(ctx, stm, l, x, k), fwd(ctx, res, l, x, k)
            check_oracle(syns[l], x, k, a)
            assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
        assert stm.cache_stats()["evictions"] > 0
        stm.cache_stats(reset=True)
        stm.pin(0, [3, 7])  # already resident: no load
        s = stm.cache_stats()
        assert s["misses"] == 0 and s["pinned"] == 2
        stm.pin(0, [3, 7], pin=False)
        assert stm.cache_stats()["pinned"] == 0
    finally:
        res.close()
        stm.close()


def test_streamed_refusals(om, ctx):
    D, H, E, k = 256, 256, 16, 8
    stm = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=False, cache_slots=6)
    try:
        stm.load_layer(0, om.SyntheticLayer(9, 0, D, H, E, True))
        x = np.random.default_rng(3).standard_normal((16, D)).astype(np.float32)
        with pytest.raises(RuntimeError, match="needs .* experts; the cache has 6 slots"):
            fwd(ctx, stm, 0, x, k)
        with pytest.raises(RuntimeError, match="ORN_MOE_GRAPH"):
            fwd(ctx, stm, 0, x[:1], k, om.MOE_GRAPH)
        res = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=False)
        try:
            with pytest.raises(RuntimeError, match="not a streamed store"):
                res.prefetch(0, [1])
        finally:
            res.close()
    finally:
        stm.close()
    # k = 2: a token needs 3 experts; 5 of 6 slots pinned to another layer
    stm = om.Store(ctx, 2, D, H, E, 2, True, prefill_layout=False, cache_slots=6)
    try:
        for l in range(2):
            stm.load_layer(l, om.SyntheticLayer(9, l, D, H, E, True))
        stm.pin(1, [0, 1, 2, 3, 4])
        with pytest.raises(RuntimeError, match="no slot to evict"):
            fwd(ctx, stm, 0, x[:1], 2)
    finally:
        stm.close()


def test_streamed_file_layout_and_device_fill(om, ctx):
    """A file-orientation streamed store, and fill_synthetic into the host
    tier, at the Ornith shape (T = 1 and 4: up to 33 experts per forward);
    the file store with as many slots as one layer has experts, over two
    layers' worth of loads."""
    D, H, E, k = 2048, 512, 256, 8
    res = om.Store(ctx, 2, D, H, E, k, True)
    stm = om.Store(ctx, 2, D, H, E, k, True, cache_slots=48)
    fres = om.Store(ctx, 1, 256, 256, 16, k, True, prefill_layout=False, file_layout=True)
    fstm = om.Store(ctx, 1, 256, 256, 16, k, True, prefill_layout=False, file_layout=True,
                    cache_slots=17)
    try:
        for l in range(2):
            res.fill_synthetic(l, 77 + l)
            stm.fill_synthetic(l, 77 + l)
        syn = om.SyntheticLayer(77, 0, D, H, E, True)
        assert np.array_equal(stm.get_experts(0, om.MAT_UP, 0, E + 1), syn.up)
        rng = np.random.default_rng(4)
        syns = [syn, om.SyntheticLayer(78, 1, D, H, E, True)]
        worst = 0.0
        for i, (l, T) in enumerate([(0, 1), (1, 4), (0, 4), (1, 1), (0, 1)]):
            x = rng.standard_normal((T, D)).astype(np.float32)
            a, b = fwd(ctx, stm, l, x, k), fwd(ctx, res, l, x, k)
            worst = max(worst, check_oracle(syns[l], x, k, a))
            for u, v in zip(a, b):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), (i, l, T)
        del syns
        say(f"  Ornith shape, 48 slots: max row err vs oracle {worst:.2e}; {stm.cache_stats()}")
        syn = om.SyntheticLayer(31, 0, 256, 256, 16, True)
        for st in (fres, fstm):
            for name, m in (("gate", om.MAT_GATE), ("up", om.MAT_UP), ("down", om.MAT_DOWN)):
                st.set_experts(0, m, 0, getattr(syn, name), 17)
            st.set_router(0, np.ascontiguousarray(syn.router.T))
        for T in (1, 2, 1):
            x = rng.standard_normal((T, 256)).astype(np.float32)
            a, b = fwd(ctx, fstm, 0, x, k), fwd(ctx, fres, 0, x, k)
            check_oracle(syn, x, k, a, layout=O.LAYOUT_FILE)
            for u, v in zip(a, b):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), T
    finally:
        for s in (res, stm, fres, fstm):
            s.close()


def test_prefetch_during_async_forward(om, ctx):
    """Prefetch, an asynchronous forward that joins it, a second prefetch
    issued before that forward has finished, then a forward of the second
    batch: the second prefetch must not rewrite the first batch's load list
    before the first gather has read it (else slots would hold the wrong
    experts while the cache maps them as correct).  Every forward against
    the resident store bit for bit and the oracle; then two more forwards
    per batch, which reuse the prefetched slots."""
    L, D, H, E, k, C = 2, 256, 256, 16, 4, 20  # room for both batches: no eviction
    res, stm, syns, _ = make_pair(om, ctx, L, D, H, E, k, C, seed=8)
    try:
        rng = np.random.default_rng(6)
        xs = [rng.standard_normal((2, D)).astype(np.float32) for _ in range(2)]
        want = [needed(*fwd(ctx, res, l, xs[l], k)[1:3], E) for l in range(2)]
        assert len(want[0]) + len(want[1]) <= C
        xb = ctx.upload(xs[0])
        ob, ib, wb = ctx.alloc(xs[0].nbytes), ctx.alloc(2 * k * 4), ctx.alloc(2 * k * 4)
        try:
            stm.prefetch(0, want[0])
            stm.forward(0, xb, 2, ob, idx=ib, w=wb, flags=om.MOE_ASYNC)
            stm.prefetch(1, want[1])  # while the forward above may still run
            second = fwd(ctx, stm, 1, xs[1], k)
            ctx.sync()
            first = (ctx.download(ob, np.float32, xs[0].shape),
                     ctx.download(ib, np.uint32, (2, k)), ctx.download(wb, np.float32, (2, k)))
        finally:
            for b in (xb, ob, ib, wb):
                b.free()
        s = stm.cache_stats()
        say(f"  prefetch/async/prefetch: {s}")
        assert s["prefetch_hits"] == len(want[0]) + len(want[1]) and s["misses"] == 0
        for l, got in ((0, first), (1, second)):
            check_oracle(syns[l], xs[l], k, got)
            ref = fwd(ctx, res, l, xs[l], k)
            for u, v in zip(got[:3], ref[:3]):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), l
        for _ in range(2):
            for l in range(2):
                a, b = fwd(ctx, stm, l, xs[l], k), fwd(ctx, res, l, xs[l], k)
                for u, v in zip(a, b):
                    assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), l
        assert stm.cache_stats()["misses"] == 0
    finally:
        res.close()
        stm.close()
