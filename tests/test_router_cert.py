"""GPU tests of the certified routing of the smallest decode batches
(T <= 4 tokens; router_cert.hip).

The reference's logit (model.c:1017-1025) is a sequential fp32 chain; the
certified kernel forms fp64 sums of the same fp32 products with a proven
bound on their distance from that chain, selects exactly when the bounds
decide the top k, and runs the chain itself for the experts they leave
undecided.  The bar is the same as for the exact routers: top-k indices
equal to the oracle's (oracle/oracle.c orc_router_logits + orc_topk_*) for
every token, in both selection modes, with the layer's rmsnorm and with a
router bias.  The weights are compared within 1e-5 relative (the logits
they come from are the sums, a few ulp from the chains); the logits
themselves within 1e-4 absolute (the bound is ~6e-5 at the Ornith shape;
the measured differences are ~1e-6).

Engineered cases force each fallback: a router column that nearly
duplicates the token's top expert (its logit a few ulp away: the bounds
cannot order them, the chains must), an exact duplicate (an exact tie: the
reference's literal selection on the chains), and a NaN activation.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

D, H, E, K = 2048, 512, 256, 8
SEED = 5150


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


@pytest.fixture(scope="module")
def store(om, ctx):
    """Layer 0: synthetic Ornith layer with rmsnorm weights; layer 1: the
    same with a Zipf(1.1) router bias."""
    st = om.Store(ctx, 2, D, H, E, K, True)
    syn, norms = [], []
    rng = np.random.default_rng(11)
    for l, z in ((0, 0.0), (1, 1.1)):
        s = om.SyntheticLayer(SEED, l, D, H, E, True, z)
        st.load_layer(l, s)
        nw = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
        st.set_norm(l, nw)
        syn.append(s)
        norms.append(nw)
    yield st, syn, norms
    st.close()


def act(om, seed, T):
    return om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)


def run(om, ctx, st, x, layer, flags, mode):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * K * 4), ctx.alloc(T * K * 4)
    st.forward(layer, xb, T, ob, idx=ib, w=wb, flags=flags, mode=mode)
    logits = st.last_logits(T)
    chained = st.last_chained()
    out = ctx.download(ob, np.float32, x.shape)
    idx = ctx.download(ib, np.uint32, (T, K))
    w = ctx.download(wb, np.float32, (T, K))
    for b in (xb, ob, ib, wb):
        b.free()
    return logits, idx, w, out, chained


def oracle_routing(xin, W, bias, mode):
    ref = O.router_logits_rows(xin, W, bias)
    T = ref.shape[0]
    ridx = np.zeros((T, K), np.uint32)
    rw = np.zeros((T, K), np.float32)
    for t in range(T):
        ridx[t], rw[t] = O.topk(ref[t], K, mode)
    return ref, ridx, rw


def check(om, ctx, store, T, layer, norm, mode, seed):
    st, syn, norms = store
    s = syn[layer]
    x = act(om, seed, T)
    flags = om.MOE_NORM if norm else 0
    logits, idx, w, out, chained = run(om, ctx, st, x, layer, flags, mode)
    xin = O.rmsnorm(x, norms[layer]) if norm else x
    ref, ridx, rw = oracle_routing(xin, s.router, s.bias, mode)
    dl = np.abs(logits.astype(np.float64) - ref).max()
    rel = (np.abs(w.astype(np.float64) - rw) / np.abs(rw)).max()
    say(f"T={T} layer={layer} norm={norm} mode={mode}: {chained} tokens chained, "
        f"max |dlogit| {dl:.2e}, max rel dw {rel:.2e}")
    assert np.array_equal(idx, ridx), np.argwhere(idx != ridx)[:5]
    assert dl <= 1e-4
    assert rel <= 1e-5
    # the same forward with the exact chains: same selection, outputs within
    # the weights' difference
    _, idx2, _, out2, ch2 = run(om, ctx, st, x, layer, flags | om.MOE_EXACT_LOGITS, mode)
    assert ch2 == 0
    assert np.array_equal(idx2, idx)
    err = (np.abs(out.astype(np.float64) - out2).max(axis=1) / np.abs(out2).max(axis=1)).max()
    say(f"  outputs vs exact-chain routing: max row err {err:.2e}")
    assert err <= 1e-5


@pytest.mark.parametrize("mode", [0, 1], ids=["renorm", "literal"])
@pytest.mark.parametrize("norm", [False, True], ids=["x", "rmsnorm"])
@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_cert_routing_matches_oracle(om, ctx, store, T, norm, mode):
    check(om, ctx, store, T, 0, norm, mode, 900 + T)


@pytest.mark.parametrize("T", [1, 4])
def test_cert_routing_bias(om, ctx, store, T):
    check(om, ctx, store, T, 1, T == 4, 0, 950 + T)


def test_cert_many_tokens(om, ctx, store):
    """512 tokens in 128 batches of 4: every selection exact; the share of
    tokens whose bounds did not decide is reported (~2% expected)."""
    st, syn, _ = store
    s = syn[0]
    n_ch = 0
    for b in range(128):
        x = act(om, 7000 + b, 4)
        _, idx, _, _, chained = run(om, ctx, st, x, 0, 0, 0)
        _, ridx, _ = oracle_routing(x, s.router, None, 0)
        assert np.array_equal(idx, ridx), (b, np.argwhere(idx != ridx)[:5])
        n_ch += chained
    say(f"512 tokens: {n_ch} needed exact chains")
    assert n_ch < 100


@pytest.fixture(scope="module")
def tie_store(om, ctx):
    """One layer whose router we rewrite per case (experts synthetic)."""
    st = om.Store(ctx, 1, D, H, E, K, True)
    s = om.SyntheticLayer(SEED + 1, 0, D, H, E, True)
    st.load_layer(0, s)
    yield st, s
    st.close()


@pytest.mark.parametrize("norm", [False, True], ids=["x", "rmsnorm"])
@pytest.mark.parametrize("mode", [0, 1], ids=["renorm", "literal"])
@pytest.mark.parametrize("kind", ["near", "exact", "near_k"])
def test_cert_engineered_ties(om, ctx, tie_store, kind, mode, norm):
    """A router column rewritten from the token's top expert (near: scaled
    by 1 + 2^-20, a logit ~1e-6 away; exact: a copy, an exact tie) or from
    its k-th (near_k: the selection boundary).  The bounds cannot decide;
    the selection must still equal the oracle's.  With the rmsnorm the
    selecting group rebuilds the normalised row from the scale the norm's
    group published, so the chained logits are the reference's bit for bit."""
    st, s = tie_store
    x = act(om, 4321, 1)
    nw = (1.0 + 0.25 * np.random.default_rng(12).standard_normal(D)).astype(np.float32)
    st.set_norm(0, nw)
    xin = O.rmsnorm(x, nw) if norm else x
    W = np.array(s.router, np.float32, copy=True)
    ref0 = O.router_logits(xin[0], W)
    order = np.argsort(-ref0.astype(np.float64), kind="stable")
    src = order[0] if kind != "near_k" else order[K - 1]
    dst = order[40]
    if kind == "exact":
        W[:, dst] = W[:, src]
    else:
        W[:, dst] = (W[:, src] * np.float32(1.0 + 2.0 ** -20)).astype(np.float32)
    st.set_router(0, W)
    try:
        logits, idx, w, _, chained = run(om, ctx, st, x, 0, om.MOE_NORM if norm else 0, mode)
        ref, ridx, rw = oracle_routing(xin, W, None, mode)
        say(f"{kind} mode={mode}: logits {ref[0, src]!r} {ref[0, dst]!r}, chained {chained}, "
            f"idx {idx[0].tolist()} ref {ridx[0].tolist()}")
        assert chained == 1
        assert np.array_equal(idx, ridx)
        # the chained experts' logits are the chain's, bit for bit
        assert logits[0, src].view(np.uint32) == ref[0, src].view(np.uint32)
        assert logits[0, dst].view(np.uint32) == ref[0, dst].view(np.uint32)
        rel = (np.abs(w.astype(np.float64) - rw) / np.abs(rw)).max()
        assert rel <= 1e-5
    finally:
        st.set_router(0, s.router)


def test_cert_nan_activation(om, ctx, tie_store):
    """A NaN in one token's activations makes its sums NaN: that token runs
    every chain and the reference's literal selection; the others certify."""
    st, s = tie_store
    x = act(om, 999, 4)
    x[2, 100] = np.nan
    _, idx, _, _, chained = run(om, ctx, st, x, 0, 0, 0)
    _, ridx, _ = oracle_routing(x, s.router, None, 0)
    say(f"NaN token: idx {idx[2].tolist()} ref {ridx[2].tolist()}, chained {chained}")
    assert chained >= 1
    assert np.array_equal(idx, ridx)
