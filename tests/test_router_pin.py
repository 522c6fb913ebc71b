"""GPU pins of the router logits the MoE forward runs on, bit for bit.

The forward computes each logit as the reference does (model.c:1017-1025:
a sequential fp32 sum from 0 of the fp32 products x[d]*W[d*E+e], d
ascending, then + bias), so the logits it selected on must equal the
oracle's (oracle/oracle.c orc_router_logits) as uint32, for every kernel
instance the forward picks:
  - k_router_pc (T <= 64), with its fused rmsnorm when ORN_MOE_NORM is set;
  - k_router_dec (64 < T < 1024), after the separate rmsnorm kernel;
  - k_router_seq (T >= 1024);
with and without a Zipf router bias, and for the file-orientation store
(router transposed at upload).  A one-ulp difference from a changed add
order fails these tests, where index equality alone would not see it.
The selection weights are compared to the oracle's within 2e-6 relative
(the device's expf against glibc's); the indices exactly.

Decode batches of up to 4 tokens route by default through the certified kernel
(router_cert.hip), whose logits are fp64 sums within a proven bound of
these chains (tests/test_router_cert.py); every call here passes
ORN_MOE_EXACT_LOGITS, which selects the exact chains at every size.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

D, H, E, K = 2048, 512, 256, 8
SEED = 4242


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
    """Two Ornith-shape layers: layer 0 plain, layer 1 with a Zipf(1.1)
    router bias; both with non-trivial rmsnorm weights."""
    st = om.Store(ctx, 2, D, H, E, K, True)
    syn = []
    rng = np.random.default_rng(7)
    norms = []
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


def forward(om, ctx, st, x, layer, flags):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * K * 4), ctx.alloc(T * K * 4)
    st.forward(layer, xb, T, ob, idx=ib, w=wb, flags=flags)
    logits = st.last_logits(T)
    idx = ctx.download(ib, np.uint32, (T, K))
    w = ctx.download(wb, np.float32, (T, K))
    for b in (xb, ob, ib, wb):
        b.free()
    return logits, idx, w


def check(om, ctx, store, T, layer, norm):
    st, syn, norms = store
    s = syn[layer]
    x = act(om, 1000 + T + 7 * layer, T)
    flags = (om.MOE_NORM if norm else 0) | om.MOE_EXACT_LOGITS
    logits, idx, w = forward(om, ctx, st, x, layer, flags)
    xin = O.rmsnorm(x, norms[layer]) if norm else x
    ref = O.router_logits_rows(xin, s.router, s.bias)
    diff = logits.view(np.uint32) != ref.view(np.uint32)
    say(f"T={T} layer={layer} norm={norm}: {int(diff.sum())} of {diff.size} logits differ")
    assert not diff.any(), np.argwhere(diff)[:5]
    ridx = np.zeros((T, K), np.uint32)
    rw = np.zeros((T, K), np.float32)
    for t in range(T):
        ridx[t], rw[t] = O.topk(ref[t], K, O.MODE_RENORM)
    assert np.array_equal(idx, ridx)
    rel = np.abs(w.astype(np.float64) - rw) / np.abs(rw)
    say(f"  weights: max rel diff {rel.max():.2e}")
    assert rel.max() <= 2e-6


@pytest.mark.parametrize("norm", [False, True], ids=["x", "rmsnorm"])
@pytest.mark.parametrize("T", [1, 16, 64])
def test_router_pc_logits_bit_exact(om, ctx, store, T, norm):
    check(om, ctx, store, T, 0, norm)


@pytest.mark.parametrize("norm", [False, True], ids=["x", "rmsnorm"])
@pytest.mark.parametrize("T", [65, 100, 256, 383])
def test_router_dec_logits_bit_exact(om, ctx, store, T, norm):
    check(om, ctx, store, T, 0, norm)


@pytest.mark.parametrize("T", [384, 400, 1023, 1024, 2048])
def test_router_seq_logits_bit_exact(om, ctx, store, T):
    """LDS-staged chains: 4 tokens per block (T < 1024), 16 (T >= 1024)."""
    check(om, ctx, store, T, 0, T == 400)


@pytest.mark.parametrize("T", [1, 16, 256])
def test_router_bias_logits_bit_exact(om, ctx, store, T):
    """The Zipf bias is added after the chain (model.c sums, then + b)."""
    check(om, ctx, store, T, 1, T == 16)


@pytest.mark.parametrize("T", [1, 16])
def test_file_orientation_router_bit_exact(om, ctx, T):
    """A file-orientation store takes ffn_gate_inp as W[e*D + d] and
    transposes it at upload; the logits are the same sequential sums."""
    st = om.Store(ctx, 1, D, H, E, K, True, prefill_layout=False, file_layout=True)
    try:
        W = om.synth_normal(SEED, om.synth_stream(0, om.SYN_ROUTER, 0), D * E, 0.02).reshape(D, E)
        st.set_router(0, np.ascontiguousarray(W.T))  # file orientation: [E][D]
        x = act(om, 77 + T, T)
        logits, idx, _ = forward(om, ctx, st, x, 0, om.MOE_EXACT_LOGITS)
        ref = O.router_logits_rows(x, W)
        assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
        for t in range(T):
            assert np.array_equal(idx[t], O.topk(ref[t], K)[0])
    finally:
        st.close()
