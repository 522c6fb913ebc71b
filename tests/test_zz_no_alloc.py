"""GPU test of gpu_moe_forward_noalloc: the forward whose work buffers live in
the device's fixed scratch array instead of an allocated workspace.

It runs the same kernels with the same plan as gpu_moe_forward, so its
outputs, indices and weights must equal gpu_moe_forward's bit for bit.  Two
calls in a row, the second with a smaller batch, check that the scratch's
leftover contents from the first call do not leak into the second.  Batches
of more than 16 tokens (separate selection and dispatch launches) and a
file-orientation store are covered too.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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


def act(om, seed, T, D):
    return om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)


def call(om, ctx, store, x, k, noalloc, flags=0, resid=None, mode=0):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * k * 4), ctx.alloc(T * k * 4)
    rb = ctx.upload(resid) if resid is not None else None
    store.forward(0, xb, T, ob, resid=rb, idx=ib, w=wb, flags=flags, mode=mode, noalloc=noalloc)
    res = (ctx.download(ob, np.float32, x.shape), ctx.download(ib, np.uint32, (T, k)),
           ctx.download(wb, np.float32, (T, k)))
    for b in (xb, ob, ib, wb, rb):
        if b is not None:
            b.free()
    return res


@pytest.mark.parametrize("shape", [(256, 256, 16, 8), (2048, 512, 256, 8)],
                         ids=["small", "ornith"])
@pytest.mark.parametrize("flags", [0, 2], ids=["plain", "norm"])
def test_noalloc_equals_forward(om, ctx, shape, flags):
    D, H, E, k = shape
    say(f"noalloc vs forward D={D} H={H} E={E} k={k} flags={flags}")
    store = om.Store(ctx, 1, D, H, E, k, True)
    try:
        store.fill_synthetic(0, 77)
        # calls in a row, each smaller than the one before, with the scratch
        # still holding the previous call's buffers (40 tokens: selection and
        # dispatch as two launches)
        for T in (40, 16, 3):
            x = act(om, 900 + T, T, D)
            resid = act(om, 950 + T, T, D) if flags else None
            got = call(om, ctx, store, x, k, True, flags, resid)
            ref = call(om, ctx, store, x, k, False, flags, resid)
            for g, r, what in zip(got, ref, ("out", "idx", "w")):
                assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (T, what)
            say(f"  T={T}: bit-identical to gpu_moe_forward")
        # and once more at the first size, after the smaller call
        x = act(om, 999, 16, D)
        got = call(om, ctx, store, x, k, True, flags)
        ref = call(om, ctx, store, x, k, False, flags)
        for g, r in zip(got, ref):
            assert np.array_equal(g.view(np.uint32), r.view(np.uint32))
    finally:
        store.close()


def test_noalloc_file_layout(om, ctx):
    """A file-orientation store (the kernels real GGUF files run): the same
    bit-for-bit equality, 40 then 16 then 3 tokens."""
    D, H, E, k = 256, 256, 16, 8
    syn = om.SyntheticLayer(41, 0, D, H, E, True)
    store = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=False, file_layout=True)
    try:
        for name, m in (("gate", om.MAT_GATE), ("up", om.MAT_UP), ("down", om.MAT_DOWN)):
            store.set_experts(0, m, 0, getattr(syn, name), E + 1)
        store.set_router(0, np.ascontiguousarray(syn.router.T))
        for T in (40, 16, 3):
            x = act(om, 700 + T, T, D)
            got = call(om, ctx, store, x, k, True)
            ref = call(om, ctx, store, x, k, False)
            for g, r, what in zip(got, ref, ("out", "idx", "w")):
                assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (T, what)
            say(f"  file layout T={T}: bit-identical to gpu_moe_forward")
    finally:
        store.close()


def test_noalloc_refuses_what_does_not_fit(om, ctx):
    """Batches whose work buffers exceed the fixed scratch, and graph replay
    (instantiation allocates), are refused with an error and run nothing."""
    D, H, E, k = 2048, 512, 256, 8
    store = om.Store(ctx, 1, D, H, E, k, True)
    try:
        store.fill_synthetic(0, 5)
        T = 2048
        xb, ob = ctx.alloc(T * D * 4), ctx.alloc(T * D * 4)
        with pytest.raises(RuntimeError, match="fixed scratch"):
            store.forward(0, xb, T, ob, noalloc=True)
        with pytest.raises(RuntimeError, match="GRAPH"):
            store.forward(0, xb, 4, ob, noalloc=True, flags=om.MOE_GRAPH)
        xb.free()
        ob.free()
        # the context still works afterwards
        x = act(om, 31, 2, D)
        got = call(om, ctx, store, x, k, True)
        ref = call(om, ctx, store, x, k, False)
        assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
    finally:
        store.close()
