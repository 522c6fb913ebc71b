"""How tight the GPU parity bar has to be (CPU; numpy emulation, no GPU).

The GPU tests compare the MFMA kernels with the oracle at
max|dy|/max|y| <= 1e-5 per row.  This file shows, at the Ornith shape
(D=2048, H=512, E=256, k=8, shared expert), that the bar catches a kernel
that drops any one term of its arithmetic while the shipped arithmetic
passes with room:

- tests/kquant_np.py's component decoders rebuild the oracle's dequantized
  weights bit for bit (so the emulation multiplies the reference's numbers);
- tests/mfma_emul.py with the shipped operands (fp16 hi + lo activations,
  exact sc*q, the q6_b2 remainder for wide Q6_K scales) lands within the
  oracle's own fp32 rounding of it;
- dropping the activation lo plane of gate/up, of the mins term or of down,
  or the q6_b2 remainder operand, each moves the output by more than 1e-5.
"""
import os

import numpy as np
import pytest

import kquant_np as KQ
import mfma_emul as M
from oracle import oracle as O

D, H, E, K = 2048, 512, 256, 8
BAR = 1e-5


@pytest.fixture(scope="module")
def om():
    import ornith_moe
    ornith_moe.lib()
    return ornith_moe


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_components_rebuild_oracle_dequant(om, golden_dir):
    """Components -> fp32 weights in the reference's order == the oracle's
    dequantization (itself pinned by the reference's goldens), on the golden
    blocks and on random blocks, including every fp16 pattern of d."""
    for name, typ, comp, wts, bs in (("dequant_q4k.npz", O.TYPE_Q4_K, KQ.q4k_components,
                                      KQ.q4k_weights, 144),
                                     ("dequant_q6k.npz", O.TYPE_Q6_K, KQ.q6k_components,
                                      KQ.q6k_weights, 210)):
        g = np.load(os.path.join(golden_dir, name), allow_pickle=False)
        blocks = g["blocks"].reshape(-1)
        n = blocks.size // bs
        assert np.array_equal(bits(wts(comp(blocks)).reshape(-1)), bits(g["expected"][:256 * n]))
        rng = np.random.default_rng(5)
        rb = rng.integers(0, 256, size=(4096, bs), dtype=np.uint8)
        doff = 0 if bs == 144 else 208
        pat = np.arange(4096, dtype=np.uint32) * 16 + 5  # spread over all 65536 patterns
        rb[:, doff] = pat & 0xFF
        rb[:, doff + 1] = pat >> 8
        ok, ref = O.dequant_tensor(rb.reshape(-1), typ, 4096 * 256)
        assert ok
        got = wts(comp(rb.reshape(-1))).reshape(-1)
        assert np.array_equal(bits(got), bits(ref))


def wide_q6_scales(blocks, rng):
    """Q6_K sub-scales over the int8 range, each block's first at -128 or 127
    (what quantizers emit)."""
    b = blocks.reshape(-1, 210).copy()
    sc = rng.integers(-128, 128, size=(b.shape[0], 16))
    sc[:, 0] = np.where(rng.random(b.shape[0]) < 0.5, -128, 127)
    b[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    return b.reshape(-1)


class SparseLayer:
    """The bench's synthetic Ornith layer (seed 1234, layer 0), with only the
    experts a batch selects generated (the others stay zero bytes, which
    neither the oracle nor the emulation reads)."""

    def __init__(self, om, x, seed=1234, wide_rng=None):
        nb = D * H // 256
        self.nb = nb
        self.router = om.synth_normal(seed, om.synth_stream(0, om.SYN_ROUTER, 0), D * E,
                                      0.02).reshape(D, E)
        self.bias = None
        self.idx = np.zeros((x.shape[0], K), np.uint32)
        self.w = np.zeros((x.shape[0], K), np.float32)
        for t in range(x.shape[0]):
            self.idx[t], self.w[t] = O.topk(O.router_logits(x[t], self.router), K, O.MODE_RENORM)
        self.arr = {"gate": np.zeros((E + 1) * nb * 144, np.uint8),
                    "up": np.zeros((E + 1) * nb * 144, np.uint8),
                    "down": np.zeros((E + 1) * nb * 210, np.uint8)}
        for e in list(np.unique(self.idx)) + [E]:
            e = int(e)
            for which, kind in (("gate", om.SYN_GATE), ("up", om.SYN_UP)):
                self.arr[which][e * nb * 144:(e + 1) * nb * 144] = om.synth_q4k(
                    seed, om.synth_stream(0, kind, e), nb)
            dn = om.synth_q6k(seed, om.synth_stream(0, om.SYN_DOWN, e), nb)
            if wide_rng is not None:
                dn = wide_q6_scales(dn, wide_rng)
            self.arr["down"][e * nb * 210:(e + 1) * nb * 210] = dn

    def routed(self, which):
        per = self.nb * (210 if which == "down" else 144)
        return self.arr[which][:E * per]

    def shared(self, which):
        per = self.nb * (210 if which == "down" else 144)
        return self.arr[which][E * per:(E + 1) * per]

    def oracle(self, x):
        out, idx, w = O.moe_layer(D=D, H=H, E=E, k=K, x=x, router_W=self.router,
                                  gate=self.routed("gate"), up=self.routed("up"),
                                  down=self.routed("down"), sh_gate=self.shared("gate"),
                                  sh_up=self.shared("up"), sh_down=self.shared("down"))
        assert np.array_equal(idx, self.idx)
        return out


def act(om, T, seed=1234):
    return om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)


def test_bar_catches_each_dropped_term(om):
    x = act(om, 3)
    L = SparseLayer(om, x)
    ref = L.oracle(x)
    variants = {"exact": None, "shipped": M.SHIPPED,
                "no activation lo (gate/up)": M.Variant(act="rtz"),
                "no mins lo (gate/up)": M.Variant(act_mins="rtz"),
                "no activation lo (down)": M.Variant(act_down="rtz")}
    res = M.layer(D=D, H=H, E=E, k=K, x=x, syn=L, idx=L.idx, w=L.w, variants=variants)
    errs = {n: M.row_err(v, ref).max() for n, v in res.items()}
    print({n: f"{e:.2e}" for n, e in errs.items()})
    # the oracle's own fp32 chains sit ~1e-6 from the fp64 products; the
    # shipped arithmetic is as close to them as the exact products are
    assert errs["exact"] < 3e-6
    assert errs["shipped"] < 3e-6
    assert M.row_err(res["shipped"], res["exact"]).max() < 1e-6
    for n in variants:
        if n.startswith("no "):
            assert errs[n] > 3 * BAR, (n, errs[n])


def test_bar_catches_dropped_q6_remainder(om):
    """Q6_K sub-scales up to 128: sc*q up to 4096 is not exact as one fp16
    operand.  The shipped form adds A_hi*b2 (the exact remainder); without
    it the output moves past the bar, with it it stays within the oracle's
    own rounding."""
    x = act(om, 3, seed=77)
    L = SparseLayer(om, x, seed=77, wide_rng=np.random.default_rng(7))
    ref = L.oracle(x)
    variants = {"exact": None, "shipped": M.SHIPPED, "no q6 remainder": M.Variant(q6="b1")}
    res = M.layer(D=D, H=H, E=E, k=K, x=x, syn=L, idx=L.idx, w=L.w, variants=variants)
    errs = {n: M.row_err(v, ref).max() for n, v in res.items()}
    print({n: f"{e:.2e}" for n, e in errs.items()})
    assert errs["exact"] < 3e-6
    assert errs["shipped"] < 3e-6
    assert errs["no q6 remainder"] > 2 * BAR, errs["no q6 remainder"]
