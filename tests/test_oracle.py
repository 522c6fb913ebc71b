"""Pins the C99 oracle (oracle/oracle.c) before it is trusted as the checker.

Every oracle function is checked against golden vectors written by the
COMPILED REFERENCE (tests/golden/make_golden.py) and, where the mathematics
fixes the answer, against an independent closed form:

  fp16 quirk        all 65536 patterns: reference golden + closed form
  Q4_K / Q6_K       reference golden (random + special halves), the
                    reference's own known-answer blocks (1.0 / -31.0), and a
                    vectorised closed form of the block layout
  element extract   equals the block dequant at all 256 positions
  expert slice      reference golden; slice identity slice[i] = full[i*E+e];
                    the reference's invalid-argument cases
  routing           reference model_get_routing golden (Ornith shape, exact
                    ties, the [1,1,9] exchange pattern)
  MoE layer         reference model_forward golden (tiny, small, tie, and the
                    full Ornith shape) in the literal mode and interleaved
                    layout; the contiguous layout and renormalised mode
                    against an fp64 brute force
"""
import hashlib
import math
import os

import numpy as np
import pytest

from oracle import oracle as O


def load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ----------------------------------------------------------------- fp16 quirk
def closed_form_half(h):
    if h == 0:
        return 0.0
    s = -1.0 if h & 0x8000 else 1.0
    e = (h >> 10) & 31
    m = h & 0x3FF
    return s * math.ldexp(1.0 + m / 1024.0, e - 15)


def test_fp16_all_patterns(golden_dir):
    g = load(golden_dir, "dequant_f16_all.npz")
    ok, out = O.dequant_tensor(g["halves"].view(np.uint8), O.TYPE_F16, 65536)
    assert ok
    assert np.array_equal(bits(out), bits(g["expected"]))
    cf = np.array([closed_form_half(h) for h in range(65536)], np.float64).astype(np.float32)
    assert np.array_equal(bits(out), bits(cf))
    # The quirks the reference has and IEEE does not (gguf.c:16-26).
    assert O.fp16_to_fp32(0x8000) == -(2.0 ** -15)
    assert O.fp16_to_fp32(0x0001) == 2.0 ** -15 * (1 + 1 / 1024)
    assert O.fp16_to_fp32(0x7C00) == 2.0 ** 16


# ----------------------------------------------------------------- K-quants
def np_scale_min(scales):
    """Vectorised 6-bit sc/m unpacking of [n,12] bytes -> ([n,8], [n,8])."""
    s = scales.astype(np.int64)
    sc = np.zeros((s.shape[0], 8), np.int64)
    m = np.zeros_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def np_half(hbytes):
    h = hbytes[:, 0].astype(np.int64) | (hbytes[:, 1].astype(np.int64) << 8)
    return np.array([closed_form_half(int(v)) for v in h], np.float64).astype(np.float32)


def np_q4k(blocks):
    b = blocks.reshape(-1, 144)
    d, dmin = np_half(b[:, 0:2]), np_half(b[:, 2:4])
    sc, m = np_scale_min(b[:, 4:16])
    qs = b[:, 16:].astype(np.int64)
    y = np.zeros((b.shape[0], 256), np.float32)
    for c in range(4):
        lo, hi = qs[:, 32 * c:32 * c + 32] & 15, qs[:, 32 * c:32 * c + 32] >> 4
        for half, q in ((0, lo), (1, hi)):
            sb = 2 * c + half
            D = (d * sc[:, sb].astype(np.float32))[:, None]
            M = (dmin * m[:, sb].astype(np.float32))[:, None]
            y[:, 64 * c + 32 * half:64 * c + 32 * half + 32] = D * q.astype(np.float32) - M
    return y.reshape(-1)


def np_q6k(blocks):
    b = blocks.reshape(-1, 210)
    d = np_half(b[:, 208:210])
    ql, qh = b[:, 0:128].astype(np.int64), b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    y = np.zeros((b.shape[0], 256), np.float32)
    for n in range(2):
        for j in range(4):
            l = np.arange(32)
            qlb = ql[:, 64 * n + (32 if j % 2 else 0) + l]
            lo = (qlb & 15) if j < 2 else (qlb >> 4)
            q = (lo | (((qh[:, 32 * n + l] >> (2 * j)) & 3) << 4)) - 32
            s = sc[:, 8 * n + 2 * j + l // 16]
            y[:, 128 * n + 32 * j + l] = (d[:, None] * s) * q.astype(np.float32)
    return y.reshape(-1)


@pytest.mark.parametrize("name,typ,npf", [("dequant_q4k.npz", O.TYPE_Q4_K, np_q4k),
                                          ("dequant_q6k.npz", O.TYPE_Q6_K, np_q6k)])
def test_kquant_golden_and_closed_form(golden_dir, name, typ, npf):
    g = load(golden_dir, name)
    blocks = g["blocks"]
    ok, out = O.dequant_tensor(blocks.reshape(-1), typ, 256 * blocks.shape[0])
    assert ok
    assert np.array_equal(bits(out), bits(g["expected"]))
    assert np.array_equal(bits(out), bits(npf(blocks)))
    # First block is the reference's own known-answer block.
    kat = 1.0 if typ == O.TYPE_Q4_K else -31.0
    assert np.all(out[:256] == kat)


@pytest.mark.parametrize("typ,bs", [(O.TYPE_Q4_K, 144), (O.TYPE_Q6_K, 210)])
def test_one_element_equals_block(golden_dir, typ, bs):
    g = load(golden_dir, "dequant_q4k.npz" if typ == O.TYPE_Q4_K else "dequant_q6k.npz")
    blocks = g["blocks"][:24]
    one = O.lib().orc_q4k_one if typ == O.TYPE_Q4_K else O.lib().orc_q6k_one
    for bi in range(blocks.shape[0]):
        b = np.ascontiguousarray(blocks[bi])
        ok, full = O.dequant_tensor(b, typ, 256)
        vals = np.array([one(b.ctypes.data, p) for p in range(256)], np.float32)
        assert np.array_equal(bits(vals), bits(full))


def test_f32_passthrough_and_unsupported(golden_dir):
    g = load(golden_dir, "dequant_f32.npz")
    ok, out = O.dequant_tensor(g["data"].view(np.uint8), O.TYPE_F32, g["data"].size)
    assert ok and np.array_equal(bits(out), bits(g["expected"]))
    ok, _ = O.dequant_tensor(np.zeros(64, np.uint8), 2, 32)  # Q4_0 is not handled (gguf.c:635-637)
    assert not ok


# ----------------------------------------------------------------- slices
def slice_fixtures(golden_dir):
    return sorted(f for f in os.listdir(golden_dir) if f.startswith("slice_"))


def test_slices_golden_and_identity(golden_dir):
    names = slice_fixtures(golden_dir)
    assert len(names) >= 9
    for name in names:
        g = load(golden_dir, name)
        typ, dims = int(g["type"]), [int(d) for d in g["dims"]]
        n = int(np.prod(dims))
        E = dims[-1]
        ok, full = O.dequant_tensor(g["data"], typ, n)
        assert ok
        for row, e in enumerate(g["experts"]):
            ok, sl = O.expert_slice(g["data"], typ, n, E, int(e))
            assert ok
            assert np.array_equal(bits(sl), bits(g["expected"][row])), (name, e)
            assert np.array_equal(bits(sl), bits(full[int(e)::E][:n // E])), (name, e)
        if name == "slice_q4k_kat.npz":
            assert np.all(g["expected"] == 1.0)


def test_slice_invalid_arguments():
    """t_gguf.c:699-735 plus E == 0 (gguf.c:656-662)."""
    data = np.zeros(144, np.uint8)
    L = O.lib()
    out = np.zeros(64, np.float32)
    assert not O.expert_slice(data, O.TYPE_Q4_K, 256, 4, -1)[0]
    assert not O.expert_slice(data, O.TYPE_Q4_K, 256, 4, 4)[0]
    assert not O.expert_slice(data, O.TYPE_Q4_K, 256, 4, 99)[0]
    assert not O.expert_slice(data, O.TYPE_Q4_K, 256, 0, 0)[0]
    assert L.orc_dequant_expert_slice(None, O.TYPE_Q4_K, 256, 4, 0, out.ctypes.data) == 0
    assert L.orc_dequant_expert_slice(data.ctypes.data, O.TYPE_Q4_K, 256, 4, 0, None) == 0
    assert not O.expert_slice(data, 2, 256, 4, 0)[0]


# ----------------------------------------------------------------- routing
def test_routing_ornith_golden(golden_dir):
    import ornith_moe as om
    g = load(golden_dir, "routing_ornith.npz")
    seed, T = int(g["seed"]), int(g["n_tokens"])
    D, E, k = 2048, 256, 8
    W = om.synth_normal(seed, om.synth_stream(0, om.SYN_ROUTER, 0), D * E, 0.02).reshape(D, E)
    X = om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)
    assert hashlib.sha256(W.tobytes() + X.tobytes()).digest() == g["sha256"].tobytes()
    for t in range(T):
        lg = O.router_logits(X[t], W)
        idx, w = O.topk(lg, k, O.MODE_RENORM)
        assert np.array_equal(idx, g["idx"][t]), t
        assert np.array_equal(bits(w), bits(g["w"][t])), t
        # fp64 cross-check of the logits the selection ran on.
        l64 = X[t].astype(np.float64) @ W.astype(np.float64)
        assert np.max(np.abs(lg - l64)) < 1e-4


@pytest.mark.parametrize("name", ["routing_ties.npz", "routing_exchange.npz"])
def test_routing_ties_golden(golden_dir, name):
    g = load(golden_dir, name)
    W, X = g["W"], g["x"]
    k = g["idx"].shape[1]
    for t in range(X.shape[0]):
        idx, w = O.topk(O.router_logits(X[t], W), k, O.MODE_RENORM)
        assert np.array_equal(idx, g["idx"][t]), (name, t, idx, g["idx"][t])
        assert np.array_equal(bits(w), bits(g["w"][t]))


def test_exchange_rule_example():
    """Exchange selection with strict '>' is not index-ordered on ties:
    logits [1, 1, 9] select 2, 1, 0 (model.c:301-305)."""
    idx, _ = O.topk(np.array([1, 1, 9], np.float32), 3, O.MODE_RENORM)
    assert list(idx) == [2, 1, 0]
    idx, _ = O.topk(np.array([1, 5, 3, 5, 9], np.float32), 3, O.MODE_RENORM)
    assert list(idx) == [4, 3, 1]


# ----------------------------------------------------------------- MoE layer
def run_literal(g):
    D, H, E, k = [int(v) for v in g["shape"]]
    if "synth_seed" in g.files:
        from tests.golden.make_golden import _synth_weights
        (gate, up, down), sh = _synth_weights(int(g["synth_seed"]), D, H, E)
        dig = hashlib.sha256()
        for a in (gate, up, down, *sh):
            dig.update(a.tobytes())
        assert dig.digest() == g["sha256"].tobytes()
    else:
        gate, up, down = g["gate"], g["up"], g["down"]
        sh = [g["sh_gate"], g["sh_up"], g["sh_down"]]
    x = g["x"]
    out, idx, w = O.moe_layer(D=D, H=H, E=E, k=k, x=x, resid=x, norm_w=g["norm_w"],
                              router_W=g["router_W"], gate=gate, up=up, down=down,
                              sh_gate=sh[0], sh_up=sh[1], sh_down=sh[2], mode=O.MODE_LITERAL,
                              layout=O.LAYOUT_INTERLEAVED)
    return out


@pytest.mark.parametrize("name", ["moe_tiny_d64.npz", "moe_small_d256.npz", "moe_tie_d64.npz"])
def test_moe_layer_golden(golden_dir, name):
    g = load(golden_dir, name)
    out = run_literal(g)
    assert np.array_equal(bits(out), bits(g["expected"]))


def test_moe_layer_golden_ornith_shape(golden_dir):
    import ornith_moe as om
    g = load(golden_dir, "moe_ornith_d2048.npz")
    seed = int(g["seed"])
    D, H, E, k = [int(v) for v in g["shape"]]
    nblk = D * H * E // 256
    fused = [fn(seed, om.synth_stream(0, kind, 0xFFFFFF), nblk) for kind, fn in
             ((om.SYN_GATE, om.synth_q4k), (om.SYN_UP, om.synth_q4k), (om.SYN_DOWN, om.synth_q6k))]
    nbs = D * H // 256
    sh = [fn(seed, om.synth_stream(0, kind, E), nbs) for kind, fn in
          ((om.SYN_GATE, om.synth_q4k), (om.SYN_UP, om.synth_q4k), (om.SYN_DOWN, om.synth_q6k))]
    W = om.synth_normal(seed, om.synth_stream(0, om.SYN_ROUTER, 0), D * E, 0.02).reshape(D, E)
    X = om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), 2 * D, 1.0).reshape(2, D)
    dig = hashlib.sha256()
    for a in (*fused, *sh, W, X):
        dig.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    assert dig.digest() == g["sha256"].tobytes()
    out, _, _ = O.moe_layer(D=D, H=H, E=E, k=k, x=X, resid=X, norm_w=np.ones(D, np.float32),
                            router_W=W, gate=fused[0], up=fused[1], down=fused[2], sh_gate=sh[0],
                            sh_up=sh[1], sh_down=sh[2], mode=O.MODE_LITERAL,
                            layout=O.LAYOUT_INTERLEAVED)
    assert np.array_equal(bits(out), bits(g["expected"]))


def np_moe_fp64(D, H, E, k, x, W, gate, up, down, sh, bias=None, shexp_gate=None):
    """fp64 brute force of the contiguous-layout, renormalised layer with an
    independent (vectorised) dequant (and, with shexp_gate, the shared
    expert scaled by sigmoid(shexp_gate . x)); returns (out, idx)."""
    nb = D * H // 256

    def mats(q4, q6):
        return (np_q4k(q4).astype(np.float64).reshape(D, H),
                np_q6k(q6).astype(np.float64).reshape(H, D))

    def ffn(xv, Wg, Wu, Wd, clamp):
        g = xv @ Wg
        u = xv @ Wu
        s = g / (1 + np.exp(-g))
        if clamp:
            s = np.where(g < -50, 0.0, np.where(g > 50, g, s))
        return (s * u) @ Wd

    out = np.zeros((x.shape[0], D))
    idx_all = []
    for t in range(x.shape[0]):
        xv = x[t].astype(np.float64)
        Wg, Wd = mats(sh[0], sh[2])
        Wu = np_q4k(sh[1]).astype(np.float64).reshape(D, H)
        y = ffn(xv, Wg, Wu, Wd, False)
        if shexp_gate is not None:
            y = y / (1.0 + np.exp(-(xv @ shexp_gate.astype(np.float64))))
        lg = xv @ W.astype(np.float64) + (0 if bias is None else bias)
        order = np.argsort(-lg, kind="stable")[:k]
        ww = np.exp(lg[order] - lg[order[0]])
        ww /= ww.sum()
        for e, wv in zip(order, ww):
            q4g = gate[e * nb * 144:(e + 1) * nb * 144]
            q4u = up[e * nb * 144:(e + 1) * nb * 144]
            q6 = down[e * nb * 210:(e + 1) * nb * 210]
            y = y + wv * ffn(xv, np_q4k(q4g).astype(np.float64).reshape(D, H),
                             np_q4k(q4u).astype(np.float64).reshape(D, H),
                             np_q6k(q6).astype(np.float64).reshape(H, D), True)
        out[t] = y
        idx_all.append(order)
    return out, np.array(idx_all)


def test_contiguous_layout_vs_fp64():
    import ornith_moe as om
    D, H, E, k, T = 256, 256, 16, 8, 6
    # with a Zipf(1.1) router bias, so the bias term of the logits is pinned too
    syn = om.SyntheticLayer(99, 0, D, H, E, True, 1.1)
    assert syn.bias is not None and np.ptp(syn.bias) > 1.0
    x = om.synth_normal(99, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)
    out, idx, w = O.moe_layer(D=D, H=H, E=E, k=k, x=x, router_W=syn.router, bias=syn.bias,
                              gate=syn.routed("gate"), up=syn.routed("up"),
                              down=syn.routed("down"), sh_gate=syn.shared("gate"),
                              sh_up=syn.shared("up"), sh_down=syn.shared("down"))
    ref, ridx = np_moe_fp64(D, H, E, k, x, syn.router, syn.routed("gate"), syn.routed("up"),
                            syn.routed("down"), [syn.shared(m) for m in ("gate", "up", "down")],
                            bias=syn.bias.astype(np.float64))
    assert np.array_equal(idx.astype(np.int64), ridx)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
    err = np.abs(out - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert err.max() < 1e-5, err


def test_shexp_gate_special_cases_and_fp64():
    """The optional shared-expert gate of orc_moe_layer_ex (no reference
    counterpart), pinned by the values sigmoid takes exactly: a dot of +huge
    (gate 1) reproduces the ungated layer bit for bit, -huge (gate 0) the
    layer without a shared expert bit for bit, a zero vector (gate 1/2 exactly)
    their mean; and a random gate against the fp64 brute force."""
    import ornith_moe as om
    D, H, E, k, T = 256, 256, 16, 8, 5
    syn = om.SyntheticLayer(7, 0, D, H, E, True)
    x = om.synth_normal(7, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)
    resid = om.synth_normal(8, om.synth_stream(0, om.SYN_ACT, 1), T * D, 1.0).reshape(T, D)
    common = dict(D=D, H=H, E=E, k=k, x=x, resid=resid, router_W=syn.router,
                  gate=syn.routed("gate"), up=syn.routed("up"), down=syn.routed("down"))
    shared = dict(sh_gate=syn.shared("gate"), sh_up=syn.shared("up"), sh_down=syn.shared("down"))
    ungated, _, _ = O.moe_layer(**common, **shared)
    no_shared, _, _ = O.moe_layer(**common)
    # per row, a gate vector along the row's sign pattern with a huge scale:
    # a dot of about +1e32 (expf(-dot) = 0: gate exactly 1) or, negated,
    # -1e32 (expf(-dot) = inf: gate exactly 0)
    for t in range(T):
        g_pos = (np.float32(1e30) * np.sign(x[t])).astype(np.float32)
        one, _, _ = O.moe_layer(**{**common, "x": x[t:t + 1], "resid": resid[t:t + 1]}, **shared,
                                shexp_gate=g_pos)
        zero, _, _ = O.moe_layer(**{**common, "x": x[t:t + 1], "resid": resid[t:t + 1]}, **shared,
                                 shexp_gate=-g_pos)
        assert np.array_equal(one.view(np.uint32), ungated[t:t + 1].view(np.uint32))
        assert np.array_equal(zero.view(np.uint32), no_shared[t:t + 1].view(np.uint32))
    half, _, _ = O.moe_layer(**common, **shared, shexp_gate=np.zeros(D, np.float32))
    mid = 0.5 * (ungated.astype(np.float64) + no_shared)
    assert np.abs(half - mid).max() <= 1e-5 * np.abs(mid).max()
    assert np.abs(half - ungated).max() > 1e-3 * np.abs(mid).max()  # the gate acts
    rng = np.random.default_rng(3)
    gv = (rng.standard_normal(D) * 0.05).astype(np.float32)
    out, idx, _ = O.moe_layer(**{**common, "resid": None}, **shared, shexp_gate=gv)
    ref, ridx = np_moe_fp64(D, H, E, k, x, syn.router, syn.routed("gate"), syn.routed("up"),
                            syn.routed("down"), [syn.shared(m) for m in ("gate", "up", "down")],
                            shexp_gate=gv)
    assert np.array_equal(idx.astype(np.int64), ridx)
    err = np.abs(out - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert err.max() < 1e-5, err
