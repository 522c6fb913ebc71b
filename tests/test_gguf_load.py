"""A model file's MoE tensors straight into a resident store
(gpu_moe_store_load_gguf, GGUF reader of csrc/host/gguf_file.c).

The file is written with the tensor names and shapes the reference loads
(model.c:707-711 routed experts ne = [D, H, E] / [H, D, E], 847-852 shared
expert ne = [D, H] / [H, D], 861 router ne = [D, E], 807 norm [D]), with
other layers' tensors and unrelated tensors around it.  The loaded store must
hold exactly the file's bytes (read back with gpu_moe_store_get_experts) and
its forwards must equal, bit for bit, those of a store filled through
set_experts / set_router / set_norm with the same bytes (a path pinned
against the oracle in the file-layout tests), and match the oracle here
too.  An f16 router goes through the reference's fp16 rule (gguf.c:16-26,
pinned on all 65,536 patterns elsewhere).  Wrong shapes, types and stores
are refused.
"""
import os
import sys
import tempfile

import numpy as np
import pytest

from oracle import gguf_writer as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5  # file-layout kernels vs the oracle (measured ~1e-6)


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


def model_file(om, path, D, H, E, layers, router_f16=False, norm=True, seed=3, shexp_gate=False):
    """Write a GGUF whose layers `layers` carry synthetic MoE tensors (the
    bytes of SyntheticLayer(seed, l)); returns {layer: (syn, router_file,
    norm_w, gate)} where router_file is the [E][D] fp32 router as stored and
    gate the shared-expert gate as the loader decodes it (with shexp_gate:
    ffn_gate_inp_shexp.weight, f16 when router_f16, else f32; else None)."""
    rng = np.random.default_rng(seed)
    md = [("general.architecture", "str", "qwen35moe"), ("qwen35moe.block_count", "u32", 40),
          ("qwen35moe.expert_count", "u32", E), ("qwen35moe.embedding_length", "u32", D),
          ("tokenizer.ggml.tokens", "arr", ("str", ["a", "b", "c"]))]
    tensors = [("token_embd.weight", om.TYPE_F32, [D, 4], rng.standard_normal(4 * D).astype(np.float32))]
    per_q4 = D * H // 256 * om.Q4K_BYTES
    per_q6 = D * H // 256 * om.Q6K_BYTES
    info = {}
    for l in layers:
        syn = om.SyntheticLayer(seed, l, D, H, E, True)
        if router_f16:
            r16 = (rng.standard_normal(E * D) * 0.02).astype(np.float16)
            rbytes, rtype = r16, om.TYPE_F16
            rfile = np.array([O.fp16_to_fp32(int(h)) for h in r16.view(np.uint16)],
                             np.float32).reshape(E, D)
        else:
            rfile = np.ascontiguousarray(syn.router.T)  # [E][D]: W[e*D + d]
            rbytes, rtype = rfile, om.TYPE_F32
        nw = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32) if norm else None
        gate = None
        if shexp_gate:
            g16 = (0.05 * rng.standard_normal(D)).astype(np.float16)
            if router_f16:
                gate = np.array([O.fp16_to_fp32(int(h)) for h in g16.view(np.uint16)], np.float32)
                tensors.append((f"blk.{l}.ffn_gate_inp_shexp.weight", om.TYPE_F16, [D], g16))
            else:
                gate = g16.astype(np.float32)
                tensors.append((f"blk.{l}.ffn_gate_inp_shexp.weight", om.TYPE_F32, [D], gate))
        tensors += [
            (f"blk.{l}.attn_norm.weight", om.TYPE_F32, [D], np.ones(D, np.float32)),
            (f"blk.{l}.ffn_gate_exps.weight", om.TYPE_Q4_K, [D, H, E], syn.gate[:E * per_q4]),
            (f"blk.{l}.ffn_up_exps.weight", om.TYPE_Q4_K, [D, H, E], syn.up[:E * per_q4]),
            (f"blk.{l}.ffn_down_exps.weight", om.TYPE_Q6_K, [H, D, E], syn.down[:E * per_q6]),
            (f"blk.{l}.ffn_gate_shexp.weight", om.TYPE_Q4_K, [D, H], syn.gate[E * per_q4:]),
            (f"blk.{l}.ffn_up_shexp.weight", om.TYPE_Q4_K, [D, H], syn.up[E * per_q4:]),
            (f"blk.{l}.ffn_down_shexp.weight", om.TYPE_Q6_K, [H, D], syn.down[E * per_q6:]),
            (f"blk.{l}.ffn_gate_inp.weight", rtype, [D, E], rbytes),
        ]
        if norm:
            tensors.append((f"blk.{l}.post_attention_norm.weight", om.TYPE_F32, [D], nw))
        info[l] = (syn, rfile, nw, gate)
    W.write_gguf(path, md, tensors)
    return info


def forward(ctx, st, layer, x, k, flags=0, resid=None):
    T = x.shape[0]
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    ib, wb = ctx.alloc(T * k * 4), ctx.alloc(T * k * 4)
    rb = ctx.upload(resid) if resid is not None else None
    st.forward(layer, xb, T, ob, resid=rb, idx=ib, w=wb, flags=flags)
    res = (ctx.download(ob, np.float32, x.shape), ctx.download(ib, np.uint32, (T, k)),
           ctx.download(wb, np.float32, (T, k)), st.last_logits(T))
    for b in (xb, ob, ib, wb, rb):
        if b is not None:
            b.free()
    return res


@pytest.fixture
def path():
    fd, p = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    yield p
    os.unlink(p)


@pytest.mark.parametrize("shape,router_f16", [((256, 256, 16), False), ((512, 256, 72), False),
                                              ((256, 256, 16), True)],
                         ids=["small", "3-chunks", "f16-router"])
def test_load_gguf_equals_set_experts(om, ctx, path, shape, router_f16):
    D, H, E = shape
    k = 8
    info = model_file(om, path, D, H, E, layers=[2, 3], router_f16=router_f16, shexp_gate=True)
    say(f"model file {os.path.getsize(path) / 1e6:.1f} MB, shape {shape}, f16 router {router_f16}")
    loaded = om.Store(ctx, 2, D, H, E, k, True, prefill_layout=False, file_layout=True)
    direct = om.Store(ctx, 2, D, H, E, k, True, prefill_layout=False, file_layout=True)
    try:
        with om.GGUF(path) as g:
            assert g.architecture == "qwen35moe" and g.param_u32("expert_count") == E
            t = g.find_tensor("blk.3.ffn_down_exps.weight")
            assert list(t.dims) == [H, D, E, 1] and t.type == om.TYPE_Q6_K
            loaded.load_gguf(g, file_first_layer=2, store_first_layer=0, n_layers=2)
        for sl, fl in ((0, 2), (1, 3)):
            syn, rfile, nw, gv = info[fl]
            for name, m in (("gate", om.MAT_GATE), ("up", om.MAT_UP), ("down", om.MAT_DOWN)):
                assert np.array_equal(loaded.get_experts(sl, m, 0, E + 1), getattr(syn, name)), name
                direct.set_experts(sl, m, 0, getattr(syn, name), E + 1)
            direct.set_router(sl, rfile)
            direct.set_norm(sl, nw)
            direct.set_shexp_gate(sl, gv)
        say("  expert bytes in the store == the file's")
        for sl, fl in ((0, 2), (1, 3)):
            syn, rfile, nw, gv = info[fl]
            # the exact chain routers, so that the logits compare bit for bit
            ex = om.MOE_EXACT_LOGITS
            for T, flags in ((1, ex), (16, om.MOE_NORM | ex), (40, ex),
                             (16, om.MOE_NORM | om.MOE_SHEXP_GATE | ex)):
                x = np.random.default_rng(100 * sl + T).standard_normal((T, D)).astype(np.float32)
                a = forward(ctx, loaded, sl, x, k, flags)
                b = forward(ctx, direct, sl, x, k, flags)
                for u, v in zip(a, b):
                    assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), (sl, T)
                xin = O.rmsnorm(x, nw) if flags & om.MOE_NORM else x
                ref, ridx, _ = O.moe_layer(D=D, H=H, E=E, k=k, x=xin,
                                           router_W=np.ascontiguousarray(rfile.T),
                                           gate=syn.routed("gate"), up=syn.routed("up"),
                                           down=syn.routed("down"), sh_gate=syn.shared("gate"),
                                           sh_up=syn.shared("up"), sh_down=syn.shared("down"),
                                           layout=O.LAYOUT_FILE,
                                           shexp_gate=gv if flags & om.MOE_SHEXP_GATE else None)
                assert np.array_equal(a[1], ridx), (sl, T)
                err = (np.abs(a[0].astype(np.float64) - ref).max(axis=1) /
                       np.abs(ref).max(axis=1)).max()
                assert err <= TOL, (sl, T, err)
                assert np.array_equal(a[3].view(np.uint32),
                                      O.router_logits_rows(xin, np.ascontiguousarray(rfile.T))
                                      .view(np.uint32))
        say("  forwards == set_experts store bit for bit; oracle indices exact, logits bit-exact")
    finally:
        loaded.close()
        direct.close()


def test_load_gguf_refusals(om, ctx, path):
    D, H, E, k = 256, 256, 16, 8
    model_file(om, path, D, H, E, layers=[0], norm=False)
    with om.GGUF(path) as g:
        vm = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=False)
        try:
            with pytest.raises(RuntimeError, match="file_layout"):
                vm.load_gguf(g)
        finally:
            vm.close()
        st = om.Store(ctx, 1, D, H, E, k, True, prefill_layout=False, file_layout=True)
        try:
            with pytest.raises(RuntimeError, match="not in the file"):
                st.load_gguf(g, file_first_layer=1)
            with pytest.raises(RuntimeError, match="past the end"):
                st.load_gguf(g, n_layers=2)
            st.load_gguf(g)  # no post_attention_norm: the norm stays all ones
        finally:
            st.close()
        other = om.Store(ctx, 1, D, H, 32, k, True, prefill_layout=False, file_layout=True)
        try:
            with pytest.raises(RuntimeError, match="ne"):
                other.load_gguf(g)
        finally:
            other.close()
    # a down projection stored as Q4_K is refused with its type
    syn = om.SyntheticLayer(3, 0, D, H, E, True)
    per = D * H // 256 * om.Q4K_BYTES
    W.write_gguf(path, [], [("blk.0.ffn_gate_exps.weight", om.TYPE_Q4_K, [D, H, E], syn.gate[:E * per]),
                            ("blk.0.ffn_up_exps.weight", om.TYPE_Q4_K, [D, H, E], syn.up[:E * per]),
                            ("blk.0.ffn_down_exps.weight", om.TYPE_Q4_K, [H, D, E], syn.gate[:E * per])])
    with om.GGUF(path) as g:
        st = om.Store(ctx, 1, D, H, E, k, False, prefill_layout=False, file_layout=True)
        try:
            with pytest.raises(RuntimeError, match="type 12"):
                st.load_gguf(g)
        finally:
            st.close()


def test_dequant_from_file_equals_goldens(om, ctx, path):
    """gpu_dequantize_tensor_gguf / gpu_dequantize_expert_slice_gguf
    (gguf_dequantize_tensor / _expert_slice, gguf.c:641-648, 714-722): the
    golden tensors the compiled reference dequantized, written into one model
    file and dequantized from it, bit for bit."""
    import ctypes as C
    gd = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    load = lambda n: np.load(os.path.join(gd, n), allow_pickle=False)  # noqa: E731
    tensors, checks = [], []
    for name, typ in (("dequant_q4k.npz", om.TYPE_Q4_K), ("dequant_q6k.npz", om.TYPE_Q6_K)):
        g = load(name)
        n = 256 * g["blocks"].shape[0]
        tensors.append((name, typ, [n], g["blocks"].reshape(-1)))
        checks.append((name, None, g["expected"]))
    for name in sorted(f for f in os.listdir(gd) if f.startswith("slice_")):
        g = load(name)
        tensors.append((name, int(g["type"]), [int(d) for d in g["dims"]], g["data"]))
        for row, e in enumerate(g["experts"]):
            checks.append((name, int(e), g["expected"][row]))
    W.write_gguf(path, [], tensors)
    L = om.lib()
    with om.GGUF(path) as gf:
        for name, e, want in checks:
            t = gf.find_tensor(name)
            out = np.zeros(want.size, np.float32)
            op = out.ctypes.data_as(C.c_void_p)
            ok = (L.gpu_dequantize_tensor_gguf(ctx.ptr, gf.ptr, C.byref(t), op) if e is None else
                  L.gpu_dequantize_expert_slice_gguf(ctx.ptr, gf.ptr, C.byref(t), e, op))
            assert ok, (name, e)
            assert np.array_equal(out.view(np.uint32), want.reshape(-1).view(np.uint32)), (name, e)
        t = gf.find_tensor("dequant_q4k.npz")
        assert not L.gpu_dequantize_expert_slice_gguf(ctx.ptr, gf.ptr, C.byref(t), -1, None)
    say(f"  {len(checks)} golden dequant/slice results reproduced from the file")
