"""GPU tests of the gpu.h backend contract and the device dequant API.

Mirrors the reference's backend tests (engine/test/t_gpu.c, t_gpu_metal.c)
and dequant tests (engine/test/t_gguf.c) against libornith_hip.so, and checks
the device dequant/slice kernels bit-exactly against the golden vectors the
compiled reference wrote (tests/golden/).
"""
import ctypes as C
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def f32p(a):
    return a.ctypes.data_as(C.c_void_p)


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


def alloc(om, ctx, n, shared=True):
    p = om.lib().gpu_alloc(ctx.ptr, n, om.GPU_BUF_SHARED if shared else om.GPU_BUF_DEFAULT)
    assert p
    return p


# ------------------------------------------------------------ t_gpu.c mirror
def test_context_and_memory_accounting(om):
    L = om.lib()
    ctx = L.gpu_init()
    assert ctx
    L.gpu_print_info(ctx)
    assert L.gpu_memory_used(ctx) == 0
    b = L.gpu_alloc(ctx, 1024, om.GPU_BUF_DEFAULT)
    assert b and L.gpu_memory_used(ctx) == 1024
    assert L.gpu_buffer_size(ctx, b) == 1024
    L.gpu_free(ctx, b)
    assert L.gpu_memory_used(ctx) == 0
    assert L.gpu_alloc(ctx, 0, 0) is None
    L.gpu_destroy(ctx)


def test_shared_cpu_ptr_and_copies(om, ctx):
    L = om.lib()
    b = alloc(om, ctx, 64)
    p = L.gpu_get_cpu_ptr(ctx.ptr, b)
    assert p
    C.memset(p, 0xAB, 64)
    raw = (C.c_ubyte * 64).from_address(p)
    assert raw[0] == 0xAB and raw[63] == 0xAB
    src = np.array([1, 2, 3, 4], np.float32)
    dev = alloc(om, ctx, 16, shared=False)
    L.gpu_copy_to_device(ctx.ptr, dev, f32p(src), 16)
    dst = np.zeros(4, np.float32)
    L.gpu_copy_to_host(ctx.ptr, f32p(dst), dev, 16)
    assert np.array_equal(dst, src)
    b2 = alloc(om, ctx, 16, shared=False)
    L.gpu_copy_buffer(ctx.ptr, b2, dev, 16)
    out = np.zeros(4, np.float32)
    L.gpu_copy_to_host(ctx.ptr, f32p(out), b2, 1000)  # clamps to the buffer size
    assert np.array_equal(out, src)
    # A host write through the SHARED pointer is seen by the next call.
    (C.c_float * 4).from_address(L.gpu_get_cpu_ptr(ctx.ptr, b))[:] = [5, 6, 7, 8]
    L.gpu_copy_buffer(ctx.ptr, b2, b, 16)
    L.gpu_copy_to_host(ctx.ptr, f32p(out), b2, 16)
    assert list(out) == [5, 6, 7, 8]
    for x in (b, dev, b2):
        L.gpu_free(ctx.ptr, x)


def test_matmul_known_answers(om, ctx):
    """t_gpu.c:127-163: C[0][0] = 74, C[1][3] = 218; t_gpu_metal.c:83-115."""
    L = om.lib()
    A = ctx.upload(np.arange(1, 7, dtype=np.float32))
    B = ctx.upload(np.arange(7, 19, dtype=np.float32))
    Cb = ctx.alloc(32)
    L.gpu_matmul(ctx.ptr, Cb.ptr, A.ptr, B.ptr, 2, 4, 3, 0, 0)
    out = ctx.download(Cb, np.float32, 8)
    assert out[0] == 74.0 and out[7] == 218.0
    v = ctx.upload(np.array([1, 2, 3], np.float32))
    m = ctx.upload(np.array([4, 5, 6, 7, 8, 9], np.float32))
    o = ctx.alloc(8)
    L.gpu_matmul(ctx.ptr, o.ptr, v.ptr, m.ptr, 1, 2, 3, 0, 0)
    assert list(ctx.download(o, np.float32, 2)) == [40.0, 46.0]
    # K=8, M=16 model-like case: bit-exact with the sequential CPU sum.
    vec = (np.arange(8) * 0.5).astype(np.float32)
    mat = (np.arange(128) * 0.01).astype(np.float32)
    exp = np.zeros(16, np.float32)
    for j in range(16):
        s = np.float32(0)
        for i in range(8):
            s = np.float32(s + np.float32(vec[i] * mat[i * 16 + j]))
        exp[j] = s
    o2 = ctx.alloc(64)
    L.gpu_matmul(ctx.ptr, o2.ptr, ctx.upload(vec).ptr, ctx.upload(mat).ptr, 1, 16, 8, 0, 0)
    assert np.array_equal(ctx.download(o2, np.float32, 16), exp)


def seq_matmul(A, B):
    """gpu.c:104-115 in numpy: every C[i][j] a sequential fp32 sum from 0 of
    the fp32 products A[i][k] * B[k][j], k ascending."""
    M, K = A.shape
    C = np.zeros((M, B.shape[1]), np.float32)
    for k in range(K):
        C = (C + (A[:, k:k + 1] * B[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    return C


@pytest.mark.parametrize("M,N,K", [(1, 4, 0), (1, 4097, 300), (1, 1000, 13), (2, 1000, 1),
                                   (3, 4096, 300), (5, 7, 257), (16, 1000, 300),
                                   (17, 4097, 13), (40, 1024, 520)])
def test_matmul_tiled_bit_exact(om, ctx, M, N, K):
    """gpu_matmul at M > 1 and odd shapes (row blocks of 1..16 rows, one or
    four columns per thread, K past one LDS chunk of 256): bit-identical to
    the CPU backend's sequential sums (gpu.c:104-115); K = 0 gives zeros."""
    rng = np.random.default_rng(M * 1000 + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    L = om.lib()
    Ab = ctx.upload(A) if K else ctx.alloc(4)
    Bb = ctx.upload(B) if K else ctx.alloc(4)
    Cb = ctx.upload(np.full((M, N), 7.0, np.float32))
    L.gpu_matmul(ctx.ptr, Cb.ptr, Ab.ptr, Bb.ptr, M, N, K, 0, 0)
    got = ctx.download(Cb, np.float32, (M, N))
    assert np.array_equal(got.view(np.uint32), seq_matmul(A, B).view(np.uint32))
    for b in (Ab, Bb, Cb):
        b.free()


@pytest.mark.parametrize("dim", [4, 64, 2048])
def test_rmsnorm(om, ctx, dim):
    """t_gpu_metal.c:189-343 (1e-5 / 1e-4) -- here bit-exact with gpu.c:144-156."""
    x = np.sin(np.arange(dim) * 0.3).astype(np.float32)
    w = (0.5 + 0.5 * np.cos(np.arange(dim) * 0.2)).astype(np.float32)
    ss = np.float32(0)
    for v in x:
        ss = np.float32(ss + np.float32(v * v))
    inv = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(dim) + np.float32(1e-6)))
    exp = (w * (x * inv)).astype(np.float32)
    o = ctx.alloc(4 * dim)
    om.lib().gpu_rmsnorm(ctx.ptr, o.ptr, ctx.upload(x).ptr, ctx.upload(w).ptr, 1, dim)
    assert np.array_equal(ctx.download(o, np.float32, dim), exp)


def test_elementwise(om, ctx):
    L = om.lib()
    g = np.linspace(-60, 60, 1001).astype(np.float32)
    u = np.linspace(2, -2, 1001).astype(np.float32)
    gb, ub, ob = ctx.upload(g), ctx.upload(u), ctx.alloc(4 * 1001)
    L.gpu_silu_mul(ctx.ptr, ob.ptr, gb.ptr, ub.ptr, 1001)
    ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert np.allclose(ctx.download(ob, np.float32, 1001), ref, rtol=2e-6, atol=1e-30)
    L.gpu_silu(ctx.ptr, ob.ptr, gb.ptr, 1001)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert np.allclose(ctx.download(ob, np.float32, 1001), ref, rtol=2e-6, atol=1e-30)
    L.gpu_add(ctx.ptr, ob.ptr, gb.ptr, ub.ptr, 1001)
    assert np.array_equal(ctx.download(ob, np.float32, 1001), g + u)
    # int4 matmul zero-fills C like the CPU backend (gpu.c:131-140).
    L.gpu_matmul_int4(ctx.ptr, ob.ptr, gb.ptr, ub.ptr, 2, 4, 3)
    assert np.all(ctx.download(ob, np.float32, 8) == 0)


def test_router_and_topk_api(om, ctx):
    from oracle import oracle as O
    L = om.lib()
    rng = np.random.default_rng(5)
    D, E, k = 2048, 256, 8
    W = (rng.standard_normal((D, E)) * 0.02).astype(np.float32)
    x = rng.standard_normal(D).astype(np.float32)
    lb = ctx.alloc(4 * E)
    L.gpu_router(ctx.ptr, lb.ptr, ctx.upload(x).ptr, ctx.upload(W).ptr, D, E)
    logits = ctx.download(lb, np.float32, E)
    assert np.array_equal(logits.view(np.uint32), O.router_logits(x, W).view(np.uint32))
    idx = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    L.gpu_topk_softmax(ctx.ptr, f32p(idx), f32p(w), lb.ptr, E, k)
    ridx, rw = O.topk(logits, k, O.MODE_RENORM)
    assert np.array_equal(idx, ridx)
    assert np.allclose(w, rw, rtol=1e-6)
    # Ties follow exchange selection: [1, 1, 9] -> 2, 1, 0.
    tb = ctx.upload(np.array([1, 1, 9], np.float32))
    idx3 = np.zeros(3, np.uint32)
    w3 = np.zeros(3, np.float32)
    L.gpu_topk_softmax(ctx.ptr, f32p(idx3), f32p(w3), tb.ptr, 3, 3)
    assert list(idx3) == [2, 1, 0]


def test_expert_mlp_api(om, ctx):
    L = om.lib()
    rng = np.random.default_rng(6)
    D, H = 64, 32
    x = rng.standard_normal(D).astype(np.float32)
    Wg, Wu = [(rng.standard_normal((D, H)) * 0.1).astype(np.float32) for _ in range(2)]
    Wd = (rng.standard_normal((H, D)) * 0.1).astype(np.float32)
    o = ctx.alloc(4 * D)
    L.gpu_expert_mlp(ctx.ptr, o.ptr, ctx.upload(x).ptr, ctx.upload(Wg).ptr, ctx.upload(Wu).ptr,
                     ctx.upload(Wd).ptr, D, H, 0)
    x64 = x.astype(np.float64)
    g, u = x64 @ Wg, x64 @ Wu
    ref = ((g / (1 + np.exp(-g))) * u) @ Wd
    assert np.allclose(ctx.download(o, np.float32, D), ref, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------ dequant API
def load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


@pytest.mark.parametrize("name,typ", [("dequant_q4k.npz", 12), ("dequant_q6k.npz", 14)])
def test_dequant_kquant_golden(om, ctx, golden_dir, name, typ):
    g = load(golden_dir, name)
    blocks = np.ascontiguousarray(g["blocks"].reshape(-1))
    n = 256 * g["blocks"].shape[0]
    info = om.tensor_info(typ, [n])
    out = np.zeros(n, np.float32)
    assert om.lib().gpu_dequantize_tensor_from_buf(ctx.ptr, f32p(blocks), C.byref(info), f32p(out))
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))
    assert np.all(out[:256] == (1.0 if typ == 12 else -31.0))


@pytest.mark.parametrize("typ,bsize,d_offs", [(12, 144, (0, 2)), (14, 210, (208,))],
                         ids=["q4k", "q6k"])
def test_dequant_random_blocks_match_oracle(om, ctx, typ, bsize, d_offs):
    """4097 random super-blocks (every scale, min and quant bit pattern;
    finite fp16 d / dmin) through the device dequant, bit for bit against the
    oracle's restatement of gguf.c:511-571 (itself pinned by the golden
    vectors above), host-pointer and device-resident calls."""
    from oracle import oracle as O
    nb = 4097
    rng = np.random.default_rng(typ)
    blocks = rng.integers(0, 256, (nb, bsize), dtype=np.uint8)
    for off in d_offs:  # finite halves: exponent field below 31
        blocks[:, off + 1] &= 0x7B
    n = 256 * nb
    ok, ref = O.dequant_tensor(blocks.reshape(-1), typ, n)
    assert ok
    info = om.tensor_info(typ, [n])
    out = np.zeros(n, np.float32)
    assert om.lib().gpu_dequantize_tensor_from_buf(ctx.ptr, f32p(blocks), C.byref(info), f32p(out))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    src, dst = ctx.upload(blocks.reshape(-1)), ctx.alloc(4 * n)
    assert om.lib().gpu_dequantize_tensor_buf(ctx.ptr, src.ptr, C.byref(info), dst.ptr)
    assert np.array_equal(ctx.download(dst, np.float32, n).view(np.uint32), ref.view(np.uint32))
    src.free()
    dst.free()


def test_dequant_f16_f32_golden(om, ctx, golden_dir):
    g = load(golden_dir, "dequant_f16_all.npz")
    info = om.tensor_info(1, [65536])
    out = np.zeros(65536, np.float32)
    h = np.ascontiguousarray(g["halves"])
    assert om.lib().gpu_dequantize_tensor_from_buf(ctx.ptr, f32p(h), C.byref(info), f32p(out))
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))
    g = load(golden_dir, "dequant_f32.npz")
    d = np.ascontiguousarray(g["data"])
    out = np.zeros(d.size, np.float32)
    assert om.lib().gpu_dequantize_tensor_from_buf(ctx.ptr, f32p(d), C.byref(om.tensor_info(0, [d.size])),
                                                   f32p(out))
    assert np.array_equal(out, g["expected"])
    bad = om.tensor_info(2, [64])
    assert not om.lib().gpu_dequantize_tensor_from_buf(ctx.ptr, f32p(d), C.byref(bad), f32p(out))


def test_slices_golden(om, ctx, golden_dir):
    names = sorted(f for f in os.listdir(golden_dir) if f.startswith("slice_"))
    for name in names:
        g = load(golden_dir, name)
        typ, dims = int(g["type"]), [int(d) for d in g["dims"]]
        info = om.tensor_info(typ, dims)
        data = np.ascontiguousarray(g["data"])
        per = int(np.prod(dims)) // dims[-1]
        for row, e in enumerate(g["experts"]):
            out = np.zeros(per, np.float32)
            ok = om.lib().gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), C.byref(info), int(e),
                                                               f32p(out))
            assert ok, (name, e)
            assert np.array_equal(out.view(np.uint32), g["expected"][row].view(np.uint32)), (name, e)


def test_slice_invalid(om, ctx):
    """t_gguf.c:699-735 -- plus E == 0 and an unsupported type."""
    L = om.lib()
    data = np.zeros(144, np.uint8)
    out = np.zeros(64, np.float32)
    info = om.tensor_info(12, [4, 16, 4])
    assert not L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, None, C.byref(info), 0, f32p(out))
    assert not L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), C.byref(info), 0, None)
    assert not L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), C.byref(info), -1, f32p(out))
    assert not L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), C.byref(info), 99, f32p(out))
    assert not L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), None, 0, f32p(out))
    z = om.tensor_info(12, [4, 16, 0])
    assert not L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), C.byref(z), 0, f32p(out))
    assert L.gpu_dequantize_expert_slice_from_buf(ctx.ptr, f32p(data), C.byref(info), 3, f32p(out))


def test_device_resident_dequant(om, ctx, golden_dir):
    g = load(golden_dir, "dequant_q4k.npz")
    blocks = np.ascontiguousarray(g["blocks"].reshape(-1))
    n = 256 * g["blocks"].shape[0]
    src = ctx.upload(blocks)
    dst = ctx.alloc(4 * n)
    info = om.tensor_info(12, [n])
    assert om.lib().gpu_dequantize_tensor_buf(ctx.ptr, src.ptr, C.byref(info), dst.ptr)
    assert np.array_equal(ctx.download(dst, np.float32, n).view(np.uint32), g["expected"].view(np.uint32))
    small = ctx.alloc(16)
    assert not om.lib().gpu_dequantize_tensor_buf(ctx.ptr, src.ptr, C.byref(info), small.ptr)


# ------------------------------------------------- measurement helper
def test_read_bandwidth_probe(om, ctx):
    """gpu_probe_read_bandwidth: a positive, physically plausible figure, and
    invalid arguments rejected without a launch."""
    gbs = ctx.read_bandwidth(64 << 20, 2)
    assert 10.0 < gbs < 100000.0
    L = om.lib()
    out = C.c_double(-1.0)
    assert L.gpu_probe_read_bandwidth(ctx.ptr, 8, 1, C.byref(out)) != 0
    assert L.gpu_probe_read_bandwidth(ctx.ptr, 1 << 20, 0, C.byref(out)) != 0
    assert out.value == -1.0


# ------------------------------------------- the reference's own contract tests
REF_BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle",
                       "_ref")


@pytest.mark.parametrize("name,n_tests", [("t_gpu_hip", 7), ("t_gpu_metal_hip", 6)])
def test_reference_contract_tests_pass(name, n_tests):
    """engine/test/t_gpu.c and t_gpu_metal.c, compiled from the reference's
    sources and linked against libornith_hip.so instead of gpu.o
    (oracle/Makefile `link`; built in the container that holds the
    reference, and shipped here as built files): every test passes on the
    GPU.  Their checks are the backend contract itself -- context and buffer
    lifecycle, gpu_memory_used, shared-buffer host pointers, copies, the
    matmul known answers 74/218 and 40/46, rmsnorm, silu, add."""
    import subprocess
    exe = os.path.join(REF_BIN, name)
    if not os.access(exe, os.X_OK):
        pytest.skip(f"{exe} not built (needs the reference tree at build time)")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    tail = r.stdout.replace("\\n", "\n")
    summary = [ln for ln in tail.splitlines() if "passed," in ln][-1]
    passed, total = summary.split("===")[1].split()[0].split("/")
    assert passed == total and " 0 failed" in summary, summary
    if n_tests is not None:
        assert int(total) == n_tests
