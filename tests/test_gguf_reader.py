"""The library's GGUF reader (orn_gguf_*, csrc/host/gguf_file.c) on the CPU.

Pinned three ways:
  * the reference's own parser tests (engine/test/t_gguf.c:74-400), restated
    on the same byte-level files: minimal header, missing file, bad magic,
    architecture / alignment / several metadata entries, tensor info, list,
    data pointer, Q4_K and Q6_K sizes;
  * the COMPILED REFERENCE parser (gguf.c, oracle/_ref) on the same files:
    every accessor of both readers must agree on files with every metadata
    value type, scalar and string arrays, many tensors of every supported
    type and rank, alignments 32/64/4096; and the two must accept and reject
    the same prefixes of a file;
  * robustness the reference does not have: malformed files (n_dims > 4, an
    alignment that is not a power of two, lengths and counts past the end of
    the file) are refused with a reason, nested arrays are skipped whole, and
    a few thousand random corruptions never crash the reader (run in a child
    process, so a crash fails this test instead of the session).
"""
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np
import pytest

from oracle import gguf_writer as W
from oracle import ref as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def om():
    import ornith_moe
    ornith_moe.lib()
    return ornith_moe


@pytest.fixture
def tmpfile():
    paths = []

    def make(data: bytes):
        fd, p = tempfile.mkstemp(suffix=".gguf")
        os.write(fd, data)
        os.close(fd)
        paths.append(p)
        return p

    yield make
    for p in paths:
        if os.path.exists(p):
            os.unlink(p)


def header(n_tensors, n_meta, version=3):
    return b"GGUF" + struct.pack("<IQQ", version, n_tensors, n_meta)


def s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def tinfo(name, dims, typ, off):
    return s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", typ, off)


# ------------------------------------------------------------ t_gguf.c cases
def test_open_minimal(om, tmpfile):
    """t_gguf.c:74-88."""
    with om.GGUF(tmpfile(header(0, 0))) as g:
        assert (g.version, g.tensor_count, g.metadata_count) == (3, 0, 0)
        assert g.architecture is None and g.alignment == 32


def test_open_nonexistent(om):
    """t_gguf.c:90-95."""
    with pytest.raises(ValueError, match="cannot open"):
        om.GGUF("/tmp/nonexistent_XXXX.gguf")


def test_open_bad_magic(om, tmpfile):
    """t_gguf.c:97-110 (and the version check, gguf.c:298-300)."""
    with pytest.raises(ValueError, match="bad magic"):
        om.GGUF(tmpfile(b"BAD!"))
    with pytest.raises(ValueError, match="bad version"):
        om.GGUF(tmpfile(header(0, 0, version=4)))
    with pytest.raises(ValueError, match="too small"):
        om.GGUF(tmpfile(b"GG"))


def test_metadata_string(om, tmpfile):
    """t_gguf.c:112-138."""
    p = tmpfile(header(0, 1) + s("general.architecture") + struct.pack("<I", 8) + s("qwen2moe"))
    with om.GGUF(p) as g:
        assert g.architecture == "qwen2moe"
        assert g.value("general.architecture") == "qwen2moe"


def test_metadata_alignment(om, tmpfile):
    """t_gguf.c:140-163."""
    p = tmpfile(header(0, 1) + s("general.alignment") + struct.pack("<II", 4, 64))
    with om.GGUF(p) as g:
        assert g.alignment == 64


def test_metadata_multiple(om, tmpfile):
    """t_gguf.c:165-216: three entries, typed lookups, a missing key."""
    body = (s("general.architecture") + struct.pack("<I", 8) + s("qwen2moe") +
            s("general.alignment") + struct.pack("<II", 4, 32) +
            s("test.custom_key") + struct.pack("<II", 4, 42))
    with om.GGUF(tmpfile(header(0, 3) + body)) as g:
        assert g.metadata_count == 3
        v = g.metadata("general.architecture")
        assert v.type == 8 and g.value("general.architecture") == "qwen2moe"
        v = g.metadata("general.alignment")
        assert v.type == 4 and v.value.uint32 == 32
        assert g.value("test.custom_key") == 42
        assert g.metadata("no.such.key") is None


def test_tensor_info(om, tmpfile):
    """t_gguf.c:219-261."""
    with om.GGUF(tmpfile(header(1, 0) + tinfo("test.weight", [256, 64], 0, 0))) as g:
        assert g.tensor_count == 1
        t = g.find_tensor("test.weight")
        assert (t.n_dims, t.dims[0], t.dims[1], t.dims[2], t.dims[3]) == (2, 256, 64, 1, 1)
        assert t.type == om.TYPE_F32 and t.n_elems == 256 * 64 and t.size_bytes == 256 * 64 * 4
        assert g.find_tensor("nonexistent") is None
        assert len(g.list_tensors()) == 1


def test_tensor_list(om, tmpfile):
    """t_gguf.c:263-305 (plus: the list is sorted by name, gguf.c:378-380)."""
    body = tinfo("output.weight", [64, 32], 2, 256 * 64 * 4) + tinfo("embd.weight", [256, 64], 0, 0)
    with om.GGUF(tmpfile(header(2, 0) + body)) as g:
        lst = g.list_tensors(10)
        assert [t.name for t in lst] == [b"embd.weight", b"output.weight"]
        assert lst[1].type == 2 and lst[1].size_bytes == 64 * 32 // 32 * 18
        assert len(g.list_tensors(1)) == 1


def test_tensor_data_ptr(om, tmpfile):
    """t_gguf.c:308-333.  Deliberate difference: that file holds tensor infos
    and no data, and the reference returns an address past the end of its
    mapping (reading it faults).  This reader returns NULL for a tensor whose
    bytes are not in the file, and the address for one whose bytes are."""
    with om.GGUF(tmpfile(header(1, 0) + tinfo("test.weight", [256, 64], 0, 0))) as g:
        assert g.tensor_data("test.weight") is None
    vals = np.arange(256 * 64, dtype=np.float32)
    p = tmpfile(W.gguf_bytes([], [("test.weight", 0, [256, 64], vals)]))
    with om.GGUF(p) as g:
        assert np.array_equal(g.tensor_data("test.weight").view(np.float32), vals)
        assert np.array_equal(g.read_tensor_data(g.find_tensor("test.weight")).view(np.float32), vals)


@pytest.mark.parametrize("typ,size", [(12, 144), (14, 210)], ids=["q4k", "q6k"])
def test_kquant_tensor_size(om, tmpfile, typ, size):
    """t_gguf.c:339-400: one 256-element K-quant block."""
    with om.GGUF(tmpfile(header(1, 0) + tinfo("q.weight", [256, 1], typ, 0))) as g:
        t = g.find_tensor("q.weight")
        assert (t.type, t.n_elems, t.size_bytes) == (typ, 256, size)


def test_param_u32(om, tmpfile):
    """gguf_get_param_u32 (gguf.h:137): "<arch>.<param>" as uint32."""
    md = [("general.architecture", "str", "qwen35moe"), ("qwen35moe.block_count", "u32", 40),
          ("qwen35moe.expert_count", "i32", 256)]
    with om.GGUF(tmpfile(W.gguf_bytes(md, []))) as g:
        assert g.param_u32("block_count") == 40
        assert g.param_u32("expert_count") is None  # not a uint32
        assert g.param_u32("missing") is None


# ------------------------------------------------- against the compiled reference
def rich_file(rng, alignment=32, n_tensors=12):
    md = [("general.architecture", "str", "qwen35moe"),
          ("general.alignment", "u32", alignment),
          ("a.u8", "u8", 200), ("a.i8", "i8", -100), ("a.u16", "u16", 60000),
          ("a.i16", "i16", -30000), ("a.u32", "u32", 4000000000), ("a.i32", "i32", -2000000000),
          ("a.f32", "f32", 1.5), ("a.bool", "bool", True), ("a.bool0", "bool", False),
          ("a.u64", "u64", 2**63 + 5), ("a.i64", "i64", -2**62), ("a.f64", "f64", -2.25),
          ("a.str_empty", "str", ""),
          ("tokenizer.ggml.tokens", "arr", ("str", ["<s>", "</s>", "", "hello", "été"])),
          ("tokenizer.ggml.scores", "arr", ("f32", [0.0, -1.5, 2.25])),
          ("tokenizer.ggml.token_type", "arr", ("i32", [1, 2, 3, 4])),
          ("a.arr_empty", "arr", ("u64", [])),
          ("a.arr_u8", "arr", ("u8", list(range(7)))),
          ("a.arr_bool", "arr", ("bool", [True, False, True]))]
    types = [(0, 4), (1, 2), (12, 144 / 256), (14, 210 / 256), (2, 18 / 32), (8, 34 / 32)]
    tensors = []
    for i in range(n_tensors):
        typ, bpe = types[i % len(types)]
        rank = 1 + i % 4
        blk = 256 if typ in (12, 14) else (32 if typ in (2, 8) else 1)
        dims = [blk * int(rng.integers(1, 3))] + [int(rng.integers(1, 4)) for _ in range(rank - 1)]
        n = int(np.prod(dims))
        raw = rng.integers(0, 256, int(n * bpe), dtype=np.uint8)
        tensors.append((f"blk.{int(rng.integers(0, 40))}.t{i}.weight", typ, dims, raw))
    return md, tensors


def C_buf():
    import ctypes
    return ctypes.create_string_buffer(256)


def ref_value(L, p, key):
    import ctypes as C
    v = om_mod().GGUFValue()  # same layout as gguf_metadata_value
    if not L.gguf_find_metadata(p, key.encode(), C.byref(v)):
        return None
    return v


def om_mod():
    import ornith_moe
    return ornith_moe


def value_bytes(v):
    """Comparable content of a GGUFValue (layout of gguf_metadata_value)."""
    import ctypes as C
    if v.type == 8:
        return (8, C.string_at(v.value.string.data, v.value.string.len))
    if v.type == 9:
        a = v.value.array
        size = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
        if a.elem_type in size:
            return (9, a.elem_type, a.count, C.string_at(a.data, a.count * size[a.elem_type]))
        out, q = [], a.data
        for _ in range(a.count):
            n = C.c_uint64.from_address(q).value
            out.append(C.string_at(q + 8, n))
            q += 8 + n
        return (9, a.elem_type, a.count, tuple(out))
    return (v.type, bytes(C.string_at(C.addressof(v.value), 8)))


def info_tuple(t):
    return (t.name, t.type, t.n_dims, tuple(t.dims), t.offset, t.size_bytes, t.n_elems)


needs_ref = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built")


@needs_ref
@pytest.mark.parametrize("alignment,seed", [(32, 1), (64, 2), (4096, 3), (32, 4)])
def test_reader_agrees_with_reference_parser(om, tmpfile, alignment, seed):
    import ctypes as C
    rng = np.random.default_rng(seed)
    md, tensors = rich_file(rng, alignment, n_tensors=6 + 6 * seed)
    p = tmpfile(W.gguf_bytes(md, tensors, alignment))
    L = R.lib()
    ref = L.gguf_open(p.encode(), C_buf(), 256)
    assert ref
    try:
        with om.GGUF(p) as g:
            assert g.version == L.gguf_version(ref)
            assert g.tensor_count == L.gguf_tensor_count(ref) == len(tensors)
            assert g.metadata_count == L.gguf_metadata_count(ref) == len(md)
            assert g.architecture.encode() == L.gguf_architecture(ref)
            assert g.alignment == L.gguf_alignment(ref) == alignment
            for key, _, _ in md + [("missing.key", None, None)]:
                a, b = g.metadata(key), ref_value(L, ref, key)
                assert (a is None) == (b is None), key
                if a is not None:
                    assert value_bytes(a) == value_bytes(b), key
            assert g.value("tokenizer.ggml.tokens") == ["<s>", "</s>", "", "hello", "été"]
            assert g.value("a.u64") == 2**63 + 5 and g.value("a.f64") == -2.25
            assert g.value("a.arr_bool") == [True, False, True]
            mine = g.list_tensors()
            arr = (C.POINTER(R.TensorInfo) * len(tensors))()
            n = L.gguf_list_tensors(ref, arr, len(tensors))
            theirs = [arr[i].contents for i in range(n)]
            assert [info_tuple(t) for t in mine] == [info_tuple(t) for t in theirs]
            for (name, typ, dims, raw) in tensors:
                t = g.find_tensor(name)
                rt = L.gguf_find_tensor(ref, name.encode()).contents
                assert info_tuple(t) == info_tuple(rt)
                got = g.read_tensor_data(t)
                buf = np.empty(rt.size_bytes, np.uint8)
                assert L.gguf_read_tensor_data(ref, C.byref(rt), buf.ctypes.data, buf.size) == buf.size
                assert np.array_equal(got, buf) and np.array_equal(got, np.asarray(raw, np.uint8))
                assert np.array_equal(g.tensor_data(name), got)
                # range reads: inside, at the end, and past it (0 from both)
                sz = t.size_bytes
                for off, ln in ((0, 1), (sz // 3, sz // 3), (sz - 7, 7), (sz, 0), (sz - 3, 4),
                                (sz + 1, 0)):
                    if off < 0 or ln < 0:
                        continue
                    mb = g.read_tensor_bytes(t, off, ln)
                    rb = np.empty(max(ln, 1), np.uint8)
                    rn = L.gguf_read_tensor_bytes(ref, C.byref(rt), off, rb.ctypes.data, ln)
                    if mb is None:
                        assert rn == 0, (off, ln)
                    else:
                        assert rn == ln and np.array_equal(mb, rb[:ln]), (off, ln)
                # too small a buffer: 0 from both
                assert L.gguf_read_tensor_data(ref, C.byref(rt), buf.ctypes.data, sz - 1) == 0
                assert g.read_tensor_data(t, sz - 1) is None
            for prm in ("block_count", "missing"):
                a, b = g.param_u32(prm), C.c_uint32(0)
                assert (a is not None) == L.gguf_get_param_u32(ref, prm.encode(), C.byref(b))
    finally:
        L.gguf_close(ref)


@needs_ref
def test_truncated_prefixes_agree_with_reference(om, tmpfile):
    """Every prefix of a small file up to the end of its header: both readers
    refuse it, or both accept it with the same counts."""
    import ctypes as C
    md = [("general.architecture", "str", "qwen35moe"), ("a.u32", "u32", 7),
          ("tok", "arr", ("str", ["ab", "c"])), ("sc", "arr", ("f32", [1.0, 2.0]))]
    tensors = [("w.a", 12, [256, 2], np.zeros(288, np.uint8)), ("w.b", 0, [4], np.zeros(16, np.uint8))]
    full = W.gguf_bytes(md, tensors)
    hdr_len = len(W.gguf_bytes(md, tensors, with_data=False))
    L = R.lib()
    for n in range(hdr_len + 1):
        p = tmpfile(full[:n])
        ref = L.gguf_open(p.encode(), C_buf(), 256)
        try:
            ok = True
            try:
                g = om.GGUF(p)
            except ValueError:
                ok = False
            assert ok == bool(ref), n
            if ok:
                assert g.tensor_count == L.gguf_tensor_count(ref)
                g.close()
        finally:
            if ref:
                L.gguf_close(ref)
        os.unlink(p)


# --------------------------------------------------------------- robustness
def test_refuses_malformed(om, tmpfile):
    cases = {
        "more than 4 dimensions": header(1, 0) + tinfo("t", [1, 1, 1, 1, 1], 0, 0),
        "not a power of two": header(0, 1) + s("general.alignment") + struct.pack("<II", 4, 48),
        "entry count": header(2**40, 0),
        "string past the end": header(0, 1) + struct.pack("<Q", 2**50) + b"abc",
        "array past the end": header(0, 1) + s("k") + struct.pack("<IIQ", 9, 6, 2**40),
        "unknown metadata value type": header(0, 1) + s("k") + struct.pack("<II", 13, 0),
        "unknown array element type": header(0, 1) + s("k") + struct.pack("<IIQ", 9, 77, 1),
        "truncated": header(1, 0) + s("t") + struct.pack("<I", 2) + struct.pack("<Q", 4),
        "overflows": header(1, 0) + tinfo("t", [2**32, 2**32, 2], 0, 0),
        # element counts that fit, byte sizes that wrap to 4 and 2 bytes
        "byte size overflows": header(1, 0) + tinfo("t", [2**62 + 1], 0, 0),
        "byte size overflows ": header(1, 0) + tinfo("t", [2**63 + 1], 1, 0),
    }
    for why, data in cases.items():
        with pytest.raises(ValueError, match=why.strip()):
            om.GGUF(tmpfile(data))


def test_nested_arrays_are_skipped_whole(om, tmpfile):
    """An array of arrays with elements: the reference skips only each inner
    array's 12-byte header (gguf.c:233-234) and misreads what follows; this
    reader skips the inner elements too."""
    md = [("nest", "arr", ("arr", [("u32", [1, 2, 3]), ("str", ["x", "yz"])])),
          ("after", "u32", 99)]
    t = [("w", 0, [8], np.arange(8, dtype=np.float32))]
    with om.GGUF(tmpfile(W.gguf_bytes(md, t))) as g:
        v = g.metadata("nest")
        assert v.type == 9 and v.value.array.elem_type == 9 and v.value.array.count == 2
        assert g.value("after") == 99
        assert np.array_equal(g.read_tensor_data(g.find_tensor("w")).view(np.float32),
                              np.arange(8, dtype=np.float32))


def test_corrupted_files_never_crash(om, tmpfile):
    """Random corruptions of a valid file, opened in a child process: each
    open either fails with a reason or yields a handle whose every accessor
    and read works."""
    rng = np.random.default_rng(11)
    md, tensors = rich_file(rng, 64, n_tensors=8)
    p = tmpfile(W.gguf_bytes(md, tensors, 64))
    code = f"""
import sys, numpy as np
sys.path.insert(0, {os.path.join(ROOT, 'ornith-flight_amd')!r})
import ornith_moe as om
data = open({p!r}, 'rb').read()
hdr = {len(W.gguf_bytes(md, tensors, 64, with_data=False))}
rng = np.random.default_rng(5)
import os, tempfile
fd, q = tempfile.mkstemp(suffix='.gguf'); os.close(fd)
opened = 0
for it in range(3000):
    b = bytearray(data)
    for _ in range(int(rng.integers(1, 4))):
        pos = int(rng.integers(0, hdr))
        if rng.random() < 0.5:
            b[pos] = int(rng.integers(0, 256))
        else:
            b[pos:pos + 8] = int(rng.integers(0, 2**63)).to_bytes(8, 'little')[:len(b[pos:pos + 8])]
    if rng.random() < 0.2:
        b = b[:int(rng.integers(0, len(b)))]
    open(q, 'wb').write(b)
    try:
        g = om.GGUF(q)
    except ValueError:
        continue
    opened += 1
    g.architecture; g.alignment; g.data_offset
    for t in g.list_tensors():
        g.find_tensor(t.name.decode(errors='replace'))
        if t.size_bytes < 1 << 24:
            g.read_tensor_data(t); g.read_tensor_bytes(t, 0, min(t.size_bytes, 64))
            g.tensor_data(t.name.decode(errors='replace'))
    g.close()
os.unlink(q)
print('opened', opened)
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "opened" in r.stdout


def test_parser_under_sanitizers(tmp_path):
    """tests/gguf_fuzz.c: the reader (gguf_file.c, built with gcc
    -fsanitize=address,undefined) over 20,000 corrupted copies of a rich
    file; any out-of-bounds access, overflow or leak fails the run."""
    import shutil
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    exe = tmp_path / "gguf_fuzz"
    src = [os.path.join(ROOT, "tests", "gguf_fuzz.c"),
           os.path.join(ROOT, "ornith-flight_amd", "csrc", "host", "gguf_file.c")]
    cmd = ["gcc", "-std=c99", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I" + os.path.join(ROOT, "include"), "-o", str(exe)] + src
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    rng = np.random.default_rng(21)
    md, tensors = rich_file(rng, 64, n_tensors=10)
    seed = tmp_path / "seed.gguf"
    seed.write_bytes(W.gguf_bytes(md, tensors, 64))
    span = len(W.gguf_bytes(md, tensors, 64, with_data=False))
    r = subprocess.run([str(exe), str(seed), str(tmp_path / "x.gguf"), "20000", str(span)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    assert "opened" in r.stdout
    print(r.stdout.strip())
