"""Bindings to the COMPILED REFERENCE (oracle/_ref/libornith_ref.so) — test
infrastructure only.

The library is compiled from the reference's own C sources by `make -C oracle
ref` (only in the container that holds /root/reference); the built .so is
what travels.  It is used to (a) write the golden vectors under tests/golden/,
(b) time the reference CPU path for bench.py's cpu_baseline leg and (c) check
the library's GGUF reader against the reference parser on the same files.

Reference entry points used (engine/src/...):
  gguf_dequantize_tensor_from_buf        gguf.c:605-638
  gguf_dequantize_expert_slice_from_buf  gguf.c:652-711
  model_load / model_unload              model.c:160-243
  model_get_routing                      model.c:264-321
  model_forward                          model.c:878-1234 (MoE block 992-1144)
  gguf_open .. gguf_get_param_u32        gguf.c:289-506, 575-601 (parser, lookups,
                                         pread reads; declared in gguf.h:67-137)
"""
from __future__ import annotations

import ctypes as C
import os
import tempfile

import numpy as np

from . import gguf_writer

HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB = os.path.join(HERE, "_ref", "libornith_ref.so")

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 12, 14
BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210}


class TensorInfo(C.Structure):
    """Mirror of gguf_tensor_info (gguf.h:15-23)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_size_t),
                ("size_bytes", C.c_size_t), ("n_elems", C.c_size_t)]


class ModelBuffers(C.Structure):
    """Mirror of model_buffers (model.h:66-73); all NULL -> attention is a no-op."""
    _fields_ = [("kv_caches", C.c_void_p), ("ssm_conv_states", C.c_void_p),
                ("ssm_h_states", C.c_void_p), ("k_cache", C.c_void_p),
                ("v_cache", C.c_void_p), ("max_cache_len", C.c_int)]


_lib = None


def available() -> bool:
    return os.path.exists(REF_LIB)


def lib():
    global _lib
    if _lib is None:
        L = C.CDLL(REF_LIB)
        L.gguf_dequantize_tensor_from_buf.restype = C.c_bool
        L.gguf_dequantize_tensor_from_buf.argtypes = [C.c_void_p, C.POINTER(TensorInfo), C.c_void_p]
        L.gguf_dequantize_expert_slice_from_buf.restype = C.c_bool
        L.gguf_dequantize_expert_slice_from_buf.argtypes = [C.c_void_p, C.POINTER(TensorInfo),
                                                            C.c_int, C.c_void_p]
        L.model_load.restype = C.c_void_p
        L.model_load.argtypes = [C.c_char_p, C.c_void_p, C.c_char_p, C.c_size_t, C.c_bool, C.c_bool]
        L.model_unload.restype = None
        L.model_unload.argtypes = [C.c_void_p]
        L.model_get_routing.restype = C.c_int
        L.model_get_routing.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        L.model_forward.restype = None
        L.model_forward.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.POINTER(ModelBuffers),
                                    C.c_int, C.c_int]
        vp, sz = C.c_void_p, C.c_size_t
        for name, res, args in (
                ("gguf_open", vp, [C.c_char_p, C.c_char_p, sz]), ("gguf_close", None, [vp]),
                ("gguf_version", C.c_uint32, [vp]), ("gguf_tensor_count", C.c_uint64, [vp]),
                ("gguf_metadata_count", C.c_uint64, [vp]),
                ("gguf_architecture", C.c_char_p, [vp]), ("gguf_alignment", sz, [vp]),
                ("gguf_find_metadata", C.c_bool, [vp, C.c_char_p, vp]),
                ("gguf_find_tensor", C.POINTER(TensorInfo), [vp, C.c_char_p]),
                ("gguf_list_tensors", C.c_uint64, [vp, C.POINTER(C.POINTER(TensorInfo)), C.c_uint64]),
                ("gguf_tensor_data", vp, [vp, C.c_char_p]),
                ("gguf_tensor_data_from_info", vp, [vp, C.POINTER(TensorInfo)]),
                ("gguf_read_tensor_data", sz, [vp, C.POINTER(TensorInfo), vp, sz]),
                ("gguf_read_tensor_bytes", sz, [vp, C.POINTER(TensorInfo), sz, vp, sz]),
                ("gguf_get_param_u32", C.c_bool, [vp, C.c_char_p, C.POINTER(C.c_uint32)])):
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _info(typ, dims):
    n = int(np.prod(dims))
    if typ == TYPE_F32:
        size = 4 * n
    elif typ == TYPE_F16:
        size = 2 * n
    else:
        size = n // 256 * BLOCK_BYTES[typ]
    arr = (C.c_uint64 * 4)(*(list(dims) + [1] * (4 - len(dims))))
    return TensorInfo(b"t", typ, len(dims), arr, 0, size, n)


def dequant_tensor(data: np.ndarray, typ: int, dims):
    info = _info(typ, dims)
    out = np.zeros(max(info.n_elems, 1), np.float32)
    d = np.ascontiguousarray(data)
    ok = lib().gguf_dequantize_tensor_from_buf(d.ctypes.data_as(C.c_void_p), C.byref(info),
                                               out.ctypes.data_as(C.c_void_p))
    return bool(ok), out[:info.n_elems]


def expert_slice(data: np.ndarray, typ: int, dims, e: int):
    info = _info(typ, dims)
    per = info.n_elems // dims[-1] if dims[-1] else 0
    out = np.zeros(max(per, 1), np.float32)
    d = np.ascontiguousarray(data)
    ok = lib().gguf_dequantize_expert_slice_from_buf(d.ctypes.data_as(C.c_void_p), C.byref(info), e,
                                                     out.ctypes.data_as(C.c_void_p))
    return bool(ok), out[:per]


class RefMoEModel:
    """A one-layer synthetic model in which model_forward reduces to the MoE
    block:  output = x + shared(norm(x)) + routed(norm(x)).

    * full_attention_interval = 1 makes layer 0 an attention layer; with
      k_cache == NULL attention_layer_forward returns before touching x
      (model.c:572-573).
    * token_embd.weight holds the T input vectors as columns (model.c:903-907).
    * output.weight is the identity with vocab = D and there is no output
      norm, so the logits are x itself (model.c:1213-1231).
    * routed experts are fused 3-D tensors whose last dim is E (interleaved,
      gguf.c:659-660).
    """

    def __init__(self, *, D, H, E, k, X, router_W, norm_w, gate, up, down,
                 sh_gate, sh_up, sh_down, types=(TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K),
                 sh_types=(TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K), path=None):
        X = np.ascontiguousarray(X, np.float32)
        T = X.shape[0]
        V = D
        assert T <= V
        emb = np.zeros((D, V), np.float32)
        emb[:, :T] = X.T
        md = [("general.architecture", "str", "qwen35moe")]
        for key, val in (("block_count", 1), ("embedding_length", D), ("attention.head_count", 1),
                         ("attention.head_count_kv", 1), ("attention.key_length", 2),
                         ("attention.value_length", 2), ("expert_count", E),
                         ("expert_used_count", k), ("feed_forward_length", H),
                         ("expert_feed_forward_length", H), ("full_attention_interval", 1),
                         ("vocab_size", V), ("rope.dimension_count", 2)):
            md.append(("qwen35moe." + key, "u32", val))
        dummy = np.zeros(4, np.float32)
        tens = [
            ("token_embd.weight", TYPE_F32, [V, D], emb),
            ("output.weight", TYPE_F32, [V, D], np.eye(D, V, dtype=np.float32)),
            ("blk.0.attn_norm.weight", TYPE_F32, [D], np.ones(D, np.float32)),
            ("blk.0.post_attention_norm.weight", TYPE_F32, [D], np.ascontiguousarray(norm_w, np.float32)),
            ("blk.0.attn_q.weight", TYPE_F32, [4], dummy),
            ("blk.0.attn_k.weight", TYPE_F32, [4], dummy),
            ("blk.0.attn_v.weight", TYPE_F32, [4], dummy),
            ("blk.0.attn_output.weight", TYPE_F32, [4], dummy),
            ("blk.0.ffn_gate_shexp.weight", sh_types[0], [H, D], sh_gate),
            ("blk.0.ffn_up_shexp.weight", sh_types[1], [H, D], sh_up),
            ("blk.0.ffn_down_shexp.weight", sh_types[2], [D, H], sh_down),
            ("blk.0.ffn_gate_inp.weight", TYPE_F32, [E, D], np.ascontiguousarray(router_W, np.float32)),
            ("blk.0.ffn_gate_exps.weight", types[0], [H, D, E], gate),
            ("blk.0.ffn_up_exps.weight", types[1], [H, D, E], up),
            ("blk.0.ffn_down_exps.weight", types[2], [D, H, E], down),
        ]
        self._own = path is None
        if path is None:
            fd, path = tempfile.mkstemp(prefix="ornith_ref_", suffix=".gguf")
            os.close(fd)
        self.path = path
        gguf_writer.write_gguf(path, md, tens)
        err = C.create_string_buffer(256)
        self.model = lib().model_load(path.encode(), None, err, 256, False, False)
        if not self.model:
            raise RuntimeError("model_load failed: " + err.value.decode())
        self.D, self.T, self.V, self.E, self.k = D, T, V, E, k

    def forward(self, t: int) -> np.ndarray:
        out = np.zeros(self.V, np.float32)
        bufs = ModelBuffers(None, None, None, None, None, 0)
        lib().model_forward(self.model, t, out.ctypes.data_as(C.c_void_p), C.byref(bufs), 1, 0)
        return out[:self.D].copy()

    def routing(self, x: np.ndarray, k=None):
        k = self.k if k is None else k
        x = np.ascontiguousarray(x, np.float32)
        idx = np.zeros(k, np.uint32)
        w = np.zeros(k, np.float32)
        n = lib().model_get_routing(self.model, x.ctypes.data_as(C.c_void_p), 0,
                                    idx.ctypes.data_as(C.c_void_p), w.ctypes.data_as(C.c_void_p), k)
        return idx[:n], w[:n]

    def close(self):
        if self.model:
            lib().model_unload(self.model)
            self.model = None
        if self._own and self.path and os.path.exists(self.path):
            os.unlink(self.path)
            self.path = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
