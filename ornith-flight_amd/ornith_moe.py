"""ctypes binding of libornith_hip.so (the C ABI in include/ornith/*.h).

Host-side mirror used by tests/, bench.py and __graft_entry__.py.  The
library is the product; this module only marshals numpy arrays to it.  If
the shared library has not been built, importing succeeds but every call
raises: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libornith_hip.so")

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 12, 14
MAT_GATE, MAT_UP, MAT_DOWN = 0, 1, 2
ROUTE_RENORM, ROUTE_LITERAL = 0, 1
MOE_ASYNC, MOE_NORM = 1, 2
MOE_PATH_VALU, MOE_PATH_MFMA, MOE_GRAPH, MOE_SHEXP_GATE = 4, 8, 16, 32
MOE_EXACT_LOGITS = 64
SYN_GATE, SYN_UP, SYN_DOWN, SYN_ROUTER, SYN_ACT, SYN_ZIPF = 1, 2, 3, 4, 5, 6
GPU_BUF_DEFAULT, GPU_BUF_SHARED, GPU_BUF_CONSTANT = 0, 1, 2
Q4K_BYTES, Q6K_BYTES = 144, 210

# Every symbol the public headers declare (include/ornith/gpu.h, ornith_hip.h).
EXPORTED = [
    "gpu_init", "gpu_destroy", "gpu_alloc", "gpu_free", "gpu_get_cpu_ptr", "gpu_buffer_size",
    "gpu_copy_to_device", "gpu_copy_to_host", "gpu_copy_buffer", "gpu_matmul", "gpu_matmul_int4",
    "gpu_rmsnorm", "gpu_silu", "gpu_silu_mul", "gpu_rope", "gpu_attention", "gpu_deltanet_step",
    "gpu_expert_mlp", "gpu_router", "gpu_topk_softmax", "gpu_add", "gpu_sync", "gpu_memory_used",
    "gpu_print_info",
    "gpu_last_error", "gpu_device_ptr", "gpu_device_info",
    "gpu_dequantize_tensor_from_buf", "gpu_dequantize_expert_slice_from_buf",
    "gpu_dequantize_tensor_buf", "gpu_dequantize_expert_slice_buf",
    "gpu_moe_store_create", "gpu_moe_store_destroy", "gpu_moe_store_bytes",
    "gpu_moe_store_set_experts", "gpu_moe_store_get_experts", "gpu_moe_store_set_router",
    "gpu_moe_store_set_norm", "gpu_moe_store_set_shexp_gate",
    "gpu_moe_store_fill_synthetic", "gpu_moe_forward", "gpu_moe_forward_noalloc",
    "gpu_moe_forward_stack",
    "gpu_moe_last_stats", "gpu_moe_last_chained", "gpu_moe_last_logits",
    "gpu_probe_read_bandwidth",
    "gpu_profile_enable", "gpu_profile_reset", "gpu_profile_count", "gpu_profile_name",
    "gpu_profile_total_ms", "gpu_profile_calls",
    "orn_synth_stream", "orn_synth_q4k", "orn_synth_q6k", "orn_synth_normal",
    "orn_synth_zipf_bias",
    "orn_gguf_open", "orn_gguf_close", "orn_gguf_version", "orn_gguf_tensor_count",
    "orn_gguf_metadata_count", "orn_gguf_architecture", "orn_gguf_alignment",
    "orn_gguf_data_offset", "orn_gguf_find_metadata", "orn_gguf_find_tensor",
    "orn_gguf_list_tensors", "orn_gguf_tensor_data", "orn_gguf_tensor_data_from_info",
    "orn_gguf_read_tensor_data", "orn_gguf_read_tensor_bytes", "orn_gguf_get_param_u32",
    "gpu_dequantize_tensor_gguf", "gpu_dequantize_expert_slice_gguf", "gpu_moe_store_load_gguf",
    "gpu_deltanet_step_gated", "gpu_kv_cache_append",
    "gpu_moe_store_prefetch", "gpu_moe_store_pin", "gpu_moe_store_cache_stats",
]


class TensorInfo(C.Structure):
    """orn_tensor_info (layout of the reference's gguf_tensor_info, gguf.h:15-23)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_size_t), ("size_bytes", C.c_size_t),
                ("n_elems", C.c_size_t)]


class _Str(C.Structure):
    _fields_ = [("data", C.c_void_p), ("len", C.c_size_t)]


class _Arr(C.Structure):
    _fields_ = [("elem_type", C.c_int), ("count", C.c_size_t), ("data", C.c_void_p)]


class _Val(C.Union):
    _fields_ = [("uint8", C.c_uint8), ("int8", C.c_int8), ("uint16", C.c_uint16),
                ("int16", C.c_int16), ("uint32", C.c_uint32), ("int32", C.c_int32),
                ("uint64", C.c_uint64), ("int64", C.c_int64), ("float32", C.c_float),
                ("float64", C.c_double), ("boolean", C.c_bool), ("string", _Str), ("array", _Arr)]


class GGUFValue(C.Structure):
    """orn_gguf_value (layout of the reference's gguf_metadata_value, gguf.h:44-66)."""
    _fields_ = [("type", C.c_int), ("value", _Val)]


class MoEShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "d_model", "hidden", "n_experts", "top_k",
                                       "has_shared", "prefill_layout", "file_layout",
                                       "cache_slots")]


class CacheStats(C.Structure):
    """ornith_moe_cache_stats (the reference's cache_stats, memory.h:40-55)."""
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("evictions", C.c_uint64),
                ("prefetches", C.c_uint64), ("prefetch_hits", C.c_uint64),
                ("bytes_uploaded", C.c_uint64), ("slots", C.c_int), ("resident", C.c_int),
                ("pinned", C.c_int), ("device_bytes", C.c_size_t), ("host_bytes", C.c_size_t)]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class MoEOpts(C.Structure):
    _fields_ = [("route_mode", C.c_int), ("flags", C.c_uint), ("ep_first", C.c_int),
                ("ep_count", C.c_int)]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-j8"], check=True)


def lib():
    """Load the built library; raise if it is missing (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    vp, sz, i, u64, f = C.c_void_p, C.c_size_t, C.c_int, C.c_uint64, C.c_float
    sig = {
        "gpu_init": (vp, []), "gpu_destroy": (None, [vp]),
        "gpu_alloc": (vp, [vp, sz, i]), "gpu_free": (None, [vp, vp]),
        "gpu_get_cpu_ptr": (vp, [vp, vp]), "gpu_buffer_size": (sz, [vp, vp]),
        "gpu_copy_to_device": (None, [vp, vp, vp, sz]), "gpu_copy_to_host": (None, [vp, vp, vp, sz]),
        "gpu_copy_buffer": (None, [vp, vp, vp, sz]),
        "gpu_matmul": (None, [vp, vp, vp, vp, i, i, i, i, i]),
        "gpu_matmul_int4": (None, [vp, vp, vp, vp, i, i, i]),
        "gpu_rmsnorm": (None, [vp, vp, vp, vp, i, i]), "gpu_silu": (None, [vp, vp, vp, i]),
        "gpu_silu_mul": (None, [vp, vp, vp, vp, i]),
        "gpu_rope": (None, [vp, vp, vp, i, i, i, i, f, i]),
        "gpu_attention": (None, [vp, vp, vp, vp, vp, i, i]),
        "gpu_deltanet_step": (None, [vp, vp, vp, vp, vp, i]),
        "gpu_expert_mlp": (None, [vp, vp, vp, vp, vp, vp, i, i, i]),
        "gpu_router": (None, [vp, vp, vp, vp, i, i]),
        "gpu_topk_softmax": (None, [vp, vp, vp, vp, i, i]),
        "gpu_add": (None, [vp, vp, vp, vp, i]), "gpu_sync": (None, [vp]),
        "gpu_memory_used": (sz, [vp]), "gpu_print_info": (None, [vp]),
        "gpu_last_error": (C.c_char_p, [vp]), "gpu_device_ptr": (vp, [vp, vp]),
        "gpu_device_info": (i, [vp, C.c_char_p, sz, C.POINTER(C.c_int), C.POINTER(C.c_size_t)]),
        "gpu_dequantize_tensor_from_buf": (C.c_bool, [vp, vp, C.POINTER(TensorInfo), vp]),
        "gpu_dequantize_expert_slice_from_buf": (C.c_bool, [vp, vp, C.POINTER(TensorInfo), i, vp]),
        "gpu_dequantize_tensor_buf": (C.c_bool, [vp, vp, C.POINTER(TensorInfo), vp]),
        "gpu_dequantize_expert_slice_buf": (C.c_bool, [vp, vp, C.POINTER(TensorInfo), i, vp]),
        "gpu_moe_store_create": (vp, [vp, C.POINTER(MoEShape)]),
        "gpu_moe_store_destroy": (None, [vp, vp]), "gpu_moe_store_bytes": (sz, [vp]),
        "gpu_moe_store_set_experts": (i, [vp, vp, i, i, i, i, vp]),
        "gpu_moe_store_get_experts": (i, [vp, vp, i, i, i, i, vp]),
        "gpu_moe_store_set_router": (i, [vp, vp, i, vp, vp]),
        "gpu_moe_store_set_norm": (i, [vp, vp, i, vp]),
        "gpu_moe_store_set_shexp_gate": (i, [vp, vp, i, vp]),
        "gpu_moe_store_fill_synthetic": (i, [vp, vp, i, u64, f]),
        "gpu_moe_forward": (i, [vp, vp, i, vp, i, vp, vp, vp, vp, C.POINTER(MoEOpts)]),
        "gpu_moe_forward_noalloc": (i, [vp, vp, i, vp, i, vp, vp, vp, vp, C.POINTER(MoEOpts)]),
        "gpu_moe_forward_stack": (i, [vp, vp, i, i, vp, vp, i, C.POINTER(MoEOpts)]),
        "gpu_moe_last_stats": (i, [vp, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "gpu_moe_last_chained": (i, [vp, C.POINTER(C.c_int)]),
        "gpu_moe_last_logits": (i, [vp, vp, sz, C.POINTER(C.c_size_t)]),
        "gpu_probe_read_bandwidth": (i, [vp, sz, i, C.POINTER(C.c_double)]),
        "gpu_profile_enable": (i, [vp, i]), "gpu_profile_reset": (None, [vp]),
        "gpu_profile_count": (i, [vp]), "gpu_profile_name": (C.c_char_p, [vp, i]),
        "gpu_profile_total_ms": (C.c_double, [vp, i]), "gpu_profile_calls": (C.c_long, [vp, i]),
        "orn_synth_stream": (u64, [i, i, i]),
        "orn_synth_q4k": (None, [u64, u64, u64, u64, vp]),
        "orn_synth_q6k": (None, [u64, u64, u64, u64, vp]),
        "orn_synth_normal": (None, [u64, u64, u64, f, vp]),
        "orn_synth_zipf_bias": (None, [u64, u64, i, f, vp]),
        "orn_gguf_open": (vp, [C.c_char_p, C.c_char_p, sz]), "orn_gguf_close": (None, [vp]),
        "orn_gguf_version": (C.c_uint32, [vp]), "orn_gguf_tensor_count": (u64, [vp]),
        "orn_gguf_metadata_count": (u64, [vp]), "orn_gguf_architecture": (C.c_char_p, [vp]),
        "orn_gguf_alignment": (sz, [vp]), "orn_gguf_data_offset": (sz, [vp]),
        "orn_gguf_find_metadata": (C.c_bool, [vp, C.c_char_p, C.POINTER(GGUFValue)]),
        "orn_gguf_find_tensor": (C.POINTER(TensorInfo), [vp, C.c_char_p]),
        "orn_gguf_list_tensors": (u64, [vp, C.POINTER(C.POINTER(TensorInfo)), u64]),
        "orn_gguf_tensor_data": (vp, [vp, C.c_char_p]),
        "orn_gguf_tensor_data_from_info": (vp, [vp, C.POINTER(TensorInfo)]),
        "orn_gguf_read_tensor_data": (sz, [vp, C.POINTER(TensorInfo), vp, sz]),
        "orn_gguf_read_tensor_bytes": (sz, [vp, C.POINTER(TensorInfo), sz, vp, sz]),
        "orn_gguf_get_param_u32": (C.c_bool, [vp, C.c_char_p, C.POINTER(C.c_uint32)]),
        "gpu_dequantize_tensor_gguf": (C.c_bool, [vp, vp, C.POINTER(TensorInfo), vp]),
        "gpu_dequantize_expert_slice_gguf": (C.c_bool, [vp, vp, C.POINTER(TensorInfo), i, vp]),
        "gpu_moe_store_load_gguf": (i, [vp, vp, vp, i, i, i]),
        "gpu_deltanet_step_gated": (i, [vp, vp, vp, vp, vp, vp, i, f]),
        "gpu_kv_cache_append": (i, [vp, vp, vp, vp, vp, i, i]),
        "gpu_moe_store_prefetch": (i, [vp, vp, i, vp, i]),
        "gpu_moe_store_pin": (i, [vp, vp, i, vp, i, i]),
        "gpu_moe_store_cache_stats": (i, [vp, vp, C.POINTER(CacheStats), i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- synthetic data
def synth_stream(layer: int, kind: int, expert: int) -> int:
    return lib().orn_synth_stream(layer, kind, expert)


def synth_q4k(seed: int, stream: int, n_blocks: int, first: int = 0) -> np.ndarray:
    out = np.empty(n_blocks * Q4K_BYTES, np.uint8)
    lib().orn_synth_q4k(seed, stream, first, n_blocks, _p(out))
    return out


def synth_q6k(seed: int, stream: int, n_blocks: int, first: int = 0) -> np.ndarray:
    out = np.empty(n_blocks * Q6K_BYTES, np.uint8)
    lib().orn_synth_q6k(seed, stream, first, n_blocks, _p(out))
    return out


def synth_normal(seed: int, stream: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orn_synth_normal(seed, stream, n, sigma, _p(out))
    return out


def synth_zipf_bias(seed: int, stream: int, n_experts: int, s: float) -> np.ndarray:
    out = np.empty(n_experts, np.float32)
    lib().orn_synth_zipf_bias(seed, stream, n_experts, s, _p(out))
    return out


class SyntheticLayer:
    """Host copy of one synthetic layer (the bytes gpu_moe_store_fill_synthetic
    uploads), for feeding the oracle."""

    def __init__(self, seed, layer, D, H, E, has_shared=True, zipf_s=0.0):
        nb = D * H // 256
        E1 = E + (1 if has_shared else 0)
        self.gate = np.concatenate([synth_q4k(seed, synth_stream(layer, SYN_GATE, e), nb) for e in range(E1)])
        self.up = np.concatenate([synth_q4k(seed, synth_stream(layer, SYN_UP, e), nb) for e in range(E1)])
        self.down = np.concatenate([synth_q6k(seed, synth_stream(layer, SYN_DOWN, e), nb) for e in range(E1)])
        self.router = synth_normal(seed, synth_stream(layer, SYN_ROUTER, 0), D * E, 0.02).reshape(D, E)
        self.bias = synth_zipf_bias(seed, synth_stream(layer, SYN_ZIPF, 0), E, zipf_s) if zipf_s > 0 else None
        self.nb, self.E, self.has_shared = nb, E, has_shared

    def routed(self, which):
        a = getattr(self, which)
        per = self.nb * (Q6K_BYTES if which == "down" else Q4K_BYTES)
        return a[: self.E * per]

    def shared(self, which):
        a = getattr(self, which)
        per = self.nb * (Q6K_BYTES if which == "down" else Q4K_BYTES)
        return a[self.E * per:(self.E + 1) * per] if self.has_shared else None


# ---------------------------------------------------------------- device side
class Buffer:
    def __init__(self, ctx, ptr, size):
        self.ctx, self.ptr, self.size = ctx, ptr, size

    def free(self):
        if self.ptr:
            lib().gpu_free(self.ctx.ptr, self.ptr)
            self.ptr = None


class Context:
    def __init__(self):
        L = lib()
        self.ptr = L.gpu_init()
        if not self.ptr:
            raise RuntimeError("gpu_init failed (no HIP device)")
        self._bufs = []

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc}): {self.last_error()}")

    def last_error(self) -> str:
        return lib().gpu_last_error(self.ptr).decode()

    def alloc(self, nbytes, shared=False) -> Buffer:
        p = lib().gpu_alloc(self.ptr, nbytes, GPU_BUF_SHARED if shared else GPU_BUF_DEFAULT)
        if not p:
            raise MemoryError(f"gpu_alloc({nbytes}) failed")
        b = Buffer(self, p, nbytes)
        self._bufs.append(b)
        return b

    def upload(self, arr: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(arr)
        b = self.alloc(max(a.nbytes, 1))
        lib().gpu_copy_to_device(self.ptr, b.ptr, _p(a), a.nbytes)
        return b

    def download(self, buf: Buffer, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        lib().gpu_copy_to_host(self.ptr, _p(out), buf.ptr, out.nbytes)
        return out

    def sync(self):
        lib().gpu_sync(self.ptr)

    def device_info(self):
        name = C.create_string_buffer(256)
        cus = C.c_int(0)
        hbm = C.c_size_t(0)
        self.check(lib().gpu_device_info(self.ptr, name, 256, C.byref(cus), C.byref(hbm)), "device_info")
        return name.value.decode(), cus.value, hbm.value

    def read_bandwidth(self, nbytes, iters=5):
        """Measured streaming-read GB/s of the device (gpu_probe_read_bandwidth)."""
        gbs = C.c_double(0.0)
        self.check(lib().gpu_probe_read_bandwidth(self.ptr, nbytes, iters, C.byref(gbs)),
                   "probe_read_bandwidth")
        return gbs.value

    def close(self):
        if self.ptr:
            for b in self._bufs:
                b.free()
            lib().gpu_destroy(self.ptr)
            self.ptr = None


class Store:
    def __init__(self, ctx: Context, n_layers, D, H, E, k, has_shared=True, prefill_layout=True,
                 file_layout=False, cache_slots=0):
        """prefill_layout: True (or 1) keeps the MFMA layouts beside the GGUF
        blocks, 2 keeps the MFMA layouts only.  file_layout: experts and
        router in GGUF file orientation (input index fastest); needs
        prefill_layout=False.  cache_slots > 0: experts in a host tier,
        streamed through that many device slots."""
        self.ctx = ctx
        pl = 2 if prefill_layout == 2 else (1 if prefill_layout else 0)
        self.shape = MoEShape(n_layers, D, H, E, k, 1 if has_shared else 0, pl,
                              1 if file_layout else 0, cache_slots)
        self.ptr = lib().gpu_moe_store_create(ctx.ptr, C.byref(self.shape))
        if not self.ptr:
            raise RuntimeError("gpu_moe_store_create failed: " + ctx.last_error())
        self.D, self.H, self.E, self.k = D, H, E, k

    def set_experts(self, layer, matrix, first, blocks: np.ndarray, n):
        b = np.ascontiguousarray(blocks, np.uint8)
        self.ctx.check(lib().gpu_moe_store_set_experts(self.ctx.ptr, self.ptr, layer, matrix, first, n, _p(b)),
                       "set_experts")

    def get_experts(self, layer, matrix, first, n):
        """The block streams of n experts (inverse of set_experts)."""
        nb = self.D * self.H // 256
        out = np.empty(n * nb * (Q6K_BYTES if matrix == MAT_DOWN else Q4K_BYTES), np.uint8)
        self.ctx.check(lib().gpu_moe_store_get_experts(self.ctx.ptr, self.ptr, layer, matrix, first,
                                                       n, _p(out)), "get_experts")
        return out

    def set_router(self, layer, W, bias=None):
        W = np.ascontiguousarray(W, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.ctx.check(lib().gpu_moe_store_set_router(self.ctx.ptr, self.ptr, layer, _p(W),
                                                      None if b is None else _p(b)), "set_router")

    def set_norm(self, layer, w):
        w = np.ascontiguousarray(w, np.float32)
        self.ctx.check(lib().gpu_moe_store_set_norm(self.ctx.ptr, self.ptr, layer, _p(w)), "set_norm")

    def set_shexp_gate(self, layer, w):
        """The layer's shared-expert gate [D] (None removes it); applied with
        MOE_SHEXP_GATE."""
        wp = None if w is None else _p(np.ascontiguousarray(w, np.float32))
        self.ctx.check(lib().gpu_moe_store_set_shexp_gate(self.ctx.ptr, self.ptr, layer, wp),
                       "set_shexp_gate")

    def fill_synthetic(self, layer, seed, zipf_s=0.0):
        self.ctx.check(lib().gpu_moe_store_fill_synthetic(self.ctx.ptr, self.ptr, layer, seed, zipf_s),
                       "fill_synthetic")

    def load_layer(self, layer, syn: SyntheticLayer):
        """Upload a host SyntheticLayer (same bytes as fill_synthetic)."""
        E1 = self.E + (1 if self.shape.has_shared else 0)
        self.set_experts(layer, MAT_GATE, 0, syn.gate, E1)
        self.set_experts(layer, MAT_UP, 0, syn.up, E1)
        self.set_experts(layer, MAT_DOWN, 0, syn.down, E1)
        self.set_router(layer, syn.router, syn.bias)

    def forward(self, layer, x: Buffer, T, out: Buffer, resid=None, idx=None, w=None,
                mode=ROUTE_RENORM, flags=0, ep=(0, 0), noalloc=False):
        """ep = (first, count): compute only that expert-parallel share (0, 0: all).
        noalloc: call gpu_moe_forward_noalloc (work buffers in the device's
        fixed scratch) instead of gpu_moe_forward."""
        o = MoEOpts(mode, flags, ep[0], ep[1])
        fn = lib().gpu_moe_forward_noalloc if noalloc else lib().gpu_moe_forward
        rc = fn(self.ctx.ptr, self.ptr, layer, x.ptr, T, resid.ptr if resid else None, out.ptr,
                idx.ptr if idx else None, w.ptr if w else None, C.byref(o))
        self.ctx.check(rc, "gpu_moe_forward_noalloc" if noalloc else "gpu_moe_forward")

    def forward_stack(self, first, n, x: Buffer, tmp: Buffer, T, mode=ROUTE_RENORM, flags=0):
        o = MoEOpts(mode, flags, 0, 0)
        self.ctx.check(lib().gpu_moe_forward_stack(self.ctx.ptr, self.ptr, first, n, x.ptr, tmp.ptr, T,
                                                   C.byref(o)), "gpu_moe_forward_stack")

    def last_stats(self):
        a, b, c = C.c_int(), C.c_int(), C.c_int()
        self.ctx.check(lib().gpu_moe_last_stats(self.ctx.ptr, C.byref(a), C.byref(b), C.byref(c)), "stats")
        return {"n_slots": a.value, "n_rows": b.value, "n_literal": c.value}

    def last_chained(self):
        """Tokens of the last forward whose certified routing ran exact chains
        (gpu_moe_last_chained)."""
        n = C.c_int()
        self.ctx.check(lib().gpu_moe_last_chained(self.ctx.ptr, C.byref(n)), "chained")
        return n.value

    def last_logits(self, T):
        """Router logits [T][E] of the context's last forward (gpu_moe_last_logits)."""
        out = np.empty((T, self.E), np.float32)
        n = C.c_size_t(0)
        self.ctx.check(lib().gpu_moe_last_logits(self.ctx.ptr, _p(out), out.size, C.byref(n)),
                       "last_logits")
        assert n.value == out.size, (n.value, out.size)
        return out

    def load_gguf(self, gguf: "GGUF", file_first_layer=0, store_first_layer=0, n_layers=1):
        """Upload MoE layers of a model file (gpu_moe_store_load_gguf)."""
        self.ctx.check(lib().gpu_moe_store_load_gguf(self.ctx.ptr, self.ptr, gguf.ptr,
                                                     file_first_layer, store_first_layer, n_layers),
                       "load_gguf")

    def bytes(self):
        return lib().gpu_moe_store_bytes(self.ptr)

    def prefetch(self, layer, experts):
        e = np.ascontiguousarray(experts, np.int32)
        self.ctx.check(lib().gpu_moe_store_prefetch(self.ctx.ptr, self.ptr, layer, _p(e), e.size),
                       "prefetch")

    def pin(self, layer, experts, pin=True):
        e = np.ascontiguousarray(experts, np.int32)
        self.ctx.check(lib().gpu_moe_store_pin(self.ctx.ptr, self.ptr, layer, _p(e), e.size,
                                               1 if pin else 0), "pin")

    def cache_stats(self, reset=False):
        st = CacheStats()
        self.ctx.check(lib().gpu_moe_store_cache_stats(self.ctx.ptr, self.ptr, C.byref(st),
                                                       1 if reset else 0), "cache_stats")
        return st.as_dict()

    def close(self):
        if self.ptr:
            lib().gpu_moe_store_destroy(self.ctx.ptr, self.ptr)
            self.ptr = None


def profile(ctx: Context):
    L = lib()
    n = L.gpu_profile_count(ctx.ptr)
    return {L.gpu_profile_name(ctx.ptr, i).decode(): (L.gpu_profile_total_ms(ctx.ptr, i),
                                                      L.gpu_profile_calls(ctx.ptr, i)) for i in range(n)}


def tensor_info(typ, dims, size_bytes=None):
    n = int(np.prod(dims)) if len(dims) else 0
    if size_bytes is None:
        size_bytes = {TYPE_F32: 4 * n, TYPE_F16: 2 * n, TYPE_Q4_K: n // 256 * Q4K_BYTES,
                      TYPE_Q6_K: n // 256 * Q6K_BYTES}.get(typ, 0)
    arr = (C.c_uint64 * 4)(*(list(dims) + [1] * (4 - len(dims))))
    return TensorInfo(b"t", typ, len(dims), arr, 0, size_bytes, n)


# ---------------------------------------------------------------- GGUF reader
class GGUF:
    """orn_gguf_* (the reference's gguf_* API, gguf.h:67-137).  open() raises
    with the reader's reason when orn_gguf_open returns NULL."""

    def __init__(self, path):
        err = C.create_string_buffer(256)
        self.ptr = lib().orn_gguf_open(os.fsencode(path), err, 256)
        if not self.ptr:
            raise ValueError(err.value.decode())

    def close(self):
        if self.ptr:
            lib().orn_gguf_close(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    version = property(lambda s: lib().orn_gguf_version(s.ptr))
    tensor_count = property(lambda s: lib().orn_gguf_tensor_count(s.ptr))
    metadata_count = property(lambda s: lib().orn_gguf_metadata_count(s.ptr))
    alignment = property(lambda s: lib().orn_gguf_alignment(s.ptr))
    data_offset = property(lambda s: lib().orn_gguf_data_offset(s.ptr))

    @property
    def architecture(self):
        a = lib().orn_gguf_architecture(self.ptr)
        return None if a is None else a.decode(errors="replace")

    def metadata(self, key):
        """The raw GGUFValue of `key`, or None."""
        v = GGUFValue()
        return v if lib().orn_gguf_find_metadata(self.ptr, key.encode(), C.byref(v)) else None

    def value(self, key):
        """`key`'s value as Python: scalars, str, or a list for arrays of
        scalars or strings; None when absent."""
        v = self.metadata(key)
        if v is None:
            return None
        scal = {0: "uint8", 1: "int8", 2: "uint16", 3: "int16", 4: "uint32", 5: "int32",
                6: "float32", 7: "boolean", 10: "uint64", 11: "int64", 12: "float64"}
        if v.type in scal:
            return getattr(v.value, scal[v.type])
        if v.type == 8:
            return C.string_at(v.value.string.data, v.value.string.len).decode()
        a = v.value.array
        dt = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32,
              6: np.float32, 7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}
        if a.elem_type in dt:
            n = a.count * np.dtype(dt[a.elem_type]).itemsize
            return np.frombuffer(C.string_at(a.data, n), dt[a.elem_type]).tolist() if n else []
        if a.elem_type == 8:
            out, p = [], a.data
            for _ in range(a.count):
                ln = C.c_uint64.from_address(p).value
                out.append(C.string_at(p + 8, ln).decode())
                p += 8 + ln
            return out
        raise ValueError(f"array of type {a.elem_type}")

    def param_u32(self, param):
        v = C.c_uint32(0)
        return v.value if lib().orn_gguf_get_param_u32(self.ptr, param.encode(), C.byref(v)) else None

    def find_tensor(self, name):
        """The TensorInfo of `name` (owned by the handle), or None."""
        p = lib().orn_gguf_find_tensor(self.ptr, name.encode())
        return p.contents if p else None

    def list_tensors(self, max_count=None):
        n = lib().orn_gguf_list_tensors(self.ptr, None, 0)
        if max_count is not None:
            n = min(n, max_count)
        arr = (C.POINTER(TensorInfo) * max(n, 1))()
        got = lib().orn_gguf_list_tensors(self.ptr, arr, n)
        return [arr[i].contents for i in range(got)]

    def read_tensor_data(self, info, buffer_size=None):
        """Bytes of a whole tensor (None when the read fails)."""
        size = info.size_bytes if buffer_size is None else buffer_size
        buf = np.empty(max(size, 1), np.uint8)
        n = lib().orn_gguf_read_tensor_data(self.ptr, C.byref(info), _p(buf), size)
        return buf[:n] if n else None

    def read_tensor_bytes(self, info, offset, n):
        buf = np.empty(max(n, 1), np.uint8)
        got = lib().orn_gguf_read_tensor_bytes(self.ptr, C.byref(info), offset, _p(buf), n)
        return buf[:got] if got else None

    def tensor_data(self, name):
        """The tensor's bytes through the file mapping (orn_gguf_tensor_data)."""
        info = self.find_tensor(name)
        p = lib().orn_gguf_tensor_data(self.ptr, name.encode())
        return None if not p else np.frombuffer(C.string_at(p, info.size_bytes), np.uint8)
