"""ORACLE bindings — test infrastructure only.

ctypes access to oracle/liboracle.so (the C99 restatement in oracle.c).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 12, 14
MODE_RENORM, MODE_LITERAL = 0, 1
LAYOUT_CONTIGUOUS, LAYOUT_INTERLEAVED, LAYOUT_FILE = 0, 1, 2

_lib = None


class MoECfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "D", "H", "E", "k", "mode", "layout",
        "gate_type", "up_type", "down_type",
        "sh_gate_type", "sh_up_type", "sh_down_type")]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        L.orc_fp16_to_fp32.restype = C.c_float
        L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.orc_dequant_tensor.restype = C.c_int
        L.orc_dequant_tensor.argtypes = [C.c_void_p, C.c_int, C.c_uint64, C.c_void_p]
        L.orc_dequant_expert_slice.restype = C.c_int
        L.orc_dequant_expert_slice.argtypes = [C.c_void_p, C.c_int, C.c_uint64, C.c_uint64,
                                               C.c_int, C.c_void_p]
        L.orc_q4k_one.restype = C.c_float
        L.orc_q4k_one.argtypes = [C.c_void_p, C.c_int]
        L.orc_q6k_one.restype = C.c_float
        L.orc_q6k_one.argtypes = [C.c_void_p, C.c_int]
        L.orc_router_logits.restype = None
        L.orc_router_logits.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_void_p, f32p]
        L.orc_rmsnorm.restype = None
        L.orc_rmsnorm.argtypes = [f32p, f32p, f32p, C.c_int]
        for fn in (L.orc_topk_renorm, L.orc_topk_literal):
            fn.restype = C.c_int
            fn.argtypes = [f32p, C.c_int, C.c_int, u32p, f32p]
        L.orc_moe_layer.restype = C.c_int
        L.orc_moe_layer.argtypes = [C.POINTER(MoECfg), C.c_int, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_moe_layer_ex.restype = C.c_int
        L.orc_moe_layer_ex.argtypes = [C.POINTER(MoECfg), C.c_int] + [C.c_void_p] * 15
        L.orc_rope.restype = None
        L.orc_rope.argtypes = [f32p, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orc_attention.restype = None
        L.orc_attention.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
        L.orc_deltanet_step.restype = None
        L.orc_deltanet_step.argtypes = [f32p, f32p, f32p, f32p, f32p, C.c_int, C.c_float]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def fp16_to_fp32(h: int) -> float:
    return lib().orc_fp16_to_fp32(h)


def dequant_tensor(data: np.ndarray, typ: int, n_elems: int):
    """Returns (ok, out)."""
    out = np.zeros(n_elems, np.float32)
    d = np.ascontiguousarray(data)
    ok = lib().orc_dequant_tensor(_ptr(d), typ, n_elems, _ptr(out))
    return bool(ok), out


def expert_slice(data: np.ndarray, typ: int, n_elems: int, n_experts: int, e: int):
    per = n_elems // n_experts if n_experts else 0
    out = np.zeros(max(per, 1), np.float32)
    d = np.ascontiguousarray(data)
    ok = lib().orc_dequant_expert_slice(_ptr(d), typ, n_elems, n_experts, e, _ptr(out))
    return bool(ok), out[:per]


def router_logits(x, W, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    D, E = W.shape
    out = np.zeros(E, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_router_logits(x, W.reshape(-1), D, E, _ptr(b), out)
    return out


def router_logits_rows(x, W, bias=None):
    """orc_router_logits for every row of x [T][D] -> [T][E]."""
    x = np.ascontiguousarray(x, np.float32)
    return np.stack([router_logits(x[t], W, bias) for t in range(x.shape[0])])


def rmsnorm(x, w):
    """orc_rmsnorm (gpu.c:144-156) of every row of x [T][D]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        row = np.empty(x.shape[1], np.float32)
        lib().orc_rmsnorm(row, x[t], w, x.shape[1])
        out[t] = row
    return out


def rope(x, pos, theta):
    """orc_rope (ops.metal:113-139) of x [n_heads][head_dim]; returns a copy."""
    y = np.array(x, np.float32, order="C", copy=True)
    lib().orc_rope(y, y.shape[0], y.shape[1], pos, theta)
    return y


def attention(Q, K, V, scale=None):
    """orc_attention (attention.metal:17-68) of one head, [seq][hd] each."""
    Q, K, V = (np.ascontiguousarray(a, np.float32) for a in (Q, K, V))
    seq, hd = Q.shape
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    out = np.empty_like(Q)
    lib().orc_attention(out, Q, K, V, seq, hd, scale)
    return out


def deltanet_step(state, q, k, v, gate):
    """orc_deltanet_step (attention.metal:80-108); returns (state', out)."""
    st = np.array(state, np.float32, order="C", copy=True)
    out = np.empty(len(q), np.float32)
    lib().orc_deltanet_step(st, *(np.ascontiguousarray(a, np.float32) for a in (q, k, v)), out,
                            len(q), gate)
    return st, out


def topk(logits, k, mode=MODE_RENORM):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    fn = lib().orc_topk_renorm if mode == MODE_RENORM else lib().orc_topk_literal
    n = fn(logits, logits.size, k, idx, w)
    assert n == k
    return idx, w


def moe_layer(*, D, H, E, k, x, router_W, gate, up, down, sh_gate=None, sh_up=None,
              sh_down=None, resid=None, norm_w=None, bias=None, mode=MODE_RENORM,
              layout=LAYOUT_CONTIGUOUS, types=(TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K),
              sh_types=(TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K), shexp_gate=None):
    """Runs orc_moe_layer (orc_moe_layer_ex with a shared-expert gate);
    returns (out[T,D], idx[T,k], w[T,k])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, D)
    T = x.shape[0]
    cfg = MoECfg(D, H, E, k, mode, layout, *types, *sh_types)
    out = np.zeros((T, D), np.float32)
    idx = np.zeros((T, k), np.uint32)
    w = np.zeros((T, k), np.float32)
    keep = [np.ascontiguousarray(a) if a is not None else None for a in
            (resid, norm_w, router_W, bias, gate, up, down, sh_gate, sh_up, sh_down)]
    if shexp_gate is None:
        rc = lib().orc_moe_layer(C.byref(cfg), T, _ptr(x), *[_ptr(a) for a in keep],
                                 _ptr(out), _ptr(idx), _ptr(w))
    else:
        g = np.ascontiguousarray(shexp_gate, np.float32)
        rc = lib().orc_moe_layer_ex(C.byref(cfg), T, _ptr(x), *[_ptr(a) for a in keep], _ptr(g),
                                    _ptr(out), _ptr(idx), _ptr(w))
    if rc != 0:
        raise RuntimeError(f"orc_moe_layer failed rc={rc}")
    return out, idx, w
