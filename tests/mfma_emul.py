"""Emulation of the matrix-core arithmetic of the vec@mat expert kernels
(test infrastructure; numpy only, no GPU).

The kernels (csrc/kernels/mfma_ops.h, expert_dec.hip, expert_mfma.hip)
compute one expert product y[r][n] = sum_k x[r][k] * W[k][n] over the
reference's dequantized weights (engine/src/gguf.c:43-86, read as vec@mat,
engine/src/model.c:351-357) as

    Q4_K:  y = ( sum_k A[r][k] * (sc*q)[k][n]  -  sum_k Am[r][k] * m[k][n] ) / s_r
    Q6_K:  y = ( sum_k A[r][k] * (sc*q)[k][n] ) / s_r

with A = x * s_r * d(k, n/256) and Am = x * s_r * dmin(k, n/256) rounded to
fp32 and then to fp16 operands, s_r a power of two per row, B = sc*q an
integer held exactly in fp16 (or, for Q6_K sub-scales above 64, as
b1 = fp16(sc*q) plus the exact remainder b2), and the sums accumulated in
fp32.  This module reproduces those operand roundings exactly (numpy fp16
conversions) and accumulates in fp64, so it differs from the kernels only by
their fp32 accumulation (~1e-7 relative).  `Variant` selects which operands
are formed and which terms are kept:

  act      "hilo"  A = hi + lo, hi = fp16 of A rounded toward zero, lo = the
                   remainder A - hi rounded toward zero (what ships);
           "rtz"   hi only, rounded toward zero;
           "rtn"   hi only, rounded to nearest;
  act_mins / act_down   the same choice for Am and the down activations;
  q6       "exact" B = sc*q exactly; "b2" b1 + b2 with the A_lo*b2 product
           dropped (what ships for |sc| > 64); "b1" b1 only.

The layer around the products follows the oracle (oracle/oracle.c,
restating engine/src/model.c:992-1144): routed experts with the clamped
SiLU, the shared expert with the plain one, the combine in selection order
skipping weights below 1e-6, then (resid + shared) + routed.  Routing is
taken from the oracle (its indices and weights), so only the expert
arithmetic is emulated.
"""
from __future__ import annotations

import dataclasses

import numpy as np

import kquant_np as KQ


@dataclasses.dataclass(frozen=True)
class Variant:
    act: str = "hilo"
    act_mins: str = "hilo"
    act_down: str = "hilo"
    q6: str = "b2"


SHIPPED = Variant()
EXACT = None  # fp64 products of the reference's fp32 weights, no operand rounding


def rtz16(a):
    """fp32 -> fp16 rounded toward zero (v_cvt_pkrtz_f16_f32), as float32."""
    a = np.asarray(a, np.float32)
    h = a.astype(np.float16)
    hf = h.astype(np.float32)
    over = np.abs(hf) > np.abs(a)
    if np.any(over):
        h = h.copy()
        h[over] = np.nextafter(h[over], np.float16(0))
    return h.astype(np.float32)


def operand(a32, how):
    """The fp16 operand(s) the kernel forms from fp32 values a32, summed in
    fp64 (the sum of two fp16 values is exact in fp64)."""
    if how == "hilo":
        hi = rtz16(a32)
        lo = rtz16((a32 - hi).astype(np.float32))  # a - hi is exact in fp32
        return hi.astype(np.float64) + lo.astype(np.float64)
    if how == "rtz":
        return rtz16(a32).astype(np.float64)
    if how == "rtn":
        return np.asarray(a32, np.float32).astype(np.float16).astype(np.float64)
    raise ValueError(how)


def hilo_parts(a32):
    hi = rtz16(a32)
    lo = rtz16((a32 - hi).astype(np.float32))
    return hi.astype(np.float64), lo.astype(np.float64)


def row_scale(amax, dmax):
    """mfma_ops.h row_scale: the power of two s with amax*dmax*s in
    [2^13, 2^14); 1 when the product is 0 or not finite."""
    t = np.float32(amax) * np.float32(dmax)
    if not (t > 0) or not np.isfinite(t):
        return np.float32(1.0)
    _, ex = np.frexp(np.float64(t))  # t = f * 2^ex, f in [0.5, 1): ilogb(t) = ex - 1
    e = 13 - (int(ex) - 1)
    e = max(-126, min(126, e))
    return np.float32(np.ldexp(1.0, e))


class Q4Matrix:
    """One Q4_K matrix [K x M] in vec@mat order, decoded into components."""

    def __init__(self, blocks, K, M):
        self.K, self.M = K, M
        self.NB = M // 256
        d, dmin, sc, m, q = KQ.q4k_components(blocks)
        # block (k, b) = flat block k*NB + b
        self.d = d.reshape(K, self.NB)
        self.dmin = dmin.reshape(K, self.NB)
        self.B = (sc * q).reshape(K, M).astype(np.float64)  # exact integers
        self.m = m.reshape(K, M).astype(np.float64)
        self.W = KQ.q4k_weights((d, dmin, sc, m, q)).reshape(K, M)
        fin = np.concatenate([np.abs(d), np.abs(dmin)])
        self.dmax = np.float32(fin[~np.isnan(fin)].max(initial=0.0))  # NaN skipped, as packed

    def apply(self, X, v):
        """X [R x K] fp32 rows -> [R x M] fp64 (variant v; None = exact)."""
        if v is None:
            return X.astype(np.float64) @ self.W.astype(np.float64)
        R = X.shape[0]
        out = np.empty((R, self.M), np.float64)
        s = np.array([row_scale(np.abs(X[r]).max(initial=0.0), self.dmax) for r in range(R)],
                     np.float32)
        xs = (X * s[:, None]).astype(np.float32)  # exact (power of two)
        for b in range(self.NB):
            cols = slice(256 * b, 256 * b + 256)
            A = (xs * self.d[None, :, b]).astype(np.float32)
            Am = (xs * self.dmin[None, :, b]).astype(np.float32)
            acc = operand(A, v.act) @ self.B[:, cols] - operand(Am, v.act_mins) @ self.m[:, cols]
            out[:, cols] = acc / s[:, None].astype(np.float64)
        return out


class Q6Matrix:
    """One Q6_K matrix [K x M] in vec@mat order."""

    def __init__(self, blocks, K, M):
        self.K, self.M = K, M
        self.NB = M // 256
        d, sc, q = KQ.q6k_components(blocks)
        self.d = d.reshape(K, self.NB)
        B = (sc * q).reshape(K, M)
        self.B = B.astype(np.float64)
        self.b1 = B.astype(np.float32).astype(np.float16).astype(np.float64)  # RN
        self.b2 = self.B - self.b1  # exact, |b2| <= 1
        self.W = KQ.q6k_weights((d, sc, q)).reshape(K, M)
        fin = np.abs(d)
        self.dmax = np.float32(fin[~np.isnan(fin)].max(initial=0.0))

    def apply(self, X, v):
        if v is None:
            return X.astype(np.float64) @ self.W.astype(np.float64)
        R = X.shape[0]
        out = np.empty((R, self.M), np.float64)
        s = np.array([row_scale(np.abs(X[r]).max(initial=0.0), self.dmax) for r in range(R)],
                     np.float32)
        xs = (X * s[:, None]).astype(np.float32)
        for b in range(self.NB):
            cols = slice(256 * b, 256 * b + 256)
            A = (xs * self.d[None, :, b]).astype(np.float32)
            if v.q6 == "exact":
                acc = operand(A, v.act_down) @ self.B[:, cols]
            elif v.q6 == "b1":
                acc = operand(A, v.act_down) @ self.b1[:, cols]
            elif v.q6 == "b2":
                a = operand(A, v.act_down)
                acc = a @ self.b1[:, cols]
                if v.act_down == "hilo":
                    hi, _ = hilo_parts(A)
                    acc += hi @ self.b2[:, cols]
                else:
                    acc += a @ self.b2[:, cols]
            else:
                raise ValueError(v.q6)
            out[:, cols] = acc / s[:, None].astype(np.float64)
        return out


def silu(g, clamp):
    g = np.asarray(g, np.float64)
    y = g / (1.0 + np.exp(-np.clip(g, -700, 700)))
    if clamp:
        y = np.where(g < -50.0, 0.0, np.where(g > 50.0, g, y))
    return y


class Expert:
    def __init__(self, gate, up, down, D, H):
        self.gate = Q4Matrix(gate, D, H)
        self.up = Q4Matrix(up, D, H)
        self.down = Q6Matrix(down, H, D)

    def ffn(self, X, v, clamp):
        g = self.gate.apply(X, v)
        u = self.up.apply(X, v)
        mid = (silu(g, clamp) * u).astype(np.float32)  # the kernels keep mid in fp32
        return self.down.apply(mid, v)


def layer(*, D, H, E, k, x, syn, idx, w, variants, resid=None, rows=None):
    """Layer outputs [T x D] (fp64) for each variant in `variants` (a dict
    name -> Variant or None for exact products), over the tokens `rows`
    (default all), with routing idx/w [T x k] (from the oracle).

    syn: an ornith_moe.SyntheticLayer-like object with routed(which) and
    shared(which) byte arrays in the contiguous per-expert layout."""
    x = np.asarray(x, np.float32)
    T = x.shape[0]
    rows = np.arange(T) if rows is None else np.asarray(rows)
    per4, per6 = (D * H // 256) * 144, (D * H // 256) * 210
    res = {n: np.zeros((len(rows), D), np.float64) for n in variants}
    base = np.zeros((len(rows), D), np.float64) if resid is None else \
        np.asarray(resid, np.float32)[rows].astype(np.float64)
    X = x[rows]
    sg, su, sd = syn.shared("gate"), syn.shared("up"), syn.shared("down")
    if sg is not None:
        ex = Expert(sg, su, sd, D, H)
        for n, v in variants.items():
            res[n] += ex.ffn(X, v, clamp=False)
    for n in variants:
        res[n] += base
    # routed: per expert, its (row, slot) pairs; then the combine in selection order
    ys = {n: np.zeros((len(rows), k, D), np.float64) for n in variants}
    sel = idx[rows]
    wt = w[rows]
    for e in np.unique(sel):
        pr, ps = np.nonzero((sel == e) & ~(wt < 1e-6))
        if len(pr) == 0:
            continue
        ex = Expert(syn.routed("gate")[e * per4:(e + 1) * per4],
                    syn.routed("up")[e * per4:(e + 1) * per4],
                    syn.routed("down")[e * per6:(e + 1) * per6], D, H)
        for n, v in variants.items():
            ys[n][pr, ps] = ex.ffn(X[pr], v, clamp=True)
    for n in variants:
        routed = np.zeros((len(rows), D), np.float64)
        for a in range(k):
            keep = ~(wt[:, a] < 1e-6)
            routed[keep] += wt[keep, a, None].astype(np.float64) * ys[n][keep, a]
        res[n] += routed
    return res


def row_err(out, ref):
    """Per-row max|out - ref| / max|ref| (the north star's metric)."""
    ref = np.asarray(ref, np.float64)
    return np.abs(np.asarray(out, np.float64) - ref).max(axis=1) / np.abs(ref).max(axis=1)
