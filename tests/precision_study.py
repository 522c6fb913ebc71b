"""Precision of the matrix-core operand choices over whole BASELINE batches
(test infrastructure: numpy on the CPU, no GPU).

Emulates the vec@mat expert kernels' operand rounding (tests/mfma_emul.py) at
the Ornith shape (D=2048, H=512, E=256, k=8, shared expert) over every token
of a batch, against the fp64 products of the reference's fp32 weights, and
prints the north star's metric (max|dy| / max|y| per token row) for each
variant:

  hilo      fp16 hi + lo activations, rounded toward zero (what ships)
  rtz       hi only, rounded toward zero
  rtn       hi only, rounded to nearest
  rtn_gu    rounded-to-nearest hi only for gate/up (main and mins), hi + lo
            for down
  rtn_main  rounded-to-nearest hi only for the gate/up main term only

Batches: BASELINE configs[3] (2048-token prefill) and configs[4] (Zipf(1.1)
256 tokens), seeded as the bench seeds them (seed 1234, layer 0).

    python tests/precision_study.py [--tokens 2048] [--zipf-tokens 256]

Routing (indices and weights) comes from the oracle's router and selection
(oracle/oracle.c), so the numbers isolate the expert arithmetic.  About five
minutes on 8 cores.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, ROOT, os.path.join(ROOT, "ornith-flight_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import mfma_emul as M  # noqa: E402

VARIANTS = {
    "exact": None,
    "hilo": M.SHIPPED,
    "rtz": M.Variant("rtz", "rtz", "rtz"),
    "rtn": M.Variant("rtn", "rtn", "rtn"),
    "rtn_gu": M.Variant("rtn", "rtn", "hilo"),
    "rtn_main": M.Variant("rtn", "hilo", "hilo"),
}


def routing(O, x, syn, k):
    T = x.shape[0]
    idx = np.zeros((T, k), np.uint32)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        lg = O.router_logits(x[t], syn.router, syn.bias)
        idx[t], w[t] = O.topk(lg, k, O.MODE_RENORM)
    return idx, w


def study(om, O, T, zipf_s, seed=1234, D=2048, H=512, E=256, k=8):
    syn = om.SyntheticLayer(seed, 0, D, H, E, True, zipf_s)
    x = om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)
    idx, w = routing(O, x, syn, k)
    res = M.layer(D=D, H=H, E=E, k=k, x=x, syn=syn, idx=idx, w=w, variants=VARIANTS)
    out = {}
    for n, v in res.items():
        if n == "exact":
            continue
        e = M.row_err(v, res["exact"])
        out[n] = (float(e.max()), float(np.percentile(e, 99)), float(np.median(e)))
    # the oracle's own fp32 chains on a few tokens, for scale
    sub = np.arange(min(T, 8))
    ref, _, _ = O.moe_layer(D=D, H=H, E=E, k=k, x=x[sub], router_W=syn.router, bias=syn.bias,
                            gate=syn.routed("gate"), up=syn.routed("up"), down=syn.routed("down"),
                            sh_gate=syn.shared("gate"), sh_up=syn.shared("up"),
                            sh_down=syn.shared("down"))
    out["oracle(first 8)"] = (float(M.row_err(ref, res["exact"][sub]).max()), float("nan"),
                              float("nan"))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=2048)
    ap.add_argument("--zipf-tokens", type=int, default=256)
    a = ap.parse_args()
    import ornith_moe as om
    from oracle import oracle as O
    for name, T, z in (("prefill", a.tokens, 0.0), ("zipf(1.1)", a.zipf_tokens, 1.1)):
        t0 = time.time()
        r = study(om, O, T, z)
        print(f"{name} T={T} ({time.time() - t0:.0f} s): worst / p99 / median row error vs fp64")
        for n, (mx, p99, med) in r.items():
            print(f"  {n:16s} {mx:.3e}  {p99:.3e}  {med:.3e}", flush=True)


if __name__ == "__main__":
    main()
