#!/usr/bin/env python3
"""Benchmark of the routed-MoE hot path on one MI355X.

Headline workload: one Ornith-shape MoE layer
(D=2048, H=512, E=256 routed + 1 shared expert, top-8, Q4_K gate/up, Q6_K
down), decode batch of 16 tokens, synthetic seeded weights resident in HBM.
A step is one gpu_moe_forward over the batch (router, top-8, dispatch,
experts, combine); inputs are already in HBM when the timed region starts.

Prints ONE JSON line (rank 0).  Also reported in "configs": the other
BASELINE configs measured the same way (1-token decode, 2048-token prefill,
Zipf-skewed 256 tokens, and the 40-layer resident stack at 1 and 16 tokens;
--no-stack skips the stack), the file-orientation store, streamed experts
(host tier + device slots), the attention-side gpu.h ops and the device
dequant API.

`roofline` is for the dominant kernel of the step: algorithmic bytes of the
expert weights that kernel streams (active experts x bytes per expert) over
its average duration, timed with HIP events recorded on the library's
stream around every launch inside the timed region.

`cpu_baseline` times the reference's own C CPU path (oracle/_ref, compiled
from the reference sources: model_forward on a one-layer Ornith-shape
model) on a bounded sample of tokens, single-threaded as the reference runs;
its "contiguous" entry times the reference's arithmetic on a contiguous
per-expert layout (the C99 oracle) for every config, on the same expert bytes.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "ornith-flight_amd"))

import numpy as np  # noqa: E402

import ornith_moe as om  # noqa: E402

D, H, E, K = 2048, 512, 256, 8
GU_BYTES = 2 * (D * H // 256) * 144      # gate + up per expert: 1,179,648
DN_BYTES = (D * H // 256) * 210          # down per expert: 860,160
EXPERT_BYTES = GU_BYTES + DN_BYTES       # 2,039,808
FLOP_PER_PAIR = 2 * (2 * D * H + H * D)  # 6,291,456
MFMA_F16_PEAK_TFLOPS = 2500.0            # MI355X dense fp16 matrix peak
VALU_F32_PEAK_TFLOPS = 157.3             # MI355X fp32 vector peak (an FMA = 2 flops)
HBM_PEAK_GBS = 8000.0
SEED = 1234


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measure(ctx, store, layer, T, steps, warmup, x_seed=1, stack_layers=0, ep=(0, 0), flags=0):
    x = om.synth_normal(x_seed, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)
    xb = ctx.upload(x)
    ob = ctx.alloc(x.nbytes)
    L = om.lib()
    opts = om.MoEOpts(om.ROUTE_RENORM, om.MOE_ASYNC | flags, ep[0], ep[1])

    def step():
        if stack_layers:
            rc = L.gpu_moe_forward_stack(ctx.ptr, store.ptr, 0, stack_layers, xb.ptr, ob.ptr, T,
                                         om.C.byref(opts))
        else:
            rc = L.gpu_moe_forward(ctx.ptr, store.ptr, layer, xb.ptr, T, None, ob.ptr, None, None,
                                   om.C.byref(opts))
        if rc:
            raise RuntimeError(ctx.last_error())

    for _ in range(warmup):
        step()
    ctx.sync()
    stats = store.last_stats()
    # Per-kernel region: HIP events on the library's stream.  Every step but
    # the input norm is launched with hipExtLaunchKernel, which stamps the
    # kernels' own start and end into the events (the duration a kernel
    # trace reports); the norm is bracketed by an event pair, which adds a
    # few microseconds to it.
    L.gpu_profile_enable(ctx.ptr, 1)
    L.gpu_profile_reset(ctx.ptr)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.sync()
    t1 = time.perf_counter()
    prof = om.profile(ctx)
    L.gpu_profile_enable(ctx.ptr, 0)
    # Same number of forwards without events: the step time.
    ctx.sync()
    t2 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.sync()
    t3 = time.perf_counter()
    xb.free()
    ob.free()
    ms = (t3 - t2) * 1e3 / steps
    kernels = {n: {"avg_us": 1e3 * tot / c, "calls_per_step": c / steps}
               for n, (tot, c) in prof.items() if c > 0}
    return ms, kernels, stats


def load_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 --pmc summary (FETCH_SIZE x counter scale + WRITE_SIZE), if
    one exists: profiles/traffic_<kernel>_<workload>.txt, a line
    'traffic_bytes_per_dispatch <N>'."""
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_{workload}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_dispatch"):
                    return int(float(line.split()[1])), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def roofline_for(kernels, stats, T, workload):
    """Dominant expert kernel against its roofline.

    Decode-shaped kernels (VALU matvec, MFMA decode instances): HBM-bound;
    achieved = algorithmic expert bytes per launch (active experts x GGUF
    bytes of the matrices the kernel streams: Q4_K gate+up, Q6_K down) /
    average launch time.  Prefill MFMA grouped GEMMs: matrix-core bound;
    achieved = useful flops per launch (token-expert rows x 2*K*N) / time,
    against the dense fp16 peak.  The MFMA kernels run two MFMAs (activation
    hi and lo halves) per useful product, so their instruction rate is twice
    the useful rate shown.
    """
    slots = stats["n_slots"]  # active experts incl. the shared one
    rows = stats["n_rows"]    # token-expert pairs incl. the shared expert's
    work = {"moe_gateup": ("hbm", slots * GU_BYTES), "moe_down": ("hbm", slots * DN_BYTES),
            "moe_gateup_dec": ("hbm", slots * GU_BYTES), "moe_down_dec": ("hbm", slots * DN_BYTES),
            "moe_gateup_mfma": ("mfma", rows * 2 * D * 2 * H), "moe_down_mfma": ("mfma", rows * 2 * H * D),
            "moe_gateup_file": ("hbm", slots * GU_BYTES), "moe_down_file": ("hbm", slots * DN_BYTES)}
    if T >= 64:  # prefill sizes: the file kernels matrix-core bound, the VALU ones vector bound
        work["moe_gateup_file"] = ("mfma", rows * 2 * D * 2 * H)
        work["moe_down_file"] = ("mfma", rows * 2 * H * D)
        work["moe_gateup"] = ("valu", rows * 2 * D * 2 * H)
        work["moe_down"] = ("valu", rows * 2 * H * D)
    present = [n for n in work if n in kernels]
    name = max(present, key=lambda n: kernels[n]["avg_us"] * kernels[n]["calls_per_step"])
    bound, amount = work[name]
    avg_s = kernels[name]["avg_us"] * 1e-6
    traffic, src = load_traffic(name, workload)
    if bound == "hbm":
        ach = amount / avg_s / 1e9
        out = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
               "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
               "kernel": name, "bytes_per_launch": amount,
               "avg_us": round(kernels[name]["avg_us"], 2)}
        if name.endswith(("_dec", "_file")):
            # the matrix-core kernels' useful flops too (both bounds reported)
            fl = rows * 2 * D * 2 * H if "gateup" in name else rows * 2 * H * D
            out["mfma"] = {"achieved": round(fl / avg_s / 1e12, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                           "unit": "TFLOP/s", "frac": round(fl / avg_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                           "flops_per_launch": fl}
    else:
        ach = amount / avg_s / 1e12
        # the same kernel's weight bytes against HBM (both bounds are reported
        # for matrix-core kernels: mixed batches sit between them)
        wbytes = slots * (GU_BYTES if "gateup" in name else DN_BYTES)
        hbm = wbytes / avg_s / 1e9
        peak = MFMA_F16_PEAK_TFLOPS if bound == "mfma" else VALU_F32_PEAK_TFLOPS
        out = {"bound": bound, "achieved": round(ach, 1), "peak": peak,
               "unit": "TFLOP/s", "frac": round(ach / peak, 4), "traffic": traffic,
               "kernel": name, "flops_per_launch": amount,
               "avg_us": round(kernels[name]["avg_us"], 2),
               "hbm": {"achieved": round(hbm, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(hbm / HBM_PEAK_GBS, 4), "bytes_per_launch": wbytes}}
    if src:
        out["traffic_source"] = src
    return name, out


def cpu_baseline(budget_s):
    """Reference CPU path (oracle/_ref model_forward), one thread, bounded sample."""
    try:
        from oracle import ref
        if not ref.available():
            raise RuntimeError("oracle/_ref not built")
        nblk = D * H * E // 256
        seed = 99
        fused = [fn(seed, om.synth_stream(0, kind, 0xFFFFFF), nblk) for kind, fn in
                 ((om.SYN_GATE, om.synth_q4k), (om.SYN_UP, om.synth_q4k), (om.SYN_DOWN, om.synth_q6k))]
        nbs = D * H // 256
        sh = [fn(seed, om.synth_stream(0, kind, E), nbs) for kind, fn in
              ((om.SYN_GATE, om.synth_q4k), (om.SYN_UP, om.synth_q4k), (om.SYN_DOWN, om.synth_q6k))]
        W = om.synth_normal(seed, om.synth_stream(0, om.SYN_ROUTER, 0), D * E, 0.02).reshape(D, E)
        X = om.synth_normal(seed, om.synth_stream(0, om.SYN_ACT, 0), 16 * D, 1.0).reshape(16, D)
        m = ref.RefMoEModel(D=D, H=H, E=E, k=K, X=X, router_W=W, norm_w=np.ones(D, np.float32),
                            gate=fused[0], up=fused[1], down=fused[2], sh_gate=sh[0], sh_up=sh[1],
                            sh_down=sh[2])
        del fused
        m.forward(0)  # warm-up (page-in)
        n, t0 = 0, time.perf_counter()
        while n < 16:
            m.forward(n)
            n += 1
            if time.perf_counter() - t0 > budget_s:
                break
        dt = time.perf_counter() - t0
        m.close()
        return {"value": round(n / dt, 4), "unit": "tokens/s", "cores": 1, "kind": "reference",
                "sample": f"{n} tokens of the 16-token decode batch through the reference's "
                          f"model_forward MoE block (interleaved fused Q4_K/Q6_K tensors, "
                          f"literal routing), {dt:.1f} s on {platform.processor() or platform.machine()}, "
                          f"host nproc={os.cpu_count()}"}
    except Exception as e:  # fall back to the C99 restatement
        log("reference CPU baseline unavailable:", e)
        from oracle import oracle as O
        syn = om.SyntheticLayer(SEED, 0, D, H, E, True)
        X = om.synth_normal(1, om.synth_stream(0, om.SYN_ACT, 0), 16 * D, 1.0).reshape(16, D)
        t0 = time.perf_counter()
        O.moe_layer(D=D, H=H, E=E, k=K, x=X, router_W=syn.router, gate=syn.routed("gate"),
                    up=syn.routed("up"), down=syn.routed("down"), sh_gate=syn.shared("gate"),
                    sh_up=syn.shared("up"), sh_down=syn.shared("down"))
        dt = time.perf_counter() - t0
        return {"value": round(16 / dt, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"16-token decode batch through the oracle restatement, {dt:.2f} s"}


def cpu_contiguous(store):
    """CPU baseline variant (ii) for every config: the reference's arithmetic
    on a contiguous per-expert layout (blockwise dequant + per-token matvec,
    no cross-token reuse; the C99 oracle, one thread) over the same expert
    bytes and activations as the GPU configs.  decode_t1 / decode_t16 run in
    full (median of 3 after one warm-up); prefill_t2048 and zipf_t256 time
    their first 32 tokens and extrapolate linearly (tokens are independent)."""
    from oracle import oracle as O
    E1 = E + 1
    layers = {}
    for l, zipf in ((0, 0.0), (1, 1.1)):
        W = om.synth_normal(SEED, om.synth_stream(l, om.SYN_ROUTER, 0), D * E, 0.02).reshape(D, E)
        bias = om.synth_zipf_bias(SEED, om.synth_stream(l, om.SYN_ZIPF, 0), E, zipf) if zipf else None
        mats = [store.get_experts(l, m, 0, E1) for m in (om.MAT_GATE, om.MAT_UP, om.MAT_DOWN)]
        layers[l] = (W, bias, mats)
    out = {}
    for label, layer, T, sample in (("decode_t1", 0, 1, 1), ("decode_t16", 0, 16, 16),
                                    ("prefill_t2048", 0, 2048, 32), ("zipf_t256", 1, 256, 32)):
        W, bias, (g, u, d) = layers[layer]
        per_g, per_d = g.size // E1, d.size // E1
        X = om.synth_normal(1, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)[:sample]

        def run():
            t0 = time.perf_counter()
            O.moe_layer(D=D, H=H, E=E, k=K, x=X, router_W=W, bias=bias, gate=g[:E * per_g],
                        up=u[:E * per_g], down=d[:E * per_d], sh_gate=g[E * per_g:],
                        sh_up=u[E * per_g:], sh_down=d[E * per_d:])
            return time.perf_counter() - t0
        run()
        dt = sorted(run() for _ in range(3 if sample <= 16 else 1))[(3 if sample <= 16 else 1) // 2]
        out[label] = {"tokens_per_s": round(sample / dt, 2),
                      "sample": f"{sample} of {T} tokens" + (", extrapolated linearly" if sample < T else ""),
                      "s_per_sample": round(dt, 3)}
    return {"variant": "contiguous layout, reference arithmetic (oracle, 1 thread)", "cores": 1,
            "configs": out}


def stack_active_experts(ctx, st, n_layers, T):
    """Active experts (incl. the shared one) of every layer of one stack
    step, from the same layers run one call at a time (x <- x +
    MoE_l(rmsnorm(x)), the stack's arithmetic) outside the timed region."""
    x = om.synth_normal(1, om.synth_stream(0, om.SYN_ACT, 0), T * D, 1.0).reshape(T, D)
    xb, ob = ctx.upload(x), ctx.alloc(x.nbytes)
    total = 0
    for l in range(n_layers):
        st.forward(l, xb, T, ob, resid=xb, flags=om.MOE_NORM)
        total += st.last_stats()["n_slots"]
        om.lib().gpu_copy_buffer(ctx.ptr, xb.ptr, ob.ptr, x.nbytes)
    xb.free()
    ob.free()
    return total


def measure_stack(ctx, steps):
    """40 Ornith-shape layers x 257 experts resident in
    HBM (generated on the device and kept in the MFMA layouts only,
    prefill_layout = 2: 23.8 GB, 1.13x the GGUF bytes), a step = one
    gpu_moe_forward_stack over all 40 layers (rmsnorm, MoE, residual per
    layer).  40 x 257 experts cannot stay in the 256 MB last-level cache
    between steps, unlike one layer's active experts."""
    n_layers = 40
    st = om.Store(ctx, n_layers, D, H, E, K, True, 2)
    t0 = time.perf_counter()
    for l in range(n_layers):
        st.fill_synthetic(l, SEED + l)
    log(f"40-layer store ({st.bytes() / 1e9:.1f} GB) filled on the device in "
        f"{time.perf_counter() - t0:.1f} s")
    out = {}
    for Ts in (1, 16):
        active = stack_active_experts(ctx, st, n_layers, Ts)
        ms_s, kern_s, _ = measure(ctx, st, 0, Ts, max(10, steps // 10), 3, stack_layers=n_layers)
        gbs = active * EXPERT_BYTES / (ms_s * 1e-3) / 1e9
        out[f"stack40_t{Ts}"] = {
            "tokens_per_s": round(Ts / (ms_s * 1e-3), 1), "ms_per_step": round(ms_s, 4),
            "us_per_layer": round(ms_s * 1e3 / n_layers, 2),
            "active_experts_per_step": active,
            "expert_bytes_per_step": active * EXPERT_BYTES,
            "hbm": {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "kernels_us": {n: round(v["avg_us"], 2) for n, v in kern_s.items()},
            "kernel_calls_per_step": {n: round(v["calls_per_step"], 1) for n, v in kern_s.items()}}
        log(f"stack40_t{Ts}", out[f"stack40_t{Ts}"]["tokens_per_s"], "tok/s")
    st.close()
    return out


def measure_streamed(ctx, steps):
    """Streamed experts (shape.cache_slots): 8 Ornith-shape layers in the
    pinned host tier, streamed through a pool of device slots.  A step is one
    forward of every layer in turn for a batch drawn from a pool of 16
    seeded batches (so routing, and with it the misses, varies).  Reported:
    layer forwards per second, the slot hit rate, and the host->device
    expert bytes per second against the PCIe Gen5 x16 peak (64 GB/s)."""
    n_layers = 8
    out = {}
    for Ts, slots in ((1, 64), (16, 192)):
        st = om.Store(ctx, n_layers, D, H, E, K, True, cache_slots=slots)
        for l in range(n_layers):
            st.fill_synthetic(l, SEED + l)
        pool = [ctx.upload(om.synth_normal(100 + i, om.synth_stream(0, om.SYN_ACT, 0), Ts * D,
                                           1.0)) for i in range(16)]
        ob = ctx.alloc(Ts * D * 4)
        L = om.lib()
        opts = om.MoEOpts(om.ROUTE_RENORM, 0, 0, 0)

        def sweep(i):
            for l in range(n_layers):
                rc = L.gpu_moe_forward(ctx.ptr, st.ptr, l, pool[i % 16].ptr, Ts, None, ob.ptr,
                                       None, None, om.C.byref(opts))
                if rc:
                    raise RuntimeError(ctx.last_error())

        for i in range(16):
            sweep(i)
        st.cache_stats(reset=True)
        n = max(8, steps // 10)
        t0 = time.perf_counter()
        for i in range(n):
            sweep(i)
        ctx.sync()
        dt = time.perf_counter() - t0
        cs = st.cache_stats()
        fwd = n * n_layers
        h2d = cs["bytes_uploaded"] / dt / 1e9
        out[f"streamed_t{Ts}_slots{slots}"] = {
            "layer_forwards_per_s": round(fwd / dt, 1),
            "tokens_per_s_per_layer": round(Ts * fwd / dt, 1),
            "us_per_layer": round(dt / fwd * 1e6, 1), "layers": n_layers, "slots": slots,
            "hit_rate": round(cs["hits"] / max(1, cs["hits"] + cs["misses"]), 4),
            "misses_per_layer": round(cs["misses"] / fwd, 2),
            "h2d": {"achieved": round(h2d, 2), "peak": 64.0, "unit": "GB/s",
                    "frac": round(h2d / 64.0, 4)},
            "host_tier_gb": round(cs["host_bytes"] / 1e9, 2),
            "slot_pool_gb": round(cs["device_bytes"] / 1e9, 3)}
        log(f"streamed_t{Ts}", out[f"streamed_t{Ts}_slots{slots}"])
        for b in pool + [ob]:
            b.free()
        st.close()
    return out


def measure_attention(ctx):
    """gpu_rope / gpu_attention (the Metal backend's semantics) at Ornith's
    head size: one head, 4096 positions, head_dim 256, on the fp32 matrix
    cores; 4*S^2*d flops per call against the MI355X dense fp32 peak
    (157.3 TFLOP/s)."""
    S, hd = 4096, 256
    rng = np.random.default_rng(0)
    bufs = [ctx.upload(rng.standard_normal((S, hd)).astype(np.float32)) for _ in range(3)]
    ob = ctx.alloc(S * hd * 4)
    L = om.lib()
    L.gpu_attention(ctx.ptr, ob.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, S, hd)
    n = 5
    t0 = time.perf_counter()
    for _ in range(n):
        L.gpu_attention(ctx.ptr, ob.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, S, hd)
    dt = (time.perf_counter() - t0) / n
    tf = 4.0 * S * S * hd / dt / 1e12
    q, k = ctx.upload(np.ones((16, 256), np.float32)), ctx.upload(np.ones((2, 256), np.float32))
    m = 200
    t0 = time.perf_counter()
    for i in range(m):
        L.gpu_rope(ctx.ptr, q.ptr, k.ptr, 1, 256, 16, 2, om.C.c_float(1e7), i)
    rope_us = (time.perf_counter() - t0) / m * 1e6
    for b in bufs + [ob, q, k]:
        b.free()
    res = {"attention_s4096_d256": {"ms": round(dt * 1e3, 3), "tflops": round(tf, 2),
                                    "bound": "mfma", "peak_fp32_tflops": 157.3,
                                    "frac": round(tf / 157.3, 4)},
           "rope_16q2k_d256_us_per_call": round(rope_us, 2)}
    log("attention", res)
    return res


def measure_lm_head(ctx):
    """gpu_matmul at the shape of the reference's LM head (model.c:1219-1231:
    logits[i] = sum_d x[d] * W[d][i], D = 2048, vocab 248,320 from
    model.c:120) for one token and for 16 (M = 1, 16): an fp32 B of 2.03 GB
    streamed once per call (per 16 rows), bit-identical to the CPU backend's
    sequential sums.  HBM-bound at M = 1: (K*N + M*K + M*N) * 4 bytes per call
    against 8 TB/s; at M = 16 also 2*M*N*K flops against the fp32 vector
    peak (157.3 TFLOP/s).  Synchronous calls, as the API is."""
    K, N = 2048, 248320
    L = om.lib()
    Bb = ctx.upload(np.full((K, N), 0.5, np.float32))
    res = {}
    for M in (1, 16):
        Ab = ctx.upload(np.full((M, K), 0.25, np.float32))
        Cb = ctx.alloc(M * N * 4)
        L.gpu_matmul(ctx.ptr, Cb.ptr, Ab.ptr, Bb.ptr, M, N, K, 0, 0)
        reps = 10
        t0 = time.perf_counter()
        for _ in range(reps):
            L.gpu_matmul(ctx.ptr, Cb.ptr, Ab.ptr, Bb.ptr, M, N, K, 0, 0)
        dt = (time.perf_counter() - t0) / reps
        moved = 4 * (K * N + M * K + M * N)
        out = {"ms": round(dt * 1e3, 3), "tokens_per_s": round(M / dt, 1),
               "hbm": {"achieved": round(moved / dt / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                       "frac": round(moved / dt / 8e12, 4), "bytes_per_call": moved}}
        if M > 1:
            tf = 2.0 * M * N * K / dt / 1e12
            out["valu"] = {"achieved": round(tf, 2), "peak": 157.3, "unit": "TFLOP/s",
                           "frac": round(tf / 157.3, 4)}
        res[f"lm_head_m{M}_k{K}_n{N}"] = out
        Ab.free()
        Cb.free()
    Bb.free()
    log("lm_head", res)
    return res


def measure_dequant(ctx):
    """The device dequant API (gpu_dequantize_tensor_buf, gguf.c:605-638) on
    one layer's expert tensor: 256 experts x 2048 x 512 weights, Q4_K (the
    gate / up layout) and Q6_K (down), to fp32.  HBM-bound: the quantized
    bytes read plus 4 bytes written per weight, per call (synchronous, as the
    API is), against 8 TB/s."""
    n = 256 * 2048 * 512
    L = om.lib()
    res = {}
    for name, typ, bsize, d_offs in (("q4k", 12, 144, (0, 2)), ("q6k", 14, 210, (208,))):
        nb = n // 256
        blocks = np.zeros((nb, bsize), np.uint8)
        for off in d_offs:
            blocks[:, off + 1] = 0x3C  # d = 1.0
        src, dst = ctx.upload(blocks.reshape(-1)), ctx.alloc(4 * n)
        del blocks
        info = om.tensor_info(typ, [n])
        if not L.gpu_dequantize_tensor_buf(ctx.ptr, src.ptr, om.C.byref(info), dst.ptr):
            raise RuntimeError(ctx.last_error())
        ctx.sync()
        reps = 10
        t0 = time.perf_counter()
        for _ in range(reps):
            L.gpu_dequantize_tensor_buf(ctx.ptr, src.ptr, om.C.byref(info), dst.ptr)
        ctx.sync()
        dt = (time.perf_counter() - t0) / reps
        moved = nb * bsize + 4 * n
        res[f"dequant_{name}_256x2048x512"] = {"ms": round(dt * 1e3, 3),
                                              "gbs": round(moved / dt / 1e9, 1),
                                              "frac": round(moved / dt / 8e12, 4),
                                              "bytes_per_call": moved}
        src.free()
        dst.free()
    log("dequant", res)
    return res


def wide_q6_store(ctx):
    """Layer 0 of the headline store with every Q6_K sub-scale redrawn over
    [-128, 127] and each block's first at -128 or 127 (a quantizer sets the
    largest sub-block of a block to the range's end): sc * q then exceeds
    fp16's exact integers and the down kernels split it in two operands."""
    st = om.Store(ctx, 1, D, H, E, K, True)
    st.fill_synthetic(0, SEED)
    blocks = st.get_experts(0, om.MAT_DOWN, 0, E + 1).reshape(-1, om.Q6K_BYTES)
    rng = np.random.default_rng(SEED)
    sc = rng.integers(-128, 128, size=(blocks.shape[0], 16))
    sc[:, 0] = np.where(rng.random(blocks.shape[0]) < 0.5, -128, 127)
    blocks[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    st.set_experts(0, om.MAT_DOWN, 0, blocks.reshape(-1), E + 1)
    return st


# Extra configs reported beside the headline: (label, store layer, tokens).
# Layer 1 carries a Zipf(1.1) router bias.
EXTRA_CONFIGS = (("decode_t1", 0, 1), ("prefill_t2048", 0, 2048), ("zipf_t256", 1, 256))
EXTRA_LABELS = [c[0] for c in EXTRA_CONFIGS] + ["valu_t1", "valu_t16", "valu_t2048", "file_t1",
                                                 "file_t16", "file_t2048", "q6wide_t1",
                                                 "q6wide_t16", "q6wide_t2048", "stack40",
                                                 "streamed", "attention", "dequant", "lm_head"]


def headline(ctx, store, args, read_gbs):
    """the 16-token decode step of one Ornith-shape layer."""
    T = 16
    ms, kernels, stats = measure(ctx, store, 0, T, args.steps, args.warmup)
    dom, roof = roofline_for(kernels, stats, T, "t16")
    roof["measured_read_peak"] = round(read_gbs, 1)
    roof["frac_of_measured"] = round(roof["achieved"] / read_gbs, 4)
    U = stats["n_slots"]
    result = {
        "metric": "MoE-layer tokens/s at batch 1/16/2048; achieved HBM GB/s & MFMA % vs peak",
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 hi+lo MFMA, f32 accumulate (Q4_K/Q6_K weights exact as f16 sc*q)",
        "data": "synthetic (seeded Q4_K/Q6_K experts; activations and router weights are "
                "Irwin-Hall(12) sums: mean 0, sd 1 (router 0.02), bounded at 6 sd)",
        "config": {"workload": "BASELINE configs[1]: single Ornith-shape MoE layer, 16-token decode",
                   "tokens": T, "d_model": D, "expert_ffn": H, "experts": E, "top_k": K,
                   "shared_experts": 1, "active_experts_incl_shared": U,
                   "expert_bytes_streamed": U * EXPERT_BYTES},
        "roofline": roof,
        "kernels_us": {n: round(v["avg_us"], 2) for n, v in kernels.items()},
        "layer_hbm_gbs": round(U * EXPERT_BYTES / (ms * 1e-3) / 1e9, 1),
    }
    return result


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-extra", action="store_true", help="only the headline config")
    ap.add_argument("--only", choices=EXTRA_LABELS, default=None,
                    help="of the extra configs, time only this one (for a kernel trace of it)")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip the 40-layer resident stack (BASELINE configs[2])")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device once: a kernel of known traffic "
                         "against which hardware byte counters are scaled")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              f"multi-GPU path (the expert-parallel shares run one GPU's part).", file=sys.stderr)
        sys.exit(2)

    ctx = om.Context()
    name, cus, hbm = ctx.device_info()
    log("device:", name, cus, "CUs", hbm >> 30, "GiB")
    if args.copy_probe:
        n = args.copy_probe << 20
        src, dst = ctx.alloc(n), ctx.alloc(n)
        om.lib().gpu_copy_buffer(ctx.ptr, dst.ptr, src.ptr, n)
        ctx.sync()
        src.free()
        dst.free()
        log(f"copy probe: {args.copy_probe} MiB device-to-device")
    # Achievable streaming-read bandwidth of this device (8 GiB, 32 x the
    # last-level cache), reported beside the spec-sheet peak.
    read_gbs = ctx.read_bandwidth(8 << 30, 5)
    log(f"measured streaming read: {read_gbs:.0f} GB/s")
    store = om.Store(ctx, 2, D, H, E, K, True)
    t0 = time.perf_counter()
    store.fill_synthetic(0, SEED)
    store.fill_synthetic(1, SEED, 1.1)  # Zipf(1.1) router bias for the skewed config
    log(f"store filled in {time.perf_counter() - t0:.1f} s ({store.bytes() / 1e9:.2f} GB)")

    T = 16
    if args.only:
        # one extra config alone (a kernel trace of it): the headline's
        # kernels are not timed, and the line carries only that config
        result = {"only": args.only, "steps": args.steps, "warmup": args.warmup}
    else:
        result = headline(ctx, store, args, read_gbs)
    if not args.no_extra:
        extra = {}
        for label, layer, Tn in EXTRA_CONFIGS:
            if args.only and label != args.only:
                continue
            steps = max(5, args.steps // (20 if Tn >= 256 else 1))
            ms_x, kern_x, st_x = measure(ctx, store, layer, Tn, steps, max(2, args.warmup // 4))
            _, roof_x = roofline_for(kern_x, st_x, Tn, label.split("_")[-1])
            if roof_x["bound"] == "hbm":
                roof_x["frac_of_measured"] = round(roof_x["achieved"] / read_gbs, 4)
            extra[label] = {"tokens_per_s": round(Tn / (ms_x * 1e-3), 1), "ms_per_step": round(ms_x, 4),
                            "active_experts": st_x["n_slots"],
                            "layer_hbm_gbs": round(st_x["n_slots"] * EXPERT_BYTES / (ms_x * 1e-3) / 1e9, 1),
                            "tflops": round(Tn * (K + 1) * FLOP_PER_PAIR / (ms_x * 1e-3) / 1e12, 2),
                            "dominant": roof_x,
                            "kernels_us": {n: round(v["avg_us"], 2) for n, v in kern_x.items()}}
            log(label, extra[label]["tokens_per_s"], "tok/s")
        # One GPU's share of an 8-way expert-parallel layer (32 experts per
        # rank, every rank routing all 16 tokens): rank 0 (also the shared
        # expert) and rank 1.  The cross-rank reduction of the T x D partial
        # outputs is not part of this one-GPU figure.
        for label, ep in (("ep8_rank0_t16", (0, E // 8)), ("ep8_rank1_t16", (E // 8, E // 8))):
            if args.only:
                break
            ms_x, kern_x, st_x = measure(ctx, store, 0, 16, args.steps, args.warmup, ep=ep)
            extra[label] = {"tokens_per_s": round(16 / (ms_x * 1e-3), 1), "ms_per_step": round(ms_x, 4),
                            "experts": list(ep), "active_experts": st_x["n_slots"],
                            "layer_hbm_gbs": round(st_x["n_slots"] * EXPERT_BYTES / (ms_x * 1e-3) / 1e9, 1),
                            "kernels_us": {n: round(v["avg_us"], 2) for n, v in kern_x.items()}}
            log(label, extra[label]["tokens_per_s"], "tok/s")
        # Experts in GGUF file orientation (input index fastest, as real
        # files store them): a store of its own, same synthetic bytes.
        def side_store(prefix, st, flags=0, close=True):
            for label, Tn in ((prefix + "t1", 1), (prefix + "t16", 16), (prefix + "t2048", 2048)):
                if args.only and label != args.only:
                    continue
                steps = max(5, args.steps // (20 if Tn >= 256 else 1))
                ms_x, kern_x, st_x = measure(ctx, st, 0, Tn, steps, max(2, args.warmup // 4),
                                             flags=flags)
                _, roof_x = roofline_for(kern_x, st_x, Tn, label.split("_")[-1])
                if roof_x["bound"] == "hbm":
                    roof_x["frac_of_measured"] = round(roof_x["achieved"] / read_gbs, 4)
                extra[label] = {"tokens_per_s": round(Tn / (ms_x * 1e-3), 1),
                                "ms_per_step": round(ms_x, 4), "active_experts": st_x["n_slots"],
                                "layer_hbm_gbs": round(st_x["n_slots"] * EXPERT_BYTES / (ms_x * 1e-3) / 1e9, 1),
                                "dominant": roof_x,
                                "kernels_us": {n: round(v["avg_us"], 2) for n, v in kern_x.items()}}
                log(label, extra[label]["tokens_per_s"], "tok/s")
            if close:
                st.close()

        # The fp32 VALU kernels on the headline layer (the path of a store
        # kept without the MFMA layouts, and the reference-order fallback).
        if not args.only or args.only.startswith("valu_"):
            side_store("valu_", store, om.MOE_PATH_VALU, close=False)
        if not args.only or args.only.startswith("file_"):
            fst = om.Store(ctx, 1, D, H, E, K, True, prefill_layout=False, file_layout=True)
            fst.fill_synthetic(0, SEED)
            side_store("file_", fst)
        # The headline layer with Q6_K sub-scales over the whole int8 range,
        # as real quantizers emit them (the down kernels' wide instances).
        if not args.only or args.only.startswith("q6wide_"):
            side_store("q6wide_", wide_q6_store(ctx))
        result["configs"] = extra
    # CPU variant (ii) reads the experts back from this store (closed next)
    cpu_contig = cpu_contiguous(store) if not args.no_cpu and not args.only else None
    store.close()
    want = lambda label: not args.only or args.only == label  # noqa: E731
    if not args.no_stack and want("stack40"):
        result.setdefault("configs", {}).update(measure_stack(ctx, args.steps))
    if not args.no_extra and want("streamed"):
        result.setdefault("configs", {}).update(measure_streamed(ctx, args.steps))
    if not args.no_extra and want("attention"):
        result.setdefault("configs", {}).update(measure_attention(ctx))
    if not args.no_extra and want("dequant"):
        result.setdefault("configs", {}).update(measure_dequant(ctx))
    if not args.no_extra and want("lm_head"):
        result.setdefault("configs", {}).update(measure_lm_head(ctx))
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_budget)
        if cpu_contig:
            result["cpu_baseline"]["contiguous"] = cpu_contig
            log("cpu contiguous", cpu_contig)
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
