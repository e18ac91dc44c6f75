#!/usr/bin/env python3
"""bench.py — DenseCore's quantized mul_mat hot path on one MI355X.

A step is one dcq_mul_mat call over one batch: Y[M, N] = W[N, K] . quantize(X[M, K])^T
(activation quantization to the vec_dot_type + the int8 dots), on inputs already
resident in HBM. Steps cycle through enough copies of W (1 GiB) to exceed the 256 MB
Infinity Cache, so every step streams its weights from HBM. Steps are captured in
one HIP graph (torch.cuda.CUDAGraph around the C ABI calls) and replayed, so host
launch overhead does not enter GPU time; HIP events on the replay stream time them.

Printed: one JSON line. `value` is the headline configuration's (
Q4_K GEMV, M = 1) weight GB/s over whole steps. `roofline` is for the dominant kernel
of that step: the whole step when it is one kernel (decode with fused activation
quantization), else the mul_mat kernel timed alone on pre-quantized activations.
Every configuration is listed under "configs", each decode config with the measured
pure-read time of its weight bytes (the ceiling any weight-streaming kernel can reach at
that size) beside the 8 TB/s peak. The CPU baseline (configs 2 and 5) is a SIMD
restatement of the reference CPU path (quantize once, row-partitioned AVX2 / AVX-512
VNNI vec_dots, one pinned worker per physical core), timed on this host.

--profile runs the same steps eagerly (no graph) followed by a device-to-device copy
of known size, for rocprofv3 counter passes (the copy calibrates FETCH_SIZE /
WRITE_SIZE); it prints no JSON line.
"""
import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quant mul_mat: weight GB/s at M=1, int8 TOPS at M=2048; % of MI355X roofline"
HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
HEADLINE = 2


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="1,2,3,4,5")
    ap.add_argument("--rotate-mb", type=int, default=1024, help="total bytes of W copies cycled through")
    ap.add_argument("--cpu-seconds", type=float, default=5.0, help="CPU baseline: time budget per config")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--replays", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true", help="skip the gate/up pair measurement")
    ap.add_argument("--profile", action="store_true", help="eager steps + a calibration copy, for rocprofv3 --pmc")
    ap.add_argument("--profile-read", action="store_true",
                    help="eager pure-read launches at each config's weight size, for rocprofv3 --kernel-trace")
    ap.add_argument("--no-read-ceiling", action="store_true", help="skip the pure-read ceiling sweep")
    ap.add_argument("--no-clocks", action="store_true", help="skip sampling the GPU clocks under load")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="CSV",
                    help="print profiles/counters.txt lines from rocprofv3 --pmc counter_collection.csv files "
                         "of --profile runs (no GPU needed)")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print profiles/traffic.txt lines from the counter_collection.csv files of a "
                         "rocprofv3 --pmc FETCH_SIZE and a --pmc WRITE_SIZE run of --profile (no GPU needed)")
    ap.add_argument("--summarize-read", metavar="CSV",
                    help="print profiles/read_ceiling.txt lines from the rocprofv3 kernel_trace.csv of a "
                         "--profile-read run made with the same --configs/--steps/--warmup (no GPU needed)")
    return ap.parse_args()


def make_config_inputs(cfg, dev):
    """W fp32 N(0, w_std) quantized on the GPU (dcq_quantize_weights) and X fp32 N(0, 1)."""
    import torch
    import densecore_amd as dc
    from densecore_amd import synth
    w = synth.normal(cfg.N * cfg.K, cfg.w_seed, 0.0, cfg.w_std).reshape(cfg.N, cfg.K)
    x = synth.normal(cfg.M * cfg.K, cfg.x_seed).reshape(cfg.M, cfg.K)
    if cfg.n_outliers:
        for m in range(cfg.M):
            synth.set_outliers(x[m], cfg.n_outliers, cfg.outlier_value, cfg.x_seed + 17 * m)
    wd = torch.from_numpy(w).to(dev)
    wq = dc.quantize_weights(cfg.wtype, wd)
    del wd
    xd = torch.from_numpy(x).to(dev)
    torch.cuda.synchronize()
    return wq, xd, {"w_f32": synth.digest(w), "x_f32": synth.digest(x)}


def _graph_kernel_nodes(g):
    """Kernel nodes in a captured graph (hipGraphGetNodes / hipGraphNodeGetType), or None."""
    try:
        import ctypes
        import torch
        raw = g.raw_cuda_graph()
        hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
        n = ctypes.c_size_t(0)
        if hip.hipGraphGetNodes(ctypes.c_void_p(raw), None, ctypes.byref(n)) != 0:
            return None
        nodes = (ctypes.c_void_p * n.value)()
        if hip.hipGraphGetNodes(ctypes.c_void_p(raw), nodes, ctypes.byref(n)) != 0:
            return None
        kinds = ctypes.c_int(0)
        kernels = 0
        for i in range(n.value):
            if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kinds)) == 0 and kinds.value == 0:
                kernels += 1
        return kernels
    except Exception:  # introspection is best-effort: timing does not depend on it
        return None


def time_graph(fn_steps, steps, warmup, replays, min_event_ms=1.0):
    """Capture `steps` calls into one graph and replay it; return (mean ms per step, kernels per
    step, graph replays per timed event).

    Each timed event pair brackets k back-to-back replays, k chosen so that it spans at least
    min_event_ms of GPU work whatever `steps` is (the fixed cost of one graph launch is then
    spread over k * steps steps). The events are recorded on the stream the graph replays on
    (the kernels' stream)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(warmup):  # eager warmup (also loads the kernels)
            fn_steps(i)
    torch.cuda.synchronize()
    try:
        g = torch.cuda.CUDAGraph(keep_graph=True)
    except TypeError:
        g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            fn_steps(i)
    torch.cuda.synchronize()
    kernels = _graph_kernel_nodes(g)

    def timed(k):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            e0.record(s)
            for _ in range(k):
                g.replay()
            e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    timed(1)  # warm replay
    k = max(1, int(np.ceil(min_event_ms / max(timed(1), 1e-3))))
    times = [timed(k) / (k * steps) for _ in range(replays)]
    del g
    return float(np.median(times)), (kernels / steps if kernels is not None else None), k


def load_traffic(cfg_index):
    """HBM bytes per launch of a config's dominant kernel from the committed PMC summary
    (profiles/traffic.txt: FETCH_SIZE / WRITE_SIZE in KiB per dispatch, each scaled by the
    same counter's reading for a device copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            kv = dict(tok.split("=", 1) for tok in line.split() if "=" in tok)
            if kv.get("config") == str(cfg_index):
                try:
                    return (float(kv["fetch_kib"]) * 1024 * float(kv["fetch_scale"]) +
                            float(kv["write_kib"]) * 1024 * float(kv["write_scale"]))
                except (KeyError, ValueError):
                    return None
    return None


def load_counters(cfg_index, key="config"):
    """The dominant kernel's utilisation counters from the committed PMC summary
    (profiles/counters.txt, written by --summarize-pmc from rocprofv3 --pmc runs of --profile),
    or None. key="extra" looks up an extra's line by its label instead of a config index."""
    path = os.path.join(ROOT, "profiles", "counters.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            kv = dict(tok.split("=", 1) for tok in line.split() if "=" in tok)
            if kv.get(key) == str(cfg_index):
                out = {}
                for k, v in kv.items():
                    try:
                        out[k] = float(v)
                    except ValueError:
                        out[k] = v
                out.pop(key, None)
                out["source"] = "profiles/counters.txt"
                return out
    return None


READ_VARIANTS = [(u, g) for u in (1, 2, 4, 8, 16) for g in (0, 1024, 2048)]


def read_ceiling(big, wbytes, copies, args):
    """The fastest pure read of wbytes over the same rotated copies the operator reads
    (dcq_probe_stream_read, include/dcq_probe.h), over a sweep of loads per lane and workgroup
    caps: the best any kernel that must stream the weights once can do at this size."""
    import torch
    import densecore_amd as dc
    sink = torch.zeros(64, dtype=torch.int32, device=big.device)
    best = None
    for u, g in READ_VARIANTS:
        def rd(i, u=u, g=g):
            dc.probe_stream_read(big[i % copies], wbytes, u, g, sink, stream=torch.cuda.current_stream().cuda_stream)
        ms, _, _ = time_graph(rd, args.steps, min(args.warmup, 5), args.replays)
        if best is None or ms < best[0]:
            best = (ms, u, g)
    ms, u, g = best
    return {"us": ms * 1e3, "GBps": wbytes / (ms * 1e-3) / 1e9, "frac_of_peak": wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "best_variant": f"{u} x 16-byte loads per lane, " + (f"at most {g} workgroups" if g else "one pass"),
            "variants": len(READ_VARIANTS)}


def sample_clocks_under_load(fn_steps, steps, seconds=5.0):
    """GPU clocks (amd-smi metric -c) sampled while a graph of `steps` calls of fn_steps replays
    back to back; None if amd-smi is unavailable. Returns the mean GFX clock over the XCDs and
    the memory clock, in MHz."""
    import re
    import subprocess
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            fn_steps(i)
    torch.cuda.synchronize()

    def replay():
        with torch.cuda.stream(s):
            for _ in range(4):
                g.replay()
    try:
        proc = subprocess.Popen(["amd-smi", "metric", "-c", "-g", "0"], stdout=subprocess.PIPE,
                                stderr=subprocess.DEVNULL, text=True)
    except OSError:
        return None
    t_end = time.time() + seconds
    while proc.poll() is None and time.time() < t_end:
        replay()
        torch.cuda.synchronize()
    try:
        out, _ = proc.communicate(timeout=max(1.0, t_end - time.time() + 1.0))
    except subprocess.TimeoutExpired:
        proc.kill()
        return None
    sections = re.findall(r"^\s*(GFX_\d+|MEM_\d+|UCLK_\d+|FCLK_\d+|SOCCLK_\d+):\s*\n\s*CLK:\s*([\d.]+)\s*MHz", out, re.M)
    gfx = [float(v) for k, v in sections if k.startswith("GFX")]
    mem = [float(v) for k, v in sections if k.startswith(("MEM", "UCLK"))]
    del g
    if not gfx:
        return None
    return {"gfx_mhz_mean": float(np.mean(gfx)), "gfx_mhz_min": min(gfx), "gfx_mhz_max": max(gfx),
            "mem_mhz": mem[0] if mem else None, "how": "amd-smi metric -c while the config's step graph replays"}


def bench_config(cfg, args, dev):
    import torch
    import densecore_amd as dc
    wq, x, digests = make_config_inputs(cfg, dev)
    rb = dc.row_size(cfg.wtype, cfg.K)
    wbytes = cfg.N * rb
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    big = torch.empty((copies, cfg.N, rb), dtype=torch.uint8, device=dev)
    for r in range(copies):
        big[r].copy_(wq)
    ws = torch.empty(dc.mul_mat_workspace_size(cfg.wtype, cfg.M, cfg.K), dtype=torch.uint8, device=dev)
    y = torch.empty((cfg.M, cfg.N), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def step(i):
        dc.mul_mat(cfg.wtype, big[i % copies], cfg.N, cfg.K, x, y=y, workspace=ws,
                   stream=torch.cuda.current_stream().cuda_stream)

    def kernel_only(i):
        dc.mul_mat_q(cfg.wtype, big[i % copies], cfg.N, cfg.K, ws, cfg.M, y=y,
                     stream=torch.cuda.current_stream().cuda_stream)

    step_ms, step_kernels, k_step = time_graph(step, args.steps, args.warmup, args.replays)
    if step_kernels == 1:
        # the whole step is one kernel (decode with the activation quantization fused in)
        dom_ms, dom = step_ms, "decode kernel with fused activation quantization (the whole step)"
    else:
        dc.quantize_src1(cfg.wtype, x, ws)
        torch.cuda.synchronize()
        dom_ms, _, _ = time_graph(kernel_only, args.steps, args.warmup, args.replays)
        dom = "mul_mat kernel on pre-quantized activations (dcq_mul_mat_q)"

    ops = 2.0 * cfg.M * cfg.N * cfg.K
    boundary = wbytes + cfg.M * cfg.K * 4 + cfg.M * cfg.N * 4
    out = {
        "config": cfg.index, "name": cfg.name, "type": dc.TYPE_NAMES[cfg.wtype], "M": cfg.M, "N": cfg.N, "K": cfg.K,
        "w_bytes": wbytes, "boundary_bytes": boundary, "w_copies": copies, "step_us": step_ms * 1e3,
        "kernels_per_step": step_kernels, "dominant_kernel": dom, "dominant_us": dom_ms * 1e3,
        "weight_GBps_step": wbytes / (step_ms * 1e-3) / 1e9,
        "boundary_GBps_step": boundary / (step_ms * 1e-3) / 1e9,
        "TOPS_step": ops / (step_ms * 1e-3) / 1e12, "digests": digests,
    }
    out["replays_per_timed_event"] = k_step
    traffic = load_traffic(cfg.index)
    counters = load_counters(cfg.index)
    if cfg.bound == "hbm":
        achieved = wbytes / (dom_ms * 1e-3) / 1e9
        out["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                           "algorithmic_bytes_per_launch": wbytes}
        if not args.no_read_ceiling:
            # the measured pure-read time of the same bytes: what any weight-streaming kernel can reach
            c = out["read_ceiling"] = read_ceiling(big, wbytes, copies, args)
            out["roofline"]["frac_of_read_ceiling"] = c["us"] / (dom_ms * 1e3)
    else:
        achieved = ops / (dom_ms * 1e-3) / 1e12
        out["roofline"] = {"bound": "mfma", "achieved": achieved, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                           "frac": achieved / INT8_PEAK_TOPS, "traffic": traffic,
                           "algorithmic_ops_per_launch": ops}
    if counters is not None:
        out["roofline"]["counters"] = counters
    if cfg.index in (HEADLINE, 5) and not args.no_clocks:
        out["clocks"] = sample_clocks_under_load(step, args.steps)
    del big, ws, y, x, wq
    torch.cuda.empty_cache()
    return out


def bench_gate_up(cfg, args, dev):
    """The SwiGLU gate/up pair at a config's shape (two weights of the same type and shape
    sharing X): one dcq_ffn_gate_up call against two dcq_mul_mat calls (the reference's two
    ggml_mul_mat nodes, without its separate silu and mul). Weight GB/s counts both matrices."""
    import torch
    import densecore_amd as dc
    wq, x, _ = make_config_inputs(cfg, dev)
    rb = dc.row_size(cfg.wtype, cfg.K)
    wbytes = cfg.N * rb
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    bg = torch.empty((copies, cfg.N, rb), dtype=torch.uint8, device=dev)
    bu = torch.empty((copies, cfg.N, rb), dtype=torch.uint8, device=dev)
    for r in range(copies):
        bg[r].copy_(wq)
        bu[r].copy_(wq.roll(1, 0))  # a different matrix of the same statistics
    ws = torch.empty(max(dc.ffn_gate_up_workspace_size(cfg.wtype, cfg.M, cfg.N, cfg.K),
                         dc.mul_mat_workspace_size(cfg.wtype, cfg.M, cfg.K)), dtype=torch.uint8, device=dev)
    y = torch.empty((cfg.M, cfg.N), dtype=torch.float32, device=dev)
    u = torch.empty_like(y)
    torch.cuda.synchronize()

    def fused(i):
        dc.ffn_gate_up(cfg.wtype, bg[i % copies], bu[i % copies], cfg.N, cfg.K, x, y=y, workspace=ws,
                       stream=torch.cuda.current_stream().cuda_stream)

    def separate(i):
        s = torch.cuda.current_stream().cuda_stream
        dc.mul_mat(cfg.wtype, bg[i % copies], cfg.N, cfg.K, x, y=y, workspace=ws, stream=s)
        dc.mul_mat(cfg.wtype, bu[i % copies], cfg.N, cfg.K, x, y=u, workspace=ws, stream=s)

    f_ms, f_k, _ = time_graph(fused, args.steps, args.warmup, args.replays)
    s_ms, s_k, _ = time_graph(separate, args.steps, args.warmup, args.replays)
    del bg, bu, ws, y, u, x, wq
    torch.cuda.empty_cache()
    return {"shape": f"config {cfg.index}: {dc.TYPE_NAMES[cfg.wtype]} M={cfg.M} N={cfg.N} K={cfg.K}, two weights",
            "fused_us": f_ms * 1e3, "fused_kernels": f_k, "separate_us": s_ms * 1e3, "separate_kernels": s_k,
            "fused_weight_GBps": 2 * wbytes / (f_ms * 1e-3) / 1e9,
            "separate_weight_GBps": 2 * wbytes / (s_ms * 1e-3) / 1e9}


def bench_qkv(args, dev, K=2560, parts=(4096, 1024, 1024), wtype=None):
    """The Q/K/V projections of one Qwen3-4B layer at decode (M = 1, Q4_K), which share X
    (core/src/inference.cpp:1128-1130): three dcq_mul_mat calls against one call over the three
    weights loaded back to back (same type and K, so one row stride). Weight GB/s counts all three."""
    import torch
    import densecore_amd as dc
    wtype = dc.TYPE_Q4_K if wtype is None else wtype
    rb = dc.row_size(wtype, K)
    n_all = sum(parts)
    w = torch.randn((n_all, K), device=dev) * 0.02
    wq = dc.quantize_weights(wtype, w)
    del w
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / (n_all * rb))))
    big = torch.empty((copies, n_all, rb), dtype=torch.uint8, device=dev)
    for r in range(copies):
        big[r].copy_(wq)
    x = torch.randn((1, K), device=dev)
    y = torch.empty((1, n_all), dtype=torch.float32, device=dev)
    ys = [torch.empty((1, n), dtype=torch.float32, device=dev) for n in parts]
    ws = torch.empty(max(dc.mul_mat_workspace_size(wtype, 1, K), 256), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def separate(i):
        s, r0 = torch.cuda.current_stream().cuda_stream, 0
        for n, yy in zip(parts, ys):
            dc.mul_mat(wtype, big[i % copies][r0:r0 + n], n, K, x, y=yy, workspace=ws, stream=s)
            r0 += n

    def fused(i):
        dc.mul_mat(wtype, big[i % copies], n_all, K, x, y=y, workspace=ws,
                   stream=torch.cuda.current_stream().cuda_stream)

    s_ms, s_k, _ = time_graph(separate, args.steps, args.warmup, args.replays)
    f_ms, f_k, _ = time_graph(fused, args.steps, args.warmup, args.replays)
    del big, wq
    torch.cuda.empty_cache()
    return {"shape": f"Q4_K q/k/v {list(parts)} x K={K}, M=1", "separate_us": s_ms * 1e3, "separate_kernels": s_k,
            "one_call_us": f_ms * 1e3, "one_call_kernels": f_k,
            "one_call_weight_GBps": n_all * rb / (f_ms * 1e-3) / 1e9}


def bench_residual(args, dev, wtype, N=2560, K=9728):
    """The FFN down projection of Qwen3-4B at decode with its residual connection
    (core/src/inference.cpp:1799-1800): dcq_mul_mat followed by torch's add, against one
    dcq_mul_mat_add call with the residual in place (R is Y)."""
    import torch
    import densecore_amd as dc
    rb = dc.row_size(wtype, K)
    w = torch.randn((N, K), device=dev) * 0.02
    wq = dc.quantize_weights(wtype, w)
    del w
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / (N * rb))))
    big = torch.empty((copies, N, rb), dtype=torch.uint8, device=dev)
    for r in range(copies):
        big[r].copy_(wq)
    x = torch.randn((1, K), device=dev)
    resid = torch.randn((1, N), device=dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    ws = torch.empty(max(dc.mul_mat_add_workspace_size(wtype, 1, N, K), 256), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def separate(i):
        dc.mul_mat(wtype, big[i % copies], N, K, x, y=y, workspace=ws, stream=torch.cuda.current_stream().cuda_stream)
        resid.add_(y)

    def fused(i):
        dc.mul_mat_add(wtype, big[i % copies], N, K, x, resid, y=resid, workspace=ws,
                       stream=torch.cuda.current_stream().cuda_stream)

    s_ms, s_k, _ = time_graph(separate, args.steps, args.warmup, args.replays)
    f_ms, f_k, _ = time_graph(fused, args.steps, args.warmup, args.replays)
    del big, wq
    torch.cuda.empty_cache()
    return {"shape": f"{dc.TYPE_NAMES[wtype]} ffn_down {N} x K={K}, M=1, residual in place",
            "mul_mat_then_add_us": s_ms * 1e3, "mul_mat_then_add_kernels": s_k,
            "mul_mat_add_us": f_ms * 1e3, "mul_mat_add_kernels": f_k}


def bench_kv_attention(args, dev, ct, n_tokens=1, n_past=4095, n_layer=36, n_head=32, n_head_kv=8, hd=128):
    """Attention of one layer over DenseCore's paged KV cache (dcq_kv_attention) at Qwen3-4B's
    heads (32 query, 8 KV, head_dim 128). Each step attends the next of n_layer layers, so the
    arenas (K and V of every layer, more than the 256 MB MALL) stream from HBM. Bytes per step:
    the K and V history of that layer plus the query, current rows and output."""
    import torch
    import densecore_amd as dc
    n_pos = n_past + n_tokens
    n_blocks = (n_pos + 15) // 16
    cache = dc.PagedKVCache(ct, n_blocks, n_layer, n_head_kv, hd, device=dev)
    table = torch.arange(n_blocks, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    row = n_head_kv * hd
    if n_past:
        hist = torch.randn((n_past, row), generator=g, device=dev)
        for layer in range(n_layer):
            cache.write("k", layer, table, 0, hist)
            cache.write("v", layer, table, 0, hist.roll(1, 1))
    q = torch.randn((n_tokens, n_head * hd), generator=g, device=dev)
    kc = torch.randn((n_tokens, row), generator=g, device=dev)
    vc = torch.randn((n_tokens, row), generator=g, device=dev)
    out = torch.empty_like(q)
    need = dc.kv_attention_workspace_size(n_head, n_head_kv, hd, n_tokens, n_past)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def step(i):
        cache.attention(i % n_layer, table, q, kc, vc, n_past, 1.0 / hd ** 0.5, out=out, workspace=ws,
                        stream=torch.cuda.current_stream().cuda_stream)

    ms, kern, _ = time_graph(step, args.steps, args.warmup, args.replays)
    hist_bytes = 2 * n_past * cache.slot_bytes
    io_bytes = 4 * (2 * q.numel() + kc.numel() + vc.numel())
    pairs = n_tokens * n_past + n_tokens * (n_tokens + 1) // 2  # (query, visible key) pairs
    flops = 4 * pairs * n_head * hd
    del cache, ws
    torch.cuda.empty_cache()
    names = {dc.TYPE_F32: "F32", dc.TYPE_F16: "F16", dc.TYPE_Q8_0: "Q8_0"}
    return {"shape": f"{names[ct]} cache, {n_head}/{n_head_kv} heads x {hd}, n_tokens={n_tokens}, "
                     f"n_past={n_past}, {n_layer} layers rotated",
            "us": ms * 1e3, "kernels": kern, "bytes": hist_bytes + io_bytes,
            "GBps": (hist_bytes + io_bytes) / (ms * 1e-3) / 1e9, "TFLOPs": flops / (ms * 1e-3) / 1e12,
            # decode streams the history (HBM-bound); a long prefill is fp32 arithmetic on the VALU
            "roofline": ({"bound": "hbm", "peak": 8000.0, "unit": "GB/s",
                          "frac": (hist_bytes + io_bytes) / (ms * 1e-3) / 1e9 / 8000.0} if n_tokens == 1 else
                         {"bound": "fp32", "peak": 157.3, "unit": "TFLOP/s",
                          "frac": flops / (ms * 1e-3) / 1e12 / 157.3})}


def random_weights(dev, wtype, N, K, copies, seed):
    """copies x N rows of valid random quants of `wtype` with small positive fp16 scales (d =
    0.0004, Q4_K / Q5_K dmin = 0.0002): the kernels' work does not depend on the values, and
    quantizing hundreds of MB of floats would dominate the run."""
    import torch
    import densecore_amd as dc
    rb = dc.row_size(wtype, K)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    big = torch.randint(0, 256, (copies, N, rb), dtype=torch.uint8, device=dev, generator=g)
    bs = {dc.TYPE_Q8_0: 34, dc.TYPE_Q4_0: 18, dc.TYPE_Q4_K: 144, dc.TYPE_Q5_K: 176, dc.TYPE_Q6_K: 210}[wtype]
    blocks = big.view(copies, N, rb // bs, bs)

    def f16(v):
        return torch.from_numpy(np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8).copy()).to(dev)

    if wtype == dc.TYPE_Q6_K:
        blocks[..., 208:210] = f16(0.0004)
    else:
        blocks[..., 0:2] = f16(0.0004)
        if wtype in (dc.TYPE_Q4_K, dc.TYPE_Q5_K):
            blocks[..., 2:4] = f16(0.0002)
    return big


def bench_lm_head(args, dev, wtype, K, M, N=151936):
    """The LM head (ggml_mul_mat(output, cur), core/src/inference.cpp:1817), the largest weight
    stream of a decode step: Qwen3's 151,936-token vocabulary, random valid quants (the kernels do
    not depend on their values), W rotated over >= 1 GiB, with the pure-read time of the same bytes."""
    import torch
    import densecore_amd as dc
    rb = dc.row_size(wtype, K)
    wbytes = N * rb
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    big = random_weights(dev, wtype, N, K, copies, 17)
    g = torch.Generator(device=dev)
    g.manual_seed(18)
    x = torch.randn((M, K), device=dev, generator=g)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(dc.mul_mat_workspace_size(wtype, M, K), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def step(i):
        dc.mul_mat(wtype, big[i % copies], N, K, x, y=y, workspace=ws, stream=torch.cuda.current_stream().cuda_stream)

    ms, kern, _ = time_graph(step, args.steps, args.warmup, args.replays)
    out = {"shape": f"{dc.TYPE_NAMES[wtype]} lm head N={N} K={K}, M={M}", "w_bytes": wbytes, "us": ms * 1e3,
           "kernels": kern, "weight_GBps": wbytes / (ms * 1e-3) / 1e9,
           "frac_of_peak": wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    if not args.no_read_ceiling:
        c = read_ceiling(big.view(copies, -1), wbytes, copies, args)
        out["read_ceiling_us"] = c["us"]
        out["frac_of_read_ceiling"] = c["us"] / (ms * 1e3)
    counters = load_counters(f"lm_head_{dc.TYPE_NAMES[wtype].lower()}_m{M}", key="extra")
    if counters is not None:
        out["counters"] = counters
    del big, ws, y, x
    torch.cuda.empty_cache()
    return out


# Batched decode (ggml MUL_MAT at small M > 1, core/src/inference.cpp:1049-1063): the batch kernels
# (and split-K) at ffn shapes of Llama 3.2 1B, 2048 x 8192 (ffn_down, few weight rows) and 8192 x 2048
BATCHED_SHAPES = [(dc_type, M, N, K) for dc_type in ("Q8_0", "Q4_K", "Q6_K")
                  for (M, N, K) in ((16, 2048, 8192), (64, 2048, 8192), (16, 8192, 2048))]


def bench_batched_decode(args, dev, tname, M, N, K):
    """One dcq_mul_mat step (activation quantization + product, + the split-K sum where used) at a
    batched-decode shape, W rotated like the configs; weight GB/s of the step."""
    import torch
    import densecore_amd as dc
    wtype = {"Q8_0": dc.TYPE_Q8_0, "Q4_K": dc.TYPE_Q4_K, "Q6_K": dc.TYPE_Q6_K}[tname]
    rb = dc.row_size(wtype, K)
    wbytes = N * rb
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    big = random_weights(dev, wtype, N, K, copies, 31)
    g = torch.Generator(device=dev)
    g.manual_seed(32)
    x = torch.randn((M, K), device=dev, generator=g)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(dc.mul_mat_workspace_size(wtype, M, K), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def step(i):
        dc.mul_mat(wtype, big[i % copies], N, K, x, y=y, workspace=ws, stream=torch.cuda.current_stream().cuda_stream)

    step_ms, kern, _ = time_graph(step, max(10, args.steps // 4), args.warmup, args.replays)
    return {"shape": f"{tname} M={M} N={N} K={K}", "step_us": step_ms * 1e3, "kernels": kern,
            "weight_GBps": wbytes / (step_ms * 1e-3) / 1e9, "TOPS": 2.0 * M * N * K / (step_ms * 1e-3) / 1e12}


def bench_kquant_prefill(args, dev, wtype, M=2048, N=8192, K=2048):
    """A K-quant prompt projection (ggml MUL_MAT at M > 1, core/src/inference.cpp:1049-1063,
    1794-1797) at config 5's shape with Q4_K / Q6_K weights (random valid quants, W rotated like
    the configs): the whole step (activation quantization + product) and the product kernel alone
    on the pre-quantized activation, against the int8 MFMA peak."""
    import torch
    import densecore_amd as dc
    rb = dc.row_size(wtype, K)
    wbytes = N * rb
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    big = random_weights(dev, wtype, N, K, copies, 29)
    g = torch.Generator(device=dev)
    g.manual_seed(30)
    x = torch.randn((M, K), device=dev, generator=g)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(dc.mul_mat_workspace_size(wtype, M, K), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def step(i):
        dc.mul_mat(wtype, big[i % copies], N, K, x, y=y, workspace=ws, stream=torch.cuda.current_stream().cuda_stream)

    def kernel_only(i):
        dc.mul_mat_q(wtype, big[i % copies], N, K, ws, M, y=y, stream=torch.cuda.current_stream().cuda_stream)

    steps = max(5, args.steps // 10)
    step_ms, kern, _ = time_graph(step, steps, args.warmup, args.replays)
    dc.quantize_src1(wtype, x, ws)
    torch.cuda.synchronize()
    k_ms, _, _ = time_graph(kernel_only, steps, args.warmup, args.replays)
    ops = 2.0 * M * N * K
    out = {"shape": f"{dc.TYPE_NAMES[wtype]} M={M} N={N} K={K}", "step_us": step_ms * 1e3, "kernels": kern,
           "kernel_us": k_ms * 1e3, "TOPS_kernel": ops / (k_ms * 1e-3) / 1e12,
           "frac_of_int8_peak": ops / (k_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS}
    counters = load_counters(f"prefill_{dc.TYPE_NAMES[wtype].lower()}", key="extra")
    if counters is not None:
        out["counters"] = counters
    del big, ws, y, x
    torch.cuda.empty_cache()
    return out


# The quantize tool's other output types (core/src/quantize.cpp:71-78: Q4_0, its default, and
# Q5_K for Q5_K_M) at the shapes of configs 2 (decode), 4 (batched) and 5 (prefill)
TOOL_TYPE_SHAPES = [(t, M, N, K) for t in ("Q4_0", "Q5_K")
                    for (M, N, K) in ((1, 9728, 2560), (64, 8192, 2048), (2048, 8192, 2048))]


def bench_tool_type(args, dev, tname, M, N, K):
    """One dcq_mul_mat step with Q4_0 or Q5_K weights (random valid quants, W rotated like the
    configs): weight GB/s against 8 TB/s and the pure-read time of the same bytes at M = 1, int8
    TOPS against the int8 MFMA peak otherwise."""
    import torch
    import densecore_amd as dc
    wtype = getattr(dc, "TYPE_" + tname)
    rb = dc.row_size(wtype, K)
    wbytes = N * rb
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    big = random_weights(dev, wtype, N, K, copies, 41)
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    x = torch.randn((M, K), device=dev, generator=g)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(dc.mul_mat_workspace_size(wtype, M, K), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def step(i):
        dc.mul_mat(wtype, big[i % copies], N, K, x, y=y, workspace=ws, stream=torch.cuda.current_stream().cuda_stream)

    ms, kern, _ = time_graph(step, max(10, args.steps // (4 if M < 2048 else 10)), args.warmup, args.replays)
    out = {"shape": f"{tname} M={M} N={N} K={K}", "step_us": ms * 1e3, "kernels": kern, "w_bytes": wbytes,
           "weight_GBps": wbytes / (ms * 1e-3) / 1e9, "frac_of_hbm_peak": wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "TOPS": 2.0 * M * N * K / (ms * 1e-3) / 1e12,
           "frac_of_int8_peak": 2.0 * M * N * K / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS}
    if M == 1 and not args.no_read_ceiling:
        c = read_ceiling(big.view(copies, -1), wbytes, copies, args)
        out["read_ceiling_us"] = c["us"]
        out["frac_of_read_ceiling"] = c["us"] / (ms * 1e3)
    del big, ws, y, x
    torch.cuda.empty_cache()
    return out


# Row-split Q8_0 (the load-time repack, dcq_repack_weights) against the GGUF Q8_0 rows: config 5's
# prefill, config 4's batched shape and config 1's decode shape
ROW_SPLIT_SHAPES = [(2048, 8192, 2048), (64, 8192, 2048), (1, 3072, 1024)]


def bench_q8_0_row_split(args, dev, M, N, K):
    """One dcq_mul_mat step on Q8_0 rows and on the same rows repacked (random valid quants, W rotated
    like the configs), alternating the two layouts twice; the repack itself is load-time work,
    outside the timed steps."""
    import torch
    import densecore_amd as dc
    q8, rs = dc.TYPE_Q8_0, dc.TYPE_Q8_0_RS
    wbytes = N * dc.row_size(q8, K)
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
    big8 = random_weights(dev, q8, N, K, copies, 43)
    bigr = torch.empty((copies, N, dc.row_size(rs, K)), dtype=torch.uint8, device=dev)
    for r in range(copies):
        dc.repack_weights(q8, big8[r], N, K, rs, out=bigr[r])
    g = torch.Generator(device=dev)
    g.manual_seed(44)
    x = torch.randn((M, K), device=dev, generator=g)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(dc.mul_mat_workspace_size(q8, M, K), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    steps = max(10, args.steps // (4 if M < 2048 else 10))
    best = {}
    for _ in range(2):
        for t, big in ((q8, big8), (rs, bigr)):
            def step(i, t=t, big=big):
                dc.mul_mat(t, big[i % copies], N, K, x, y=y, workspace=ws, stream=torch.cuda.current_stream().cuda_stream)
            ms, _, _ = time_graph(step, steps, args.warmup, args.replays)
            best[t] = min(best.get(t, float("inf")), ms)
    out = {"shape": f"Q8_0 M={M} N={N} K={K}", "gguf_step_us": best[q8] * 1e3, "row_split_step_us": best[rs] * 1e3,
           "row_split_speedup": best[q8] / best[rs], "w_bytes": wbytes}
    del big8, bigr, ws, y, x
    torch.cuda.empty_cache()
    return out


def bench_gguf_load(args, dev, mib=512):
    """GGUF ingest: a file of Q4_K tensors (mib MiB, in the page cache after it is written) loaded
    tensor by tensor into HBM with dcq_gguf_load_tensor; host-to-device GB/s (PCIe bound)."""
    import tempfile
    import torch
    import densecore_amd as dc
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from gguf_writer import write_gguf
    rb = dc.row_size(dc.TYPE_Q4_K, 4096)
    rows = (mib << 20) // (8 * rb)
    rng = np.random.default_rng(5)
    payload = rng.integers(0, 256, size=rows * rb, dtype=np.uint8).tobytes()
    tensors = [(f"blk.{i}.ffn_up.weight", dc.TYPE_Q4_K, [4096, rows], payload) for i in range(8)]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "bench.gguf")
        write_gguf(path, [], tensors)
        dst = torch.empty(len(payload), dtype=torch.uint8, device=dev)
        with dc.GGUF(path) as g:
            g.load(0, dst=dst)  # warm
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(len(tensors)):
                g.load(i, dst=dst)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
    total = len(payload) * len(tensors)
    return {"bytes": total, "tensors": len(tensors), "seconds": dt, "GBps": total / dt / 1e9,
            "note": "file in the page cache; read into two pinned 32 MB chunks, each copied while the next is read"}


def bench_weight_quantizer(args, dev):
    """dcq_quantize_weights (ggml_quantize_chunk's algorithms on the GPU) at the weight shapes of
    BASELINE configs 1-3 (their types), and Q4_0 / Q5_K at config 2's: ms per matrix and GB/s of
    fp32 input (load-time work, off the hot path)."""
    import torch
    import densecore_amd as dc
    from densecore_amd import synth
    out = {}
    cases = [(dc.by_index(ci), dc.by_index(ci).wtype) for ci in (1, 2, 3)]
    cases += [(dc.by_index(2), dc.TYPE_Q4_0), (dc.by_index(2), dc.TYPE_Q5_K)]
    for cfg, wtype in cases:
        w = torch.from_numpy(synth.normal(cfg.N * cfg.K, cfg.w_seed, 0.0, cfg.w_std).reshape(cfg.N, cfg.K)).to(dev)
        q = dc.quantize_weights(wtype, w)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        e0.record()
        for _ in range(reps):
            dc.quantize_weights(wtype, w, out=q)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[dc.TYPE_NAMES[wtype].lower()] = {"shape": f"{cfg.N}x{cfg.K}", "ms": ms,
                                             "GBps_fp32_in": cfg.N * cfg.K * 4 / (ms * 1e-3) / 1e9}
    return out


def profile_config(cfg, args, dev):
    """Eager steps of one config (counter collection needs plain dispatches)."""
    import torch
    import densecore_amd as dc
    wq, x, _ = make_config_inputs(cfg, dev)
    rb = dc.row_size(cfg.wtype, cfg.K)
    copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / (cfg.N * rb))))
    big = torch.empty((copies, cfg.N, rb), dtype=torch.uint8, device=dev)
    for r in range(copies):
        big[r].copy_(wq)
    ws = torch.empty(dc.mul_mat_workspace_size(cfg.wtype, cfg.M, cfg.K), dtype=torch.uint8, device=dev)
    y = torch.empty((cfg.M, cfg.N), dtype=torch.float32, device=dev)
    for i in range(args.warmup + args.steps):
        dc.mul_mat(cfg.wtype, big[i % copies], cfg.N, cfg.K, x, y=y, workspace=ws)
    torch.cuda.synchronize()
    print(f"# profiled config {cfg.index}: {args.warmup + args.steps} eager steps", file=sys.stderr, flush=True)
    del big, ws, y, x, wq
    torch.cuda.empty_cache()


# Extras whose kernels the counter passes cover: (label, kernel, weight type, M, N, K). The LM heads
# share their kernels with configs 1 and 3 and are told apart by grid size (PROFILED below).
PROFILE_EXTRAS = [("lm_head_q8_0_m1", "decode_q8_0_kernel", "Q8_0", 1, 151936, 1024),
                  ("lm_head_q6_k_m1", "decode_q6k_mfma_kernel", "Q6_K", 1, 151936, 2560),
                  ("prefill_q4_k", "prefill_q4_k_kernel", "Q4_K", 2048, 8192, 2048),
                  ("prefill_q6_k", "prefill_q6_k_kernel", "Q6_K", 2048, 8192, 2048)]


def profile_extras(args, dev):
    """Eager calls of the PROFILE_EXTRAS shapes (random valid quants, W rotated like the configs)."""
    import torch
    import densecore_amd as dc
    for label, _, tname, M, N, K in PROFILE_EXTRAS:
        wt = getattr(dc, "TYPE_" + tname)
        copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / (N * dc.row_size(wt, K)))))
        big = random_weights(dev, wt, N, K, copies, 41)
        x = torch.randn((M, K), device=dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        ws = torch.empty(dc.mul_mat_workspace_size(wt, M, K), dtype=torch.uint8, device=dev)
        for i in range(args.warmup + args.steps):
            dc.mul_mat(wt, big[i % copies], N, K, x, y=y, workspace=ws)
        torch.cuda.synchronize()
        print(f"# profiled {label}: {args.warmup + args.steps} eager calls", file=sys.stderr, flush=True)
        del big, ws, y, x
        torch.cuda.empty_cache()


def profile_read(args, dev):
    """Eager pure-read launches (dcq_probe_stream_read) at each config's weight size over the same
    rotation as the operator, every sweep variant, for rocprofv3 --kernel-trace: the per-size
    read ceiling in the committed profile."""
    import torch
    import densecore_amd as dc
    wanted = [int(c) for c in args.configs.split(",") if c.strip()]
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    for cfg in dc.CONFIGS:
        if cfg.index not in wanted:
            continue
        wbytes = cfg.N * dc.row_size(cfg.wtype, cfg.K)
        copies = max(2, int(np.ceil(args.rotate_mb * 2 ** 20 / wbytes)))
        big = torch.empty((copies, wbytes), dtype=torch.uint8, device=dev)
        for u, g in READ_VARIANTS:
            for i in range(args.warmup + args.steps):
                dc.probe_stream_read(big[i % copies], wbytes, u, g, sink)
        torch.cuda.synchronize()
        print(f"# read probe: config {cfg.index}, {wbytes} bytes, {len(READ_VARIANTS)} variants x "
              f"{args.warmup + args.steps} launches", file=sys.stderr, flush=True)
        del big
        torch.cuda.empty_cache()


def summarize_read(path, configs, launches):
    """profiles/read_ceiling.txt lines from the rocprofv3 kernel trace of a --profile-read run:
    per config, the mean duration of each read variant (its first two launches skipped) and the
    best. Dispatches are assigned to configs and variants by their order, as --profile-read issues
    them (configs ascending, READ_VARIANTS in order, `launches` launches each)."""
    import csv
    import densecore_amd as dc
    rows = [r for r in csv.DictReader(open(path)) if "stream_read_kernel" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    wanted = [c for c in dc.CONFIGS if c.index in configs]
    per_cfg = len(READ_VARIANTS) * launches
    if len(rows) != per_cfg * len(wanted):
        raise SystemExit(f"{len(rows)} probe dispatches in the trace, expected {per_cfg * len(wanted)}")
    lines = ["# config bytes | mean us per variant (loads per lane x workgroup cap; 0 = one pass) | best"]
    for ci, cfg in enumerate(wanted):
        wbytes = cfg.N * dc.row_size(cfg.wtype, cfg.K)
        means = []
        for vi, (u, g) in enumerate(READ_VARIANTS):
            sub = rows[ci * per_cfg + vi * launches: ci * per_cfg + (vi + 1) * launches][2:]
            means.append(float(np.mean([(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in sub])))
        b = int(np.argmin(means))
        lines.append(f"config={cfg.index} bytes={wbytes} " +
                     " ".join(f"u{u}g{g}={m:.2f}" for (u, g), m in zip(READ_VARIANTS, means)) +
                     f" best_us={means[b]:.2f} best_GBps={wbytes / means[b] / 1e3:.0f} "
                     f"best=u{READ_VARIANTS[b][0]}g{READ_VARIANTS[b][1]}")
    return "\n".join(lines)


# the kernel that dominates each config's step (for --summarize-pmc)
DOMINANT = {1: "decode_q8_0_kernel", 2: "decode_kq_kernel", 3: "decode_q6k_lds_kernel", 4: "batch_q4k_kernel",
            5: "prefill_q8_0_kernel"}
# counter summary lines: (label, kernel, smallest and largest grid in threads). The Q8_0 LM head
# shares its kernel with config 1 and is told apart by grid size: the configs' decode grids stay
# below 300 k threads, the Q8_0 LM head's (151936 rows) is above. The other extras' kernels are
# their own.
LM_GRID = 300_000
_SHARED = {k for _, k, *_ in PROFILE_EXTRAS} & set(DOMINANT.values())
PROFILED = ([(f"config={i}", k, 0, LM_GRID if k in _SHARED else 1 << 62) for i, k in sorted(DOMINANT.items())] +
            [(f"extra={lab}", k, LM_GRID if k in _SHARED else 0, 1 << 62) for lab, k, *_ in PROFILE_EXTRAS])


def summarize_traffic(fetch_csv, write_csv):
    """profiles/traffic.txt lines: per PROFILED kernel, the median over its dispatches (the first two
    of each skipped) of FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled by what the same
    counter reads for the run's last dispatch, calibration_copy's device copy of 64 MiB (read and
    written once), against the algorithmic bytes (quantized W + fp32 X + fp32 Y) of one launch."""
    import csv
    import collections
    import densecore_amd as dc

    def per_dispatch(path, counter):
        rows = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                rows[int(r["Dispatch_Id"])] = (r["Kernel_Name"], int(r["Grid_Size"]), float(r["Counter_Value"]))
        return rows

    fetch, write = per_dispatch(fetch_csv, "FETCH_SIZE"), per_dispatch(write_csv, "WRITE_SIZE")
    copy_kib = (64 << 20) / 1024
    fetch_scale = copy_kib / fetch[max(fetch)][2]
    write_scale = copy_kib / write[max(write)][2]
    shapes = {f"config={c.index}": (c.wtype, c.M, c.N, c.K) for c in dc.CONFIGS}
    shapes.update({f"extra={lab}": (getattr(dc, "TYPE_" + t), M, N, K) for lab, _, t, M, N, K in PROFILE_EXTRAS})
    lines = [f"# scale: the calibration copy of 64 MiB reads FETCH_SIZE={fetch[max(fetch)][2]:.1f} KiB and "
             f"WRITE_SIZE={write[max(write)][2]:.1f} KiB: fetch_scale={fetch_scale:.4f}, write_scale={write_scale:.4f}",
             "# traffic (bytes) = fetch_kib*1024*fetch_scale + write_kib*1024*write_scale; medians over each "
             "kernel's dispatches after its first two"]
    for label, kname, gmin, gmax in PROFILED:
        vals = collections.defaultdict(list)
        for name, table in (("fetch", fetch), ("write", write)):
            for d in sorted(table):
                k, grid, v = table[d]
                if kname in k and gmin <= grid < gmax:
                    vals[name].append(v)
        if not vals["fetch"] or not vals["write"]:
            continue
        f_kib = float(np.median(vals["fetch"][2:] or vals["fetch"]))
        w_kib = float(np.median(vals["write"][2:] or vals["write"]))
        wt, M, N, K = shapes[label]
        algo = N * dc.row_size(wt, K) + M * K * 4 + M * N * 4
        traffic = f_kib * 1024 * fetch_scale + w_kib * 1024 * write_scale
        lines.append(f"{label} kernel={kname} fetch_kib={f_kib:.1f} write_kib={w_kib:.1f} fetch_scale={fetch_scale:.4f} "
                     f"write_scale={write_scale:.4f} traffic_bytes={traffic:.0f} algorithmic_bytes={algo}")
    return "\n".join(lines)


def summarize_pmc(paths):
    """profiles/counters.txt lines from rocprofv3 --pmc counter_collection.csv files of --profile
    runs (one pass per file; passes are joined by kernel name). Per config, the medians over that
    kernel's dispatches of:
      mfma_busy_pct  = 100 * sum SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs * GRBM_GUI_ACTIVE per XCD)
                       (rocprofv3's MfmaUtil)
      valu_busy_pct  = 100 * sum SQ_ACTIVE_INST_VALU / (CUs * GRBM_GUI_ACTIVE per XCD)
                       (rocprofv3's VALUBusy: quad-cycles over the CU's 4 SIMDs)
      valu_per_mfma  = SQ_INSTS_VALU / SQ_INSTS_MFMA (SQ_INSTS_VALU counts the MFMAs too)
      coexec_pct     = 100 * SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES
    GRBM_GUI_ACTIVE is reported summed over the XCDs and covers the counting window around the
    dispatch, which adds a few microseconds to short kernels: their busy percentages are lower
    bounds."""
    import csv
    import collections
    per = collections.defaultdict(dict)  # (file, dispatch) -> counters
    names = {}
    agent = {"simds": 1024, "cus": 256, "xcds": 8}
    for p in paths:
        info = os.path.join(os.path.dirname(p), os.path.basename(p).replace("counter_collection", "agent_info"))
        if os.path.exists(info):
            for a in csv.DictReader(open(info)):
                if a.get("Agent_Type") == "GPU":
                    agent = {"simds": int(a["Simd_Count"]), "cus": int(a["Cu_Count"]), "xcds": int(a["Num_Xcc"])}
        for r in csv.DictReader(open(p)):
            key = (p, r["Dispatch_Id"])
            per[key][r["Counter_Name"]] = float(r["Counter_Value"])
            names[key] = (r["Kernel_Name"], int(r["Grid_Size"]))
    lines = [f"# per-dispatch medians; {agent['simds']} SIMDs, {agent['cus']} CUs, {agent['xcds']} XCDs"]
    for label, kname, gmin, gmax in PROFILED:
        rows = collections.defaultdict(list)
        for key, cnt in per.items():
            if kname in names[key][0] and gmin <= names[key][1] < gmax:
                for c, v in cnt.items():
                    rows[c].append(v)
        if not rows:
            continue
        med = {c: float(np.median(v)) for c, v in rows.items()}
        n_disp = max(len(v) for v in rows.values())
        gui = med.get("GRBM_GUI_ACTIVE")
        kv = [label, f"kernel={kname}", f"samples={n_disp}"]
        if gui:
            gui_x = gui / agent["xcds"]
            kv.append(f"gui_cycles_per_xcd={gui_x:.0f}")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
                kv.append(f"mfma_busy_pct={100 * med['SQ_VALU_MFMA_BUSY_CYCLES'] / (agent['simds'] * gui_x):.2f}")
            if "SQ_ACTIVE_INST_VALU" in med:
                kv.append(f"valu_busy_pct={100 * med['SQ_ACTIVE_INST_VALU'] / (agent['cus'] * gui_x):.2f}")
        if med.get("SQ_INSTS_MFMA"):
            kv.append(f"valu_per_mfma={med['SQ_INSTS_VALU'] / med['SQ_INSTS_MFMA']:.2f}")
        if med.get("SQ_VALU_MFMA_BUSY_CYCLES") and "SQ_VALU_MFMA_COEXEC_CYCLES" in med:
            kv.append(f"coexec_pct={100 * med['SQ_VALU_MFMA_COEXEC_CYCLES'] / med['SQ_VALU_MFMA_BUSY_CYCLES']:.2f}")
        if med.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_ANY" in med:
            # share of the waves' lifetime spent in s_waitcnt (loads, LDS, scalar memory)
            kv.append(f"wait_inst_pct={100 * med['SQ_WAIT_INST_ANY'] / med['SQ_WAVE_CYCLES']:.2f}")
        for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_I8", "SQ_VALU_MFMA_BUSY_CYCLES",
                  "SQ_ACTIVE_INST_VALU", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES",
                  "SQ_WAIT_INST_ANY", "SQ_INSTS_SALU"):
            if c in med:
                kv.append(f"{c}={med[c]:.6g}")
        lines.append(" ".join(kv))
    return "\n".join(lines)


def calibration_copy(dev, nbytes=64 << 20):
    """One device-to-device copy of nbytes: the known-size kernel the traffic counters are scaled by."""
    import torch
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"# calibration copy: {nbytes} bytes read, {nbytes} bytes written", file=sys.stderr, flush=True)


def host_cpu_info():
    """Model name (lscpu), logical CPUs in this process's affinity mask, and one logical CPU per
    physical core among them (sysfs topology)."""
    import subprocess
    from oracle import oracle as O
    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), "")
    except (OSError, subprocess.SubprocessError):
        pass
    cpus, logical = O.physical_cpus()
    return {"model": model, "logical_cpus": logical, "physical_cores": len(cpus), "cpus": cpus,
            "nproc": os.cpu_count()}


def cpu_baseline(cfg, seconds, threads, host):
    """The reference CPU path restated with SIMD int8 dots (oracle/dcq_cpu_simd.c: quantize X once,
    then row-partitioned AVX2 / AVX-512 VNNI vec_dots on a persistent pool pinned one worker per
    physical core, as core/src/worker.cpp:63-77 sizes the reference's pool), on the full config:
    3 warm-up runs, then the median of at least 10 runs (more while under `seconds`)."""
    from oracle import oracle as O
    from densecore_amd import synth
    w = synth.normal(cfg.N * cfg.K, cfg.w_seed, 0.0, cfg.w_std).reshape(cfg.N, cfg.K)
    wq = O.quantize_matrix(cfg.wtype, w)
    x = synth.normal(cfg.M * cfg.K, cfg.x_seed).reshape(cfg.M, cfg.K)
    if cfg.n_outliers:
        for m in range(cfg.M):
            synth.set_outliers(x[m], cfg.n_outliers, cfg.outlier_value, cfg.x_seed + 17 * m)
    # one worker per physical core, within the box's CPU share of 16
    nt = threads or min(16, host["physical_cores"])
    cpus = host["cpus"][:nt] if len(host["cpus"]) >= nt else None
    isa = O.simd_isa()
    for _ in range(3):
        O.simd_mul_mat(cfg.wtype, wq, x, nthreads=nt, cpus=cpus, isa=isa)
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 10 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        O.simd_mul_mat(cfg.wtype, wq, x, nthreads=nt, cpus=cpus, isa=isa)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    if cfg.bound == "hbm":
        value, unit = wq.nbytes / med / 1e9, "GB/s"
    else:
        value, unit = 2.0 * cfg.M * cfg.N * cfg.K / med / 1e12, "TOPS"
    return {"value": value, "unit": unit, "cores": nt, "kind": "port",
            "sample": f"config {cfg.index} in full ({cfg.M}x{cfg.N}x{cfg.K} {dc_type_name(cfg.wtype)}): CPU restatement "
                      f"(not ggml) of the reference path, quantize X once + row-partitioned {O.ISA_NAMES[isa]} "
                      f"vec_dots on {nt} workers pinned to distinct physical cores; median of {len(times)} runs "
                      f"({sum(times):.1f} s), {med * 1e3:.3f} ms per run",
            "ms_per_run": med * 1e3, "isa": O.ISA_NAMES[isa], "host_cpu": host["model"],
            "physical_cores": host["physical_cores"], "logical_cpus": host["logical_cpus"], "nproc": host["nproc"]}


def dc_type_name(t):
    import densecore_amd as dc
    return dc.TYPE_NAMES[t]


def main():
    args = parse()
    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc))
        return 0
    if args.summarize_traffic:
        print(summarize_traffic(*args.summarize_traffic))
        return 0
    if args.summarize_read:
        print(summarize_read(args.summarize_read, [int(c) for c in args.configs.split(",") if c.strip()],
                             args.warmup + args.steps))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    import densecore_amd as dc
    dc.lib()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    wanted = [int(c) for c in args.configs.split(",") if c.strip()]
    if args.profile:
        for c in dc.CONFIGS:
            if c.index in wanted:
                profile_config(c, args, dev)
        if not args.no_extras:
            profile_extras(args, dev)
        calibration_copy(dev)
        return 0
    if args.profile_read:
        profile_read(args, dev)
        return 0
    results = []
    for c in dc.CONFIGS:
        if c.index in wanted:
            r = bench_config(c, args, dev)
            results.append(r)
            print(f"# config {c.index} {c.name}: step {r['step_us']:.2f} us ({r['kernels_per_step']} kernels), "
                  f"dominant kernel {r['dominant_us']:.2f} us, roofline {r['roofline']['achieved']:.1f} "
                  f"{r['roofline']['unit']} ({100 * r['roofline']['frac']:.1f} %)", file=sys.stderr, flush=True)
    extras = {}
    if HEADLINE in wanted and not args.no_extras:
        extras["ffn_gate_up"] = bench_gate_up(dc.by_index(HEADLINE), args, dev)
        g = extras["ffn_gate_up"]
        print(f"# gate/up pair at config {HEADLINE}: fused {g['fused_us']:.2f} us ({g['fused_kernels']} kernels), "
              f"two mul_mat calls {g['separate_us']:.2f} us", file=sys.stderr, flush=True)
    if not args.no_extras:
        q = extras["qkv_projections"] = bench_qkv(args, dev)
        print(f"# q/k/v projections: three calls {q['separate_us']:.2f} us, one call over the concatenated "
              f"weights {q['one_call_us']:.2f} us", file=sys.stderr, flush=True)
        for wt in (dc.TYPE_Q6_K, dc.TYPE_Q4_K):
            e = extras[f"ffn_down_residual_{dc.TYPE_NAMES[wt].lower()}"] = bench_residual(args, dev, wt)
            print(f"# {e['shape']}: mul_mat + add {e['mul_mat_then_add_us']:.2f} us "
                  f"({e['mul_mat_then_add_kernels']} kernels), mul_mat_add {e['mul_mat_add_us']:.2f} us "
                  f"({e['mul_mat_add_kernels']} kernels)", file=sys.stderr, flush=True)
        for name, kw in (("kv_attention_decode_q8_0", dict(ct=dc.TYPE_Q8_0)),
                         ("kv_attention_decode_f16", dict(ct=dc.TYPE_F16)),
                         ("kv_attention_prefill_q8_0", dict(ct=dc.TYPE_Q8_0, n_tokens=2048, n_past=0, n_layer=2)),
                         ("kv_attention_chunk_q8_0", dict(ct=dc.TYPE_Q8_0, n_tokens=256, n_past=4096, n_layer=2))):
            e = extras[name] = bench_kv_attention(args, dev, **kw)
            print(f"# {name}: {e['us']:.2f} us ({e['kernels']} kernels), {e['GBps']:.0f} GB/s, "
                  f"{e['TFLOPs']:.2f} TFLOP/s", file=sys.stderr, flush=True)
        for wt, K in ((dc.TYPE_Q8_0, 1024), (dc.TYPE_Q6_K, 2560)):
            for M in (1, 4):
                e = extras[f"lm_head_{dc.TYPE_NAMES[wt].lower()}_m{M}"] = bench_lm_head(args, dev, wt, K, M)
                print(f"# {e['shape']}: {e['us']:.2f} us ({e['kernels']} kernels), {e['weight_GBps']:.0f} GB/s "
                      f"({100 * e['frac_of_peak']:.1f} % of 8 TB/s; read ceiling {e.get('read_ceiling_us', 0):.2f} us)",
                      file=sys.stderr, flush=True)
        for wt in (dc.TYPE_Q4_K, dc.TYPE_Q6_K):
            e = extras[f"prefill_{dc.TYPE_NAMES[wt].lower()}"] = bench_kquant_prefill(args, dev, wt)
            print(f"# {e['shape']}: kernel {e['kernel_us']:.1f} us ({e['TOPS_kernel']:.0f} TOPS, "
                  f"{100 * e['frac_of_int8_peak']:.1f} % of int8 peak), step {e['step_us']:.1f} us "
                  f"({e['kernels']} kernels)", file=sys.stderr, flush=True)
        for tname, M, N, K in BATCHED_SHAPES:
            e = extras[f"batched_{tname.lower()}_m{M}_{N}x{K}"] = bench_batched_decode(args, dev, tname, M, N, K)
            print(f"# batched decode {e['shape']}: {e['step_us']:.2f} us ({e['kernels']} kernels), "
                  f"{e['weight_GBps']:.0f} GB/s of weights, {e['TOPS']:.1f} TOPS", file=sys.stderr, flush=True)
        for tname, M, N, K in TOOL_TYPE_SHAPES:
            e = extras[f"tool_type_{tname.lower()}_m{M}_{N}x{K}"] = bench_tool_type(args, dev, tname, M, N, K)
            print(f"# {e['shape']}: {e['step_us']:.2f} us ({e['kernels']} kernels), {e['weight_GBps']:.0f} GB/s "
                  f"of weights ({100 * e['frac_of_hbm_peak']:.1f} % of 8 TB/s; read ceiling "
                  f"{e.get('read_ceiling_us', 0):.2f} us), {e['TOPS']:.1f} TOPS", file=sys.stderr, flush=True)
        for M, N, K in ROW_SPLIT_SHAPES:
            e = extras[f"q8_0_row_split_m{M}_{N}x{K}"] = bench_q8_0_row_split(args, dev, M, N, K)
            print(f"# {e['shape']}: GGUF rows {e['gguf_step_us']:.2f} us, row-split {e['row_split_step_us']:.2f} us "
                  f"({e['row_split_speedup']:.3f}x)", file=sys.stderr, flush=True)
        extras["weight_quantizer"] = bench_weight_quantizer(args, dev)
        extras["gguf_load"] = bench_gguf_load(args, dev)
        print(f"# GGUF ingest: {extras['gguf_load']['GBps']:.1f} GB/s host-to-HBM over "
              f"{extras['gguf_load']['bytes'] >> 20} MiB", file=sys.stderr, flush=True)
    head = next((r for r in results if r["config"] == HEADLINE), results[0])
    hcfg = dc.by_index(head["config"])
    line = {
        "metric": METRIC,
        "value": head["weight_GBps_step"] if hcfg.bound == "hbm" else head["TOPS_step"],
        "unit": "GB/s" if hcfg.bound == "hbm" else "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["step_us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded SplitMix64/Box-Muller; W quantized on the GPU by dcq_quantize_weights)",
        "config": {"workload": f"config {hcfg.index}: {dc.TYPE_NAMES[hcfg.wtype]} mul_mat M={hcfg.M} "
                               f"N={hcfg.N} K={hcfg.K} ({hcfg.name}); a step is one dcq_mul_mat call "
                               f"(activation quantization + dots, {head['kernels_per_step']} kernel(s)); "
                               f"W rotated over {head['w_copies']} copies ({head['w_copies'] * head['w_bytes'] >> 20} MiB)",
                   "M": hcfg.M, "N": hcfg.N, "K": hcfg.K, "type": dc.TYPE_NAMES[hcfg.wtype]},
        "roofline": head["roofline"],
        "device": props.name, "gcn_arch": getattr(props, "gcnArchName", ""), "host": platform.node(),
        "configs": results,
        "extras": extras,
    }
    if not args.no_cpu_baseline:
        host = host_cpu_info()
        for r in results:
            if r["config"] in (HEADLINE, 5):
                cb = r["cpu_baseline"] = cpu_baseline(dc.by_index(r["config"]), args.cpu_seconds, args.cpu_threads, host)
                print(f"# CPU baseline config {r['config']}: {cb['value']:.3g} {cb['unit']} on {cb['cores']} cores "
                      f"({cb['ms_per_run']:.3f} ms per run)", file=sys.stderr, flush=True)
        line["cpu_baseline"] = head.get("cpu_baseline")
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
