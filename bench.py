#!/usr/bin/env python3
"""Benchmark of the quantized decode matmul path on one MI355X.

Headline (default): batch-1 Q4_0 GEMV over every linear layer of Llama-3-8B
decode - 32 layers x {q, k, v, o, gate, up, down}, K x N = 4096x4096,
4096x1024 (k, v), 4096x14336 (gate, up), 14336x4096 (down) - with 32
distinct weight copies resident in HBM (3.9 GB, 15x the 256 MB Infinity
Cache, so every weight byte comes from HBM).  One step = one decode token
through all 224 GEMVs, replayed as a HIP graph.  value = algorithmic bytes
(weights + scales + x + y) / step time, in GB/s.

Also reported on the same JSON line:
  roofline      the dominant kernel (Q4_0 GEMV at 14336 x 4096, the gate/up
                shape) timed with HIP events around graph replays of
                back-to-back launches over rotating weight copies;
  ceiling       a plain streaming read of the same weight bytes in the same
                timing at each shape (per_shape.*.frac_of_ceiling = read
                time / GEMV time): what one launch per GEMV can reach;
  cpu_baseline  the C restatement of the reference CPU engine's Q4_0 GEMV
                (GemmF32Q4NT, internal/xblas/gemm_quant.go:81-157) on the
                host cores, over one layer's seven matrices;
  configs       every benchmark configuration's shapes and batches as the
                engine runs them (batched W4A16 / IQ4_NL on the row-block
                GEMM or the tiled layouts, whichever the engine picks):
                [format, "KxN", batch, us per matmul, % of peak]
                (skipped with --no-configs);
  configs_cpu   the CPU restatement of each configuration's reference CPU
                path on one representative shape, about 2 s each (skipped
                with --no-configs or --no-cpu-baseline).

`python bench.py --suite` instead prints one line per benchmark
configuration (W4A16, Q4_0, Q8_0, ternary, IQ4_NL, and the K-quant / Q5_0
formats at the Llama-3-8B shapes) with us per matmul and effective GB/s;
those are supporting numbers, not the headline line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "quant GEMV effective HBM GB/s (% of peak) at Llama-3-8B decode shapes, batch 1"
PEAK_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 MFMA
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
LLAMA3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
             ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]  # (name, rows=N_out, K)
MALL_BYTES = 256 << 20


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------ device setup

class Q4Matrix:
    """One Q4_0 weight matrix uploaded in the RawBytesGPU layout."""

    def __init__(self, torch, lib, rows: int, K: int, seed: int, copies: int):
        from ztensor_amd import synth

        self.rows, self.K = rows, K
        w = synth.q4_0(rows, K, seed)
        self.raw = w.raw
        nblk = rows * K // 32
        host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
        lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
        base = torch.from_numpy(host).cuda()
        self.copies = [base] + [base.clone() for _ in range(copies - 1)]
        self.off = lib.zt_q4_gpu_data_offset(nblk)
        self.x = torch.from_numpy(synth.x_f32(K, seed)).cuda()
        self.y = [torch.empty(rows, dtype=torch.float32, device="cuda") for _ in range(copies)]
        from ztensor_amd.synth import algorithmic_bytes

        self.bytes = algorithmic_bytes("q4_0", rows, K)

    def launch(self, lib, i: int, stream: int) -> None:
        rc = lib.zt_gemm_q4_f32(self.copies[i].data_ptr(), self.x.data_ptr(), self.y[i].data_ptr(), self.rows,
                                self.K, 1, self.off, stream)
        if rc != 0:
            raise RuntimeError(f"zt_gemm_q4_f32 returned {rc}")


def graph_of(torch, fn):
    """Captures fn() (which launches on torch's current stream) into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up launch outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps: int) -> float:
    """Average ms per replay, HIP events on the replay stream."""
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


# ------------------------------------------------------------ HBM traffic

TRAFFIC_FILE = ROOT / "profiles" / "q4_0_gemv_14336x4096_traffic.md"


def measured_traffic(kernel: str):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (a line starting with
    'traffic_json: '), or None when it is absent or was taken on another
    kernel build."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_json: "):
                t = json.loads(line[len("traffic_json: "):])
                if t.get("kernel") == kernel:
                    return t["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        pass
    return None


def calibration_copy(torch) -> None:
    """Device-to-device copies of 64 MiB, the known-size reference kernel that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE readings to bytes."""
    src = torch.ones(64 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


# ------------------------------------------------------------ CPU baseline

def cpu_baseline(mats, budget_s: float = 15.0) -> dict:
    from oracle import oracle

    threads = min(16, oracle.nthreads())
    total_bytes, t_total, reps = 0, 0.0, 0
    xs = {m.K: m.x.cpu().numpy() for m in mats}
    while t_total < budget_s:
        for m in mats:
            t0 = time.perf_counter()
            oracle.gemm_f32_q4_nt(xs[m.K], m.raw, 1, m.rows, m.K, threads=threads)
            t_total += time.perf_counter() - t0
            total_bytes += m.bytes
        reps += 1
    try:
        cpu = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        cpu = "unknown"
    return {
        "value": round(total_bytes / t_total / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} passes over one Llama-3-8B layer's 7 Q4_0 GEMVs (batch 1) with the C restatement of "
                  f"GemmF32Q4NT (scalar q4DotRow, N split over min(threads, N/4) workers); {t_total:.1f} s on {cpu}",
    }


# ------------------------------------------------------------ headline run

def run_headline(args) -> dict:
    import torch

    from ztensor_amd import _lib

    lib = _lib.load()
    if args.calibration_copy:
        calibration_copy(torch)
    layers = args.layers
    log(f"bench: generating Llama-3-8B Q4_0 weights, {layers} layer copies")
    mats = [Q4Matrix(torch, lib, rows, K, 0x5EED0020 + i, layers) for i, (_, rows, K) in enumerate(LLAMA3_8B)]
    step_bytes = layers * sum(m.bytes for m in mats)
    resident = layers * sum(m.copies[0].numel() for m in mats)
    log(f"bench: {resident / 1e9:.2f} GB of weights resident; {step_bytes / 1e6:.1f} MB per step")

    def step():
        s = torch.cuda.current_stream().cuda_stream
        for layer in range(layers):
            for m in mats:
                m.launch(lib, layer, s)

    g = graph_of(torch, step)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = time_graph(torch, g, args.steps)
    wall = time.perf_counter() - t0
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"bench: {ms * 1e3:.1f} us/step, {value:.1f} GB/s ({100 * value / PEAK_GBS:.1f}% of peak), wall {wall:.2f}s")

    # Per-shape and dominant-kernel timings: graphs of back-to-back launches
    # rotating over the layer copies, each beside the ceiling: a plain
    # 16-byte-a-lane streaming read of the same weight buffers in the same
    # graph timing (zt_bench_stream_read).
    per_shape = {}
    ceiling = {"kernel": "zt_bench_stream_read: nontemporal 16-byte loads a lane, no arithmetic, over the same "
                         "rotating weight buffers and graph timing as the GEMV", "per_shape": {}}
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    dom = None
    for (name, rows, K), m in zip(LLAMA3_8B, mats):
        if name in ("k", "up"):
            continue  # same shapes as v / gate
        n = 8 * layers

        def loop(m=m, n=n):
            s = torch.cuda.current_stream().cuda_stream
            for i in range(n):
                m.launch(lib, i % layers, s)

        gl = graph_of(torch, loop)
        gl.replay()
        us = time_graph(torch, gl, max(3, args.steps // 20)) * 1e3 / n
        gbs = m.bytes / (us * 1e-6) / 1e9

        def read_loop(m=m, n=n):
            s = torch.cuda.current_stream().cuda_stream
            for i in range(n):
                buf = m.copies[i % layers]
                if lib.zt_bench_stream_read(buf.data_ptr(), buf.numel(), sink.data_ptr(), s) != 0:
                    raise RuntimeError("zt_bench_stream_read failed")

        gr = graph_of(torch, read_loop)
        gr.replay()
        cus = time_graph(torch, gr, max(3, args.steps // 20)) * 1e3 / n
        wbytes = m.copies[0].numel()
        ceiling["per_shape"][f"{name} {K}x{rows}"] = {
            "us": round(cus, 3), "bytes_read": wbytes, "GB/s": round(wbytes / (cus * 1e-6) / 1e9, 1),
            "pct_peak": round(100 * wbytes / (cus * 1e-6) / 1e9 / PEAK_GBS, 1)}
        per_shape[f"{name} {K}x{rows}"] = {"us": round(us, 3), "GB/s": round(gbs, 1),
                                           "pct_peak": round(100 * gbs / PEAK_GBS, 1), "bytes": m.bytes,
                                           "ceiling_us": round(cus, 3), "frac_of_ceiling": round(cus / us, 3)}
        if name == "gate":
            dom = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                   "frac": round(gbs / PEAK_GBS, 4), "frac_of_ceiling": round(cus / us, 4), "traffic": None,
                   "kernel": "gemv_q4_steps_kernel<S=1, R=8> (zt_gemm_q4_f32), K=4096 x N=14336, batch 1",
                   "bytes_per_launch": m.bytes, "us_per_launch": round(us, 3)}
        log(f"bench: {name:5s} K={K:5d} N={rows:5d}: {us:7.2f} us  {gbs:7.1f} GB/s  (streaming read of the same "
            f"bytes: {cus:.2f} us)")

    if dom is not None:
        dom["traffic"] = measured_traffic(dom["kernel"])

    grouped = run_grouped_step(torch, lib, args, mats, step_bytes)
    merged = run_merged_step(torch, lib, args) if args.merged else None
    bitnet = run_bitnet_step(torch, lib, args) if args.merged else None
    w4step = run_w4a16_step(torch, lib, args) if args.merged else None

    # Parity spot check of the last replayed outputs against the oracle.
    from oracle import oracle

    m = mats[0]
    ref = oracle.gemm_f32_q4_nt(m.x.cpu().numpy(), m.raw, 1, m.rows, m.K, threads=8)
    err = float(np.max(np.abs(m.y[0].cpu().numpy() - ref)) / np.max(np.abs(ref)))
    if err > 1e-3:
        raise SystemExit(f"bench: parity check failed (rel err {err:.2e})")

    cpu = cpu_baseline(mats[:7]) if args.cpu_baseline else None
    return {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_0 nibbles U[0,15], fp16 scales |N(0,1)|*0.02, fp32 x ~ N(0,1))",
        "config": {
            "workload": f"Llama-3-8B decode, {layers} layers x {{q,k,v,o,gate,up,down}} Q4_0 GEMV, batch 1, "
                        "weights resident in HBM (distinct copy per layer)",
            "format": "Q4_0 (RawBytesGPU layout)",
            "batch": 1,
            "layers": layers,
            "shapes_KxN": [f"{K}x{rows}" for _, rows, K in LLAMA3_8B],
            "bytes_per_step": step_bytes,
            "pct_of_peak": round(100 * value / PEAK_GBS, 1),
            "parity_rel_err": err,
        },
        "per_shape": per_shape,
        "ceiling": ceiling,
        "grouped_projections": grouped,
        "merged_projections": merged,
        "bitnet_layer_step": bitnet,
        "w4a16_70b_layer_step": w4step,
        "roofline": dom,
        "cpu_baseline": cpu,
    }


def run_grouped_step(torch, lib, args, mats, step_bytes: int) -> dict:
    """The headline's decode step over the same resident weights with the
    matrices that share an activation vector launched together through
    zt_gemm_q4_group_f32: per layer group(q, k, v), o, group(gate, up),
    down - 4 launches instead of 7, each matrix still in its own upload."""
    from ztensor_amd import _lib as zl

    by = {name: m for (name, _, _), m in zip(LLAMA3_8B, mats)}
    layers = args.layers
    plan = []  # per layer: ("group", descs, n, x, K) or ("one", matrix)
    for layer in range(layers):
        for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            if len(names) == 1:
                plan.append(("one", by[names[0]]))
                continue
            ms = [by[n] for n in names]
            descs = zl.q4_gemv_descs([(m.copies[layer].data_ptr(), m.off, m.y[layer].data_ptr(), m.rows)
                                      for m in ms])
            plan.append(("group", descs, len(ms), ms[0].x, ms[0].K))

    def step():
        s = torch.cuda.current_stream().cuda_stream
        for i, item in enumerate(plan):
            if item[0] == "one":
                item[1].launch(lib, i // 4, s)
            else:
                _, descs, n, x, K = item
                rc = lib.zt_gemm_q4_group_f32(descs, n, x.data_ptr(), K, s)
                if rc != 0:
                    raise RuntimeError(f"zt_gemm_q4_group_f32 returned {rc}")

    g = graph_of(torch, step)
    for _ in range(args.warmup):
        g.replay()
    ms = time_graph(torch, g, args.steps)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"bench: grouped Q/K/V and Gate/Up launches: {ms * 1e3:.1f} us/step, {value:.1f} GB/s "
        f"({100 * value / PEAK_GBS:.1f}%)")
    return {"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "bytes_per_step": step_bytes,
            "pct_of_peak": round(100 * value / PEAK_GBS, 1), "launches_per_layer": 4,
            "workload": "the headline step, q/k/v and gate/up each one zt_gemm_q4_group_f32 launch over the "
                        "separate uploads"}


def run_w4a16_step(torch, lib, args, layers: int = 4) -> dict:
    """A Llama-3-70B W4A16 decode step at batch 1 (configuration 4's shapes,
    group 128, fp16 activations, packed (scale, zero) dwords): per layer q,
    o (8192 x 8192), k, v (1024 x 8192), gate, up (28672 x 8192) and down
    (8192 x 28672) as rows x K, `layers` distinct layer copies resident (1.7
    GB at 4, beyond the Infinity Cache).  Timed as 7 zt_gemv_w4a16sz_f32
    launches a layer, and as 4 with q/k/v and gate/up each one
    zt_gemv_w4a16sz_group_f32 launch over the same uploads."""
    from ztensor_amd import _lib as zl
    from ztensor_amd import synth

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
    s0 = torch.cuda.current_stream().cuda_stream
    shapes = [("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192), ("gate", 28672, 8192),
              ("up", 28672, 8192), ("down", 8192, 28672)]
    mats = {}
    for i, (name, rows, K) in enumerate(shapes):
        w = synth.w4a16(rows, K, 0x5EED0090 + i)
        p, sc, z = dev(w.packed), dev(w.scales), dev(w.zeros)
        szr = torch.empty(w.scales.size, dtype=torch.int32, device="cuda")
        if lib.zt_w4a16_pack_szr(sc.data_ptr(), z.data_ptr(), rows, K, 128, szr.data_ptr(), s0) != 0:
            raise RuntimeError("zt_w4a16_pack_szr failed")
        mats[name] = {"rows": rows, "K": K, "w": [p] + [p.clone() for _ in range(layers - 1)],
                      "szr": [szr] + [szr.clone() for _ in range(layers - 1)],
                      "y": [torch.empty(rows, dtype=torch.float32, device="cuda") for _ in range(layers)]}
        del sc, z
    xs = {K: dev(synth.x_f16(K, 0x5EED0098 + K)) for K in (8192, 28672)}
    step_bytes = layers * sum(synth.algorithmic_bytes("w4a16", rows, K, 1) for _, rows, K in shapes)

    def single(name, layer, s):
        m = mats[name]
        rc = lib.zt_gemv_w4a16sz_f32(m["w"][layer].data_ptr(), m["szr"][layer].data_ptr(), xs[m["K"]].data_ptr(),
                                     m["y"][layer].data_ptr(), m["rows"], m["K"], 128, s)
        if rc != 0:
            raise RuntimeError(f"zt_gemv_w4a16sz_f32 returned {rc}")

    plan = []
    for layer in range(layers):
        for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            if len(names) == 1:
                plan.append(("one", names[0], layer))
                continue
            descs = zl.w4a16_gemv_descs([(mats[n]["w"][layer].data_ptr(), mats[n]["szr"][layer].data_ptr(),
                                          mats[n]["y"][layer].data_ptr(), mats[n]["rows"]) for n in names])
            plan.append(("group", descs, len(names), 8192))

    def step_single():
        s = torch.cuda.current_stream().cuda_stream
        for layer in range(layers):
            for name, _, _ in shapes:
                single(name, layer, s)

    def step_grouped():
        s = torch.cuda.current_stream().cuda_stream
        for item in plan:
            if item[0] == "one":
                single(item[1], item[2], s)
            else:
                _, descs, n, K = item
                rc = lib.zt_gemv_w4a16sz_group_f32(descs, n, xs[K].data_ptr(), K, 128, s)
                if rc != 0:
                    raise RuntimeError(f"zt_gemv_w4a16sz_group_f32 returned {rc}")

    out = {"workload": f"Llama-3-70B decode step, {layers} layers x {{q,o 8192x8192; k,v 1024x8192; gate,up "
                       "28672x8192; down 8192x28672}} (rows x K) W4A16 GEMVs (group 128, packed scale/zero), batch 1",
           "bytes_per_step": step_bytes}
    for key, fn, launches in (("per_gemv", step_single, 7), ("grouped", step_grouped, 4)):
        g = graph_of(torch, fn)
        for _ in range(args.warmup):
            g.replay()
        ms = time_graph(torch, g, args.steps)
        out[key] = {"us_per_layer": round(ms * 1e3 / layers, 3), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                    "pct_peak": round(100 * step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 1), "launches_per_layer": launches}
        log(f"bench: W4A16 70B step, {key}: {ms * 1e3 / layers:.2f} us per layer")
    del mats
    torch.cuda.empty_cache()
    return out


def run_bitnet_step(torch, lib, args, layers: int = 32) -> dict:
    """A BitNet-2B decode step over the configuration-3 shapes with int8
    activations: per layer q, k, v, o (2560 x 2560), gate, up (6912 x 2560)
    and down (2560 x 6912) as rows x K, 32 distinct layer copies resident
    (about 630 MB, beyond the Infinity Cache).  Timed as 7 zt_ternary_gemv_i8
    launches a layer, and as 4 with q/k/v and gate/up each one
    zt_ternary_gemv_i8_group launch over the same uploads."""
    from ztensor_amd import _lib as zl
    from ztensor_amd import synth
    from ztensor_amd.storage import TernaryStorage

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
    shapes = [("q", 2560, 2560), ("k", 2560, 2560), ("v", 2560, 2560), ("o", 2560, 2560), ("gate", 6912, 2560),
              ("up", 6912, 2560), ("down", 2560, 6912)]
    mats = {}
    for i, (name, rows, K) in enumerate(shapes):
        t = synth.ternary(rows, K, 0x5EED0070 + i)
        w = dev(TernaryStorage(t.raw, rows * K).row_aligned(rows, K))
        mats[name] = {"rows": rows, "K": K, "w": [w] + [w.clone() for _ in range(layers - 1)],
                      "ws": torch.tensor([t.w_scale], dtype=torch.float32, device="cuda"),
                      "y": [torch.empty(rows, dtype=torch.float32, device="cuda") for _ in range(layers)]}
    xq = {}
    for K in (2560, 6912):
        q, xs = synth.x_i8(K, 0x5EED0078 + K)
        xq[K] = (dev(q), torch.tensor([xs], dtype=torch.float32, device="cuda"))
    step_bytes = layers * sum(synth.algorithmic_bytes("ternary_i8", rows, K, 1) for _, rows, K in shapes)

    def single(name, layer, s):
        m = mats[name]
        x, xs = xq[m["K"]]
        rc = lib.zt_ternary_gemv_i8(m["w"][layer].data_ptr(), x.data_ptr(), xs.data_ptr(), m["ws"].data_ptr(),
                                    m["y"][layer].data_ptr(), m["rows"], m["K"], s)
        if rc != 0:
            raise RuntimeError(f"zt_ternary_gemv_i8 returned {rc}")

    plan = []
    for layer in range(layers):
        for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            if len(names) == 1:
                plan.append(("one", names[0], layer))
                continue
            descs = zl.ternary_gemv_descs([(mats[n]["w"][layer].data_ptr(), mats[n]["ws"].data_ptr(),
                                           mats[n]["y"][layer].data_ptr(), mats[n]["rows"]) for n in names])
            plan.append(("group", descs, len(names), 2560))

    def step_single():
        s = torch.cuda.current_stream().cuda_stream
        for layer in range(layers):
            for name, _, _ in shapes:
                single(name, layer, s)

    def step_grouped():
        s = torch.cuda.current_stream().cuda_stream
        for item in plan:
            if item[0] == "one":
                single(item[1], item[2], s)
            else:
                _, descs, n, K = item
                x, xs = xq[K]
                rc = lib.zt_ternary_gemv_i8_group(descs, n, x.data_ptr(), xs.data_ptr(), K, s)
                if rc != 0:
                    raise RuntimeError(f"zt_ternary_gemv_i8_group returned {rc}")

    out = {"workload": f"BitNet-2B decode step, {layers} layers x {{q,k,v,o 2560x2560; gate,up 6912x2560; "
                       "down 2560x6912}} (rows x K) ternary GEMVs, int8 activations", "bytes_per_step": step_bytes}
    for key, fn, launches in (("per_gemv", step_single, 7), ("grouped", step_grouped, 4)):
        g = graph_of(torch, fn)
        for _ in range(args.warmup):
            g.replay()
        ms = time_graph(torch, g, args.steps)
        out[key] = {"us_per_layer": round(ms * 1e3 / layers, 3), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                    "launches_per_layer": launches}
        log(f"bench: BitNet step, {key}: {ms * 1e3 / layers:.2f} us per layer")
    del mats
    torch.cuda.empty_cache()
    return out


def run_merged_step(torch, lib, args) -> dict:
    """The same 32-layer decode step with Q/K/V and Gate/Up merged row-wise
    (MergeQ4Storage, tensor/quantized.go:224-242): 4 GEMVs per layer
    (6144x4096, 4096x4096, 28672x4096, 4096x14336 as rows x K) moving the
    same bytes as the 7 separate ones.  Reported beside the headline, which
    keeps one GEMV per projection."""
    layers = args.layers
    shapes = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]
    mats = [Q4Matrix(torch, lib, rows, K, 0x5EED0040 + i, layers) for i, (_, rows, K) in enumerate(shapes)]
    step_bytes = layers * sum(m.bytes for m in mats)

    def step():
        s = torch.cuda.current_stream().cuda_stream
        for layer in range(layers):
            for m in mats:
                m.launch(lib, layer, s)

    g = graph_of(torch, step)
    for _ in range(args.warmup):
        g.replay()
    ms = time_graph(torch, g, args.steps)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"bench: merged Q/K/V and Gate/Up: {ms * 1e3:.1f} us/step, {value:.1f} GB/s ({100 * value / PEAK_GBS:.1f}%)")
    del mats
    torch.cuda.empty_cache()
    return {"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "bytes_per_step": step_bytes,
            "pct_of_peak": round(100 * value / PEAK_GBS, 1),
            "shapes_rows_x_K": [f"{rows}x{K}" for _, rows, K in shapes]}


# ------------------------------------------------------------ suite mode

SUITE = {
    # name: (format, [(rows = N_out, K)], batches)
    "w4a16_c1": ("w4a16", [(4096, 4096)], [1]),
    "w4a16sz_c1": ("w4a16sz", [(4096, 4096)], [1]),
    "q4_0": ("q4_0", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q4_0_merged": ("q4_0", [(6144, 4096), (28672, 4096)], [1]),
    "q8_0": ("q8_0", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [1]),
    "rbf8": ("q4_0", [(4096, 4096), (14336, 4096), (4096, 14336)], [8, 16]),
    "q4_0_prefill": ("q4_0", [(4096, 4096), (14336, 4096), (4096, 14336)], [32, 64, 128, 512]),
    "q8_0_prefill": ("q8_0", [(4096, 4096), (14336, 4096), (4096, 14336)], [32, 64, 128, 512]),
    "q8_0_raw_prefill": ("q8_0_raw", [(4096, 4096), (14336, 4096), (4096, 14336)], [32, 64, 128, 512]),
    "q8_0_raw": ("q8_0_raw", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [1]),
    "ternary": ("ternary_i8", [(2560, 2560), (6912, 2560), (2560, 6912)], [1]),
    "ternary_f32": ("ternary_f32", [(2560, 2560), (6912, 2560), (2560, 6912)], [1]),
    "w4a16_70b": ("w4a16", [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)], [1, 4, 8, 16]),
    "w4a16sz_70b": ("w4a16sz", [(8192, 8192), (1024, 8192), (28672, 8192)], [1]),
    "w4a16sz_70b_k28672": ("w4a16sz", [(8192, 28672)], [1]),
    "w4a16sz_70b_batched": ("w4a16sz", [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)], [4, 8]),
    "w4a16sz_70b_wide": ("w4a16sz", [(8192, 8192), (1024, 8192), (28672, 8192)], [12, 16]),
    "w4a16sz_8b_wide": ("w4a16sz", [(4096, 4096), (1024, 4096), (14336, 4096)], [12, 16]),
    "w4a16sz_8b_batched": ("w4a16sz", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8]),
    "w4a16_8b_batched": ("w4a16", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [12, 16]),
    "w4a16t_8b": ("w4a16t", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8, 12, 16]),
    "w4a16_70b_k28672": ("w4a16", [(8192, 28672)], [1]),
    "w4a16t_70b": ("w4a16t", [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)], [4, 8, 16]),
    "iq4nl": ("iq4nl", [(3584, 3584), (18944, 3584), (3584, 18944)], [1, 8]),
    "iq4nlt": ("iq4nlt", [(3584, 3584), (18944, 3584), (3584, 18944)], [8]),
    "iq4nlt_b4": ("iq4nlt", [(3584, 3584), (18944, 3584), (3584, 18944)], [4]),
    # the engine's dispatch (row-block or tiled) at the configuration shapes
    "w4a16_70b_engine": ("w4a16_engine", [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)], [1, 4, 8, 16]),
    "iq4nl_engine": ("iq4nl_engine", [(3584, 3584), (18944, 3584), (3584, 18944)], [1, 4, 8]),
    "iq4nl_batched": ("iq4nl", [(3584, 3584), (18944, 3584), (3584, 18944)], [4, 8]),
    "iq4nl_wide": ("iq4nl", [(3584, 3584), (18944, 3584), (1024, 4096), (4096, 4096)], [12, 16]),
    "iq4nlt_wide": ("iq4nlt", [(3584, 3584), (1024, 4096), (4096, 4096)], [12, 16]),
    # zt_gemm_iq4nl_f32: fp32 activations (the reference's IQ4_NL matmul input type)
    # zt_gemm_q4_f16: Q4_0 with fp16 activations (Float16Storage activations on the Q4_0 path)
    "q4_0h": ("q4_0h", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [1]),
    "iq4nl32_batched": ("iq4nl32", [(3584, 3584), (18944, 3584), (3584, 18944)], [1, 4, 8]),
    "q4_k": ("q4_k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q5_k": ("q5_k", [(4096, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q6_k": ("q6_k", [(4096, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q6_ks": ("q6_ks", [(4096, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q5_0": ("q5_0", [(4096, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q8_0_gguf": ("q8_0_gguf", [(4096, 4096), (14336, 4096), (4096, 14336)], [1]),
    "q4_0_batched": ("q4_0", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8, 16]),
    # gemm_int4.cu / gemm_int8.cu: decode shapes, and the reference benchmark's square GEMMs
    # (gemm_bench_test.go:159-165, batch = rows)
    "int4": ("int4", [(4096, 4096), (14336, 4096)], [1, 4]),
    "int4_rmul": ("int4_rmul", [(4096, 4096)], [1, 4]),
    "int4_rmul_shapes": ("int4_rmul", [(4096, 4096), (14336, 4096), (4096, 14336)], [1, 2, 3, 4]),
    "int4_rmul_batched": ("int4_rmul", [(4096, 4096), (14336, 4096), (4096, 14336)], [8, 16, 32]),
    "int8": ("int8", [(4096, 4096), (4096, 14336)], [1, 4]),
    "int4_batched": ("int4", [(4096, 4096), (14336, 4096), (4096, 14336)], [4, 8, 12, 16, 32, 64]),
    "int8_batched": ("int8", [(4096, 4096), (14336, 4096), (4096, 14336)], [4, 8, 12, 16, 32, 64]),
    "int4_gemm": ("int4", [(1024, 1024), (2048, 2048), (4096, 4096)], ["square"]),
    "int4_rmul_gemm": ("int4_rmul", [(1024, 1024), (2048, 2048), (4096, 4096)], ["square"]),
    "int8_gemm": ("int8", [(1024, 1024), (2048, 2048), (4096, 4096)], ["square"]),
    "intq_mid": ("int4", [(4096, 4096), (14336, 4096)], [96, 128, 256]),
    "int8_mid": ("int8", [(4096, 4096), (4096, 14336)], [96, 128, 256]),
    "q8_0_batched": ("q8_0", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8, 16]),
    "q8_0_raw_batched": ("q8_0_raw", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8]),
    "q4_0t": ("q4_0t", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8, 16]),
    "q8_0t": ("q8_0t", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)], [4, 8, 16]),
    "q4_kt": ("q4_kt", [(4096, 4096), (14336, 4096), (4096, 14336)], [8, 16]),
    "q5_0t": ("q5_0t", [(4096, 4096), (14336, 4096), (4096, 14336)], [8, 16]),
    "q5_kt": ("q5_kt", [(4096, 4096), (14336, 4096), (4096, 14336)], [8, 16]),
    "q6_kt": ("q6_kt", [(4096, 4096), (14336, 4096), (4096, 14336)], [8, 16]),
}


def _suite_case(torch, lib, fmt: str, rows: int, K: int, N: int, seed: int, eager: int = 0) -> dict:
    """One suite measurement.  With eager > 0 the case instead runs that many
    plain launches (no graph, no timing) over its rotating copies, the
    workload of a rocprofv3 counter pass."""
    from ztensor_amd import synth

    s = torch.cuda.current_stream().cuda_stream
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
    if fmt == "w4a16_engine":  # the kernel ROCmEngine picks for this batch
        from ztensor_amd.engine import _w4a16_rowblock

        fmt = "w4a16sz" if N == 1 or (N in (4, 8, 12, 16) and _w4a16_rowblock(rows, K, N)) else "w4a16t"
    elif fmt == "iq4nl_engine":
        fmt = "iq4nl" if N == 1 or (N in (4, 8) and K <= 8192) else "iq4nlt"
    if fmt in ("q4_0", "q4_0h", "iq4nl", "iq4nl32"):
        w = synth.q4_0(rows, K, seed) if fmt in ("q4_0", "q4_0h") else synth.iq4nl(rows, K, seed)
        nblk = rows * K // 32
        host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
        lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
        wbufs = [dev(host)]
        off = lib.zt_q4_gpu_data_offset(nblk)
        if fmt == "q4_0":
            x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
            fn = lambda wb, y: lib.zt_gemm_q4_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, off, s)
        elif fmt == "q4_0h":
            x = dev(synth.x_f16(K * N, seed))
            fn = lambda wb, y: lib.zt_gemm_q4_f16(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, off, s)
        elif fmt == "iq4nl32":
            x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
            fn = lambda wb, y: lib.zt_gemm_iq4nl_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, off,
                                                     s)
        else:
            x = dev(synth.x_f16(K * N, seed))
            fn = lambda wb, y: lib.zt_gemm_iq4nl_f16(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, off,
                                                     s)
        nbytes = synth.algorithmic_bytes(fmt, rows, K, N)
    elif fmt in ("q8_0", "q8_0_raw"):
        w = synth.q8_0(rows, K, seed)
        nblk = rows * K // 32
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        if fmt == "q8_0":
            host = np.empty(lib.zt_q8_gpu_bytes(nblk), np.uint8)
            lib.zt_q8_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
            off = lib.zt_q8_gpu_data_offset(nblk)
            wbufs = [dev(host)]
            fn = lambda wb, y: lib.zt_gemm_q8sep_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, off, s)
        else:
            wbufs = [dev(w.raw)]
            fn = lambda wb, y: lib.zt_gemm_q8_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, s)
        nbytes = synth.algorithmic_bytes("q8_0", rows, K, N)
    elif fmt in ("q4_0t", "q8_0t"):
        # the tiled upload layouts (zt_q4_tile / zt_q8_tile), built once outside the timing
        f = fmt[:2]
        w = synth.q4_0(rows, K, seed) if f == "q4" else synth.q8_0(rows, K, seed)
        nblk = rows * K // 32
        host = np.empty(getattr(lib, f"zt_{f}_gpu_bytes")(nblk), np.uint8)
        getattr(lib, f"zt_{f}_raw_to_gpu")(w.raw.ctypes.data, nblk, host.ctypes.data)
        sep = dev(host)
        wt = torch.empty(getattr(lib, f"zt_{f}_tiled_bytes")(rows, K), dtype=torch.uint8, device="cuda")
        st = torch.empty(getattr(lib, f"zt_{f}_tiled_scale_bytes")(rows, K), dtype=torch.uint8, device="cuda")
        lib.call(f"zt_{f}_tile", sep.data_ptr(), rows, K, getattr(lib, f"zt_{f}_gpu_data_offset")(nblk), wt.data_ptr(),
                 st.data_ptr(), s)
        torch.cuda.synchronize()
        del sep
        wbufs = [wt, st]
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        gemm = getattr(lib, f"zt_gemm_{f}t_f32")
        wsb = getattr(lib, f"zt_gemm_{f}t_workspace_bytes")(rows, K, N)
        wsbuf = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")  # launches run in order on one stream
        fn = lambda wb, y: gemm(wb[0].data_ptr(), wb[1].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N,
                                wsbuf.data_ptr(), wsb, s)
        nbytes = synth.algorithmic_bytes(fmt[:4], rows, K, N)
    elif fmt == "q5_0t":
        # batched Q5_0 on the tiled layout (zt_q5_0_tile), built once outside the timing
        w = synth.kquant("q5_0", rows, K, seed)
        nblk = rows * K // 32
        host = np.empty(lib.zt_q5_0_gpu_bytes(nblk), np.uint8)
        lib.zt_q5_0_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
        sep = dev(host)
        wbufs = [torch.empty(f(rows, K), dtype=torch.uint8, device="cuda")
                 for f in (lib.zt_q5_0_tiled_bytes, lib.zt_q5_0_tiled_scale_bytes, lib.zt_q5_0_tiled_qh_bytes)]
        lib.call("zt_q5_0_tile", sep.data_ptr(), rows, K, lib.zt_q5_0_gpu_qh_offset(nblk),
                 lib.zt_q5_0_gpu_qs_offset(nblk), *(t.data_ptr() for t in wbufs), s)
        torch.cuda.synchronize()
        del sep
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        wsb = lib.zt_gemm_q5_0t_workspace_bytes(rows, K, N)
        wsbuf = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")
        fn = lambda wb, y: lib.zt_gemm_q5_0t_f32(wb[0].data_ptr(), wb[1].data_ptr(), wb[2].data_ptr(), x.data_ptr(),
                                                 y.data_ptr(), rows, K, N, wsbuf.data_ptr(), wsb, s)
        nbytes = synth.algorithmic_bytes("q5_0", rows, K, N)
    elif fmt in ("q4_kt", "q5_kt", "q6_kt"):
        # batched K-quants on the tiled layouts (zt_q4k_tile / zt_q5k_tile / zt_q6k_tile), built once outside the timing
        f = fmt[:4].replace("_", "")
        w = synth.kquant(fmt[:4], rows, K, seed)
        raw = dev(w.raw)
        parts = (["tiled_bytes", "tiled_scale_bytes"] if f == "q6k" else
                 ["tiled_bytes", "tiled_header_bytes"] + (["tiled_qh_bytes"] if f == "q5k" else []))
        wbufs = [torch.empty(getattr(lib, f"zt_{f}_{p}")(rows, K), dtype=torch.uint8, device="cuda") for p in parts]
        lib.call(f"zt_{f}_tile", raw.data_ptr(), rows, K, *(t.data_ptr() for t in wbufs), s)
        torch.cuda.synchronize()
        del raw
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        wsb = getattr(lib, f"zt_gemm_{f}t_workspace_bytes")(rows, K, N)
        wsbuf = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")
        gemm = getattr(lib, f"zt_gemm_{f}t_f32")
        fn = lambda wb, y: gemm(*(t.data_ptr() for t in wb), x.data_ptr(), y.data_ptr(), rows, K, N, wsbuf.data_ptr(),
                                wsb, s)
        nbytes = synth.algorithmic_bytes(fmt[:4], rows, K, N)
    elif fmt == "w4a16":
        w = synth.w4a16(rows, K, seed)
        wbufs = [dev(w.packed), dev(w.scales), dev(w.zeros)]
        x = dev(synth.x_f16(K * N, seed))
        fn = lambda wb, y: lib.zt_gemm_w4a16_f32(wb[0].data_ptr(), wb[1].data_ptr(), wb[2].data_ptr(), x.data_ptr(),
                                                 y.data_ptr(), rows, K, N, 128, s)
        nbytes = synth.algorithmic_bytes("w4a16", rows, K, N)
    elif fmt == "iq4nlt":
        # the tiled upload layout (zt_iq4nl_tile), built once outside the timing
        w = synth.iq4nl(rows, K, seed)
        nblk = rows * K // 32
        host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
        lib.zt_iq4nl_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
        sep = dev(host)
        wt = torch.empty(lib.zt_iq4nl_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
        st = torch.empty(lib.zt_iq4nl_tiled_scale_bytes(rows, K), dtype=torch.uint8, device="cuda")
        if lib.zt_iq4nl_tile(sep.data_ptr(), rows, K, lib.zt_q4_gpu_data_offset(nblk), wt.data_ptr(), st.data_ptr(),
                             s) != 0:
            raise RuntimeError("zt_iq4nl_tile failed")
        torch.cuda.synchronize()
        del sep
        wbufs = [wt, st]
        x = dev(synth.x_f16(K * N, seed))
        wsb = lib.zt_gemm_iq4nlt_workspace_bytes(rows, K, N)
        wsbuf = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")  # launches run in order on one stream
        fn = lambda wb, y: lib.zt_gemm_iq4nlt_f16(wb[0].data_ptr(), wb[1].data_ptr(), x.data_ptr(), y.data_ptr(), rows,
                                                  K, N, wsbuf.data_ptr(), wsb, s)
        nbytes = synth.algorithmic_bytes("iq4nl", rows, K, N)
    elif fmt == "w4a16sz":
        # batch 1 on the packed (scale, zero) dwords (zt_w4a16_pack_szr), built outside the timing
        w = synth.w4a16(rows, K, seed)
        sc, zr = dev(w.scales), dev(w.zeros)
        szr = torch.empty(w.scales.size, dtype=torch.int32, device="cuda")
        if lib.zt_w4a16_pack_szr(sc.data_ptr(), zr.data_ptr(), rows, K, 128, szr.data_ptr(), s) != 0:
            raise RuntimeError("zt_w4a16_pack_szr failed")
        wbufs = [dev(w.packed), szr]
        x = dev(synth.x_f16(K * N, seed))
        # batch 1: zt_gemv_w4a16sz_f32; batches of 4 and 8: the single-launch row-block MFMA GEMM
        fn = lambda wb, y: lib.zt_gemm_w4a16sz_f32(wb[0].data_ptr(), wb[1].data_ptr(), x.data_ptr(), y.data_ptr(),
                                                   rows, K, N, 128, s)
        nbytes = synth.algorithmic_bytes("w4a16", rows, K, N)
    elif fmt == "w4a16t":
        # the tiled upload layout (zt_w4a16_tile), built once outside the timing
        w = synth.w4a16(rows, K, seed)
        p, sc, zr = dev(w.packed), dev(w.scales), dev(w.zeros)
        wt = torch.empty(lib.zt_w4a16_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
        sz = torch.empty(lib.zt_w4a16_sz_bytes(rows, K, 128), dtype=torch.uint8, device="cuda")
        if lib.zt_w4a16_tile(p.data_ptr(), sc.data_ptr(), zr.data_ptr(), rows, K, 128, wt.data_ptr(), sz.data_ptr(),
                             s) != 0:
            raise RuntimeError("zt_w4a16_tile failed")
        del p, sc, zr
        wbufs = [wt, sz]
        x = dev(synth.x_f16(K * N, seed))
        wsb = lib.zt_gemm_w4a16t_workspace_bytes(rows, K, N)
        wsbuf = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")  # launches run in order on one stream
        fn = lambda wb, y: lib.zt_gemm_w4a16t_f32(wb[0].data_ptr(), wb[1].data_ptr(), x.data_ptr(), y.data_ptr(), rows,
                                                  K, N, 128, wsbuf.data_ptr(), wsb, s)
        nbytes = synth.algorithmic_bytes("w4a16", rows, K, N)
    elif fmt == "ternary_i8":
        t = synth.ternary(rows, K, seed)
        from ztensor_amd.storage import TernaryStorage

        wbufs = [dev(TernaryStorage(t.raw, rows * K).row_aligned(rows, K))]
        q, xs = synth.x_i8(K, seed)
        x = dev(q)
        sc = torch.tensor([xs, t.w_scale], dtype=torch.float32, device="cuda")
        fn = lambda wb, y: lib.zt_ternary_gemv_i8(wb[0].data_ptr(), x.data_ptr(), sc.data_ptr(), sc.data_ptr() + 4,
                                                  y.data_ptr(), rows, K, s)
        nbytes = synth.algorithmic_bytes("ternary_i8", rows, K, N)
    elif fmt == "ternary_f32":
        t = synth.ternary(rows, K, seed)
        from ztensor_amd.storage import TernaryStorage

        wbufs = [dev(TernaryStorage(t.raw, rows * K).row_aligned(rows, K))]
        x = torch.from_numpy(synth.x_f32(K, seed)).cuda()
        fn = lambda wb, y: lib.zt_ternary_gemv_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, s)
        nbytes = synth.algorithmic_bytes("ternary_f32", rows, K, N)
    elif fmt in ("q4_k", "q5_k", "q6_k"):
        w = synth.kquant(fmt, rows, K, seed)
        wbufs = [dev(w.raw)]
        x = torch.from_numpy(synth.x_f32(K, seed)).cuda()
        name = f"zt_gemv_{fmt.replace('_', '')}_f32"
        fn = lambda wb, y: getattr(lib, name)(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, s)
        nbytes = synth.algorithmic_bytes(fmt, rows, K, N)
    elif fmt == "q6_ks":
        # Q6_K batch 1 on the split layout (zt_q6k_split), the same bytes regrouped
        w = synth.kquant("q6_k", rows, K, seed)
        raw = dev(w.raw)
        sp = torch.empty(lib.zt_q6k_split_bytes(rows, K), dtype=torch.uint8, device="cuda")
        lib.call("zt_q6k_split", raw.data_ptr(), rows, K, sp.data_ptr(), s)
        wbufs = [sp]
        x = torch.from_numpy(synth.x_f32(K, seed)).cuda()
        fn = lambda wb, y: lib.zt_gemv_q6ks_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, s)
        nbytes = synth.algorithmic_bytes("q6_k", rows, K, N)
    elif fmt == "q8_0_gguf":
        raw = synth.gguf_q8_0(rows, K, seed)
        nblk = rows * K // 32
        host = np.empty(lib.zt_q8gguf_gpu_bytes(nblk), np.uint8)
        lib.zt_q8gguf_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
        wbufs = [dev(host)]
        off = lib.zt_q8gguf_gpu_data_offset(nblk)
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        fn = lambda wb, y: lib.zt_gemm_q8gguf_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, off, s)
        nbytes = synth.algorithmic_bytes(fmt, rows, K, N)
    elif fmt in ("int4", "int4_rmul"):
        # the reference benchmark's group size (gemm_bench_test.go:47); int4: A [rows, K]; rmul: W [K, rows]
        gs = 32
        w = synth.int4(rows, K, gs, seed) if fmt == "int4" else synth.int4(K, rows, gs, seed)
        wbufs = [dev(w.packed), dev(w.scales), dev(w.zeros)]
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        if fmt == "int4":
            fn = lambda wb, y: lib.zt_gemm_int4_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), wb[1].data_ptr(),
                                                    wb[2].data_ptr(), rows, K, N, gs, s)
        else:
            fn = lambda wb, y: lib.zt_gemm_int4_f32_rmul(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(),
                                                         wb[1].data_ptr(), wb[2].data_ptr(), N, K, rows, gs, s)
        nbytes = synth.algorithmic_bytes("int4", rows, K, N, group=gs)
    elif fmt == "int8":
        wbufs = [dev(synth.int8(rows, K, seed))]
        x = torch.from_numpy(synth.x_f32(K * N, seed)).cuda()
        fn = lambda wb, y: lib.zt_gemm_int8_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, s)
        nbytes = synth.algorithmic_bytes("int8", rows, K, N)
    elif fmt == "q5_0":
        w = synth.kquant(fmt, rows, K, seed)
        nblk = rows * K // 32
        host = np.empty(lib.zt_q5_0_gpu_bytes(nblk), np.uint8)
        lib.zt_q5_0_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
        wbufs = [dev(host)]
        qh, qs = lib.zt_q5_0_gpu_qh_offset(nblk), lib.zt_q5_0_gpu_qs_offset(nblk)
        x = torch.from_numpy(synth.x_f32(K, seed)).cuda()
        fn = lambda wb, y: lib.zt_gemv_q5_0_f32(wb[0].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, qh, qs, s)
        nbytes = synth.algorithmic_bytes(fmt, rows, K, N)
    else:
        raise ValueError(fmt)
    wbytes = sum(b.numel() for b in wbufs)
    copies = int(min(64, max(2, -(-2 * MALL_BYTES // wbytes) + 1)))
    sets = [wbufs] + [[b.clone() for b in wbufs] for _ in range(copies - 1)]
    ys = [torch.empty(rows * N, dtype=torch.float32, device="cuda") for _ in range(copies)]
    # at least 256 launches a graph, two untimed replays, then 10 timed: 60-128-launch
    # graphs measured 5-10% slower per launch and varied more between runs
    n = copies * max(1, -(-256 // copies))
    if eager:
        torch.cuda.synchronize()
        for i in range(eager):
            rc = fn(sets[i % copies], ys[i % copies])
            if rc != 0:
                raise RuntimeError(f"{fmt} launch returned {rc}")
        torch.cuda.synchronize()
        return {"format": fmt, "K": K, "N": rows, "batch": N, "launches": eager, "rotating_copies": copies}

    def loop():
        nonlocal s
        s = torch.cuda.current_stream().cuda_stream
        for i in range(n):
            rc = fn(sets[i % copies], ys[i % copies])
            if rc != 0:
                raise RuntimeError(f"{fmt} launch returned {rc}")

    g = graph_of(torch, loop)
    g.replay()
    g.replay()
    us = time_graph(torch, g, 10) * 1e3 / n
    gbs = nbytes / (us * 1e-6) / 1e9
    r = {"format": fmt, "K": K, "N": rows, "batch": N, "us": round(us, 3), "GB/s": round(gbs, 1),
         "pct_peak": round(100 * gbs / PEAK_GBS, 1), "bytes": nbytes, "rotating_copies": copies}
    rowblock = (fmt in ("int4", "int8") and N % 4 == 0 and K % 32 == 0 and K <= 32768
                and (N <= 16 or (N <= 64 and rows * N <= (1 << 19 if fmt == "int4" else 1 << 18))))
    if rowblock and N > 4:
        # the row-block MFMA GEMM (zt_intq.hip's dispatch): one launch per 4 or 8 columns, HBM-bound
        r["kernel"] = "rowblock"
    elif fmt == "int4_rmul" and N > 4 and ((K <= 8192 and rows % 32 == 0 and N <= 64) or N <= 16):
        # X W past batch 4: the batch-4 kernels once per group of up to 4 rows of X (zt_intq.hip's dispatch)
        r["kernel"] = "rmul_groups_of_4"
    elif fmt in ("int4", "int4_rmul", "int8") and N > 4:
        # useful flops 2 M K N; the MFMA unit the call runs on (zt_intq.hip's dispatch) and its
        # actual MFMA work: bf16 runs 3 MFMAs per product (int4: plus 3 all-ones MFMAs per column
        # tile and step, over TI row tiles), fp32 one
        tf = 2.0 * rows * K * N / (us * 1e-6) / 1e12
        r["TFLOP/s"] = round(tf, 2)
        bf16 = fmt != "int4_rmul" and K % 32 == 0 and N % 2 == 0
        if bf16:
            ti = (4 if -(-rows // 128) * -(-N // 128) >= 256
                  else 1 if -(-rows // 64) * -(-N // 64) < (192 if fmt == "int4" else 256) else 2)
            work = 3.0 if fmt == "int8" else 3.0 + 3.0 / ti
            r["mfma"] = "bf16"
            r["mfma_TFLOP/s"] = round(tf * work, 1)
            r["pct_peak_mfma"] = round(100 * tf * work / PEAK_BF16_TFLOPS, 1)
        else:
            r["mfma"] = "fp32"
            r["mfma_TFLOP/s"] = round(tf, 1)
            r["pct_peak_mfma"] = round(100 * tf / PEAK_FP32_TFLOPS, 1)
    return r


SUITE_FORMATS = ("w4a16_engine", "iq4nl_engine", "int4", "int4_rmul", "int8", "q4_0", "q4_0h", "iq4nl", "iq4nl32", "q8_0", "q8_0_raw", "q4_0t", "q8_0t", "q5_0t", "q4_kt", "q5_kt", "q6_kt", "w4a16",
                 "iq4nlt", "w4a16sz", "w4a16t", "ternary_i8", "ternary_f32", "q4_k", "q5_k", "q6_k", "q6_ks", "q8_0_gguf", "q5_0")


def _pmc_case_arg(v: str) -> str:
    if v in ("q4_0", "w4a16_b8", "w4a16t_b8", "q4_0t_b8"):
        return v
    parts = v.split(":")
    if len(parts) == 4 and parts[0] in SUITE_FORMATS and all(p.isdigit() for p in parts[1:]):
        return v
    raise argparse.ArgumentTypeError(f"not a pmc case: {v}")


def run_pmc_case(args) -> None:
    """A short, fixed workload for rocprofv3 counter passes: the 64 MiB
    calibration copies, then 40 launches of the dominant Q4_0 GEMV (14336 x
    4096, batch 1) rotating over 20 weight copies (660 MB, beyond the
    Infinity Cache)."""
    import torch

    from ztensor_amd import _lib

    lib = _lib.load()
    calibration_copy(torch)
    if ":" in args.pmc_case:
        fmt, rows, K, N = args.pmc_case.split(":")
        if fmt not in SUITE_FORMATS:
            raise SystemExit(f"bench: unknown pmc format {fmt}")
        r = _suite_case(torch, lib, fmt, int(rows), int(K), int(N), 0x5EED0060, eager=40)
        log(f"bench: pmc case {r}")
        return
    if args.pmc_case in ("w4a16_b8", "w4a16t_b8"):
        run_pmc_case_w4a16(torch, lib, tiled=args.pmc_case == "w4a16t_b8")
        return
    if args.pmc_case == "q4_0t_b8":
        run_pmc_case_q4t(torch, lib)
        return
    m = Q4Matrix(torch, lib, 14336, 4096, 0x5EED0024, 20)
    s = torch.cuda.current_stream().cuda_stream
    for i in range(40):
        m.launch(lib, i % 20, s)
    torch.cuda.synchronize()
    log("bench: pmc case done")


def run_pmc_case_w4a16(torch, lib, tiled: bool) -> None:
    """40 launches of the batch-8 W4A16 MFMA GEMM at the Llama-3-70B down
    projection (28672 rows, K = 8192, group 128), rotating over 3 weight
    copies (352 MB, beyond the Infinity Cache), on the row-major layout or
    on the tiled layout (built before the launches)."""
    from ztensor_amd import synth

    rows, K, N = 28672, 8192, 8
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
    s = torch.cuda.current_stream().cuda_stream
    copies = []
    for c in range(3):
        w = synth.w4a16(rows, K, 0x5EED0040 + c)
        bufs = (dev(w.packed), dev(w.scales), dev(w.zeros))
        if tiled:
            wt = torch.empty(lib.zt_w4a16_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
            sz = torch.empty(lib.zt_w4a16_sz_bytes(rows, K, 128), dtype=torch.uint8, device="cuda")
            if lib.zt_w4a16_tile(*(b.data_ptr() for b in bufs), rows, K, 128, wt.data_ptr(), sz.data_ptr(), s) != 0:
                raise SystemExit("bench: zt_w4a16_tile failed")
            bufs = (wt, sz)
        copies.append(bufs)
    x = dev(synth.x_f16(K * N, 0x5EED0043))
    y = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    wsb = lib.zt_gemm_w4a16t_workspace_bytes(rows, K, N)
    wsbuf = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for i in range(40):
        b = copies[i % 3]
        if tiled:
            rc = lib.zt_gemm_w4a16t_f32(b[0].data_ptr(), b[1].data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, 128,
                                        wsbuf.data_ptr(), wsb, s)
        else:
            rc = lib.zt_gemm_w4a16_f32(b[0].data_ptr(), b[1].data_ptr(), b[2].data_ptr(), x.data_ptr(), y.data_ptr(),
                                       rows, K, N, 128, s)
        if rc != 0:
            raise SystemExit(f"bench: W4A16 GEMM returned {rc}")
    torch.cuda.synchronize()
    log(f"bench: pmc case {'w4a16t_b8' if tiled else 'w4a16_b8'} done")


def run_pmc_case_q4t(torch, lib) -> None:
    """40 launches of the batch-8 Q4_0 MFMA GEMM on the tiled layout at the
    Llama-3-8B gate/up shape (14336 rows, K = 4096), rotating over 20 weight
    copies (700 MB, beyond the Infinity Cache); K is split 8 ways, so each
    launch is the GEMM and the split-K reduction."""
    from ztensor_amd import synth

    rows, K, N = 14336, 4096, 8
    s = torch.cuda.current_stream().cuda_stream
    w = synth.q4_0(rows, K, 0x5EED0050)
    nblk = rows * K // 32
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    sep = torch.from_numpy(host).cuda()
    wt = torch.empty(lib.zt_q4_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
    st = torch.empty(lib.zt_q4_tiled_scale_bytes(rows, K), dtype=torch.uint8, device="cuda")
    if lib.zt_q4_tile(sep.data_ptr(), rows, K, lib.zt_q4_gpu_data_offset(nblk), wt.data_ptr(), st.data_ptr(), s) != 0:
        raise SystemExit("bench: zt_q4_tile failed")
    copies = [(wt, st)] + [(wt.clone(), st.clone()) for _ in range(19)]
    x = torch.from_numpy(synth.x_f32(K * N, 0x5EED0051)).cuda()
    y = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    wsb = lib.zt_gemm_q4t_workspace_bytes(rows, K, N)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for i in range(40):
        a, b = copies[i % 20]
        rc = lib.zt_gemm_q4t_f32(a.data_ptr(), b.data_ptr(), x.data_ptr(), y.data_ptr(), rows, K, N, ws.data_ptr(), wsb,
                                 s)
        if rc != 0:
            raise SystemExit(f"bench: Q4_0 tiled GEMM returned {rc}")
    torch.cuda.synchronize()
    log("bench: pmc case q4_0t_b8 done")


def run_suite(args) -> None:
    import torch

    from ztensor_amd import _lib

    lib = _lib.load()
    only = set(args.only.split(",")) if args.only else None
    for ci, (name, (fmt, shapes, batches)) in enumerate(SUITE.items()):
        if only and name not in only:
            continue
        for si, (rows, K) in enumerate(shapes):
            for N in batches:
                N = rows if N == "square" else N
                r = _suite_case(torch, lib, fmt, rows, K, N, 0x5EED0000 + 16 * ci + si)
                r["config"] = name
                print(json.dumps(r), flush=True)
                log(f"suite: {name:10s} K={K:5d} N={rows:5d} batch={N:2d}: {r['us']:8.2f} us {r['GB/s']:8.1f} GB/s "
                    f"({r['pct_peak']:.1f}%)")
                torch.cuda.empty_cache()


# The five benchmark configurations of this path (W4A16 GEMV, Q4_0 / Q8_0 at
# the Llama-3-8B shapes, BitNet ternary, W4A16 at the Llama-3-70B shapes,
# IQ4_NL at the Qwen2-7B shapes) as run by the engine's dispatch (batch-1
# W4A16 on packed (scale, zero) dwords, batched W4A16 and IQ4_NL on their
# tiled layouts), reported beside the headline.
CONFIGS = {
    "1_w4a16_gemv": ["w4a16sz_c1"],
    "2_q4_0_q8_0_llama3_8b": ["q4_0", "q8_0"],
    "3_ternary_bitnet": ["ternary"],
    "4_w4a16_llama3_70b": ["w4a16_70b_engine"],
    "5_iq4nl_qwen2_7b": ["iq4nl_engine"],
}


def run_configs(torch, lib) -> dict:
    """Per-configuration timings (graph replays over rotating weight copies,
    as --suite): {config: [[format, "KxN", batch, us, pct_of_peak], ...]}."""
    out = {}
    names = list(SUITE)
    for cfg, entries in CONFIGS.items():
        rows_out = []
        for e in entries:
            name, only_batches = (e if isinstance(e, tuple) else (e, None))
            fmt, shapes, batches = SUITE[name]
            ci = names.index(name)
            for si, (rows, K) in enumerate(shapes):
                for N in batches:
                    if only_batches is not None and N not in only_batches:
                        continue
                    r = _suite_case(torch, lib, fmt, rows, K, N, 0x5EED0000 + 16 * ci + si)
                    rows_out.append([r["format"], f"{K}x{rows}", N, r["us"], r["pct_peak"]])
                    torch.cuda.empty_cache()
        out[cfg] = rows_out
        log(f"bench: config {cfg}: " + ", ".join(f"{f} {s} b{n} {us:.2f}us {p:.1f}%" for f, s, n, us, p in rows_out))
    return out


def cpu_configs(budget_s: float = 2.0) -> dict:
    """The CPU restatement of each configuration's reference CPU path on one
    representative shape, timed on the host (about budget_s each):
    W4A16 and IQ4_NL dequantize then SgemmSimd (compute/w4a16.go:71-119,
    compute/cpu_engine.go:1215-1245), Q8_0 GemmF32Q8NT
    (internal/xblas/gemm_quant.go:163-264), ternary TernaryGEMV
    (compute/ternary_gemv.go:12-77)."""
    from oracle import oracle
    from ztensor_amd import synth

    th = min(16, oracle.nthreads())
    w1 = synth.w4a16(4096, 4096, 0x5EED0011)
    x1 = synth.x_f16(4096, 0x5EED0011)
    q8 = synth.q8_0(14336, 4096, 0x5EED0012)
    x2 = synth.x_f32(4096, 0x5EED0012)
    t3 = synth.ternary(6912, 2560, 0x5EED0013)
    x3 = synth.x_f32(2560, 0x5EED0013)
    w4 = synth.w4a16(8192, 8192, 0x5EED0014)
    x4 = synth.x_f16(8192 * 8, 0x5EED0014)
    i5 = synth.iq4nl(18944, 3584, 0x5EED0015)
    x5 = synth.x_f16(3584 * 8, 0x5EED0015)
    cases = {
        "1_w4a16_gemv": ("w4a16 4096x4096 batch 1, dequantize + SgemmSimd", 1,
                         synth.algorithmic_bytes("w4a16", 4096, 4096, 1),
                         lambda: oracle.w4a16_matmul(w1.packed, w1.scales, w1.zeros, x1, 4096, 4096, 1, 128)),
        "2_q4_0_q8_0_llama3_8b": ("q8_0 4096x14336 batch 1, GemmF32Q8NT", th,
                                  synth.algorithmic_bytes("q8_0", 14336, 4096, 1),
                                  lambda: oracle.gemm_f32_q8_nt(x2, q8.raw, 1, 14336, 4096, threads=th)),
        "3_ternary_bitnet": ("ternary 2560x6912 batch 1, TernaryGEMV", 1, 6912 * 640 + 4 * 2560 + 4 * 6912,
                             lambda: oracle.ternary_gemv(t3.raw, x3, 6912, 2560)),
        "4_w4a16_llama3_70b": ("w4a16 8192x8192 batch 8, dequantize + SgemmSimd", 1,
                               synth.algorithmic_bytes("w4a16", 8192, 8192, 8),
                               lambda: oracle.w4a16_matmul(w4.packed, w4.scales, w4.zeros, x4, 8192, 8192, 8, 128)),
        "5_iq4nl_qwen2_7b": ("iq4nl 3584x18944 batch 8, dequantize + SgemmSimd", 1,
                             synth.algorithmic_bytes("iq4nl", 18944, 3584, 8),
                             lambda: oracle.iq4nl_matmul(i5.raw, x5, 18944, 3584, 8)),
    }
    out = {}
    for cfg, (case, threads, nbytes, fn) in cases.items():
        reps, t = 0, 0.0
        while t < budget_s or reps == 0:
            t0 = time.perf_counter()
            fn()
            t += time.perf_counter() - t0
            reps += 1
        us = t / reps * 1e6
        out[cfg] = {"case": case, "us": round(us, 1), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 3), "threads": threads,
                    "kind": "port", "calls": reps}
        log(f"bench: cpu {cfg}: {case}: {us:.0f} us/call on {threads} thread(s)")
    return out


def summarize_trace(path: str) -> None:
    """Per-launch-shape durations from a rocprofv3 kernel-trace CSV, as a
    markdown table: kernel, grid and block size, calls, median and mean us.
    The --stats averages mix every shape a kernel runs; this splits them."""
    import csv
    import statistics

    groups: dict = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            key = (r["Kernel_Name"][:60], int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
            groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("| kernel | grid (threads) | block | calls | median us | mean us |")
    print("|---|---|---|---|---|---|")
    for (name, grid, block), v in sorted(groups.items()):
        print(f"| `{name}` | {grid} | {block} | {len(v)} | {statistics.median(v):.3f} | {statistics.fmean(v):.3f} |")


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    ap.add_argument("--no-merged", dest="merged", action="store_false",
                    help="skip the merged Q/K/V + Gate/Up variant reported beside the headline")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="skip the per-configuration timings reported beside the headline")
    ap.add_argument("--suite", action="store_true", help="per-configuration table instead of the headline")
    ap.add_argument("--only", default="", help="comma-separated suite entries (with --suite)")
    ap.add_argument("--pmc-case", nargs="?", const="q4_0", type=_pmc_case_arg,
                    help="short fixed workload for rocprofv3 counter passes: copies + 40 launches of the dominant "
                         "Q4_0 GEMV (default), of the W4A16 batch-8 MFMA GEMM at 28672 x 8192 on the row-major "
                         "(w4a16_b8) or tiled (w4a16t_b8) layout, or of the batch-8 Q4_0 tiled GEMM at "
                         "14336 x 4096 (q4_0t_b8); FORMAT:ROWS:K:BATCH runs 40 launches of any suite "
                         "format at that shape (e.g. iq4nlt:3584:3584:8)")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="run 64 MiB device copies first (reference kernel for rocprofv3 byte counters)")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print per-launch-shape durations of a rocprofv3 kernel-trace CSV and exit (no GPU)")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this path runs on one GPU; multi-GPU runs are not part of this build. "
              "Sharded, each GPU would run the same kernels on its slice: output rows for q/k/v/gate/up, "
              "K for o/down followed by an all-reduce of the partial outputs", file=sys.stderr)
        raise SystemExit(2)
    if args.suite:
        run_suite(args)
        return
    if args.pmc_case:
        run_pmc_case(args)
        return
    result = run_headline(args)
    if args.configs:
        import torch

        from ztensor_amd import _lib

        result["configs"] = run_configs(torch, _lib.load())
        if args.cpu_baseline:
            result["configs_cpu"] = cpu_configs()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
