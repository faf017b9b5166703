#!/usr/bin/env python3
"""Benchmark of the fused per-layer kernels on one MI355X.

Workload ("step"): one call of each fused kernel at the BASELINE.json configs,
inputs resident in HBM:
  C1  rmsnorm fp32 [36 x 2048]
  C2  Q/K head RMSNorm + partial RoPE, Q [512x16x256], K [512x2x256] (in place)
  C3a residual add + RMSNorm, bf16 [4096 x 2048]
  C3b SwiGLU bf16 [4096 x 8 x 512]
  C3c shared-expert SwiGLU x sigmoid(logit), bf16 [4096 x 512]
  C4a GDN conv1d(k=4) + SiLU + Q/K L2, fp32 [4096 x 8192]
  C4b GDN gated per-head RMSNorm, fp32 [4096 x 32 x 128]
  C5  Q4_K and Q6_K embedding dequant-gather, 8192 ids from 248320 x 2048

The timed region replays the step as one HIP graph (the nine launches with no
host work between them), K times, bracketed by torch.cuda.synchronize();
value = algorithmic bytes per step / wall time per step.

Per-kernel figures (the metric's "GB/s and us/call per kernel"): each kernel is
timed on its own stream with HIP events around single launches, each launch
preceded by a 512 MiB read of an unrelated buffer so that neither L2 nor the
256 MB MALL holds the kernel's inputs (a cold, HBM-bound call), and a spin
kernel ahead of each batch so all launches are queued before the GPU reaches
them. Algorithmic bytes count every input read once and every output written
once. The roofline object reports the kernel with the largest time per step.

CPU baseline: the oracle (oracle/liboracle.so, a C++ restatement of the
reference kernels) timed on this host on a bounded sample of each config.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen-3.5-cuda_amd"))

METRIC = "achieved HBM GB/s (% of MI355X peak) + µs/call per fused norm/RoPE/act kernel"
PEAK_GBPS = 8000.0  # MI355X HBM3E
FLUSH_BYTES = 512 << 20


class Kernel:
    def __init__(self, name, config, nbytes, launch, cpu=None):
        self.name, self.config, self.bytes, self.launch, self.cpu = name, config, nbytes, launch, cpu
        self.us = None
        self.us_warm = None


def build_workload(torch, ops, synth, with_host: bool):
    """Returns [Kernel] with device buffers bound into each launch closure, and
    the host inputs needed by the CPU baseline."""
    dev = torch.device("cuda:0")

    def d(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
        return torch.from_numpy(a).to(dev)

    ks: list[Kernel] = []
    host = {}

    c = synth.c1_rmsnorm()
    x, w = d(c["x"]), d(c["w"])
    out = torch.empty_like(x)
    nb = 2 * x.numel() * 4 + w.numel() * 4
    ks.append(Kernel("rmsnorm", "C1 f32 [36x2048]", nb, lambda x=x, w=w, out=out: ops.rmsnorm_rows(x, w, out)))
    host["rmsnorm"] = c

    c = synth.c2_qk_rope()
    q, k, qw, kw, pos = d(c["q"]), d(c["k"]), d(c["qw"]), d(c["kw"]), d(c["pos"])
    nb = 2 * (q.numel() + k.numel()) * 4 + (qw.numel() + kw.numel()) * 4 + pos.numel() * 4
    ks.append(Kernel("qk_norm_rope", "C2 f32 Q[512x16x256] K[512x2x256] rd64 theta1e7", nb,
                     lambda: ops.attn_qk_norm_rope_rows(q, k, qw, kw, pos=pos, rope_dim=64, theta=1e7)))
    host["qk_norm_rope"] = c

    c = synth.c3_residual()
    xr, br, wr = d(c["x"]), d(c["branch"]), d(c["w"])
    resid, normed = torch.empty_like(xr), torch.empty_like(xr)
    nb = 4 * xr.numel() * 2 + wr.numel() * 4
    ks.append(Kernel("residual_rmsnorm_bf16", "C3a bf16 [4096x2048]", nb,
                     lambda: ops.residual_rmsnorm_rows(xr, br, wr, resid, normed)))
    host["residual_rmsnorm_bf16"] = c

    c = synth.c3_swiglu()
    g, u = d(c["g"]), d(c["u"])
    h = torch.empty_like(g)
    nb = 3 * g.numel() * 2
    ks.append(Kernel("swiglu_bf16", "C3b bf16 [4096x8x512]", nb, lambda: ops.swiglu_bf16(g, u, h)))
    host["swiglu_bf16"] = c

    c = synth.c3_shared()
    gs, us_, lg = d(c["g"]), d(c["u"]), d(c["logits"])
    hs = torch.empty_like(gs)
    nb = 3 * gs.numel() * 2 + lg.numel() * 4
    ks.append(Kernel("shared_swiglu_sigmoid_bf16", "C3c bf16 [4096x512] + logits", nb,
                     lambda: ops.shared_swiglu_sigmoid_rows_bf16(gs, us_, lg, hs)))
    host["shared_swiglu_sigmoid_bf16"] = c

    c = synth.c4_frontend()
    xc, wc, hin = d(c["x"]), d(c["w"]), d(c["hist"])
    hout, yc = torch.empty_like(hin), torch.empty_like(xc)
    nb = 2 * xc.numel() * 4 + wc.numel() * 4 + 2 * hin.numel() * 4
    ks.append(Kernel("gdn_frontend", "C4a f32 [4096x8192] k4, 16 key heads x128", nb,
                     lambda: ops.gdn_frontend_rows(xc, wc, hin, hout, yc, k_heads=16, key_dim=128)))
    host["gdn_frontend"] = c

    c = synth.c4_norm_gate()
    xg, zg, wg = d(c["x"]), d(c["z"]), d(c["w"])
    og = torch.empty_like(xg)
    nb = 3 * xg.numel() * 4 + wg.numel() * 4
    ks.append(Kernel("gdn_norm_gate", "C4b f32 [4096x32x128]", nb, lambda: ops.gdn_norm_gate_rows(xg, zg, wg, og)))
    host["gdn_norm_gate"] = c

    vocab, cols = 248320, 2048
    ids_h = synth.token_ids(8192, vocab)
    ids = d(ids_h)
    for kind, make, bpr in (("Q4_K", synth.q4k_table, 1152), ("Q6_K", synth.q6k_table, 1680)):
        tab_h = make(vocab, cols)
        tab = d(tab_h)
        o = torch.empty((8192, cols), dtype=torch.float32, device=dev)
        nb = 8192 * bpr + ids.numel() * 4 + o.numel() * 4
        name = f"dequant_gather_{kind.lower()}"
        ks.append(Kernel(name, f"C5 {kind} 248320x2048, 8192 ids", nb,
                         lambda tab=tab, kind=kind, o=o: ops.dequant_gather_rows(tab, kind, vocab * cols, ids, cols, o)))
        host[name] = {"table": tab_h if with_host else None, "ids": ids_h, "type": ops.GGML_TYPES[kind]}
    return ks, host


def spin_cycles_per_ms(torch) -> float:
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)
    s.record()
    torch.cuda._sleep(2_000_000)
    e.record()
    torch.cuda.synchronize()
    return 2_000_000 / max(s.elapsed_time(e), 1e-3)


def time_kernel(torch, k: Kernel, flush, spin, reps: int, batch: int, cold: bool) -> float:
    """Median event-timed duration (us) of single launches of k."""
    times = []
    done = 0
    while done < reps:
        n = min(batch, reps - done)
        torch.cuda._sleep(spin)
        evs = []
        for _ in range(n):
            if cold:
                flush()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            k.launch()
            e1.record()
            evs.append((e0, e1))
        torch.cuda.synchronize()
        times += [a.elapsed_time(b) * 1e3 for a, b in evs]
        done += n
    return statistics.median(times)


def cpu_baseline(host, kernels, threads: int, budget_s: float):
    """Times the oracle on a bounded sample of every config; returns per-kernel
    (GB/s, sample description) and the aggregate."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle as orc

    orc.lib()
    by = {k.name: k for k in kernels}
    frac_rows = {  # sample size per config
        "rmsnorm": 36, "qk_norm_rope": 64, "residual_rmsnorm_bf16": 512, "swiglu_bf16": 512,
        "shared_swiglu_sigmoid_bf16": 4096, "gdn_frontend": 256, "gdn_norm_gate": 512,
        "dequant_gather_q4_k": 1024, "dequant_gather_q6_k": 1024,
    }
    full_rows = {"rmsnorm": 36, "qk_norm_rope": 512, "residual_rmsnorm_bf16": 4096, "swiglu_bf16": 4096,
                 "shared_swiglu_sigmoid_bf16": 4096, "gdn_frontend": 4096, "gdn_norm_gate": 4096,
                 "dequant_gather_q4_k": 8192, "dequant_gather_q6_k": 8192}

    def runner(name, rows, th):
        c = host[name]
        if name == "rmsnorm":
            return lambda: orc.rmsnorm_rows(c["x"][:rows], c["w"], threads=th)
        if name == "qk_norm_rope":
            return lambda: orc.qk_norm_rope_rows(c["q"][:rows], c["k"][:rows], c["qw"], c["kw"], pos=c["pos"][:rows],
                                                 rope_dim=64, theta=1e7, threads=th)
        if name == "residual_rmsnorm_bf16":
            return lambda: orc.residual_rmsnorm_rows(c["x"][:rows], c["branch"][:rows], c["w"], threads=th)
        if name == "swiglu_bf16":
            return lambda: orc.swiglu_bf16(c["g"][:rows], c["u"][:rows], threads=th)
        if name == "shared_swiglu_sigmoid_bf16":
            return lambda: orc.shared_swiglu_sigmoid_bf16(c["g"][:rows], c["u"][:rows], c["logits"][:rows], threads=th)
        if name == "gdn_frontend":
            return lambda: orc.gdn_frontend_rows(c["x"][:rows], c["w"], c["hist"], threads=th)
        if name == "gdn_norm_gate":
            return lambda: orc.norm_gate_rows(c["x"][:rows], c["z"][:rows], c["w"], threads=th)
        return lambda: orc.dequant_gather(c["table"], c["type"], c["ids"][:rows], 2048, threads=th)

    per, tot_b, tot_t = {}, 0.0, 0.0
    per_budget = budget_s / len(by)
    for name, k in by.items():
        rows = frac_rows[name]
        fn = runner(name, rows, threads)
        fn()  # warm
        t0 = time.perf_counter()
        n = 0
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el > per_budget or n >= 200:
                break
        sec = el / n
        b = k.bytes * rows / full_rows[name]
        per[name] = {"gbps": b / sec / 1e9, "us_per_call_full": sec * full_rows[name] / rows * 1e6,
                     "sample_rows": rows}
        tot_b += k.bytes
        tot_t += sec * full_rows[name] / rows
    return per, tot_b / tot_t / 1e9


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=40, help="event-timed launches per kernel")
    ap.add_argument("--kernels", default="", help="comma list: only these kernels (profiling)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a graph replay")
    ap.add_argument("--json-out", default="", help="also write the JSON line to this file")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every kernel is row-local and the multi-GPU path is not built)", file=sys.stderr)
        return 2

    import torch

    from qwen35_hip import load, ops, synth

    load()  # fail loudly if the HIP library is missing
    torch.cuda.set_device(0)
    t_setup = time.perf_counter()
    kernels, host = build_workload(torch, ops, synth, with_host=not args.no_cpu)
    if args.kernels:
        keep = set(args.kernels.split(","))
        kernels = [k for k in kernels if k.name in keep]
    torch.cuda.synchronize()
    print(f"# setup {time.perf_counter() - t_setup:.1f}s, {len(kernels)} kernels", file=sys.stderr, flush=True)

    flush_buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device="cuda:0")
    flush_out = torch.empty((), dtype=torch.float32, device="cuda:0")

    def flush():
        torch.sum(flush_buf, dtype=torch.float32, out=flush_out)

    spin = int(spin_cycles_per_ms(torch) * 4.0)  # ~4 ms of spin ahead of each batch

    for k in kernels:  # warm-up: first launches load code objects
        k.launch()
    torch.cuda.synchronize()

    # ---- per-kernel cold-cache timing
    for k in kernels:
        k.us = time_kernel(torch, k, flush, spin, args.reps, 10, cold=True)
        k.us_warm = time_kernel(torch, k, flush, spin, max(args.reps // 2, 5), 20, cold=False)
        print(f"# {k.name:28s} {k.us:9.2f} us cold ({k.bytes / k.us / 1e3:7.1f} GB/s, "
              f"{k.bytes / k.us / 1e3 / PEAK_GBPS:6.1%}), {k.us_warm:9.2f} us warm", file=sys.stderr, flush=True)

    # ---- timed steps (the contract): K graph replays of the whole step
    graph = None
    if not args.eager:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for k in kernels:
                k.launch()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for k in kernels:
                k.launch()

    def step():
        if graph is not None:
            graph.replay()
        else:
            for k in kernels:
                k.launch()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    bytes_step = sum(k.bytes for k in kernels)
    value = bytes_step / (ms_per_step * 1e-3) / 1e9
    print(f"# step: {ms_per_step * 1e3:.1f} us, {value:.1f} GB/s aggregate", file=sys.stderr, flush=True)

    # ---- roofline of the dominant kernel
    dom = max(kernels, key=lambda k: k.us)
    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get(dom.name, {}).get("bytes_per_launch")
    roofline = {"kernel": dom.name, "bound": "hbm", "achieved": round(dom.bytes / dom.us / 1e3, 1),
                "peak": PEAK_GBPS, "unit": "GB/s", "frac": round(dom.bytes / dom.us / 1e3 / PEAK_GBPS, 4),
                "traffic": traffic, "algorithmic_bytes": dom.bytes, "us_per_call": round(dom.us, 3)}

    # ---- CPU baseline
    cpu = None
    if not args.no_cpu and not args.kernels:
        threads = max(1, min(16, os.cpu_count() or 1))
        per, agg = cpu_baseline(host, kernels, threads, args.cpu_seconds)
        cpu = {"value": round(agg, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": ("oracle/liboracle.so (C++ restatement of the reference kernels, -O2) on the first rows "
                          "of each config: " + ", ".join(f"{n} {p['sample_rows']}" for n, p in per.items())
                          + f"; row-parallel std::threads; host CPU {cpu_model()}"),
               "per_kernel_gbps": {n: round(p["gbps"], 3) for n, p in per.items()}}

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: splitmix64 + Box-Muller inputs, seeds 0x5EED0000+k, BASELINE.json configs C1-C5",
        "config": {"workload": "one call of each of the 9 fused kernels at BASELINE configs C1-C5 "
                               "(HIP graph replay; storage f32/bf16/Q4_K/Q6_K, math f32)",
                   "bytes_per_step": bytes_step, "parallelism": "single GPU",
                   "graph": graph is not None},
        "kernels": {k.name: {"config": k.config, "bytes": k.bytes, "us_per_call": round(k.us, 3),
                             "gbps": round(k.bytes / k.us / 1e3, 1),
                             "frac_peak": round(k.bytes / k.us / 1e3 / PEAK_GBPS, 4),
                             "us_per_call_warm_cache": round(k.us_warm, 3)} for k in kernels},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    text = json.dumps(line)
    print(text, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
