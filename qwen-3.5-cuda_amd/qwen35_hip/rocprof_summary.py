"""Summarise rocprofv3 outputs of bench.py runs into the profile tables.

  python -m qwen35_hip.rocprof_summary stats   KERNEL_STATS.csv
      per-kernel dispatch count and average / min / max duration (us)
  python -m qwen35_hip.rocprof_summary steady KERNEL_TRACE.csv TIMED.json
      per-kernel duration (us) over the dispatches of the steady-state timed
      batches only: the last N dispatches of each kernel, N from the counts
      bench.py --timed-counts wrote (no step-graph, warm-up or eager dispatches)
  python -m qwen35_hip.rocprof_summary traffic FETCH.csv WRITE.csv COPY_BYTES [--json OUT]
      per-kernel FETCH_SIZE / WRITE_SIZE (KiB per dispatch, from two --pmc runs),
      scaled to bytes by the factor that makes the reference copy of COPY_BYTES
      read + COPY_BYTES written read exactly its known traffic, next to each
      kernel's algorithmic bytes
  python -m qwen35_hip.rocprof_summary counters COUNTERS.csv [...] [--match SYM] [--stages N]
      mean per dispatch of every counter of the --pmc runs for the kernels whose
      symbol contains SYM; per wave and stage (N stages per wave: K / 32 of the
      prefill GEMM, the chunks of the chunked GDN state walk) with SQ_WAVES; the MFMA-busy
      share (SQ_VALU_MFMA_BUSY_CYCLES over 1024 SIMDs x SQ_BUSY_CYCLES / 32 SEs)

Kernel symbols are mapped to the bench.py kernel names; the reference copies are
"copy16" and "copy_form" (libqwen35_benchutil.so).
"""

from __future__ import annotations

import argparse
import csv
import hashlib
import json
import sys
from collections import defaultdict
from pathlib import Path

# symbol substring -> bench.py kernel name (first match wins)
NAMES = [
    ("gdn_frontend_k4", "gdn_frontend"),
    ("norm_gate_v4", "gdn_norm_gate"),
    ("swiglu_routed_shared_v8", "swiglu_routed_shared_bf16"),
    ("swiglu_bf16_v8ILi2ELb1", "shared_swiglu_sigmoid_bf16"),
    ("swiglu_bf16_v8ILi2ELb0", "swiglu_bf16"),
    ("swiglu_bf16_v8<2, true>", "shared_swiglu_sigmoid_bf16"),
    ("swiglu_bf16_v8<2, false>", "swiglu_bf16"),
    ("gather_q4k", "dequant_gather_q4_k"),
    ("gather_q6k", "dequant_gather_q6_k"),
    ("residual_rmsnorm_bf16_v8", "residual_rmsnorm_bf16"),
    ("qk_norm_rope_grouped", "qk_norm_rope"),
    ("qk_norm_rope_v4", "qk_norm_rope"),
    ("rmsnorm_rows_split", "rmsnorm"),
    ("rmsnorm_rows_v4", "rmsnorm"),
    ("copy16", "copy"),
    ("copy_form", "copy"),
    # next rows (kernel symbols; several bench shapes can share one instantiation)
    ("gemv_mfma<14, 2>", "gemv Q6_K MFMA, 2-block k-slices (LM head)"),
    ("gemv_mfma<12, 2>", "gemv Q4_K MFMA, 2-block k-slices"),
    ("gemv_q4k_direct_swiglu", "gemv Q4_K direct, MoE SwiGLU rows (moe_route_swiglu)"),
    ("gemv_q4k_norm_gate", "gemv Q4_K direct after the gated norm (gdn_norm_gate_matmul)"),
    ("moe_down_combine_q4k", "moe_down_combine, Q4_K direct (routed + shared down, combine)"),
    ("gemv_q4k_direct_multi", "gemv Q4_K direct, several matrices of one x (matmul_dispatch_multi)"),
    ("gemv_q4k_direct_gate_up", "gemv Q4_K direct, routed experts' gate + up (moe_expert_gate_up)"),
    ("gemv_q4k_direct<2, 1,", "gemv Q4_K direct, 2 rows/wave (GDN qkv)"),
    ("gemv_q4k_direct<2, 2,", "gemv Q4_K direct, 2 rows/wave, 2-unit rows (out proj)"),
    ("gemv_q4k_direct<1, 1,", "gemv Q4_K direct, 1 row/wave (experts)"),
    ("gemv_q4k_direct", "gemv Q4_K direct, other shapes"),
    ("gemv_q6k_direct_multi", "gemv Q6_K direct, several matrices of one x (matmul_dispatch_multi)"),
    ("gemv_q6k_direct<2,", "gemv Q6_K direct, 2 rows/wave (8192-row matrices)"),
    ("gemv_q6k_direct<1,", "gemv Q6_K direct, 1 row/wave"),
    ("gemv_q6k_direct", "gemv Q6_K direct, other shapes"),
    ("gemv_kquant<14, 4>", "gemv Q6_K per-row, 4 units/wave"),
    ("gemv_kquant<12, 2>", "gemv Q4_K per-row, 2 units/wave (GDN qkv)"),
    ("gemv_kquant<12, 1>", "gemv Q4_K per-row, 1 unit/wave (out proj, experts)"),
    ("gemv_kquant_multi", "gemv per-row, several matrices of one x (matmul_dispatch_multi)"),
    ("gemv_kquant_gate_up", "gemv per-row, routed experts' gate + up (moe_expert_gate_up)"),
    ("moe_down_combine_kernel", "moe_down_combine (routed + shared down, combine)"),
    ("gdn_step_tile", "gdn_recurrent step (decode, 16-column tiles)"),
    ("gdn_recurrent_v4", "gdn_recurrent step (decode, 4-column slices)"),
    ("gdn_decode_fused", "gdn_decode_step (front end + gated step, one launch)"),
    ("gdn_recurrent_g", "gdn_recurrent token loop (4096 tokens)"),
    ("gdn_chunk_prep", "gdn_recurrent chunked: per-chunk prep"),
    ("gdn_chunk_state", "gdn_recurrent chunked: state walk"),
    ("decode_split", "attn_decode split-K pass"),
    ("decode_combine", "attn_decode combine"),
    ("scores_split", "attn_scores (drop-in, MFMA tiles)"),
    ("scores_kernel", "attn_scores (drop-in, other shapes)"),
    ("softmax_regs", "attn_softmax (drop-in, row in registers)"),
    ("softmax_loop", "attn_softmax (drop-in, long rows)"),
    ("values_cols", "attn_values (drop-in)"),
    ("topk_group_kernel", "moe_topk, two rows per wave (top-k of <= 256)"),
    ("topk_rows_kernel", "moe_topk_rows"),
    ("weighted_sum_v4", "moe_weighted_sum_rows"),
    ("gates_kernel", "gdn gates (decode, separate launch)"),
    ("sigmoid_gate_kernel", "attn sigmoid gate (drop-in)"),
    ("gemm_prep_x", "matmul_rows prep (x to fp16 parts)"),
    ("gemm_q4k", "matmul_rows Q4_K GEMM, fp16 MFMA"),
    ("gemm_q6k", "matmul_rows Q6_K GEMM, fp16 MFMA"),
]

# algorithmic bytes per call at the BASELINE configs (bench.py computes the same)
ALGORITHMIC = {
    "rmsnorm": 598016, "qk_norm_rope": 18878464, "residual_rmsnorm_bf16": 67117056, "swiglu_bf16": 100663296,
    "shared_swiglu_sigmoid_bf16": 12599296, "gdn_frontend": 268763136, "gdn_norm_gate": 201327104,
    "dequant_gather_q4_k": 76578816, "dequant_gather_q6_k": 80904192, "swiglu_routed_shared_bf16": 113262592,
    # the LM-head GEMV (bench.py next rows: Q6_K 248320 x 2048, x and y fp32)
    "gemv Q6_K MFMA, 2-block k-slices (LM head)": 418179072,
}


# Source files (qwen-3.5-cuda_amd/csrc) each counted kernel is compiled from,
# with the headers they include. The traffic summary records their digest, so a
# counter figure is used (bench.py) only while the kernel source is the one it
# was measured on.
CSRC = Path(__file__).resolve().parents[1] / "csrc"
_COMMON = ["capi_common.hpp", "device_common.hpp", "../../include/qwen35_hip.h"]
KERNEL_SOURCES = {
    "rmsnorm": ["norm.hip"], "residual_rmsnorm_bf16": ["norm.hip"], "qk_norm_rope": ["attn.hip", "attn_common.hpp"],
    "swiglu_bf16": ["moe.hip"], "shared_swiglu_sigmoid_bf16": ["moe.hip"], "swiglu_routed_shared_bf16": ["moe.hip"],
    "gdn_frontend": ["gdn.hip", "gdn_common.hpp"], "gdn_norm_gate": ["gdn.hip", "gdn_common.hpp"],
    "dequant_gather_q4_k": ["dequant.hip", "ggml_common.hpp"], "dequant_gather_q6_k": ["dequant.hip", "ggml_common.hpp"],
    "gemv Q6_K MFMA, 2-block k-slices (LM head)": ["gemv.hip", "ggml_common.hpp", "moe_common.hpp"],
}


def sources_digest(name: str) -> str | None:
    """sha256 (16 hex digits) over the kernel's source files, or None for a kernel
    without a source list."""
    files = KERNEL_SOURCES.get(name)
    if files is None:
        return None
    h = hashlib.sha256()
    for f in sorted(files + _COMMON):
        h.update(f.encode())
        h.update((CSRC / f).read_bytes())
    return h.hexdigest()[:16]


def kernel_name(symbol: str) -> str | None:
    for key, name in NAMES:
        if key in symbol:
            return name
    return None


def stats(path: str) -> dict:
    out = {}
    for r in csv.DictReader(open(path)):
        name = kernel_name(r["Name"])
        if name is None:
            continue
        out.setdefault(name, []).append(r)
    table = {}
    for name, rs in out.items():
        calls = sum(int(r["Calls"]) for r in rs)
        total = sum(float(r["TotalDurationNs"]) for r in rs)
        table[name] = {"calls": calls, "avg_us": total / calls / 1e3, "min_us": min(float(r["MinNs"]) for r in rs) / 1e3,
                       "max_us": max(float(r["MaxNs"]) for r in rs) / 1e3}
    return table


def steady(trace_csv: str, timed_json: str) -> dict:
    """Duration statistics over each kernel's last N dispatches, N = the number
    of launches in its timed batches (bench.py --timed-counts): in a run that
    measures each kernel once, those are exactly the timed graph replays."""
    timed = json.load(open(timed_json))
    disp = defaultdict(list)
    for r in csv.DictReader(open(trace_csv)):
        name = kernel_name(r["Kernel_Name"])
        if name in timed:
            disp[name].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out = {}
    for name, n in timed.items():
        d = sorted(disp.get(name, []))[-n:]
        if not d:
            continue
        us = sorted((e - b) / 1e3 for b, e in d)
        out[name] = {"dispatches": len(us), "of_total": len(disp[name]), "avg_us": sum(us) / len(us),
                     "median_us": us[len(us) // 2], "min_us": us[0], "max_us": us[-1]}
    return out


def counter_means(path: str, counter: str) -> dict:
    """Mean counter value per dispatch, per kernel name (copy16 split by grid size)."""
    acc = defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r.get("Counter_Name") != counter:
            continue
        name = kernel_name(r["Kernel_Name"])
        if name is None:
            continue
        if name == "copy":
            name = f"copy:{r.get('Grid_Size', '')}"
        acc[name].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def traffic(fetch_csv: str, write_csv: str, copy_bytes: int) -> dict:
    fetch = counter_means(fetch_csv, "FETCH_SIZE")
    write = counter_means(write_csv, "WRITE_SIZE")
    # the calibration copy is the largest copy16 dispatch
    ck = max((k for k in fetch if k.startswith("copy:")), key=lambda k: fetch[k])
    f_scale = copy_bytes / (fetch[ck] * 1024.0)
    w_scale = copy_bytes / (write[ck] * 1024.0)
    out = {"_calibration": {"copy_bytes_each_way": copy_bytes, "copy_fetch_kib": fetch[ck], "copy_write_kib": write[ck],
                            "fetch_bytes_per_kib": f_scale * 1024.0, "write_bytes_per_kib": w_scale * 1024.0}}
    for name, alg in ALGORITHMIC.items():
        if name not in fetch or name not in write:
            continue
        fb = fetch[name] * 1024.0 * f_scale
        wb = write[name] * 1024.0 * w_scale
        out[name] = {"fetch_kib": fetch[name], "write_kib": write[name], "fetch_bytes": round(fb),
                     "write_bytes": round(wb), "bytes_per_launch": round(fb + wb), "algorithmic_bytes": alg,
                     "traffic_over_algorithmic": round((fb + wb) / alg, 4), "sources_sha256": sources_digest(name)}
    return out


# SIMDs and shader engines of an MI355X (256 CUs x 4 SIMDs, 8 XCDs x 4 SEs):
# SQ_VALU_MFMA_BUSY_CYCLES sums over SIMDs, SQ_BUSY_CYCLES over shader engines.
MI355X_SIMDS = 1024
MI355X_SES = 32


def counters(paths: list[str], match: str, stages: int) -> dict:
    """Mean per dispatch of every counter in the given counter_collection CSVs, for the
    kernels whose symbol contains `match`; with SQ_WAVES, per wave and per K stage
    (`stages` stages per wave) figures; with SQ_VALU_MFMA_BUSY_CYCLES and SQ_BUSY_CYCLES,
    the MFMA-busy share of the kernel's SIMD cycles."""
    acc = defaultdict(lambda: defaultdict(list))
    for path in paths:
        for r in csv.DictReader(open(path)):
            sym = r["Kernel_Name"]
            if match not in sym:
                continue
            name = kernel_name(sym) or sym[:60]
            acc[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
    out = {}
    for name, cs in acc.items():
        m = {c: sum(v) / len(v) for c, v in cs.items()}
        d = {"mean_per_dispatch": m, "dispatches": {c: len(v) for c, v in cs.items()}}
        waves = m.get("SQ_WAVES")
        if waves:
            d["per_wave_stage"] = {c: m[c] / waves / stages for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS",
                                                                      "SQ_INSTS_SALU", "SQ_INSTS_VMEM",
                                                                      "SQ_VALU_MFMA_BUSY_CYCLES") if c in m}
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m and "SQ_BUSY_CYCLES" in m:
            cycles = m["SQ_BUSY_CYCLES"] / MI355X_SES
            d["kernel_cycles"] = cycles
            d["mfma_busy"] = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (MI355X_SIMDS * cycles)
        if "SQ_WAIT_ANY" in m and "SQ_WAVE_CYCLES" in m:
            d["wait_share"] = m["SQ_WAIT_ANY"] / m["SQ_WAVE_CYCLES"]
        out[name] = d
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("csv")
    c = sub.add_parser("steady")
    c.add_argument("trace_csv")
    c.add_argument("timed_json")
    b = sub.add_parser("traffic")
    b.add_argument("fetch_csv")
    b.add_argument("write_csv")
    b.add_argument("copy_bytes", type=int)
    b.add_argument("--json", default="")
    k = sub.add_parser("counters")
    k.add_argument("csv", nargs="+")
    k.add_argument("--match", default="gemm_")
    k.add_argument("--stages", type=int, default=64,
                   help="stages per wave: K / 32 for the prefill GEMM, chunks for the chunked GDN state walk")
    args = ap.parse_args(argv)
    if args.cmd == "counters":
        for name, d in counters(args.csv, args.match, args.stages).items():
            print(name)
            for c, v in sorted(d["mean_per_dispatch"].items()):
                print(f"   {c:28s} {v:16.6g}   ({d['dispatches'][c]} dispatches)")
            for c, v in d.get("per_wave_stage", {}).items():
                print(f"   per wave and stage: {c:28s} {v:10.1f}")
            if "mfma_busy" in d:
                print(f"   kernel cycles (SQ_BUSY_CYCLES / {MI355X_SES} SEs): {d['kernel_cycles']:.0f}; MFMA busy "
                      f"{100 * d['mfma_busy']:.1f}% of {MI355X_SIMDS} SIMDs")
            if "wait_share" in d:
                print(f"   SQ_WAIT_ANY / SQ_WAVE_CYCLES: {100 * d['wait_share']:.1f}%")
        return 0
    if args.cmd == "stats":
        t = stats(args.csv)
        print(f"{'kernel':44s} {'calls':>6s} {'avg us':>9s} {'min us':>9s} {'max us':>9s} {'GB/s (avg)':>11s}")
        for name, r in sorted(t.items(), key=lambda kv: -kv[1]["avg_us"]):
            gbps = ALGORITHMIC.get(name, 0) / r["avg_us"] / 1e3 if name in ALGORITHMIC else float("nan")
            print(f"{name[:44]:44s} {r['calls']:6d} {r['avg_us']:9.2f} {r['min_us']:9.2f} {r['max_us']:9.2f} "
                  f"{gbps:11.1f}")
        return 0
    if args.cmd == "steady":
        t = steady(args.trace_csv, args.timed_json)
        print(f"{'kernel':44s} {'timed':>6s} {'of':>6s} {'avg us':>8s} {'median':>8s} {'min us':>8s} {'max us':>8s} "
              f"{'GB/s (avg)':>11s}")
        for name, r in sorted(t.items(), key=lambda kv: -kv[1]["avg_us"]):
            gbps = ALGORITHMIC[name] / r["avg_us"] / 1e3 if name in ALGORITHMIC else float("nan")
            print(f"{name[:44]:44s} {r['dispatches']:6d} {r['of_total']:6d} {r['avg_us']:8.2f} {r['median_us']:8.2f} "
                  f"{r['min_us']:8.2f} {r['max_us']:8.2f} {gbps:11.1f}")
        return 0
    t = traffic(args.fetch_csv, args.write_csv, args.copy_bytes)
    cal = t["_calibration"]
    print(f"calibration: copy of {cal['copy_bytes_each_way']} B each way read as FETCH {cal['copy_fetch_kib']:.0f} KiB, "
          f"WRITE {cal['copy_write_kib']:.0f} KiB -> {cal['fetch_bytes_per_kib']:.1f} / {cal['write_bytes_per_kib']:.1f} "
          "bytes per counter KiB")
    print(f"{'kernel':44s} {'fetch B':>12s} {'write B':>12s} {'total B':>12s} {'algorithmic':>12s} {'ratio':>7s}")
    for name, r in t.items():
        if name.startswith("_"):
            continue
        print(f"{name[:44]:44s} {r['fetch_bytes']:12d} {r['write_bytes']:12d} {r['bytes_per_launch']:12d} "
              f"{r['algorithmic_bytes']:12d} {r['traffic_over_algorithmic']:7.3f}")
    if args.json:
        with open(args.json, "w") as f:
            json.dump(t, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
