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

Timed region (the contract): the step captured as one HIP graph (eight launches:
C3b and C3c run as one routed + shared SwiGLU launch; no host work between them) replayed K times, bracketed by
torch.cuda.synchronize(); value = algorithmic bytes per step / wall time per step.
One step touches ~830 MB, more than the 256 MB MALL, so every call reads its
inputs from HBM and pays for writing its outputs back.

Per-kernel figures (the metric's "GB/s and us/call per kernel"), steady state:
each kernel gets enough copies of its buffers that consecutive launches touch
>= 1 GiB of distinct memory (4x the MALL); the rotating launches are captured in
a graph and timed with HIP events around R replays on the launching stream;
us/call = elapsed / launches. The same measurement of a plain 16-byte-vector
copy of the same byte count (the fastest of three launch shapes, COPY_FORMS) is
reported beside each kernel as the box's practical ceiling. Algorithmic bytes count every input read once and every
output written once. The roofline object reports the kernel with the largest
time per step; its "traffic" comes from the committed rocprofv3 counter runs
(profiles/traffic.json), and only while the kernel's source files have the
digest recorded with those counts ("traffic_source" says which run and whether
it applies; otherwise traffic is null).

CPU baseline: the oracle (oracle/liboracle_fp32.so, a C++ restatement of the
reference kernels) timed on this host's cores over the full configs.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import struct
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen-3.5-cuda_amd"))

METRIC = "achieved HBM GB/s (% of MI355X peak) + µs/call per fused norm/RoPE/act kernel"
PEAK_GBPS = 8000.0  # MI355X HBM3E
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA
ROTATE_BYTES = 1 << 30


class Kernel:
    """A config: `make(i)` returns a launch closure bound to buffer set i
    (set 0 = the base buffers; i > 0 = fresh copies)."""

    def __init__(self, name, config, nbytes, footprint, make, in_step=True):
        self.name, self.config, self.bytes, self.footprint, self.make = name, config, nbytes, footprint, make
        self.in_step = in_step  # False: measured per kernel, its work done in the step by another entry point
        self.us = None
        self.copy_us = None


def build_workload(torch, ops, synth):
    dev = torch.device("cuda:0")

    def d(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
        return torch.from_numpy(a).to(dev)

    def cp(t, i):
        return t if i == 0 else t.clone()

    def new(t, i, keep):
        return keep if i == 0 else torch.empty_like(t)

    ks: list[Kernel] = []
    host = {}

    c = synth.c1_rmsnorm()
    host["rmsnorm"] = c
    x1, w1 = d(c["x"]), d(c["w"])
    o1 = torch.empty_like(x1)

    def mk_rms(i, x=x1, w=w1, o=o1):
        xx, oo = cp(x, i), new(o, i, o)
        return lambda: ops.rmsnorm_rows(xx, w, oo)
    nb = 2 * x1.numel() * 4 + w1.numel() * 4
    ks.append(Kernel("rmsnorm", "C1 f32 [36x2048] eps 1e-6", nb, nb, mk_rms))

    c = synth.c2_qk_rope()
    host["qk_norm_rope"] = c
    q2, k2, qw2, kw2, pos2 = d(c["q"]), d(c["k"]), d(c["qw"]), d(c["kw"]), d(c["pos"])

    def mk_rope(i):
        qq, kk = cp(q2, i), cp(k2, i)
        return lambda: ops.attn_qk_norm_rope_rows(qq, kk, qw2, kw2, pos=pos2, rope_dim=64, theta=1e7)
    nb = 2 * (q2.numel() + k2.numel()) * 4 + (qw2.numel() + kw2.numel()) * 4 + pos2.numel() * 4
    ks.append(Kernel("qk_norm_rope", "C2 f32 Q[512x16x256] K[512x2x256] rope 64 theta 1e7", nb, nb, mk_rope))

    c = synth.c3_residual()
    host["residual_rmsnorm_bf16"] = c
    x3, b3, w3 = d(c["x"]), d(c["branch"]), d(c["w"])
    r3, n3 = torch.empty_like(x3), torch.empty_like(x3)

    def mk_res(i):
        xx, bb, rr, nn = cp(x3, i), cp(b3, i), new(r3, i, r3), new(n3, i, n3)
        return lambda: ops.residual_rmsnorm_rows(xx, bb, w3, rr, nn)
    nb = 4 * x3.numel() * 2 + w3.numel() * 4
    ks.append(Kernel("residual_rmsnorm_bf16", "C3a bf16 [4096x2048]", nb, nb, mk_res))

    c = synth.c3_swiglu()
    host["swiglu_bf16"] = c
    g4, u4 = d(c["g"]), d(c["u"])
    h4 = torch.empty_like(g4)

    def mk_sw(i):
        gg, uu, hh = cp(g4, i), cp(u4, i), new(h4, i, h4)
        return lambda: ops.swiglu_bf16(gg, uu, hh)
    nb = 3 * g4.numel() * 2
    ks.append(Kernel("swiglu_bf16", "C3b bf16 [4096x8x512]", nb, nb, mk_sw, in_step=False))

    c = synth.c3_shared()
    host["shared_swiglu_sigmoid_bf16"] = c
    g5, u5, l5 = d(c["g"]), d(c["u"]), d(c["logits"])
    h5 = torch.empty_like(g5)

    def mk_sh(i):
        gg, uu, ll, hh = cp(g5, i), cp(u5, i), cp(l5, i), new(h5, i, h5)
        return lambda: ops.shared_swiglu_sigmoid_rows_bf16(gg, uu, ll, hh)
    nb = 3 * g5.numel() * 2 + l5.numel() * 4
    ks.append(Kernel("shared_swiglu_sigmoid_bf16", "C3c bf16 [4096x512] + logits [4096]", nb, nb, mk_sh,
                     in_step=False))

    # C3b + C3c as the MoE layer runs them: one launch (src/layer_moe.cpp:135,149,153)
    def mk_rs(i):
        gg, uu, hh = cp(g4, i), cp(u4, i), new(h4, i, h4)
        sg, su, sl, sh = cp(g5, i), cp(u5, i), cp(l5, i), new(h5, i, h5)
        return lambda: ops.swiglu_routed_shared_bf16(gg, uu, sg, su, sl, out=hh, shared_out=sh)
    nb = 3 * g4.numel() * 2 + 3 * g5.numel() * 2 + l5.numel() * 4
    ks.append(Kernel("swiglu_routed_shared_bf16", "C3b+C3c bf16 routed [4096x8x512] + shared [4096x512] x sigmoid, "
                     "one launch", nb, nb, mk_rs))

    c = synth.c4_frontend()
    host["gdn_frontend"] = c
    x6, w6, hi6 = d(c["x"]), d(c["w"]), d(c["hist"])
    ho6, y6 = torch.empty_like(hi6), torch.empty_like(x6)

    def mk_fe(i):
        xx, hi, ho, yy = cp(x6, i), cp(hi6, i), new(ho6, i, ho6), new(y6, i, y6)
        return lambda: ops.gdn_frontend_rows(xx, w6, hi, ho, yy, k_heads=16, key_dim=128)
    nb = 2 * x6.numel() * 4 + w6.numel() * 4 + 2 * hi6.numel() * 4
    ks.append(Kernel("gdn_frontend", "C4a f32 [4096x8192] kernel 4, 16 key heads x 128", nb, nb, mk_fe))

    c = synth.c4_norm_gate()
    host["gdn_norm_gate"] = c
    x7, z7, w7 = d(c["x"]), d(c["z"]), d(c["w"])
    o7 = torch.empty_like(x7)

    def mk_ng(i):
        xx, zz, oo = cp(x7, i), cp(z7, i), new(o7, i, o7)
        return lambda: ops.gdn_norm_gate_rows(xx, zz, w7, oo)
    nb = 3 * x7.numel() * 4 + w7.numel() * 4
    ks.append(Kernel("gdn_norm_gate", "C4b f32 [4096x32x128]", nb, nb, mk_ng))

    vocab, cols = 248320, 2048
    ids_h = synth.token_ids(8192, vocab)
    ids = d(ids_h)
    for kind, make, bpr in (("Q4_K", synth.q4k_table, 1152), ("Q6_K", synth.q6k_table, 1680)):
        tab_h = make(vocab, cols)
        tab = d(tab_h)
        out = torch.empty((8192, cols), dtype=torch.float32, device=dev)
        name = f"dequant_gather_{kind.lower()}"
        host[name] = {"table": tab_h, "ids": ids_h, "type": ops.GGML_TYPES[kind]}

        def mk_ga(i, tab=tab, kind=kind, out=out):
            ii, oo = cp(ids, i), new(out, i, out)
            return lambda: ops.dequant_gather_rows(tab, kind, vocab * cols, ii, cols, oo)
        nb = 8192 * bpr + ids.numel() * 4 + out.numel() * 4
        ks.append(Kernel(name, f"C5 {kind} table 248320x2048, 8192 ids -> f32", nb, nb, mk_ga))
        host[name]["device_table"] = tab
    return ks, host


def build_next_rows(torch, ops, synth, host):
    """The next rows of the path, measured alone (not part of the step). GDN
    recurrent state update at the Qwen3.5 GDN shape; decode-step GEMVs
    (matmul_dispatch) at the model's real shapes
    (include/config.hpp:40-60 of the reference: d_model 2048, vocab 248320, GDN
    conv dim 8192, value dim 4096, 256 experts x 512): one token's x [K] f32 ->
    y [M] f32. Bytes = weight bytes + 4K + 4M. Not part of the step."""
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(2048)
    ks: list[Kernel] = []

    def add(name, config, kind, tab, n_el, M, K, offsets, bpb, host_tab):
        x = torch.from_numpy(rng.standard_normal(K).astype(np.float32)).to(dev)
        y = torch.empty(M, dtype=torch.float32, device=dev)
        wbytes = M * (K // 256) * bpb
        nb = wbytes + 4 * K + 4 * M
        copies = {}

        def mk(i):
            # launch i reads weight slice offsets[i % len] of copy i // len
            c, o = divmod(i, len(offsets))
            if c not in copies:
                copies[c] = tab if c == 0 else tab.clone()
            t, yy = copies[c], (y if i == 0 else torch.empty_like(y))
            return lambda: ops.matmul_dispatch(t, kind, n_el, x, M, K, element_offset=offsets[o], out=yy)
        k = Kernel(name, config, nb, nb, mk)
        k.gemv = {"type": ops.GGML_TYPES[kind], "table": host_tab, "M": M, "K": K, "x": x.cpu().numpy()}
        ks.append(k)

    q6 = host["dequant_gather_q6_k"]
    add("gemv_lm_head_q6_k", "Q6_K [248320 x 2048] x f32 [2048] (model.cpp:216 LM head)", "Q6_K",
        q6["device_table"], 248320 * 2048, 248320, 2048, [0], 210, q6["table"])
    t = synth.q4k_table(8192, 2048, seed_tensor=16)
    add("gemv_qkv_q4_k", "Q4_K [8192 x 2048] x f32 [2048] (layer_gdn.cpp:83 qkv projection)", "Q4_K",
        torch.from_numpy(t).to(dev), 8192 * 2048, 8192, 2048, [0], 144, t)
    t = synth.q4k_table(2048, 4096, seed_tensor=20)
    add("gemv_out_q4_k", "Q4_K [2048 x 4096] x f32 [4096] (layer_gdn.cpp:112 output projection)", "Q4_K",
        torch.from_numpy(t).to(dev), 2048 * 4096, 2048, 4096, [0], 144, t)
    # A Q6_K projection at the qkv shape (Q4_K_M files hold some projections as
    # Q6_K): the direct per-row kernel.
    t = synth.q6k_table(8192, 2048, seed_tensor=24)
    add("gemv_qkv_q6_k", "Q6_K [8192 x 2048] x f32 [2048] (a Q6_K projection at the qkv shape)", "Q6_K",
        torch.from_numpy(t).to(dev), 8192 * 2048, 8192, 2048, [0], 210, t)
    # Prefill: the same projections for 4096 tokens in one matmul_rows call (prep
    # kernel + matrix-core GEMM). Compute-bound: reported as algorithmic TFLOP/s
    # (2 M K per token) and as the share of the dense fp16 MFMA peak that the two
    # exact fp16 parts of x use (2x the algorithmic flops).
    T = 4096
    xg = torch.from_numpy(rng.standard_normal((T, 2048)).astype(np.float32)).to(dev)
    for name, kind, make, M, K, bpb, seed in (("gemm_qkv_q4_k_4096", "Q4_K", synth.q4k_table, 8192, 2048, 144, 16),
                                              ("gemm_qkv_q6_k_4096", "Q6_K", synth.q6k_table, 8192, 2048, 210, 17)):
        wt = torch.from_numpy(make(M, K, seed_tensor=seed)).to(dev)
        yg = torch.empty((T, M), dtype=torch.float32, device=dev)
        wsg = torch.empty(ops.matmul_rows_workspace_bytes(T, K), dtype=torch.uint8, device=dev)

        def mk_gemm(i, wt=wt, yg=yg, wsg=wsg, kind=kind, M=M, K=K):
            xx = xg if i == 0 else xg.clone()
            yy = yg if i == 0 else torch.empty_like(yg)
            return lambda: ops.matmul_rows(wt, kind, M * K, xx, M, K, out=yy, workspace=wsg)
        nb = M * (K // 256) * bpb + 4 * T * K + 4 * T * M
        k = Kernel(name, f"{kind} [{M} x {K}] x f32 [{T} x {K}] (layer_gdn.cpp:83 qkv projection over a "
                   f"{T}-token prompt, one matmul_rows call)", nb, nb, mk_gemm)
        k.flops = 2 * T * M * K
        k.no_cpu = True
        ks.append(k)
    # GDN recurrent state (gdn.cu:108-172): 16 key / 32 value heads of 128, state 2 MB.
    kh, vh, dk, dv = 16, 32, 128, 128
    c = host["gdn_frontend"]
    for rows in (1, 4096):
        # Front-end-shaped rows [rows x 8192]: q | k scaled to about unit norm per
        # head so that the recurrence stays bounded over 4096 steps.
        qkv_h = np.array(c["x"][:rows], dtype=np.float32)
        qkv_h[:, :2 * kh * dk] *= dk ** -0.5
        qkv = torch.from_numpy(np.ascontiguousarray(qkv_h)).to(dev)
        beta = torch.full((rows, vh), 0.5, device=dev)
        decay = torch.full((rows, vh), 0.95, device=dev)
        st0 = torch.from_numpy((0.1 * rng.standard_normal(vh * dk * dv)).astype(np.float32)).to(dev)
        o = torch.empty((rows, vh * dv), dtype=torch.float32, device=dev)
        nb = 2 * st0.numel() * 4 + rows * (2 * kh * dk + 2 * vh * dv + 2 * vh) * 4

        def mk_gdn(i, qkv=qkv, beta=beta, decay=decay, st0=st0, o=o, rows=rows):
            ss = st0 if i == 0 else st0.clone()
            qq = qkv if i == 0 or rows == 1 else qkv.clone()
            oo = o if i == 0 else torch.empty_like(o)
            return lambda: ops.gdn_recurrent_rows(ss, qq, beta, decay, kh, vh, dk, dv, oo)
        name = "gdn_recurrent_step" if rows == 1 else "gdn_recurrent_rows_4096"
        desc = ("one decode step, state [32 x 128 x 128] f32 (layer_gdn.cpp:100)" if rows == 1 else
                "4096 sequential steps in one launch over front-end rows [4096 x 8192] f32")
        k = Kernel(name, desc, nb, nb, mk_gdn)
        k.gdn = {"rows": rows, "qkv": qkv_h, "beta": np.full((rows, vh), 0.5, np.float32),
                 "decay": np.full((rows, vh), 0.95, np.float32), "state": st0.cpu().numpy()}
        ks.append(k)
        if rows == 1:
            # The layer's gates + step (layer_gdn.cpp:100-106): two launches, or the
            # fused-gate form in one (raw gates in, no beta / decay buffers).
            braw = torch.from_numpy(rng.standard_normal((1, vh)).astype(np.float32)).to(dev)
            araw = torch.from_numpy(rng.standard_normal((1, vh)).astype(np.float32)).to(dev)
            ag = torch.from_numpy(-np.exp(rng.standard_normal(vh)).astype(np.float32)).to(dev)
            dtg = torch.from_numpy(rng.uniform(-1, 1, vh).astype(np.float32)).to(dev)
            bt1, dc1 = torch.empty((1, vh), device=dev), torch.empty((1, vh), device=dev)
            nbg = nb + 2 * vh * 4   # raw gates in place of beta / decay (same count)
            for gname, fused in (("gdn_gates_step_2_launches", False), ("gdn_gated_step", True)):
                def mk_g(i, qkv=qkv, st0=st0, o=o, fused=fused):
                    ss = st0 if i == 0 else st0.clone()
                    oo = o if i == 0 else torch.empty_like(o)
                    if fused:
                        return lambda: ops.gdn_gated_recurrent_rows(ss, qkv, braw, araw, ag, dtg, kh, vh, dk, dv, oo)

                    def run():
                        ops.gdn_gate_values_rows(braw, araw, ag, dtg, beta=bt1, decay=dc1)
                        ops.gdn_recurrent_rows(ss, qkv, bt1, dc1, kh, vh, dk, dv, oo)
                    return run
                kg = Kernel(gname, "one decode step with its gates from the raw projections: " +
                            ("gate kernel + step kernel" if not fused else "fused-gate step, one launch"),
                            nbg, nbg, mk_g)
                kg.no_cpu = True
                ks.append(kg)
            # The whole decode step after the input projections (layer_gdn.cpp:89-106):
            # conv + SiLU + Q/K L2 norm + gates + recurrence in one launch.
            C = 2 * kh * dk + vh * dv
            cw = torch.from_numpy((0.5 * rng.standard_normal((C, 4))).astype(np.float32)).to(dev)
            hin = torch.from_numpy(rng.standard_normal((C, 3)).astype(np.float32)).to(dev)
            xin = torch.from_numpy(rng.standard_normal(C).astype(np.float32)).to(dev)
            ybuf = torch.empty(C, dtype=torch.float32, device=dev)
            nbd = (2 * st0.numel() + C * 4 + 2 * C * 3 + 2 * C + 4 * vh + vh * dv) * 4

            def mk_d(i, st0=st0, o=o):
                ss = st0 if i == 0 else st0.clone()
                hout = torch.empty_like(hin)
                oo = o if i == 0 else torch.empty_like(o)
                return lambda: ops.gdn_decode_step(xin, cw, hin, hout, ss, braw.view(-1), araw.view(-1), ag, dtg, kh, vh, dk, dv,
                                                   y=ybuf, out=oo)
            kd = Kernel("gdn_decode_step_fused", "one decode step after the input projections: conv + SiLU + Q/K "
                        "L2 norm + gates + recurrence, one launch (layer_gdn.cpp:89-106)", nbd, nbd, mk_d)
            kd.no_cpu = True
            ks.append(kd)
        if rows > 1:
            # The chunked form on the same inputs (its workspace outside the bytes).
            ws = torch.empty(ops.load().qwen_gdn_recurrent_chunked_workspace_bytes(rows, vh), dtype=torch.uint8,
                             device=dev)

            def mk_chunk(i, qkv=qkv, beta=beta, decay=decay, st0=st0, o=o, ws=ws):
                ss = st0 if i == 0 else st0.clone()
                qq = qkv if i == 0 else qkv.clone()
                oo = o if i == 0 else torch.empty_like(o)
                return lambda: ops.gdn_recurrent_chunked(ss, qq, beta, decay, kh, vh, dk, dv, oo, workspace=ws)
            kc = Kernel("gdn_recurrent_chunked_4096", "the same 4096 tokens in the chunked form (64-token chunks, "
                        "fp16-pair MFMA for the long products, 2 launches)", nb, nb, mk_chunk)
            kc.gdn = k.gdn
            ks.append(kc)

    # Decode attention (attn_kernels.cu:72-195): 16 query / 2 kv heads of 256,
    # 4096 cached keys, sigmoid gate; fused split-K path and the reference's
    # staged launches (scores, softmax, values, gate) on the same inputs.
    H, Hkv, D, pos = 16, 2, 256, 4095
    qa = torch.from_numpy(rng.standard_normal(H * D).astype(np.float32)).to(dev)
    ga = torch.from_numpy(rng.standard_normal(H * D).astype(np.float32)).to(dev)
    kc0 = torch.from_numpy(rng.standard_normal((pos + 1) * Hkv * D).astype(np.float32)).to(dev)
    vc0 = torch.from_numpy(rng.standard_normal((pos + 1) * Hkv * D).astype(np.float32)).to(dev)
    ws = torch.empty(ops.attn_decode_workspace_bytes(H, Hkv, D, pos), dtype=torch.uint8, device=dev)
    nb = 2 * kc0.numel() * 4 + 3 * H * D * 4
    for name, staged in (("attn_decode_4096", False), ("attn_decode_staged_4096", True)):
        def mk_att(i, staged=staged):
            kc, vc = (kc0, vc0) if i == 0 else (kc0.clone(), vc0.clone())
            o = torch.empty(H * D, dtype=torch.float32, device=dev)
            sc = torch.empty(H * (pos + 1), dtype=torch.float32, device=dev)
            if not staged:
                return lambda: ops.attn_decode(qa, kc, vc, H, Hkv, D, pos, gate=ga, workspace=ws, out=o)

            def run():
                ops.attn_scores(qa, kc, H, Hkv, D, pos, out=sc)
                ops.attn_softmax(sc, H, pos + 1)
                ops.attn_values(sc, vc, H, Hkv, D, pos, out=o)
                ops.attn_sigmoid_gate(o, ga, out=o)
            return run
        desc = ("fused split-K decode, q [16 x 256] vs K/V cache [4096 x 2 x 256] f32, sigmoid gate" if not staged else
                "the reference's four launches (scores, softmax, values, gate) on the same inputs")
        k = Kernel(name, desc, nb, nb, mk_att)
        k.attn = {"q": qa.cpu().numpy(), "K": kc0.cpu().numpy(), "V": vc0.cpu().numpy(), "g": ga.cpu().numpy()}
        ks.append(k)

    # MoE routing (moe.cu:7-86, layer_moe.cpp:98-140) with the routing kept on the device.
    T, E, k_sel, Dm = 4096, 256, 8, 2048
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    ti = torch.empty((T, k_sel), dtype=torch.int32, device=dev)
    tw = torch.empty((T, k_sel), dtype=torch.float32, device=dev)

    def mk_topk(i):
        ll = lg if i == 0 else lg.clone()
        return lambda: ops.moe_topk_rows(ll, k_sel, idx=ti, weights=tw)
    nb = lg.numel() * 4 + 2 * ti.numel() * 4
    k = Kernel("moe_topk_4096", "router logits [4096 x 256] f32 -> top-8 ids + softmax weights", nb, nb, mk_topk)
    k.route = {"logits": lg.cpu().numpy()}
    ks.append(k)
    ye = torch.from_numpy(rng.standard_normal((T, k_sel, Dm)).astype(np.float32)).to(dev)
    acc0 = torch.zeros((T, Dm), dtype=torch.float32, device=dev)
    wts = torch.full((T, k_sel), 0.125, device=dev)

    def mk_wsum(i):
        yy, aa = (ye, acc0) if i == 0 else (ye.clone(), acc0.clone())
        return lambda: ops.moe_weighted_sum_rows(aa, yy, wts)
    nb = ye.numel() * 4 + 2 * acc0.numel() * 4 + wts.numel() * 4
    k = Kernel("moe_weighted_sum_4096", "acc [4096 x 2048] += sum of 8 weighted expert rows [4096 x 8 x 2048] f32",
               nb, nb, mk_wsum)
    k.route = {"y": ye[:64].cpu().numpy(), "w": wts[:64].cpu().numpy()}
    ks.append(k)

    t = synth.q4k_table(256 * 512, 2048, seed_tensor=24)
    add("gemv_expert_q4_k", "Q4_K expert e of [256 x 512 x 2048] x f32 [2048] (layer_moe.cpp:131 gate, "
        "element offset e*512*2048)", "Q4_K", torch.from_numpy(t).to(dev), 256 * 512 * 2048, 512, 2048,
        [e * 512 * 2048 for e in range(256)], 144, t)
    # the 8 routed experts' gate projections of one token in one launch, ids on the device
    qt = torch.from_numpy(t).to(dev)
    ids8 = torch.from_numpy(np.array([3, 77, 141, 200, 9, 250, 31, 128], np.int32)).to(dev)
    x8 = torch.from_numpy(rng.standard_normal(2048).astype(np.float32)).to(dev)
    y8 = torch.empty((8, 512), dtype=torch.float32, device=dev)

    def mk_ex(i):
        # one 151 MB table; each buffer set picks other experts so the rotation still
        # walks distinct weight bytes
        ii = ids8 if i == 0 else (ids8 + 8 * i) % 256
        return lambda: ops.moe_expert_matmul(qt, "Q4_K", 256 * 512 * 2048, 512 * 2048, 256, ii, x8, 0, 512, 2048,
                                             out=y8)
    nb = 8 * 512 * 8 * 144 + 2048 * 4 + 8 * 512 * 4
    k = Kernel("moe_expert_gate_8", "8 routed experts' Q4_K gate projections [8 x 512 x 2048], ids on the device",
               nb, nb, mk_ex)
    k.gemv = {"type": 12, "table": t[:8 * 512 * 8 * 144], "M": 8 * 512, "K": 2048, "x": x8.cpu().numpy()}
    ks.append(k)

    # A GDN layer's four input projections of one token (layer_gdn.cpp:83-86: qkv 8192, z 4096,
    # beta 32 and alpha 32 rows of 2048, Q4_K): the reference's four matmul_dispatch calls
    # against one matmul_dispatch_multi call (one launch). No CPU figure (it would be the
    # GEMV rows above again).
    proj = [(8192, 30), (4096, 31), (32, 32), (32, 33)]
    ptabs = [torch.from_numpy(synth.q4k_table(M, 2048, seed_tensor=s)).to(dev) for M, s in proj]
    xp = torch.from_numpy(rng.standard_normal(2048).astype(np.float32)).to(dev)
    ys = [torch.empty(M, dtype=torch.float32, device=dev) for M, _ in proj]
    nb = sum(M * 8 * 144 + 4 * M for M, _ in proj) + 4 * 2048
    for name, multi in (("gdn_in_proj_4_calls", False), ("gdn_in_proj_multi", True)):
        def mk_p(i, multi=multi):
            tt = ptabs if i == 0 else [tb.clone() for tb in ptabs]
            if multi:
                jobs = [(tb, "Q4_K", M * 2048, M, 0, y) for tb, (M, _), y in zip(tt, proj, ys)]
                return lambda: ops.matmul_dispatch_multi(jobs, xp, 2048)

            def run():
                for tb, (M, _), y in zip(tt, proj, ys):
                    ops.matmul_dispatch(tb, "Q4_K", M * 2048, xp, M, 2048, out=y)
            return run
        desc = ("GDN input projections qkv/z/beta/alpha, Q4_K [8192|4096|32|32 x 2048], " +
                ("one matmul_dispatch_multi launch" if multi else "four matmul_dispatch calls (the reference's)"))
        k = Kernel(name, desc, nb, nb, mk_p)
        k.no_cpu = True
        ks.append(k)

    # One GDN layer's decode step (layer_gdn.cpp:78-113) composed from the library: the
    # reference's ten calls against the fused five (qwen35_hip.decode_layers). Bytes: the
    # five Q4_K projections, the state read and written, conv weights and history.
    from qwen35_hip.decode_layers import GdnLayerDecode
    cdim, vdim = 2 * kh * dk + vh * dv, vh * dv
    lw = [torch.from_numpy(synth.q4k_table(M, K, seed_tensor=s)).to(dev)
          for M, K, s in ((cdim, 2048, 40), (vdim, 2048, 41), (vh, 2048, 42), (vh, 2048, 43), (2048, vdim, 44))]
    conv_w = torch.from_numpy((0.5 * rng.standard_normal((cdim, 4))).astype(np.float32)).to(dev)
    la = torch.from_numpy(-np.exp(rng.standard_normal(vh)).astype(np.float32)).to(dev)
    ldt = torch.from_numpy(rng.uniform(-1, 1, vh).astype(np.float32)).to(dev)
    lnw = torch.from_numpy((1 + 0.1 * rng.standard_normal(dv)).astype(np.float32)).to(dev)
    lx = torch.from_numpy((0.3 * rng.standard_normal(2048)).astype(np.float32)).to(dev)
    lout = torch.empty(2048, dtype=torch.float32, device=dev)
    nb = (sum(t.numel() for t in lw) + 2 * vh * dk * dv * 4 + cdim * 4 * 4 + 2 * cdim * 3 * 4 + 2048 * 4 * 2)
    for name, fused in (("gdn_layer_decode_10_calls", False), ("gdn_layer_decode_fused", True)):
        def mk_l(i, fused=fused):
            ww = lw if i == 0 else [t.clone() for t in lw]
            layer = GdnLayerDecode(*ww, conv_w, la, ldt, lnw)
            return (lambda: layer.forward(lx, lout)) if fused else (lambda: layer.forward_reference_launches(lx, lout))
        desc = ("one GDN layer decode step, Q4_K weights, 16/32 heads of 128: " +
                ("fused entry points, 3 launches" if fused else "the reference's sequence of 10 calls"))
        k = Kernel(name, desc, nb, nb, mk_l)
        k.layer = True
        k.no_cpu = True
        ks.append(k)

    # The same GDN layer over a 4096-token prompt in one pass (GdnLayerDecode.prefill: GEMM
    # projections, front end over all rows, chunked recurrence); the reference runs the
    # decode step 4096 times. Bytes: weights once, x and out, the state read and written.
    TP = 4096
    lxs = torch.from_numpy((0.3 * rng.standard_normal((TP, 2048))).astype(np.float32)).to(dev)
    lpo = torch.empty((TP, 2048), dtype=torch.float32, device=dev)

    def mk_pre(i):
        layer = GdnLayerDecode(*lw, conv_w, la, ldt, lnw)
        return lambda: layer.prefill(lxs, lpo)
    nbp = sum(t.numel() for t in lw) + 2 * TP * 2048 * 4 + 2 * vh * dk * dv * 4
    k = Kernel("gdn_layer_prefill_4096", "one GDN layer over a 4096-token prompt in one pass (matmul_rows "
               "projections, front end, chunked recurrence, gated norm), eager wall clock per call", nbp, 1 << 30,
               mk_pre)
    k.layer = True
    k.no_cpu = True
    k.eager = True
    ks.append(k)

    # One full-attention layer's decode step (layer_attn.cpp:63-111) at position 2047 of a
    # 4096-row cache: the reference's fifteen calls against the fused five. Bytes: the four
    # Q4_K projections and the 2048 K and V rows read.
    from qwen35_hip.decode_layers import AttnLayerDecode
    apos = 2047
    aw = [torch.from_numpy(synth.q4k_table(M, K, seed_tensor=s)).to(dev)
          for M, K, s in ((8192, 2048, 50), (512, 2048, 51), (512, 2048, 52), (2048, 4096, 53))]
    aqn = torch.from_numpy((1 + 0.1 * rng.standard_normal(256)).astype(np.float32)).to(dev)
    akn = torch.from_numpy((1 + 0.1 * rng.standard_normal(256)).astype(np.float32)).to(dev)
    akv = torch.from_numpy(rng.standard_normal((2, apos, 512)).astype(np.float32)).to(dev)
    nb = sum(t.numel() for t in aw) + 2 * (apos + 1) * 512 * 4 + 4 * 2048 * 2
    for name, fused in (("attn_layer_decode_15_calls", False), ("attn_layer_decode_fused", True)):
        def mk_a(i, fused=fused):
            ww = aw if i == 0 else [t.clone() for t in aw]
            layer = AttnLayerDecode(*ww, aqn, akn)
            layer.k_cache[:apos].copy_(akv[0])
            layer.v_cache[:apos].copy_(akv[1])
            return ((lambda: layer.forward(lx, apos, lout)) if fused else
                    (lambda: layer.forward_reference_launches(lx, apos, lout)))
        desc = ("one attention layer decode step at position 2047, Q4_K weights, 16 query / 2 KV heads of 256: " +
                ("fused entry points, 3 calls" if fused else "the reference's sequence of 15 calls"))
        k = Kernel(name, desc, nb, nb, mk_a)
        k.layer = True
        k.no_cpu = True
        ks.append(k)

    # One MoE layer's decode step (layer_moe.cpp:80-159): 256 experts, top 8, Q4_K. The
    # reference's sequence synchronises with the host to read the expert ids, so it cannot
    # be captured: it is timed eagerly (wall clock per call), and the fused path both
    # eagerly and captured. Each buffer set has its own token (so its own experts) and its
    # own copy of the router and shared expert. Bytes: router, 8 x 3 expert matrices,
    # the shared expert's four, the 8 expert outputs written and read.
    from qwen35_hip.decode_layers import MoeLayerDecode
    E, I, S = 256, 512, 2048
    ew = [torch.from_numpy(synth.q4k_table(E * M, K, seed_tensor=s)).to(dev)
          for M, K, s in ((I, 2048, 61), (I, 2048, 62), (2048, I, 63))]
    sw = [torch.from_numpy(synth.q4k_table(M, K, seed_tensor=s)).to(dev)
          for M, K, s in ((E, 2048, 60), (1, 2048, 64), (S, 2048, 65), (S, 2048, 66), (2048, S, 67))]
    q4 = lambda M, K: M * K // 256 * 144  # noqa: E731
    nb = (q4(E, 2048) + 8 * 3 * q4(I, 2048) + q4(1, 2048) + 3 * q4(S, 2048) + 2 * 8 * 2048 * 4 + 4 * 2048 * 2)
    for name, fused, eager in (("moe_layer_decode_reference_calls", False, True),
                               ("moe_layer_decode_fused_eager", True, True),
                               ("moe_layer_decode_fused", True, False)):
        def mk_m(i, fused=fused):
            s = sw if i == 0 else [t.clone() for t in sw]
            layer = MoeLayerDecode(s[0], *ew, *s[1:])
            xm = torch.from_numpy((0.05 * np.random.default_rng(1000 + i).standard_normal(2048))
                                  .astype(np.float32)).to(dev)
            om = torch.empty(2048, dtype=torch.float32, device=dev)
            return (lambda: layer.forward(xm, om)) if fused else (lambda: layer.forward_reference_launches(xm, om))
        desc = ("one MoE layer decode step, 256 experts top 8, 512-wide experts, 2048-wide shared expert, Q4_K: " +
                ("fused entry points, 3 launches, expert ids on the device" if fused else
                 "the reference's sequence (8 + 5 x 8 calls and a host round trip for the expert ids)") +
                ("; eager, wall clock per call" if eager else ""))
        k = Kernel(name, desc, nb, nb, mk_m)
        k.layer = True
        k.no_cpu = True
        k.eager = eager
        ks.append(k)
    return ks


def spin_cycles_per_ms(torch) -> float:
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)
    s.record()
    torch.cuda._sleep(2_000_000)
    e.record()
    torch.cuda.synchronize()
    return 2_000_000 / max(s.elapsed_time(e), 1e-3)


GRAPH_LAUNCHES = 64  # kernel launches per captured graph in the steady-state timing
TIMED_LAUNCHES: dict[str, int] = {}  # kernel name -> launches in its timed batches (for --timed-counts)


def steady_state_us(torch, launches, replays: int, spin: int, repeats: int = 5, name: str | None = None) -> float:
    """us per launch of `launches` (one per buffer set, cycled through the sets
    until the graph holds at least GRAPH_LAUNCHES launches, so the gap between
    two graph launches is spread over that many kernels rather than over a
    handful), captured as one graph and replayed; events bracket each batch of
    replays on the capturing stream. The median over `repeats` batches is
    returned (single batches of a few ms vary by a few percent on this box)."""
    cycle = max(1, -(-GRAPH_LAUNCHES // len(launches)))
    launches = list(launches) * cycle
    replays = max(1, -(-replays // cycle))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in launches:
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in launches:
            f()
    g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(spin)
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / (replays * len(launches)))
    del g
    if name:
        TIMED_LAUNCHES[name] = repeats * replays * len(launches)
    return sorted(times)[len(times) // 2]


def n_sets(footprint: int) -> int:
    return max(2, min(2048, -(-ROTATE_BYTES // footprint)))


def eager_us(torch, launches, calls: int, repeats: int = 5) -> float:
    """Wall-clock us per call of `launches` called eagerly in turn (for a sequence
    that synchronises with the host inside, which no graph can hold), the device
    synchronised before and after each batch; median over `repeats` batches."""
    for f in launches:
        f()
    torch.cuda.synchronize()
    n = max(len(launches), calls)
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        for j in range(n):
            launches[j % len(launches)]()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e6 / n)
    return sorted(times)[len(times) // 2]


def measure_kernel(torch, k: Kernel, spin: int, min_launches: int) -> float:
    sets = n_sets(k.footprint)
    launches = [k.make(i) for i in range(sets)]
    replays = max(1, -(-min_launches // sets))
    if getattr(k, "eager", False):
        us = eager_us(torch, launches, max(min_launches, 200))
        del launches
        torch.cuda.empty_cache()
        return us
    us = steady_state_us(torch, launches, replays, spin, name=k.name)
    del launches
    torch.cuda.empty_cache()
    return us


# Copy forms the per-kernel ceiling takes the best of (unroll, block): the
# reference streaming copy (8 x 16 B per thread, 256 threads: the fastest form
# from ~64 MB up) and the two forms the small-size sweep found fastest below
# that (one vector per thread in 256-thread workgroups; four per thread in
# single-wave workgroups).
COPY_FORMS = [(8, 256), (1, 256), (4, 64)]


def measure_copy(torch, bench_lib, nbytes: int, spin: int, min_launches: int) -> float:
    """us per launch of the fastest COPY_FORMS copy of nbytes (half read, half
    written), timed like a kernel."""
    half = (nbytes // 2 + 15) // 16 * 16
    sets = n_sets(2 * half)
    bufs = [(torch.empty(half, dtype=torch.uint8, device="cuda:0"), torch.empty(half, dtype=torch.uint8, device="cuda:0"))
            for _ in range(sets)]
    fn = bench_lib.qwen_bench_copy_form
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int, ctypes.c_void_p]

    def launcher(src, dst, u, b):
        def f():
            if fn(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), half, u, b, 0, 1,
                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)):
                raise RuntimeError("qwen_bench_copy_form failed")
        return f
    us = min(steady_state_us(torch, [launcher(s, d, u, b) for s, d in bufs], max(1, -(-min_launches // sets)), spin)
             for u, b in COPY_FORMS)
    del bufs
    torch.cuda.empty_cache()
    return us


SWEEP_SIZES = [598_016, 1 << 20, 2 << 20, 4 << 20, 8 << 20, 12_599_296, 16 << 20, 18_878_464, 32 << 20, 64 << 20]


def copy_sweep(torch, bench_lib, spin: int, min_launches: int) -> list[dict]:
    """Streaming-copy forms at the small sizes where the fused kernels miss 70% of
    peak (C1 0.6 MB, C3c 12.6 MB, C2 18.9 MB) and around them: one-shot grids of
    1..16 16-byte vectors per thread and 64/256/1024-thread workgroups, with and
    without the nontemporal hint; persistent (grid-stride) grids of 256..2048
    workgroups; and the in-place form (src == dst, as C2 reads and writes the same
    lines). `bytes` counts the read and the write, as the kernels' algorithmic
    bytes do; each form is timed like a kernel (steady state, >= 1 GiB rotated)."""
    forms = [(u, b, 0, nt, False) for nt in (1, 0) for b in (64, 256, 1024) for u in (1, 2, 4, 8, 16)]
    forms += [(u, 256, g, 1, False) for u in (1, 4) for g in (256, 512, 1024, 2048)]
    forms += [(u, 256, 0, 1, True) for u in (1, 2, 8)]
    fn = bench_lib.qwen_bench_copy_form
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int, ctypes.c_void_p]
    out = []
    for nbytes in SWEEP_SIZES:
        half = (nbytes // 2 + 15) // 16 * 16
        sets = n_sets(2 * half)
        bufs = [(torch.empty(half, dtype=torch.uint8, device="cuda:0"),
                 torch.empty(half, dtype=torch.uint8, device="cuda:0")) for _ in range(sets)]
        best = None
        for u, b, g, nt, inplace in forms:
            def launcher(src, dst, u=u, b=b, g=g, nt=nt, inplace=inplace):
                d = src if inplace else dst

                def f():
                    if fn(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(d.data_ptr()), half, u, b, g, nt,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)):
                        raise RuntimeError("qwen_bench_copy_form failed")
                return f
            us = steady_state_us(torch, [launcher(a, c) for a, c in bufs], max(1, -(-min_launches // sets)), spin,
                                 repeats=3)
            rec = {"bytes": 2 * half, "unroll": u, "block": b, "grid_cap": g, "nt": nt, "inplace": inplace,
                   "us": round(us, 3), "gbps": round(2 * half / us / 1e3, 1)}
            out.append(rec)
            if not inplace and (best is None or us < best["us"]):
                best = rec
        print(f"# copy sweep {2 * half:>10d} B: best {best['us']:7.2f} us {best['gbps']:7.1f} GB/s "
              f"(unroll {best['unroll']}, block {best['block']}, grid cap {best['grid_cap']}, nt {best['nt']})",
              file=sys.stderr, flush=True)
        mine = sorted((r for r in out if r["bytes"] == 2 * half), key=lambda r: r["us"])
        std = next(r for r in mine if (r["unroll"], r["block"], r["grid_cap"], r["nt"], r["inplace"]) ==
                   (8, 256, 0, 1, False))
        for r in mine[:5] + [std]:
            print(f"#   {r['us']:8.3f} us {r['gbps']:8.1f} GB/s  unroll {r['unroll']:2d} block {r['block']:4d} "
                  f"grid cap {r['grid_cap']:4d} nt {r['nt']} {'in place' if r['inplace'] else ''}"
                  f"{'  <- bench.py reference copy form' if r is std else ''}", file=sys.stderr, flush=True)
        del bufs
        torch.cuda.empty_cache()
    return out


def cpu_rates_sampled(host, kernels, threads: int, budget_s: float, gemv=None):
    """The oracle's CPU rate for the next-row kernels (decode GEMVs, routing,
    attention, recurrence; not part of the step), timed on a bounded sample of
    rows and scaled to the full shape; returns per-kernel results and the
    aggregate GB/s."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle as orc

    orc.lib()
    sample = {"rmsnorm": 36, "qk_norm_rope": 64, "residual_rmsnorm_bf16": 512, "swiglu_bf16": 512,
              "shared_swiglu_sigmoid_bf16": 4096, "gdn_frontend": 256, "gdn_norm_gate": 512,
              "dequant_gather_q4_k": 1024, "dequant_gather_q6_k": 1024}
    gemv = gemv or {}
    for name, g in gemv.items():
        sample[name] = (min(g["M"], 4096) if "M" in g else min(g["rows"], 4) if "rows" in g else
                        64 if "y" in g else 4096)
    full = {"rmsnorm": 36, "qk_norm_rope": 512, "residual_rmsnorm_bf16": 4096, "swiglu_bf16": 4096,
            "shared_swiglu_sigmoid_bf16": 4096, "gdn_frontend": 4096, "gdn_norm_gate": 4096,
            "dequant_gather_q4_k": 8192, "dequant_gather_q6_k": 8192}
    full.update({name: g["M"] if "M" in g else g["rows"] if "rows" in g else 4096 for name, g in gemv.items()})

    def runner(name, rows, th):
        if name in gemv and "table" in gemv[name]:
            g = gemv[name]
            return lambda: orc.gemv(g["table"], g["type"], g["x"], rows, g["K"], threads=th)
        if name == "moe_topk_4096":
            g = gemv[name]
            return lambda: orc.moe_topk_rows(g["logits"][:rows], 8)
        if name == "moe_weighted_sum_4096":
            g = gemv[name]
            return lambda: orc.moe_weighted_sum_rows(np.zeros((rows, 2048), np.float32), g["y"][:rows], g["w"][:rows])
        if name.startswith("attn_decode"):
            g = gemv[name]
            n = min(rows, 4096)
            return lambda: orc.attn_decode(g["q"], g["K"][:n * 512], g["V"][:n * 512], 16, 2, 256, n - 1, gate=g["g"])
        if name.startswith("gdn_recurrent"):
            g = gemv[name]
            st = g["state"].copy()
            return lambda: orc.gdn_recurrent_rows(st, g["qkv"][:rows], g["beta"][:rows], g["decay"][:rows],
                                                  16, 32, 128, 128)
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
    budget = budget_s / len(kernels)
    for k in kernels:
        rows = sample[k.name]
        fn = runner(k.name, rows, threads)
        fn()
        t0 = time.perf_counter()
        n = 0
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el > budget or n >= 200:
                break
        sec_full = el / n * full[k.name] / rows
        per[k.name] = {"gbps": k.bytes / sec_full / 1e9, "us_per_call": sec_full * 1e6, "sample_rows": rows}
        tot_b += k.bytes
        tot_t += sec_full
    return per, tot_b / tot_t / 1e9


def cpu_step_fns(orc, host, th: int) -> dict:
    """The CPU restatement of every step kernel on its full BASELINE config, in
    the reference's form: C3b and C3c are the two calls the reference makes
    (src/layer_moe.cpp:135,149), C2 is per head norm + RoPE (layer_attn.cpp:91-96)."""
    c = host
    f = {
        "rmsnorm": lambda: orc.rmsnorm_rows(c["rmsnorm"]["x"], c["rmsnorm"]["w"], threads=th),
        "qk_norm_rope": lambda: orc.qk_norm_rope_rows(
            c["qk_norm_rope"]["q"], c["qk_norm_rope"]["k"], c["qk_norm_rope"]["qw"], c["qk_norm_rope"]["kw"],
            pos=c["qk_norm_rope"]["pos"], rope_dim=64, theta=1e7, threads=th),
        "residual_rmsnorm_bf16": lambda: orc.residual_rmsnorm_rows(
            c["residual_rmsnorm_bf16"]["x"], c["residual_rmsnorm_bf16"]["branch"], c["residual_rmsnorm_bf16"]["w"],
            threads=th),
        "swiglu_bf16": lambda: orc.swiglu_bf16(c["swiglu_bf16"]["g"], c["swiglu_bf16"]["u"], threads=th),
        "shared_swiglu_sigmoid_bf16": lambda: orc.shared_swiglu_sigmoid_bf16(
            c["shared_swiglu_sigmoid_bf16"]["g"], c["shared_swiglu_sigmoid_bf16"]["u"],
            c["shared_swiglu_sigmoid_bf16"]["logits"], threads=th),
        "gdn_frontend": lambda: orc.gdn_frontend_rows(c["gdn_frontend"]["x"], c["gdn_frontend"]["w"],
                                                      c["gdn_frontend"]["hist"], threads=th),
        "gdn_norm_gate": lambda: orc.norm_gate_rows(c["gdn_norm_gate"]["x"], c["gdn_norm_gate"]["z"],
                                                    c["gdn_norm_gate"]["w"], threads=th),
    }
    f["swiglu_routed_shared_bf16"] = lambda: (f["swiglu_bf16"](), f["shared_swiglu_sigmoid_bf16"]())
    for name in ("dequant_gather_q4_k", "dequant_gather_q6_k"):
        g = c[name]
        f[name] = lambda g=g: orc.dequant_gather(g["table"], g["type"], g["ids"], 2048, threads=th)
    return f


def cpu_baseline(host, kernels, threads: int, repeats: int = 3) -> tuple[dict, float]:
    """The reference CPU path on this host: the float-math build of the oracle
    (oracle/liboracle_fp32.so: the same restatement of the reference kernels,
    float expf / sqrtf / sinf / cosf and float sums, -O2, no fast-math) run on
    the FULL config of every kernel, row-parallel over `threads` std::threads;
    each kernel warmed once, then the median of `repeats` calls. Returns
    per-kernel {us_per_call, gbps} and the step's aggregate GB/s (step bytes over
    the sum of the step kernels' times)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle as orc

    per, tot_b, tot_t = {}, 0.0, 0.0
    with orc.fp32_math():
        fns = cpu_step_fns(orc, host, threads)
        for k in kernels:
            fn = fns[k.name]
            fn()
            times = []
            for _ in range(repeats):
                t0 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t0)
            sec = sorted(times)[len(times) // 2]
            per[k.name] = {"gbps": k.bytes / sec / 1e9, "us_per_call": sec * 1e6}
            if k.in_step:
                tot_b += k.bytes
                tot_t += sec
    return per, tot_b / tot_t / 1e9


def cpu_threads() -> tuple[int, int, int]:
    """(threads used, CPUs this process may run on, logical CPUs of the host).
    The pool is the CPUs this process may run on, capped by OMP_NUM_THREADS when
    the environment sets it (the GPU box sets it to its CPU share per GPU)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    used = min(avail, int(cap)) if cap.isdigit() and int(cap) > 0 else avail
    return max(1, used), avail, os.cpu_count() or avail


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, family / model /
    stepping, cache and clock of the first processor entry."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            k, _, v = line.partition(":")
            fields[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    return (f"{fields.get('model name', 'unknown')} (vendor {fields.get('vendor_id', '?')}, family "
            f"{fields.get('cpu family', '?')}, model {fields.get('model', '?')}, stepping {fields.get('stepping', '?')}, "
            f"cache {fields.get('cache size', '?')}, {fields.get('cpu MHz', '?')} MHz)")


def measure_gguf_load(torch, host, path: Path) -> dict:
    """GGUF file -> device memory (the loader row, src/loader_gguf.cpp:322-381):
    a file holding the C5 tables as token_embd.weight (Q4_K) and output.weight
    (Q6_K), 703 MB, written to `path` and loaded three times by the library
    (median); beside it the reference's scheme (per tensor: read into a host
    buffer, allocate, synchronous pageable copy) run through torch on the same
    file. The file sits in the page cache after writing, so both figures are
    host memory -> PCIe -> HBM, not disk."""
    sys.path.insert(0, str(ROOT / "tests"))
    import gguf_writer as gw
    from qwen35_hip.gguf import GgufFile

    q4, q6 = host["dequant_gather_q4_k"]["table"], host["dequant_gather_q6_k"]["table"]
    ts = [("token_embd.weight", (2048, 248320), 12, memoryview(q4)), ("output.weight", (2048, 248320), 14,
                                                                       memoryview(q6))]
    offs = [0, (q4.nbytes + 31) // 32 * 32]
    head = (b"GGUF" + struct.pack("<IQQ", 3, len(ts), 1) + gw.kv_bytes("general.architecture", gw.STR, "qwen35moe") +
            b"".join(gw.tensor_info_bytes(n, shp, t, o) for (n, shp, t, _), o in zip(ts, offs)))
    with open(path, "wb") as f:   # header (tensor infos), then the payload written in place
        f.write(head)
        payload = (len(head) + 31) // 32 * 32
        f.write(b"\0" * (payload - len(head)))
        f.write(ts[0][3])
        f.write(b"\0" * ((q4.nbytes + 31) // 32 * 32 - q4.nbytes))
        f.write(ts[1][3])
    nbytes = q4.nbytes + q6.nbytes
    times = []
    with GgufFile(path) as g:
        for _ in range(3):
            t0 = time.perf_counter()
            g.load()
            times.append(time.perf_counter() - t0)
            g.unload()
    ours = sorted(times)[1]
    ref_times = []
    for _ in range(2):
        t0 = time.perf_counter()
        with open(path, "rb") as f:
            for k, (_, _, _, b) in enumerate(ts):
                f.seek(payload + offs[k])
                buf = bytearray(len(b))
                f.readinto(buf)
                d = torch.frombuffer(buf, dtype=torch.uint8).to("cuda:0")
                torch.cuda.synchronize()
                del d
        ref_times.append(time.perf_counter() - t0)
    ref = min(ref_times)
    path.unlink()
    return {"config": "GGUF with the C5 tables (Q4_K token_embd 248320x2048 + Q6_K output), page-cache warm",
            "bytes": nbytes, "ms": round(ours * 1e3, 2), "gbps": round(nbytes / ours / 1e9, 2),
            "reference_scheme_ms": round(ref * 1e3, 2), "reference_scheme_gbps": round(nbytes / ref / 1e9, 2)}



def main() -> int:
    ap = argparse.ArgumentParser(description="Fused per-layer kernels on one MI355X")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--launches", type=int, default=64, help="min launches per kernel for the per-kernel timing")
    ap.add_argument("--kernels", default="", help="comma list: only these kernels (profiling runs)")
    ap.add_argument("--no-per-kernel", action="store_true", help="skip the per-kernel and copy measurements")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-next", action="store_true", help="skip the decode GEMV measurements (not part of the step)")
    ap.add_argument("--no-layers", action="store_true",
                    help="skip the layer-composition rows (their 1-token calls of the step kernels would mix into a "
                         "kernel trace of the step kernels)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget")
    ap.add_argument("--json-out", default="", help="also write the JSON line to this file")
    ap.add_argument("--profile-gemv", type=int, default=0, metavar="N",
                    help="also run the LM-head GEMV N times after the step (counter runs)")
    ap.add_argument("--timed-counts", default="", metavar="JSON",
                    help="write each kernel's number of launches in its timed batches (for a steady-state trace)")
    ap.add_argument("--no-step", action="store_true",
                    help="skip the step graph (a trace of the per-kernel steady state only)")
    ap.add_argument("--step-all", action="store_true",
                    help="counter runs: put every kernel in the step graph, also those whose work the step does "
                         "through another entry point (C3b and C3c, done in the step by the routed+shared launch)")
    ap.add_argument("--copy-sweep", default="", metavar="JSON",
                    help="only run the streaming-copy sweep at small sizes and write its records to JSON")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="also run the reference copy of BYTES (read) + BYTES (write) three times, for "
                         "calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE against known traffic")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every kernel is row-local; the multi-GPU path is not built)", file=sys.stderr)
        return 2

    import torch

    from qwen35_hip import PACKAGE_DIR, load, ops, synth

    load()  # fail loudly if the HIP library is missing
    bench_lib = ctypes.CDLL(str(PACKAGE_DIR / "libqwen35_benchutil.so"))
    bench_lib.qwen_bench_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    torch.cuda.set_device(0)
    if args.copy_sweep:
        recs = copy_sweep(torch, bench_lib, int(spin_cycles_per_ms(torch) * 2.0), args.launches)
        Path(args.copy_sweep).write_text(json.dumps(recs, indent=0) + "\n")
        return 0
    t_setup = time.perf_counter()
    kernels, host = build_workload(torch, ops, synth)
    if args.kernels:
        keep = set(args.kernels.split(","))
        kernels = [k for k in kernels if k.name in keep]
    torch.cuda.synchronize()
    print(f"# setup {time.perf_counter() - t_setup:.1f}s, {len(kernels)} kernels", file=sys.stderr, flush=True)
    spin = int(spin_cycles_per_ms(torch) * 2.0)

    # ---- the step: K graph replays (the contract)
    step = [k for k in kernels if k.in_step or args.step_all]
    ms_per_step, value, bytes_step = 0.0, 0.0, sum(k.bytes for k in step)
    if step and not args.no_step:  # (empty only in a profiling run of the decode GEMVs)
        base = [k.make(0) for k in step]
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in base:
                f()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for f in base:
                f()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_per_step = wall / args.steps * 1e3
        value = bytes_step / (ms_per_step * 1e-3) / 1e9
        print(f"# step: {ms_per_step * 1e3:.1f} us, {value:.1f} GB/s aggregate", file=sys.stderr, flush=True)
        del graph

    if args.profile_gemv:
        lm = [k for k in build_next_rows(torch, ops, synth, host) if k.name == "gemv_lm_head_q6_k"][0]
        f = lm.make(0)
        for _ in range(args.profile_gemv):
            f()
        torch.cuda.synchronize()
        print(f"# LM-head GEMV: {args.profile_gemv} launches", file=sys.stderr, flush=True)

    if args.calibrate_copy:
        n = args.calibrate_copy // 16 * 16
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty(n, dtype=torch.uint8, device="cuda:0")
        for _ in range(3):
            if bench_lib.qwen_bench_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), n,
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)):
                raise RuntimeError("qwen_bench_copy failed")
            torch.cuda.synchronize()
        print(f"# calibration copy: {n} bytes read + {n} bytes written per launch, 3 launches", file=sys.stderr,
              flush=True)
        del src, dst

    # ---- per-kernel steady state and the copy ceiling at the same bytes
    if not args.no_per_kernel:
        for k in kernels:
            k.us = measure_kernel(torch, k, spin, args.launches)
            k.copy_us = measure_copy(torch, bench_lib, k.bytes, spin, args.launches)
            print(f"# {k.name:28s} {k.us:9.2f} us  {k.bytes / k.us / 1e3:7.1f} GB/s ({k.bytes / k.us / 1e3 / PEAK_GBPS:6.1%})"
                  f"   copy of same bytes {k.copy_us:8.2f} us {k.bytes / k.copy_us / 1e3:7.1f} GB/s",
                  file=sys.stderr, flush=True)
        big = 1 << 30
        copy_big = measure_copy(torch, bench_lib, big, spin, 16)
        print(f"# copy 1 GiB: {big / copy_big / 1e3:.1f} GB/s", file=sys.stderr, flush=True)

    # ---- decode GEMVs (matmul_dispatch): measured alone, not part of the step
    nxt = []
    if not args.no_next and not args.no_per_kernel:
        nxt = build_next_rows(torch, ops, synth, host)
        if args.kernels:
            nxt = [k for k in nxt if k.name in keep]
        if args.no_layers:
            nxt = [k for k in nxt if not getattr(k, "layer", False)]
        for k in nxt:
            k.us = measure_kernel(torch, k, spin, args.launches)
            k.copy_us = measure_copy(torch, bench_lib, k.bytes, spin, args.launches)
            print(f"# {k.name:28s} {k.us:9.2f} us  {k.bytes / k.us / 1e3:7.1f} GB/s ({k.bytes / k.us / 1e3 / PEAK_GBPS:6.1%})"
                  f"   copy of same bytes {k.copy_us:8.2f} us {k.bytes / k.copy_us / 1e3:7.1f} GB/s" +
                  (f"   {k.flops / k.us / 1e6:.1f} TFLOP/s" if getattr(k, "flops", None) else ""),
                  file=sys.stderr, flush=True)

    gguf = None
    if not args.no_next and not args.no_per_kernel and not args.kernels:
        gguf = measure_gguf_load(torch, host, Path(os.environ.get("TMPDIR", "/tmp")) / f"qwen35_bench_{os.getpid()}.gguf")
        print(f"# gguf load: {gguf['ms']:.1f} ms ({gguf['gbps']:.1f} GB/s); reference scheme "
              f"{gguf['reference_scheme_ms']:.1f} ms ({gguf['reference_scheme_gbps']:.1f} GB/s)", file=sys.stderr,
              flush=True)

    # ---- roofline of the dominant kernel
    roofline = None
    if not args.no_per_kernel and kernels:
        dom = max(kernels, key=lambda k: k.us)
        # HBM bytes per launch from the committed counter runs (FETCH_SIZE and
        # WRITE_SIZE, calibrated on a copy): used only when the kernel's source
        # files still have the digest recorded with the counts, else null.
        from qwen35_hip.rocprof_summary import sources_digest
        traffic, tsrc = None, {"file": "profiles/traffic.json"}
        tf = ROOT / "profiles" / "traffic.json"
        if tf.exists():
            tj = json.loads(tf.read_text())
            rec = tj.get(dom.name, {})
            tsrc["measured_at_commit"] = tj.get("_provenance", {}).get("commit")
            tsrc["sources_sha256"] = rec.get("sources_sha256")
            tsrc["current_sources_sha256"] = sources_digest(dom.name)
            if rec.get("sources_sha256") and rec["sources_sha256"] == tsrc["current_sources_sha256"]:
                traffic = rec.get("bytes_per_launch")
            else:
                tsrc["note"] = "counted on other kernel sources: traffic left null"
        roofline = {"kernel": dom.name, "bound": "hbm", "achieved": round(dom.bytes / dom.us / 1e3, 1),
                    "peak": PEAK_GBPS, "unit": "GB/s", "frac": round(dom.bytes / dom.us / 1e3 / PEAK_GBPS, 4),
                    "traffic": traffic, "traffic_source": tsrc, "algorithmic_bytes": dom.bytes,
                    "us_per_call": round(dom.us, 3),
                    "copy_same_bytes_gbps": round(dom.bytes / dom.copy_us / 1e3, 1),
                    "copy_1gib_gbps": round(big / copy_big / 1e3, 1)}

    # ---- CPU baseline: the reference path on this host's cores, full configs
    cpu = None
    if not args.no_cpu and not args.kernels:
        threads, avail, logical = cpu_threads()
        t_cpu = time.perf_counter()
        per, agg = cpu_baseline(host, kernels, threads)
        # the reference's own host code is one thread: the same full configs on one core
        per1, agg1 = cpu_baseline(host, kernels, 1, repeats=1)
        print(f"# cpu baseline: {agg:.2f} GB/s on {threads} threads, {agg1:.2f} GB/s on 1 "
              f"({time.perf_counter() - t_cpu:.1f} s)", file=sys.stderr, flush=True)
        cpu = {"value": round(agg, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": ("full configs C1-C5 (every row of every config, no extrapolation; C3 as the reference's "
                          "two SwiGLU calls): oracle/liboracle_fp32.so, the C++ restatement of the reference kernels "
                          "with float math, -O2, row-parallel std::threads; step GB/s = step bytes / summed "
                          "per-kernel median time"),
               "host_cpu": cpu_model(), "host_logical_cpus": logical, "cpus_available": avail,
               "per_kernel": {n: {"gbps": round(p["gbps"], 3), "us_per_call": round(p["us_per_call"], 1)}
                              for n, p in per.items()},
               "single_thread": {"value": round(agg1, 3), "cores": 1,
                                 "per_kernel": {n: {"gbps": round(p["gbps"], 3),
                                                    "us_per_call": round(p["us_per_call"], 1)}
                                                for n, p in per1.items()}}}

    next_rows = None
    if nxt:
        cpu_next = {}
        if not args.no_cpu:
            threads = cpu_threads()[0]
            nxt_cpu = [k for k in nxt if not getattr(k, "no_cpu", False)]
            cpu_next, _ = cpu_rates_sampled(host, nxt_cpu, threads, args.cpu_seconds / 3,
                                       gemv={k.name: getattr(k, "gemv", None) or getattr(k, "gdn", None) or
                                             getattr(k, "attn", None) or k.route for k in nxt_cpu})
        next_rows = {
            k.name: {"config": k.config, "bytes": k.bytes, "us_per_call": round(k.us, 3),
                     "gbps": round(k.bytes / k.us / 1e3, 1), "frac_peak": round(k.bytes / k.us / 1e3 / PEAK_GBPS, 4),
                     "copy_same_bytes_us": round(k.copy_us, 3),
                     "cpu_gbps": round(cpu_next[k.name]["gbps"], 3) if k.name in cpu_next else None,
                     **({"tflops": round(k.flops / k.us / 1e6, 1),
                         "mfma_f16_frac": round(2 * k.flops / k.us / 1e6 / PEAK_F16_TFLOPS, 4)}
                        if getattr(k, "flops", None) else {})}
            for k in nxt}

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
        "config": {"workload": "one call of each of the 9 fused kernels at BASELINE configs C1-C5 as one HIP graph "
                               "(storage f32/bf16/Q4_K/Q6_K, math f32)",
                   "bytes_per_step": bytes_step, "parallelism": "single GPU"},
        "kernels": None if args.no_per_kernel else {
            k.name: {"config": k.config, "bytes": k.bytes, "us_per_call": round(k.us, 3),
                     "gbps": round(k.bytes / k.us / 1e3, 1), "frac_peak": round(k.bytes / k.us / 1e3 / PEAK_GBPS, 4),
                     "copy_same_bytes_us": round(k.copy_us, 3)} for k in kernels},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "next_rows": next_rows,
        "gguf_load": gguf,
    }
    if args.timed_counts:
        Path(args.timed_counts).write_text(json.dumps(TIMED_LAUNCHES, indent=1) + "\n")
    text = json.dumps(line)
    print(text, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
