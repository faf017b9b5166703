"""HIP graph capture of the library's entry points.

The kernel entry points enqueue work on the caller's stream and allocate,
memset and synchronise nothing, so a caller can capture them into a graph (the
bench does, for the step). This test captures one call of the fused kernels
and of the next-row kernels (GEMV on both kernels, attention decode with its
workspace, top-k routing, the chunked GDN recurrence with its workspace, the
in-place Q/K norm + RoPE) into one graph, replays it three times with eager
work between the replays (restoring the in-place buffers, an unrelated torch
kernel), and requires every replay to reproduce the eager results bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from qwen35_hip import ops, synth

pytestmark = pytest.mark.gpu

F32 = np.float32


def _dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    if t.dtype in (torch.float32, torch.int32):
        return t.view(torch.int32).cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu()
    return t.cpu()


def test_graph_capture_and_replay():
    r = np.random.default_rng(77)
    n = lambda *s: r.standard_normal(s).astype(F32)  # noqa: E731

    # fused kernels
    x1, w1 = _dev(n(64, 2048)), _dev(1 + 0.1 * n(2048))
    o1 = torch.empty_like(x1)
    xb, bb = _dev(synth.to_bf16_bits(n(256, 2048))), _dev(synth.to_bf16_bits(n(256, 2048)))
    rb, nb = torch.empty_like(xb), torch.empty_like(xb)
    g3, u3 = _dev(synth.to_bf16_bits(2 * n(256, 8 * 512))), _dev(synth.to_bf16_bits(2 * n(256, 8 * 512)))
    h3 = torch.empty_like(g3)
    xc, wc, hin = _dev(n(256, 8192)), _dev(0.5 * n(8192, 4)), _dev(n(8192, 3))
    hout, yc = torch.empty_like(hin), torch.empty_like(xc)
    xg, zg, wg = _dev(n(256, 32, 128)), _dev(n(256, 32, 128)), _dev(1 + 0.1 * n(128))
    og = torch.empty_like(xg)
    tab6 = synth.q6k_table(4096, 2048, seed_tensor=3)
    t6 = _dev(tab6)
    ids = _dev(r.integers(0, 4096, 300).astype(np.int32))
    emb = torch.empty((300, 2048), device="cuda")
    qq0, kk0 = _dev(n(64, 16, 256)), _dev(n(64, 2, 256))
    qq, kk = qq0.clone(), kk0.clone()
    qw, kw = _dev(1 + 0.1 * n(256)), _dev(1 + 0.1 * n(256))
    posv = _dev(np.arange(64, dtype=np.int32) * 7)
    # next rows
    w6 = _dev(synth.q6k_table(16384, 2048, seed_tensor=5))        # int8-MFMA GEMV
    w4 = _dev(synth.q4k_table(8192, 2048, seed_tensor=6))         # per-row GEMV
    xv = _dev(n(2048))
    y6, y4 = torch.empty(16384, device="cuda"), torch.empty(8192, device="cuda")
    heads, kvh, dim, pos = 16, 2, 256, 1000
    q, kc, vc, gate = _dev(n(heads * dim)), _dev(n((pos + 1) * kvh * dim)), _dev(n((pos + 1) * kvh * dim)), \
        _dev(n(heads * dim))
    ws_a = torch.empty(ops.attn_decode_workspace_bytes(heads, kvh, dim, pos), dtype=torch.uint8, device="cuda")
    oa = torch.empty(heads * dim, device="cuda")
    logits = _dev(n(512, 256))
    ti, tw = torch.empty((512, 8), dtype=torch.int32, device="cuda"), torch.empty((512, 8), device="cuda")
    rows, HK, HV, D = 200, 16, 32, 128
    qkv = n(rows, 2 * HK * D + HV * D)
    qkv[:, :2 * HK * D] /= 11.3
    qkv = _dev(qkv)
    beta, decay = _dev(r.uniform(0, 1, (rows, HV)).astype(F32)), _dev(r.uniform(0.9, 1, (rows, HV)).astype(F32))
    st0 = _dev(0.1 * n(HV, D, D))
    st = st0.clone()
    ws_g = torch.empty(ops.load().qwen_gdn_recurrent_chunked_workspace_bytes(rows, HV), dtype=torch.uint8,
                       device="cuda")
    og2 = torch.empty((rows, HV * D), device="cuda")

    outs = [o1, rb, nb, h3, hout, yc, og, emb, qq, kk, y6, y4, oa, ti, tw, st, og2]

    def restore():
        qq.copy_(qq0)
        kk.copy_(kk0)
        st.copy_(st0)

    def run():
        ops.rmsnorm_rows(x1, w1, out=o1)
        ops.residual_rmsnorm_rows(xb, bb, w1, resid=rb, normed=nb)
        ops.swiglu_bf16(g3, u3, out=h3)
        ops.gdn_frontend_rows(xc, wc, hin, hist_out=hout, y=yc)
        ops.gdn_norm_gate_rows(xg, zg, wg, out=og)
        ops.dequant_gather_rows(t6, "Q6_K", 4096 * 2048, ids, 2048, out=emb)
        ops.attn_qk_norm_rope_rows(qq, kk, qw, kw, pos=posv)
        ops.matmul_dispatch(w6, "Q6_K", 16384 * 2048, xv, 16384, 2048, out=y6)
        ops.matmul_dispatch(w4, "Q4_K", 8192 * 2048, xv, 8192, 2048, out=y4)
        ops.attn_decode(q, kc, vc, heads, kvh, dim, pos, gate=gate, workspace=ws_a, out=oa)
        ops.moe_topk_rows(logits, 8, idx=ti, weights=tw)
        ops.gdn_recurrent_chunked(st, qkv, beta, decay, HK, HV, D, D, out=og2, workspace=ws_g)

    restore()
    run()
    torch.cuda.synchronize()
    ref = [_bits(t) for t in outs]

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        restore()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    for rep in range(3):
        for t in outs:                              # eager work between the replays; every
            t.view(torch.uint8).fill_(0x7f)         # replay must write all its outputs again
        restore()
        torch.cuda.synchronize()
        _ = (xv * 3.0).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        for i, t in enumerate(outs):
            assert torch.equal(_bits(t), ref[i]), f"replay {rep}: output {i} differs from the eager call"
