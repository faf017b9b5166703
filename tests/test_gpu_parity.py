"""GPU parity: every C entry point against the CPU oracle on identical inputs.

Bars: fp32 within 1e-5 relative (row-rms floor for cancelling sums), bf16
within 1 ulp, dequant-gather bit-exact. Inputs are the seeded BASELINE configs
(qwen35_hip.synth) at full size plus edge shapes that route through the
scalar / generic paths (odd lengths, unaligned pointers, other head sizes,
kernel sizes and GGML types).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_bf16_close, assert_bits_equal, assert_f32_close, floor_audit
from qwen35_hip import ops, synth

pytestmark = pytest.mark.gpu
THREADS = 16
F32 = np.float32


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ RMSNorm family
def test_rmsnorm_config_c1(oracle):
    c = synth.c1_rmsnorm()
    got = host(ops.rmsnorm_rows(dev(c["x"]), dev(c["w"]), eps=c["eps"]))
    assert_f32_close(got, oracle.rmsnorm_rows(c["x"], c["w"], c["eps"]), what="C1")


@pytest.mark.parametrize("rows,n", [(1, 2), (3, 7), (5, 64), (2, 1000), (9, 1001), (4, 4096), (3, 8192), (1100, 512)])
def test_rmsnorm_shapes(oracle, rows, n):
    r = rng(rows * 100003 + n)
    x = r.standard_normal((rows, n)).astype(F32)
    w = (1 + 0.1 * r.standard_normal(n)).astype(F32)
    got = host(ops.rmsnorm_rows(dev(x), dev(w)))
    assert_f32_close(got, oracle.rmsnorm_rows(x, w), what=f"rmsnorm {rows}x{n}")


def test_rmsnorm_unaligned_and_reference_fixture(oracle):
    r = rng(5)
    buf = dev(r.standard_normal(2049).astype(F32))
    x = buf[1:]  # 4-byte aligned only: the scalar path
    w = dev((1 + 0.1 * r.standard_normal(2048)).astype(F32))
    got = host(ops.rmsnorm_rows(x.view(1, 2048), w))
    assert_f32_close(got, oracle.rmsnorm_rows(host(x).reshape(1, 2048), host(w)), what="unaligned")
    # tests/kernel_tests.cu:301-325 through the single-row entry point
    xf, wf = dev(np.array([3.0, 4.0], F32)), dev(np.array([2.0, 0.5], F32))
    out = torch.empty(2, device="cuda")
    ops.check(ops.load().qwen_rmsnorm_forward(ops._p(xf), ops._p(wf), ops._p(out), 2, 1e-6, ops._stream(None)))
    r_ = 1.0 / np.sqrt(np.float32(12.5) + np.float32(1e-6))
    assert np.max(np.abs(host(out) - np.array([3 * r_ * 2, 4 * r_ * 0.5], F32))) < 1e-5


# 1031 rows: the weight-staging launch shape with a partly filled last workgroup
@pytest.mark.parametrize("rows,n", [(36, 2048), (3, 1001), (8, 8192), (1031, 2048)])
def test_rmsnorm_gated(oracle, rows, n):
    r = rng(n)
    x = r.standard_normal((rows, n)).astype(F32)
    g = (2 * r.standard_normal((rows, n))).astype(F32)
    w = (1 + 0.1 * r.standard_normal(n)).astype(F32)
    got = host(ops.rmsnorm_gated_rows(dev(x), dev(g), dev(w)))
    assert_f32_close(got, oracle.rmsnorm_gated_rows(x, g, w), what="gated")


@pytest.mark.parametrize("n", [2048, 1000, 64, 8192])
@pytest.mark.parametrize("gated", [False, True])
def test_rmsnorm_rows_bits_independent_of_row_count(n, gated):
    """A row normalised alone (the two-wave form below 256 rows) and among 300 or 1100
    rows (one wave per row; weights staged in LDS from 1024 rows) gives the same bits:
    every form adds the squares in one order."""
    r = rng(n + gated)
    x = r.standard_normal((1100, n)).astype(F32)
    g = r.standard_normal((1100, n)).astype(F32)
    w = (1 + 0.1 * r.standard_normal(n)).astype(F32)
    dx, dg, dw = dev(x), dev(g), dev(w)

    def run(rows):
        if gated:
            return host(ops.rmsnorm_gated_rows(dx[:rows].contiguous(), dg[:rows].contiguous(), dw))
        return host(ops.rmsnorm_rows(dx[:rows].contiguous(), dw))
    alone = np.concatenate([run(1)] + [host(ops.rmsnorm_gated_rows(dx[i:i + 1].contiguous(), dg[i:i + 1].contiguous(),
                                                                    dw) if gated else
                                            ops.rmsnorm_rows(dx[i:i + 1].contiguous(), dw)) for i in (1, 299, 1099)])
    few, many, most = run(36), run(300), run(1100)
    for got in (few[:2], many[:2], most[:2]):
        assert_bits_equal(got, alone[:2], what=f"first rows, n {n}")
    assert_bits_equal(many[299], alone[2], what="row 299")
    assert_bits_equal(most[299], alone[2], what="row 299 of 1100")
    assert_bits_equal(most[1099], alone[3], what="row 1099")


@pytest.mark.parametrize("n", [2048, 1001, 1 << 20])
def test_residual_add(oracle, n):
    r = rng(n)
    a, b = r.standard_normal(n).astype(F32), r.standard_normal(n).astype(F32)
    assert_bits_equal(host(ops.residual_add(dev(a), dev(b))), oracle.residual_add(a, b))


def test_residual_rmsnorm_bf16_config_c3a(oracle):
    c = synth.c3_residual()
    resid, normed = ops.residual_rmsnorm_rows(dev(c["x"]), dev(c["branch"]), dev(c["w"]), eps=c["eps"])
    r_ref, n_ref = oracle.residual_rmsnorm_rows(c["x"], c["branch"], c["w"], c["eps"], threads=THREADS)
    assert np.array_equal(host(resid), r_ref), "resid must be the exact RNE of the fp32 sum"
    assert_bf16_close(host(normed), n_ref, what="C3a normed")


# 1025 / 1030 rows: the weight-staging launch shape with a partly filled last workgroup
@pytest.mark.parametrize("rows,n", [(7, 2048), (3, 1000), (2, 6000), (64, 4096), (1025, 4096), (1030, 1000),
                                    (1027, 256)])
def test_residual_rmsnorm_shapes(oracle, rows, n):
    r = rng(rows + n)
    x, b = r.standard_normal((rows, n)).astype(F32), r.standard_normal((rows, n)).astype(F32)
    w = (1 + 0.1 * r.standard_normal(n)).astype(F32)
    resid, normed = ops.residual_rmsnorm_rows(dev(x), dev(b), dev(w))
    r_ref, n_ref = oracle.residual_rmsnorm_rows(x, b, w)
    assert_bits_equal(host(resid), r_ref)
    assert_f32_close(host(normed), n_ref, what="f32 normed")
    xb, bb = synth.to_bf16_bits(x), synth.to_bf16_bits(b)
    resid, normed = ops.residual_rmsnorm_rows(dev(xb), dev(bb), dev(w))
    r_ref, n_ref = oracle.residual_rmsnorm_rows(xb, bb, w)
    assert np.array_equal(host(resid), r_ref)
    assert_bf16_close(host(normed), n_ref, what="bf16 normed")


def test_encoder_forward(oracle):
    table = rng(9).standard_normal((100, 2048)).astype(F32)
    t = dev(table)
    ids = np.array([0, 57, 99, 57], np.int32)
    want = oracle.encoder_rows(ids, table)
    for j, tok in enumerate(ids):
        assert_bits_equal(host(ops.encoder_forward(int(tok), t)), want[j])


# ------------------------------------------------------------------ attention
def test_qk_norm_rope_config_c2(oracle):
    c = synth.c2_qk_rope()
    q, k = dev(c["q"]), dev(c["k"])
    ops.attn_qk_norm_rope_rows(q, k, dev(c["qw"]), dev(c["kw"]), pos=dev(c["pos"]), rope_dim=c["rope_dim"],
                               theta=c["theta"], eps=c["eps"])
    rq, rk = oracle.qk_norm_rope_rows(c["q"], c["k"], c["qw"], c["kw"], pos=c["pos"], rope_dim=c["rope_dim"],
                                      theta=c["theta"], eps=c["eps"], threads=THREADS)
    gq, gk = host(q), host(k)
    assert_f32_close(gq, rq, group=256, what="C2 q")
    assert_f32_close(gk, rk, group=256, what="C2 k")
    # The rms floor must only carry near-zero outputs of the rotation: every
    # element that passes only through it sits far below its head's rms, and its
    # error is within the bar measured against that rms.
    for name, g, r in (("C2 q", gq, rq), ("C2 k", gk, rk)):
        a = floor_audit(g, r, 256, name)
        assert a["floor_only"] <= 1e-3 * a["elements"], a
        assert a["floor_only_max_abs_ref_over_rms"] < 0.05, a


@pytest.mark.parametrize("hd,rd,qh,kh", [(128, 64, 4, 2), (128, 128, 3, 1), (64, 32, 5, 3), (256, 256, 2, 1),
                                         (256, 0, 2, 2), (96, 32, 2, 1), (256, 60, 2, 1)])
def test_qk_norm_rope_shapes(oracle, hd, rd, qh, kh):
    r = rng(hd * 7 + rd)
    rows = 33
    q, k = r.standard_normal((rows, qh, hd)).astype(F32), r.standard_normal((rows, kh, hd)).astype(F32)
    qw, kw = (1 + 0.1 * r.standard_normal(hd)).astype(F32), (1 + 0.1 * r.standard_normal(hd)).astype(F32)
    pos = r.integers(0, 40000, size=rows).astype(np.int32)
    dq, dk = dev(q), dev(k)
    ops.attn_qk_norm_rope_rows(dq, dk, dev(qw), dev(kw), pos=dev(pos), rope_dim=rd, theta=1e6)
    rq, rk = oracle.qk_norm_rope_rows(q, k, qw, kw, pos=pos, rope_dim=rd, theta=1e6)
    assert_f32_close(host(dq), rq, group=hd, what="q")
    assert_f32_close(host(dk), rk, group=hd, what="k")


def test_rope_forward_reference_fixture_and_drop_in(oracle):
    import json
    from pathlib import Path

    fx = json.loads((Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())["rope"]
    x = dev(np.array(fx["x"], F32).reshape(fx["heads"], fx["head_dim"]))
    ops.rope_forward(x, fx["pos"], rope_dim=fx["rope_dim"], theta=fx["theta"])
    assert np.max(np.abs(host(x).ravel() - np.array(fx["expected"], F32))) < fx["tol"]
    # the production shape: 16 heads x 256, rope 64, theta 1e7, pos 511
    v = rng(3).standard_normal((16, 256)).astype(F32)
    d = dev(v)
    ops.rope_forward(d, 511, rope_dim=64, theta=1e7)
    assert_f32_close(host(d), oracle.rope_rows(v[None], pos0=511, rope_dim=64, theta=1e7)[0], group=256)


@pytest.mark.parametrize("heads,dim", [(16, 256), (2, 256), (3, 100)])
def test_attn_head_norm(oracle, heads, dim):
    r = rng(heads * dim)
    x, w = r.standard_normal((heads, dim)).astype(F32), (1 + 0.1 * r.standard_normal(dim)).astype(F32)
    d = dev(x)
    ops.attn_head_norm(d, dev(w))
    assert_f32_close(host(d), oracle.head_norm_rows(x, w), what="head_norm")


# ------------------------------------------------------------------ Gated DeltaNet
@pytest.mark.parametrize("random_history", [False, True])
def test_gdn_frontend_config_c4a(oracle, random_history):
    c = synth.c4_frontend(random_history=random_history)
    hist = dev(c["hist"])
    y, h = ops.gdn_frontend_rows(dev(c["x"]), dev(c["w"]), hist, hist_out=hist, k_heads=c["k_heads"],
                                 key_dim=c["key_dim"], eps=c["eps"])
    ry, rh = oracle.gdn_frontend_rows(c["x"], c["w"], c["hist"], c["k_heads"], c["key_dim"], c["eps"],
                                      threads=THREADS)
    gy = host(y)
    assert_f32_close(gy, ry, group=128, what="C4a y")
    assert_bits_equal(host(h), rh, "C4a history")
    a = floor_audit(gy, ry, 128, f"C4a y (random history {random_history})")
    assert a["floor_only"] <= 1e-3 * a["elements"], a
    assert a["floor_only_max_abs_ref_over_rms"] < 0.05, a


@pytest.mark.parametrize("rows,channels,kernel,heads,dim", [
    (1, 8192, 4, 16, 128), (2, 1024, 4, 2, 128), (65, 1024, 4, 2, 128), (200, 640, 4, 1, 64),
    (130, 768, 4, 3, 128), (50, 8192, 4, 0, 0), (40, 1000, 4, 2, 100), (70, 512, 3, 2, 64), (9, 255, 5, 1, 32)])
def test_gdn_frontend_shapes(oracle, rows, channels, kernel, heads, dim):
    r = rng(rows * 31 + channels + kernel)
    x = r.standard_normal((rows, channels)).astype(F32)
    w = (0.5 * r.standard_normal((channels, kernel))).astype(F32)
    hist = r.standard_normal((channels, kernel - 1)).astype(F32)
    y, h = ops.gdn_frontend_rows(dev(x), dev(w), dev(hist), k_heads=heads, key_dim=dim)
    ry, rh = oracle.gdn_frontend_rows(x, w, hist, heads, dim)
    assert_f32_close(host(y), ry, group=channels, what="y")
    assert_bits_equal(host(h), rh, "history")


def test_gdn_frontend_chunked_equals_one_shot(oracle):
    c = synth.c4_frontend(rows=300, channels=1024, random_history=True)
    x, w = dev(c["x"]), dev(c["w"])
    hist = dev(c["hist"])
    y1, _ = ops.gdn_frontend_rows(x[:100], w, hist, hist_out=hist, k_heads=2, key_dim=128)
    y2, _ = ops.gdn_frontend_rows(x[100:], w, hist, hist_out=hist, k_heads=2, key_dim=128)
    y, h = ops.gdn_frontend_rows(x, w, dev(c["hist"]), k_heads=2, key_dim=128)
    assert_bits_equal(torch.cat([y1, y2]).cpu().numpy(), host(y))
    assert_bits_equal(host(hist), host(h))


def test_gdn_conv_step_sequence_and_qk_normalize(oracle):
    r = rng(77)
    C, T = 8192, 5
    x = r.standard_normal((T, C)).astype(F32)
    w = (0.5 * r.standard_normal((C, 4))).astype(F32)
    hist = dev(np.zeros((C, 3), F32))
    dw = dev(w)
    ys = [host(ops.gdn_conv_step(dev(x[t]), dw, hist)) for t in range(T)]
    ry, rh = oracle.conv_rows(x, w, np.zeros((C, 3), F32))
    assert_f32_close(np.stack(ys), ry, group=C)
    assert_bits_equal(host(hist), rh)
    q = r.standard_normal((16, 128)).astype(F32)
    k = r.standard_normal((16, 128)).astype(F32)
    dq, dk = dev(q), dev(k)
    ops.gdn_qk_normalize(dq, dk)
    rq, rk = oracle.qk_l2_rows(q[None], k[None])
    assert_f32_close(host(dq), rq[0])
    assert_f32_close(host(dk), rk[0])


def test_gdn_norm_gate_config_c4b(oracle):
    c = synth.c4_norm_gate()
    got = host(ops.gdn_norm_gate_rows(dev(c["x"]), dev(c["z"]), dev(c["w"]), eps=c["eps"]))
    assert_f32_close(got, oracle.norm_gate_rows(c["x"], c["z"], c["w"], c["eps"], threads=THREADS), what="C4b")


@pytest.mark.parametrize("shape", [(1, 32, 128), (3, 7, 64), (5, 3, 256), (2, 4, 100)])
def test_gdn_norm_gate_shapes(oracle, shape):
    r = rng(sum(shape))
    x, z = r.standard_normal(shape).astype(F32), r.standard_normal(shape).astype(F32)
    w = (1 + 0.1 * r.standard_normal(shape[-1])).astype(F32)
    got = host(ops.gdn_norm_gate_rows(dev(x), dev(z), dev(w)))
    assert_f32_close(got, oracle.norm_gate_rows(x, z, w), what="norm_gate")


# ------------------------------------------------------------------ MoE
def test_swiglu_config_c3b(oracle):
    c = synth.c3_swiglu()
    got = host(ops.swiglu_bf16(dev(c["g"]), dev(c["u"])))
    assert_bf16_close(got, oracle.swiglu_bf16(c["g"], c["u"], threads=THREADS), what="C3b")


def test_shared_swiglu_config_c3c(oracle):
    c = synth.c3_shared()
    got = host(ops.shared_swiglu_sigmoid_rows_bf16(dev(c["g"]), dev(c["u"]), dev(c["logits"])))
    assert_bf16_close(got, oracle.shared_swiglu_sigmoid_bf16(c["g"], c["u"], c["logits"]), what="C3c")


def test_swiglu_routed_shared_config_c3(oracle):
    """C3's routed [4096 x 8 x 512] and shared [4096 x 512] SwiGLU in one launch:
    each output within 1 bf16 ulp of the oracle and bit-equal to the separate
    entry points (the same per-chunk code runs in both)."""
    c, cs = synth.c3_swiglu(), synth.c3_shared()
    g, u, sg, su, lg = dev(c["g"]), dev(c["u"]), dev(cs["g"]), dev(cs["u"]), dev(cs["logits"])
    h, hs = ops.swiglu_routed_shared_bf16(g, u, sg, su, lg)
    got, got_s = host(h), host(hs)
    assert_bf16_close(got, oracle.swiglu_bf16(c["g"], c["u"], threads=THREADS), what="C3 routed")
    assert_bf16_close(got_s, oracle.shared_swiglu_sigmoid_bf16(cs["g"], cs["u"], cs["logits"]), what="C3 shared")
    assert np.array_equal(got, host(ops.swiglu_bf16(g, u)))
    assert np.array_equal(got_s, host(ops.shared_swiglu_sigmoid_rows_bf16(sg, su, lg)))


@pytest.mark.parametrize("n,rows,dim,offset", [
    (8 * 1000, 3, 520, 0),      # ragged last workgroup in both parts
    (4096, 1, 8, 0),            # one shared row of one chunk
    (37 * 3, 3, 37, 0),         # not whole chunks: the two separate launches
    (8 * 64, 5, 64, 1),         # misaligned routed pointers: the two separate launches
    (0, 7, 512, 0),             # routed part empty
    (8 * 512, 0, 512, 0),       # shared part empty
])
def test_swiglu_routed_shared_shapes(oracle, n, rows, dim, offset):
    r = rng(n + rows * 7 + dim)
    g = synth.to_bf16_bits(2 * r.standard_normal(n + offset).astype(F32))
    u = synth.to_bf16_bits(2 * r.standard_normal(n + offset).astype(F32))
    sg = synth.to_bf16_bits(2 * r.standard_normal((rows, dim)).astype(F32))
    su = synth.to_bf16_bits(2 * r.standard_normal((rows, dim)).astype(F32))
    lg = r.standard_normal(rows).astype(F32)
    dg, du = dev(g)[offset:], dev(u)[offset:]
    h, hs = ops.swiglu_routed_shared_bf16(dg, du, dev(sg), dev(su), dev(lg))
    if n:
        assert_bf16_close(host(h), oracle.swiglu_bf16(g[offset:], u[offset:]), what="routed")
    if rows:
        assert_bf16_close(host(hs), oracle.shared_swiglu_sigmoid_bf16(sg, su, lg), what="shared")


def test_swiglu_exhaustive_and_odd(oracle):
    g = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    u = np.full_like(g, 0x3F80)
    assert_bf16_close(host(ops.swiglu_bf16(dev(g), dev(u))), oracle.swiglu_bf16(g, u), what="all bf16 g")
    r = rng(4)
    g2 = synth.to_bf16_bits(2 * r.standard_normal((3, 37)).astype(F32))
    u2 = synth.to_bf16_bits(2 * r.standard_normal((3, 37)).astype(F32))
    lg = r.standard_normal(3).astype(F32)
    assert_bf16_close(host(ops.swiglu_bf16(dev(g2), dev(u2))), oracle.swiglu_bf16(g2, u2))
    assert_bf16_close(host(ops.shared_swiglu_sigmoid_rows_bf16(dev(g2), dev(u2), dev(lg))),
                      oracle.shared_swiglu_sigmoid_bf16(g2, u2, lg))


@pytest.mark.parametrize("n", [512, 2047, 1 << 20])
def test_moe_silu_mul(oracle, n):
    r = rng(n)
    g, u = (2 * r.standard_normal(n)).astype(F32), (2 * r.standard_normal(n)).astype(F32)
    assert_f32_close(host(ops.moe_silu_mul(dev(g), dev(u))), oracle.silu_mul(g, u))


@pytest.mark.parametrize("rows,n", [(1, 2048), (4096, 2048), (3, 1001)])
def test_moe_shared_add(oracle, rows, n):
    r = rng(rows + n)
    acc, x = r.standard_normal((rows, n)).astype(F32), r.standard_normal((rows, n)).astype(F32)
    gate = r.standard_normal(rows).astype(F32)
    got = host(ops.moe_shared_add_rows(dev(acc), dev(x), dev(gate)))
    assert_f32_close(got, oracle.shared_add_rows(acc, x, gate), group=n)


# ------------------------------------------------------------------ dequant gather
@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_gather_config_c5(oracle, kind):
    vocab, cols = 248320, 2048
    table = synth.q4k_table(vocab, cols) if kind == "Q4_K" else synth.q6k_table(vocab, cols)
    ids = synth.token_ids(8192, vocab)
    t = ops.GGML_TYPES[kind]
    got = host(ops.dequant_gather_rows(dev(table), kind, vocab * cols, dev(ids), cols))
    assert_bits_equal(got, oracle.dequant_gather(table, t, ids, cols, threads=THREADS), f"C5 {kind}")


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K", "Q4_0", "Q5_0", "Q8_0", "Q5_K", "F16", "BF16", "F32"])
@pytest.mark.parametrize("cols", [2048, 768, 256])
def test_gather_types(oracle, kind, cols):
    import ggml_blocks

    t = ops.GGML_TYPES[kind]
    r = rng(t * 1000 + cols)
    vocab = 300
    if t in ggml_blocks.BLOCK:
        elems = ggml_blocks.BLOCK[t][0]
        table = ggml_blocks.random_blocks(r, t, vocab * cols // elems)
    else:
        width = 4 if kind == "F32" else 2
        table = r.integers(0, 256, size=vocab * cols * width, dtype=np.uint8)
        if kind != "BF16":  # keep floats finite
            table = (r.standard_normal(vocab * cols).astype(np.float32 if kind == "F32" else np.float16)).view(np.uint8)
    ids = r.integers(0, vocab, size=77).astype(np.int32)
    got = host(ops.dequant_gather_rows(dev(table), t, vocab * cols, dev(ids), cols))
    ref = oracle.dequant_gather(table, t, ids, cols)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_bits_equal(np.where(nan, 0, got), np.where(nan, 0, ref), f"{kind} cols {cols}")


def test_gather_out_of_range_ids_give_nan(oracle):
    table = synth.q4k_table(16, 2048)
    ids = np.array([3, -1, 16, 15, 1 << 30], dtype=np.int32)
    got = host(ops.dequant_gather_rows(dev(table), "Q4_K", 16 * 2048, dev(ids), 2048))
    assert np.isnan(got[[1, 2, 4]]).all()
    assert_bits_equal(got[[0, 3]], oracle.dequant_gather(table, 12, ids[[0, 3]], 2048))


@pytest.mark.parametrize("kind,cols,row", [("Q4_K", 2048, 5), ("Q6_K", 2048, 0), ("Q4_K", 100, 7), ("Q6_K", 300, 3),
                                           ("Q8_0", 50, 9), ("F16", 33, 4)])
def test_dequantize_row(oracle, kind, cols, row):
    import ggml_blocks

    t = ops.GGML_TYPES[kind]
    r = rng(cols + row)
    n_el = 16 * 2048
    if t in ggml_blocks.BLOCK:
        table = ggml_blocks.random_blocks(r, t, n_el // ggml_blocks.BLOCK[t][0])
    else:
        table = r.standard_normal(n_el).astype(np.float16).view(np.uint8)
    got = host(ops.dequantize_row(dev(table), kind, n_el, row, cols))
    assert_bits_equal(got, oracle.dequant_span(table, t, row * cols, cols), f"{kind} row {row}")


@pytest.mark.parametrize("kind", ["Q4_0", "Q5_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K"])
def test_reference_quant_fixtures_on_gpu(kind):
    """The reference's own block fixtures (tests/kernel_tests.cu:116-223, frozen in
    tests/golden/reference_fixtures.json) through every GPU dequant path: rows of
    8 copies of the block via dequantize_row, the gather, and the GEMV with one-hot
    x (which reads exactly one weight per row: w_j = (d*sc)*q - dmin*m, bit for bit);
    for Q4_K and Q6_K also at a row count that takes the int8-MFMA GEMV."""
    import json
    from pathlib import Path

    fx = json.loads((Path(__file__).resolve().parent / "golden" / "reference_fixtures.json").read_text())["quant"][kind]
    blk = np.frombuffer(bytes.fromhex(fx["bytes_hex"]), np.uint8)
    exp_row = np.tile(np.asarray(fx["expected"], F32), 8)
    cols = exp_row.size

    def table(rows):
        return dev(np.tile(blk, 8 * rows))

    tab = table(4)
    got = host(ops.dequantize_row(tab, kind, 4 * cols, 2, cols))
    assert np.array_equal(got, exp_row), np.argwhere(got != exp_row)[:5]
    ids = dev(np.array([0, 3, 1, 2, 2], np.int32))
    got = host(ops.dequant_gather_rows(tab, kind, 4 * cols, ids, cols))
    assert np.array_equal(got, np.tile(exp_row, (5, 1)))
    sizes = [64] + ({"Q4_K": [65536], "Q6_K": [16384]}.get(kind, []) if cols == 2048 else [])
    for M in sizes:
        w = table(M)
        for j in (0, 1, 37, cols // 2 + 5, cols - 1):
            x = np.zeros(cols, F32)
            x[j] = 1.0
            y = host(ops.matmul_dispatch(w, kind, M * cols, dev(x), M, cols))
            assert np.array_equal(y, np.full(M, exp_row[j], F32)), (M, j, y[:4], exp_row[j])


# ------------------------------------------------------------------ GDN gates + recurrent state
def _gdn_inputs(r, rows, kh, vh, dk, dv, extra=0):
    """Front-end-like rows (unit-norm k, q scaled by dk^-1/2, v ~ N(0,1)), gates from raw
    projections through the oracle's gate formula, and a random state."""
    kd = kh * dk
    qkv = r.standard_normal((rows, 2 * kd + vh * dv + extra)).astype(F32)
    for t in range(rows):
        for part, scale in ((0, dk ** -0.5), (kd, 1.0)):
            seg = qkv[t, part:part + kd].reshape(kh, dk)
            seg /= np.linalg.norm(seg, axis=1, keepdims=True)
            seg *= scale
    b = r.standard_normal((rows, vh)).astype(F32)
    alpha = (2 * r.standard_normal((rows, vh))).astype(F32)
    a = -np.exp(r.standard_normal(vh)).astype(F32)
    dt = r.uniform(-1, 1, vh).astype(F32)
    state = (0.5 * r.standard_normal(vh * dk * dv)).astype(F32)
    return qkv, b, alpha, a, dt, state


def test_gdn_gate_values(oracle):
    r = rng(31)
    rows, heads = 64, 32
    b = (4 * r.standard_normal((rows, heads))).astype(F32)
    alpha = (8 * r.standard_normal((rows, heads))).astype(F32)
    alpha[0, :4] = [25.0, 20.5, 19.5, -90.0]  # both sides of the softplus threshold
    a = -np.exp(r.standard_normal(heads)).astype(F32)
    dt = r.uniform(-1, 1, heads).astype(F32)
    beta, decay = ops.gdn_gate_values_rows(dev(b), dev(alpha), dev(a), dev(dt))
    rb, rd = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    assert_f32_close(host(beta), rb, what="beta")
    assert_f32_close(host(decay), rd, what="decay")


def test_gdn_recurrent_reference_fixture():
    """tests/kernel_tests.cu:225-262 (kh=2, vh=4, dk=4, dv=3: the generic path), three steps."""
    import json
    from pathlib import Path

    fx = json.loads((Path(__file__).resolve().parent / "golden" / "reference_fixtures.json").read_text())["gdn_recurrent"]
    kh, vh, dk, dv = fx["key_heads"], fx["value_heads"], fx["key_dim"], fx["value_dim"]
    state = torch.zeros(vh * dk * dv, dtype=torch.float32, device="cuda")
    for st in fx["steps"]:
        out = ops.gdn_recurrent_step(state, *(dev(np.array(st[n], dtype=F32)) for n in ("q", "k", "v", "beta", "decay")),
                                     kh, vh, dk, dv)
        assert np.max(np.abs(host(out) - np.array(st["expected"], dtype=F32))) < fx["tol"]


@pytest.mark.parametrize("kh,vh,dk,dv,rows", [(16, 32, 128, 128, 1), (16, 32, 128, 128, 37), (4, 8, 64, 64, 9),
                                              (2, 4, 96, 100, 5), (3, 6, 128, 256, 3), (4, 8, 64, 64, 1),
                                              (3, 6, 128, 256, 1), (3, 6, 128, 36, 1), (2, 4, 64, 100, 1),
                                              (3, 6, 128, 48, 1), (1, 5, 64, 80, 1)])
def test_gdn_recurrent_rows(oracle, kh, vh, dk, dv, rows):
    """Qwen3.5 GDN shape (16 key / 32 value heads of 128), a token count that is not a
    multiple of the 4-deep prefetch, key dim 64, and generic shapes (dk 96, dv 100 / 256);
    one token on the 16-column tile (key dim 64 / 128, dv 64 / 256; dv 48 / 80, whose
    18 / 25 tiles leave 2 / 9 outside the XCD-paired groups of 16) and on the 4-column
    slices (dv 36 / 100)."""
    r = rng(kh * 1000 + rows)
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, rows, kh, vh, dk, dv, extra=8)
    beta, decay = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    ds = dev(state)
    out = host(ops.gdn_recurrent_rows(ds, dev(qkv), dev(beta), dev(decay), kh, vh, dk, dv))
    # Oracle token by token, keeping each readout's condition scale sum_i |q_i| |S_ij|:
    # out_j is a dot product that can cancel (a strongly decayed head reads ~1e-4 from
    # terms ~4e-3), so its fp32 error is bounded relative to that scale, not to |out_j|.
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, out, host(ds), kh, vh, dk, dv)


def _check_gdn_recurrence(oracle, qkv, beta, decay, state, out, new_state, kh, vh, dk, dv):
    """The oracle token by token, keeping each readout's condition scale
    sum_i |q_i| |S_ij|: out_j is a dot product that can cancel (a strongly decayed
    head reads ~1e-4 from terms ~4e-3), so its fp32 error is bounded relative to
    that scale, not to |out_j|."""
    rows = qkv.shape[0]
    ref_state = state.copy()
    kd = kh * dk
    ref = np.empty_like(out)
    scale = np.empty(out.shape, dtype=np.float64)
    src = np.arange(vh) % kh
    for t in range(rows):
        q, k, v = qkv[t, :kd], qkv[t, kd:2 * kd], qkv[t, 2 * kd:2 * kd + vh * dv]
        ref[t] = oracle.gdn_recurrent_step(ref_state, q, k, v, beta[t], decay[t], kh, vh, dk, dv)
        aq = np.abs(q.astype(np.float64)).reshape(kh, dk)[src]                       # [vh, dk]
        aS = np.abs(ref_state.astype(np.float64)).reshape(vh, dk, dv)
        scale[t] = np.einsum("hi,hij->hj", aq, aS).reshape(-1)
    err = np.abs(out.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), scale)
    worst = np.unravel_index(int(np.argmax(err)), err.shape)
    assert err[worst] <= 1e-5, f"out rel err {err[worst]:.3e} at {worst}: got {out[worst]!r} ref {ref[worst]!r}"
    assert_f32_close(new_state, ref_state, group=dv, what="state")


@pytest.mark.parametrize("rows,gates", [(1, "normal"), (63, "normal"), (64, "normal"), (200, "normal"),
                                        (700, "normal"), (150, "fast_decay"), (150, "beta_one"),
                                        (128, "tiny_late_beta")])
def test_gdn_recurrent_chunked(oracle, rows, gates):
    """The chunked prefill form against the oracle's token loop at the Qwen3.5 GDN shape:
    partial last chunks, several chunks, decays that underflow to zero inside a chunk
    (the ratios are running products), beta near 1 (the triangular solve's
    largest off-diagonal terms), and fast decay with beta ~1e-17 on the second half of
    each chunk, ending in that half: the final state (~1e-23 for some heads) is then
    R[C-1] Delta of the last tokens alone, whose fp16 scale must come from a bound
    that pairs each token's factors (pairing the largest of each overstated it by
    ~1e17) and be undone exactly at any magnitude (a float multiplier clamped to stay
    normal lost those heads; both flushed the state to zeros in a CPU emulation)."""
    kh, vh, dk, dv = 16, 32, 128, 128
    r = rng(rows * 3 + len(gates))
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, rows, kh, vh, dk, dv)
    if gates in ("fast_decay", "tiny_late_beta"):
        alpha = (alpha + 60.0).astype(F32)      # softplus ~ 60: decay exp(a * 60) underflows for a < -1.6
    if gates == "beta_one":
        b = (b + 12.0).astype(F32)
    elif gates == "tiny_late_beta":
        late = (np.arange(rows) % 64) >= 32
        b = np.where(late[:, None], b - 40.0, b).astype(F32)
    beta, decay = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    if gates == "fast_decay":
        assert (decay == 0).any() and (decay > 0).any()
    ds = dev(state)
    ws = torch.empty(ops.load().qwen_gdn_recurrent_chunked_workspace_bytes(rows, vh), dtype=torch.uint8,
                     device="cuda")
    out = host(ops.gdn_recurrent_chunked(ds, dev(qkv), dev(beta), dev(decay), kh, vh, dk, dv, workspace=ws))
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, out, host(ds), kh, vh, dk, dv)


@pytest.mark.parametrize("kh,vh", [(4, 4), (2, 6), (2, 3), (4, 2)])
def test_gdn_recurrent_chunked_head_maps(oracle, kh, vh):
    """Value head h reads key head h % key_heads (src/cuda/gdn.cu:108-151); the
    chunked prep computes K K^T and Q K^T once per key head for every value head
    that reads it: one, three, an uneven split (2 key heads, 3 value heads) and
    more key heads than value heads, over a ragged second chunk."""
    dk, dv, rows = 128, 32, 100
    r = rng(kh * 16 + vh)
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, rows, kh, vh, dk, dv)
    beta, decay = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    ds = dev(state)
    out = host(ops.gdn_recurrent_chunked(ds, dev(qkv), dev(beta), dev(decay), kh, vh, dk, dv))
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, out, host(ds), kh, vh, dk, dv)


def test_gdn_recurrent_chunked_strides(oracle):
    """Row strides the chunked state walk addresses with 32-bit lane offsets from a
    per-chunk base: a qkv row padded past q | k | v and an output row padded past its
    values (the padding stays untouched); one row with strides 0 (the walk reads a
    range one stride long, so the library widens it to the row); and a qkv stride past
    the walk's 32-bit limit, which runs the token loop (the same bits as calling it)."""
    import ctypes
    from qwen35_hip._lib import check

    lib = ops.load()
    kh, vh, dk, dv = 4, 8, 128, 32
    kd = kh * dk
    vp = lambda t: ctypes.c_void_p(t.data_ptr())

    def call(fn, state, qkv_t, beta, decay, out_t, rows, qs, os, ws=True):
        base = qkv_t.data_ptr()
        args = [vp(state), ctypes.c_void_p(base), ctypes.c_void_p(base + 4 * kd), ctypes.c_void_p(base + 8 * kd),
                vp(beta), vp(decay), vp(out_t), rows, kh, vh, dk, dv, qs, os]
        if ws:
            w = torch.empty(lib.qwen_gdn_recurrent_chunked_workspace_bytes(rows, vh), dtype=torch.uint8, device="cuda")
            args += [vp(w), w.numel()]
        check(fn(*args, None))
        torch.cuda.synchronize()

    r = rng(977)
    # padded rows: qkv stride 2 kd + vh dv + 12, output stride vh dv + 20 (two chunks, the second ragged)
    rows = 100
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, rows, kh, vh, dk, dv, extra=12)
    beta, decay = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    ds = dev(state)
    out = torch.full((rows, vh * dv + 20), 7.0, device="cuda")
    call(lib.qwen_gdn_recurrent_chunked, ds, dev(qkv), dev(beta), dev(decay), out, rows, qkv.shape[1], out.shape[1])
    o = host(out)
    assert (o[:, vh * dv:] == 7.0).all(), "output padding written"
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, np.ascontiguousarray(o[:, :vh * dv]), host(ds), kh, vh, dk, dv)
    # one row, strides 0
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, 1, kh, vh, dk, dv)
    beta, decay = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    ds = dev(state)
    out = torch.empty((1, vh * dv), device="cuda")
    call(lib.qwen_gdn_recurrent_chunked, ds, dev(qkv), dev(beta), dev(decay), out, 1, 0, 0)
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, host(out), host(ds), kh, vh, dk, dv)
    # qkv stride 8,400,000 floats (past 2^31 bytes over 64 rows): the token loop, bit for bit
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, 2, kh, vh, dk, dv)
    beta, decay = (dev(x) for x in oracle.gdn_gate_values_rows(b, alpha, a, dt))
    wide = torch.zeros((2, 8_400_000), device="cuda")
    wide[:, :qkv.shape[1]] = dev(qkv)
    s1, s2 = dev(state), dev(state)
    o1, o2 = torch.empty((2, vh * dv), device="cuda"), torch.empty((2, vh * dv), device="cuda")
    call(lib.qwen_gdn_recurrent_chunked, s1, wide, beta, decay, o1, 2, wide.shape[1], vh * dv)
    call(lib.qwen_gdn_recurrent_rows, s2, wide, beta, decay, o2, 2, wide.shape[1], vh * dv, ws=False)
    assert_bits_equal(host(o1), host(o2), "long-stride fallback outputs")
    assert_bits_equal(host(s1), host(s2), "long-stride fallback state")


def test_gdn_recurrent_chunked_long_and_fallback(oracle):
    """2048 tokens (32 chunks): the chunked form and the token-loop kernel both
    against the oracle's token loop (condition-scale bar: late outputs of strongly
    decayed heads are tiny cancelling sums); key dim 64 (not chunked) runs the
    token loop; a short workspace is rejected."""
    from qwen35_hip._lib import QwenError

    kh, vh, dk, dv, T = 16, 32, 128, 128, 2048
    r = rng(4096)
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, T, kh, vh, dk, dv)
    beta, decay = oracle.gdn_gate_values_rows(b, alpha, a, dt)
    s1, s2, dq = dev(state), dev(state), dev(qkv)
    o1 = host(ops.gdn_recurrent_chunked(s1, dq, dev(beta), dev(decay), kh, vh, dk, dv))
    o2 = host(ops.gdn_recurrent_rows(s2, dq, dev(beta), dev(decay), kh, vh, dk, dv))
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, o1, host(s1), kh, vh, dk, dv)
    _check_gdn_recurrence(oracle, qkv, beta, decay, state, o2, host(s2), kh, vh, dk, dv)
    kh, vh, dk, dv, T = 4, 8, 64, 64, 9
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, T, kh, vh, dk, dv)
    beta, decay = ops.gdn_gate_values_rows(dev(b), dev(alpha), dev(a), dev(dt))
    s1, s2, dq = dev(state), dev(state), dev(qkv)
    o1 = host(ops.gdn_recurrent_chunked(s1, dq, beta, decay, kh, vh, dk, dv,
                                        workspace=torch.empty(16, dtype=torch.uint8, device="cuda")))
    o2 = host(ops.gdn_recurrent_rows(s2, dq, beta, decay, kh, vh, dk, dv))
    assert_bits_equal(o1, o2, "fallback")
    with pytest.raises(QwenError):
        qkv, b, alpha, a, dt, state = _gdn_inputs(r, 100, 16, 32, 128, 128)
        beta, decay = ops.gdn_gate_values_rows(dev(b), dev(alpha), dev(a), dev(dt))
        ops.gdn_recurrent_chunked(dev(state), dev(qkv), beta, decay, 16, 32, 128, 128,
                                  workspace=torch.empty(1024, dtype=torch.uint8, device="cuda"))


def test_gdn_recurrent_rows_equals_steps():
    """One launch over T tokens matches T single-step launches (the decode path's
    kernel) to fp32 rounding: the two kernels sum a column's rows in different
    orders."""
    kh, vh, dk, dv, T = 16, 32, 128, 128, 6
    r = rng(77)
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, T, kh, vh, dk, dv)
    beta, decay = ops.gdn_gate_values_rows(dev(b), dev(alpha), dev(a), dev(dt))
    s1, s2 = dev(state), dev(state)
    dq = dev(qkv)
    out = host(ops.gdn_recurrent_rows(s1, dq, beta, decay, kh, vh, dk, dv))
    kd = kh * dk
    for t in range(T):
        o = ops.gdn_recurrent_step(s2, dq[t, :kd].contiguous(), dq[t, kd:2 * kd].contiguous(),
                                   dq[t, 2 * kd:].contiguous(), beta[t].contiguous(), decay[t].contiguous(),
                                   kh, vh, dk, dv)
        assert_f32_close(host(o), out[t], group=dv, rtol=1e-5, what=f"token {t}")
    assert_f32_close(host(s1), host(s2), group=dv, what="state")


@pytest.mark.parametrize("kind,heads,hd,K", [("Q4_K", 16, 256, 2048), ("Q6_K", 4, 256, 2048), ("Q4_K", 8, 64, 512),
                                             ("Q8_0", 4, 32, 256)])
def test_matmul_dispatch_multi_split_equals_projection_then_split(kind, heads, hd, K):
    """A descriptor with split = head_dim writes the fused query | gate
    projection in attn_split_qg's layout: bit-equal to matmul_dispatch followed
    by attn_split_qg (src/layer_attn.cpp:85,90), on the per-row kernel (Q4_K,
    Q6_K, packed rows at K = 512) and the generic one (Q8_0); an unsplit
    descriptor in the same call is unaffected."""
    r = rng(heads * hd + K)
    M = 2 * heads * hd
    t = ops.GGML_TYPES[kind]
    w = dev(_gemv_weight(kind, M, K, r))
    w2 = dev(_gemv_weight(kind, 96, K, r))
    x = dev(r.standard_normal(K).astype(F32))
    ys, y2 = torch.empty(M, device="cuda"), torch.empty(96, device="cuda")
    ops.matmul_dispatch_multi([(w, t, M * K, M, 0, ys, hd), (w2, t, 96 * K, 96, 0, y2)], x, K)
    full = ops.matmul_dispatch(w, t, M * K, x, M, K)
    q, g = ops.attn_split_qg(full, heads, hd)
    assert_bits_equal(host(ys[:M // 2]), host(q), what=f"{kind} q")
    assert_bits_equal(host(ys[M // 2:]), host(g), what=f"{kind} gate")
    assert_bits_equal(host(y2), host(ops.matmul_dispatch(w2, t, 96 * K, x, 96, K)), what=f"{kind} unsplit")


def test_matmul_dispatch_multi_rejects_unpaired_split():
    from qwen35_hip._lib import QwenError

    w = dev(synth.q4k_table(96, 2048, seed_tensor=1))
    x = torch.zeros(2048, device="cuda")
    with pytest.raises(QwenError, match="descriptor 0: split 64 does not pair the 96 rows"):
        ops.matmul_dispatch_multi([(w, "Q4_K", 96 * 2048, 96, 0, None, 64)], x, 2048)


@pytest.mark.parametrize("kh,vh,dk,dv,alias", [(16, 32, 128, 128, False), (4, 8, 128, 64, False),
                                               (16, 32, 128, 128, True), (2, 4, 64, 32, False),
                                               (2, 4, 128, 36, False), (2, 6, 128, 256, False),
                                               (3, 6, 128, 48, False)])
def test_gdn_decode_step_equals_frontend_then_gated_recurrence(kh, vh, dk, dv, alias):
    """The one-launch decode step (front end + fused-gate recurrence) gives the
    bits of gdn_frontend_rows (one row) followed by gdn_gated_recurrent_rows:
    conv output, new history, state and output, over three tokens with the
    history carried; an in-place history (alias), key dim 64 and a value dim
    that is not a multiple of 32 take the two calls inside the same entry point."""
    r = rng(kh * vh + dk + dv + alias)
    C = 2 * kh * dk + vh * dv
    cw = dev((0.5 * r.standard_normal((C, 4))).astype(F32))
    a = dev(-np.exp(r.standard_normal(vh)).astype(F32))
    dt = dev(r.uniform(-1, 1, vh).astype(F32))
    st_f = dev((0.1 * r.standard_normal((vh, dk, dv))).astype(F32))
    st_r = st_f.clone()
    hist_f = dev(r.standard_normal((C, 3)).astype(F32))
    hist_r = hist_f.clone()
    spare = torch.empty_like(hist_f)
    for t in range(3):
        x = dev(r.standard_normal(C).astype(F32))
        br, ar = dev(r.standard_normal(vh).astype(F32)), dev(r.standard_normal(vh).astype(F32))
        # reference: the two calls, history in place
        y_r, _ = ops.gdn_frontend_rows(x.view(1, C), cw, hist_r, hist_out=hist_r, k_heads=kh, key_dim=dk)
        o_r = ops.gdn_gated_recurrent_rows(st_r, y_r, br.view(1, vh), ar.view(1, vh), a, dt, kh, vh, dk, dv)
        y_f = torch.empty(C, device="cuda")
        hout = hist_f if alias else spare
        o_f = ops.gdn_decode_step(x, cw, hist_f, hout, st_f, br, ar, a, dt, kh, vh, dk, dv, y=y_f)
        if not alias:
            hist_f, spare = spare, hist_f
        assert_bits_equal(host(y_f), host(y_r).reshape(-1), what=f"token {t} conv output")
        assert_bits_equal(host(hist_f), host(hist_r), what=f"token {t} history")
        assert_bits_equal(host(o_f), host(o_r).reshape(-1), what=f"token {t} output")
        assert_bits_equal(host(st_f), host(st_r), what=f"token {t} state")


@pytest.mark.parametrize("rows,kh,vh,dk,dv", [(1, 16, 32, 128, 128), (1, 4, 8, 64, 64), (37, 16, 32, 128, 128),
                                               (5, 2, 4, 100, 48), (1, 3, 6, 128, 36)])
def test_gdn_gated_recurrent_equals_gates_then_recurrence(rows, kh, vh, dk, dv):
    """The fused-gate recurrence (qwen_gdn_gated_recurrent_rows) gives the bits of
    gdn_gate_values_rows followed by gdn_recurrent_rows on every kernel path (one
    token, the token loop, the generic form), with gates that reach the softplus
    threshold (alpha + dt > 20) and saturated betas."""
    r = rng(rows * 1000 + dk)
    qkv, b, alpha, a, dt, state = _gdn_inputs(r, rows, kh, vh, dk, dv)
    alpha[:, 0] = 25.0          # softplus(x) = x branch
    b[:, 1 % vh] = -30.0        # beta ~ 0
    beta, decay = ops.gdn_gate_values_rows(dev(b), dev(alpha), dev(a), dev(dt))
    s1, s2 = dev(state), dev(state)
    dq = dev(qkv)
    ref = host(ops.gdn_recurrent_rows(s1, dq, beta, decay, kh, vh, dk, dv))
    got = host(ops.gdn_gated_recurrent_rows(s2, dq, dev(b), dev(alpha), dev(a), dev(dt), kh, vh, dk, dv))
    assert_bits_equal(got, ref, "out")
    assert_bits_equal(host(s2), host(s1), "state")


@pytest.mark.parametrize("kind,heads,dim,M,off_rows", [("Q4_K", 32, 128, 2048, 0), ("Q4_K", 16, 128, 96, 3),
                                                        ("Q4_K", 32, 64, 1000, 0), ("Q4_K", 16, 256, 4100, 0),
                                                        ("Q4_K", 16, 128, 16400, 0),
                                                        ("Q6_K", 32, 128, 64, 0), ("Q4_K", 3, 128, 40, 0)])
def test_gdn_norm_gate_matmul_equals_norm_gate_then_matmul(kind, heads, dim, M, off_rows):
    """The gated norm and output projection in one entry point (src/layer_gdn.cpp:
    109-112) give the bits of gdn_norm_gate_rows followed by matmul_dispatch, normed
    included: the one-launch form (Q4_K, K = heads * dim a multiple of 2048, dim 64 /
    128 / 256, R = 1, 2 and 4 rows per wave, a row offset into the tensor) and the two
    calls it falls back to (Q6_K; K = 384)."""
    r = rng(heads * dim + M)
    K = heads * dim
    t = ops.GGML_TYPES[kind]
    w = dev(_gemv_weight(kind, M + off_rows, K, r))
    n_el = (M + off_rows) * K
    x = dev(r.standard_normal((heads, dim)).astype(F32))
    z = dev((2 * r.standard_normal((heads, dim))).astype(F32))
    nw = dev((1 + 0.1 * r.standard_normal(dim)).astype(F32))
    ref_n = ops.gdn_norm_gate_rows(x, z, nw)
    ref_y = ops.matmul_dispatch(w, t, n_el, ref_n.view(-1), M, K, element_offset=off_rows * K)
    got_n, got_y = ops.gdn_norm_gate_matmul(x, z, nw, w, t, n_el, M, element_offset=off_rows * K)
    assert_bits_equal(host(got_n), host(ref_n), what=f"{kind} normed")
    assert_bits_equal(host(got_y), host(ref_y), what=f"{kind} {M}x{K} out")


def test_gdn_layer_decode_fused_equals_reference_launches():
    """A GDN layer's decode step (src/layer_gdn.cpp:78-113) through the fused
    entry points (three launches) against the reference's sequence of calls on the
    same library (ten launches), three tokens in a row with the conv history and
    the recurrent state carried: same outputs, state and history (the fused
    front end's L2 norm sums in another order, so fp32 tolerance)."""
    from qwen35_hip.decode_layers import GdnLayerDecode

    r = rng(31)
    dm, kh, vh, dk, dv = 2048, 16, 32, 128, 128
    cd, vd = 2 * kh * dk + vh * dv, vh * dv

    def q4(M, K, s):
        return dev(synth.q4k_table(M, K, seed_tensor=s))
    wq, wz, wb, wa, wo = q4(cd, dm, 40), q4(vd, dm, 41), q4(vh, dm, 42), q4(vh, dm, 43), q4(dm, vd, 44)
    conv_w = dev((0.5 * r.standard_normal((cd, 4))).astype(F32))
    a = dev(-np.exp(r.standard_normal(vh)).astype(F32))
    dt = dev(r.uniform(-1, 1, vh).astype(F32))
    nw = dev((1 + 0.1 * r.standard_normal(dv)).astype(F32))
    ref = GdnLayerDecode(wq, wz, wb, wa, wo, conv_w, a, dt, nw)
    fus = GdnLayerDecode(wq, wz, wb, wa, wo, conv_w, a, dt, nw)
    for t in range(3):
        x = dev((0.3 * r.standard_normal(dm)).astype(F32))
        o_ref = host(ref.forward_reference_launches(x, torch.empty(dm, device="cuda")))
        o_fus = host(fus.forward(x, torch.empty(dm, device="cuda")))
        assert_f32_close(o_fus, o_ref, group=dm, what=f"token {t} output")
        assert_f32_close(host(fus.state), host(ref.state), group=dv, what=f"token {t} state")
        assert np.array_equal(host(fus.history), host(ref.history)), f"token {t} history"


@pytest.mark.parametrize("T", [16, 100, 200])
def test_gdn_layer_prefill_equals_decode_steps(T):
    """A prompt of T tokens through a GDN layer in one pass (GEMM projections,
    front end over all rows, chunked recurrence) against T decode steps of the
    same layer (src/layer_gdn.cpp:78-113 per token), from the same random
    history and state: outputs, final state and history. The two sum the
    projections, the L2 norms and the recurrence in different orders. The
    synthetic Q4_K weights have a mean near +1, so each projection of a
    zero-mean x cancels ~45x over K = 2048 and the two paths' inputs to the
    recurrence differ by ~1e-6 relative; the recurrence carries that into its
    state. Bars: outputs 1e-4 of the row rms, state 2e-3 of the head rms (small
    entries of strongly decayed heads, measured up to 1e-3 of their row rms), history
    (projection outputs) 1e-5 of the token's rms. A wiring mistake (a layout, a carried buffer)
    gives errors of order 1."""
    from qwen35_hip.decode_layers import GdnLayerDecode

    r = rng(T + 5)
    dm, kh, vh, dk, dv = 2048, 16, 32, 128, 128
    cd, vd = 2 * kh * dk + vh * dv, vh * dv

    def q4(M, K, s):
        return dev(synth.q4k_table(M, K, seed_tensor=s))
    wq, wz, wb, wa, wo = q4(cd, dm, 40), q4(vd, dm, 41), q4(vh, dm, 42), q4(vh, dm, 43), q4(dm, vd, 44)
    conv_w = dev((0.5 * r.standard_normal((cd, 4))).astype(F32))
    a = dev(-np.exp(r.standard_normal(vh)).astype(F32))
    dt = dev(r.uniform(-1, 1, vh).astype(F32))
    nw = dev((1 + 0.1 * r.standard_normal(dv)).astype(F32))
    step = GdnLayerDecode(wq, wz, wb, wa, wo, conv_w, a, dt, nw)
    pre = GdnLayerDecode(wq, wz, wb, wa, wo, conv_w, a, dt, nw)
    hist0 = dev(r.standard_normal((cd, 3)).astype(F32))
    st0 = dev((0.05 * r.standard_normal((vh, dk, dv))).astype(F32))
    for layer in (step, pre):
        layer.history.copy_(hist0)
        layer.state.copy_(st0)
    xs = dev((0.3 * r.standard_normal((T, dm))).astype(F32))
    o_step = np.stack([host(step.forward(xs[t], torch.empty(dm, device="cuda"))) for t in range(T)])
    o_pre = host(pre.prefill(xs))
    assert_f32_close(o_pre, o_step, group=dm, rtol=1e-4, what=f"{T} tokens output")
    assert_f32_close(host(pre.state), host(step.state), group=dk * dv, rtol=2e-3, what="state")
    # history [C, 3] holds the last 3 tokens' qkv projections: compare per token (rms over its C channels)
    assert_f32_close(np.ascontiguousarray(host(pre.history).T), np.ascontiguousarray(host(step.history).T), group=cd,
                     what="history")


def _attn_layer_pair(r, max_seq_len):
    from qwen35_hip.decode_layers import AttnLayerDecode

    dm, h, kvh, hd = 2048, 16, 2, 256
    ws = [dev(synth.q4k_table(M, K, seed_tensor=s)) for M, K, s in
          ((2 * h * hd, dm, 50), (kvh * hd, dm, 51), (kvh * hd, dm, 52), (dm, h * hd, 53))]
    qn, kn = dev((1 + 0.1 * r.standard_normal(hd)).astype(F32)), dev((1 + 0.1 * r.standard_normal(hd)).astype(F32))
    return (AttnLayerDecode(*ws, qn, kn, max_seq_len=max_seq_len),
            AttnLayerDecode(*ws, qn, kn, max_seq_len=max_seq_len))


@pytest.mark.parametrize("start", [0, 700])
def test_attn_layer_decode_fused_equals_reference_launches(start):
    """A full-attention layer's decode step (src/layer_attn.cpp:63-111) through
    the fused entry points (three calls: projections with the query | gate
    rows written split and K, V straight into the cache rows, Q/K norm + RoPE
    folded into the attention decode, output projection) against the
    reference's sequence of fifteen calls on the same library, three tokens in a
    row from position `start` (0, and 700 over a cache whose earlier rows hold the
    same random keys and values in both layers): same output and cache rows
    within fp32 tolerance (the attention sums run in another order), the V rows
    bit for bit."""
    r = rng(37 + start)
    ref, fus = _attn_layer_pair(r, 1024)
    if start:
        kv = dev((r.standard_normal((2, start, 512))).astype(F32))
        for layer in (ref, fus):
            layer.k_cache[:start].copy_(kv[0])
            layer.v_cache[:start].copy_(kv[1])
    for pos in range(start, start + 3):
        x = dev((0.3 * r.standard_normal(2048)).astype(F32))
        o_ref = host(ref.forward_reference_launches(x, pos, torch.empty(2048, device="cuda")))
        o_fus = host(fus.forward(x, pos, torch.empty(2048, device="cuda")))
        assert_f32_close(o_fus, o_ref, group=2048, what=f"pos {pos} output")
        assert_f32_close(host(fus.k_cache[pos]), host(ref.k_cache[pos]), group=256, what=f"pos {pos} K row")
        assert np.array_equal(host(fus.v_cache[pos]), host(ref.v_cache[pos])), f"pos {pos} V row"


def test_attn_layer_decode_rejects_position_past_context():
    r = rng(38)
    _, fus = _attn_layer_pair(r, 16)
    x = torch.zeros(2048, device="cuda")
    with pytest.raises(ValueError, match="attention position exceeds configured context"):
        fus.forward(x, 16, torch.empty(2048, device="cuda"))


def test_moe_layer_decode_fused_equals_reference_launches():
    """A MoE layer's decode step (src/layer_moe.cpp:80-159, 256 experts, top 8,
    512-wide experts, 2048-wide shared expert) through the fused entry points (three
    launches, the expert ids staying on the device) against the reference's
    sequence (router, top-k, host round trip and check, five calls per routed
    expert, the shared expert's six calls): same routing, same output within fp32
    tolerance, over three tokens."""
    from qwen35_hip.decode_layers import MoeLayerDecode

    r = rng(39)
    dm, E, k, I, S = 2048, 256, 8, 512, 2048

    def q4(M, K, s):
        return dev(synth.q4k_table(M, K, seed_tensor=s))
    ws = [q4(E, dm, 60), q4(E * I, dm, 61), q4(E * I, dm, 62), q4(E * dm, I, 63), q4(1, dm, 64), q4(S, dm, 65),
          q4(S, dm, 66), q4(dm, S, 67)]
    ref, fus = MoeLayerDecode(*ws), MoeLayerDecode(*ws)
    for t in range(3):
        x = dev((0.05 * r.standard_normal(dm)).astype(F32))
        o_ref = host(ref.forward_reference_launches(x, torch.empty(dm, device="cuda")))
        o_fus = host(fus.forward(x, torch.empty(dm, device="cuda")))
        assert np.array_equal(host(fus.top_idx), host(ref.top_idx)), f"token {t} routing"
        assert len(set(host(fus.top_idx).tolist())) == k
        assert_f32_close(o_fus, o_ref, group=dm, what=f"token {t} output")


def test_gdn_recurrent_rejects_wide_values():
    from qwen35_hip._lib import QwenError

    s = torch.zeros(1 * 4 * 260, device="cuda")
    x = torch.zeros(1040, device="cuda")
    with pytest.raises(QwenError, match="GDN value dimension exceeds kernel limit"):
        ops.gdn_recurrent_step(s, x, x, x, x, x, 1, 1, 4, 260)


# ------------------------------------------------------------------ attention core (decode)
def _attn_inputs(r, heads, kv_heads, dim, n_keys):
    q = r.standard_normal(heads * dim).astype(F32)
    K = r.standard_normal((n_keys, kv_heads * dim)).astype(F32)
    V = r.standard_normal((n_keys, kv_heads * dim)).astype(F32)
    g = (2 * r.standard_normal(heads * dim)).astype(F32)
    return q, K, V, g


def _attn_scale(oracle, q, K, V, heads, kv_heads, dim, pos, gate=None):
    """Condition scale of each output: sum_t p_t |v_tj| (times the gate's sigmoid)."""
    p = oracle.attn_softmax(oracle.attn_scores(q, K, heads, kv_heads, dim, pos), heads, pos + 1)
    Vh = np.abs(V.reshape(pos + 1, kv_heads, dim).astype(np.float64))
    sc = np.stack([p.reshape(heads, -1)[h].astype(np.float64) @ Vh[:, h // (heads // kv_heads)]
                   for h in range(heads)]).reshape(-1)
    if gate is not None:
        sc = sc / (1.0 + np.exp(-gate.astype(np.float64)))
    return sc


def _assert_scaled(got, ref, scale, what, rtol=1e-5):
    err = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), scale)
    w = int(np.argmax(err))
    assert err[w] <= rtol, f"{what}: rel err {err[w]:.3e} at {w}: got {got[w]!r} ref {ref[w]!r}"


def test_attn_split_qg_gate_and_kv_store(oracle):
    from qwen35_hip._lib import QwenError

    r = rng(5)
    heads, dim = 16, 256
    qg = r.standard_normal(2 * heads * dim).astype(F32)
    q, g = ops.attn_split_qg(dev(qg), heads, dim)
    rq, rg = oracle.attn_split_qg(qg, heads, dim)
    assert_bits_equal(host(q), rq)
    assert_bits_equal(host(g), rg)
    x = r.standard_normal(heads * dim).astype(F32)
    assert_f32_close(host(ops.attn_sigmoid_gate(dev(x), g)), oracle.attn_sigmoid_gate(x, rg), what="gate")
    kd, max_len = 512, 8
    kc, vc = torch.zeros(max_len * kd, device="cuda"), torch.zeros(max_len * kd, device="cuda")
    k, v = r.standard_normal(kd).astype(F32), r.standard_normal(kd).astype(F32)
    ops.attn_kv_store(dev(k), dev(v), kc, vc, 5, max_len)
    assert_bits_equal(host(kc).reshape(max_len, kd)[5], k)
    assert_bits_equal(host(vc).reshape(max_len, kd)[5], v)
    assert not host(kc).reshape(max_len, kd)[[4, 6]].any()
    for bad in (-1, max_len):
        with pytest.raises(QwenError, match="attention position exceeds configured context"):
            ops.attn_kv_store(dev(k), dev(v), kc, vc, bad, max_len)


# 16 / 2 heads of 256 and 32 / 2: the tiled scores (32 and 16 keys per split),
# the register softmax (1 to 16 values per thread) and the 16-byte values form;
# 9001 keys: more than 8 values per softmax thread and a partial last split;
# 20000: the softmax past the register form; head dims 128 and 100 (scores one
# wave per head and key; values over 16-column blocks with dead column quads)
# and 102 (values with scalar loads).
@pytest.mark.parametrize("heads,kv,dim,pos", [
    (16, 2, 256, 0), (16, 2, 256, 40), (16, 2, 256, 1000), (16, 2, 256, 4095), (16, 2, 256, 9000),
    (32, 2, 256, 100), (32, 2, 256, 2047), (16, 1, 256, 517), (16, 2, 256, 19999),
    (8, 2, 128, 200), (6, 2, 100, 50), (4, 1, 102, 20)])
def test_attn_stages(oracle, heads, kv, dim, pos):
    """The reference's three launches (src/layer_attn.cpp:103-105): scores, softmax and
    values each against the oracle on the oracle's inputs, then the GPU chain of the
    four calls (with the gate) against the oracle's decode."""
    q, K, V, g = _attn_inputs(rng(pos + 1 + heads + dim), heads, kv, dim, pos + 1)
    dq, dK, dV = dev(q), dev(K), dev(V)
    s = ops.attn_scores(dq, dK, heads, kv, dim, pos)
    rs = oracle.attn_scores(q, K, heads, kv, dim, pos)
    # a score is a dot product: bound its error by sum |q_i k_i| / sqrt(D)
    grp = heads // kv
    ks = np.abs(K.reshape(pos + 1, kv, dim).astype(np.float64))
    sscale = np.stack([ks[:, h // grp] @ np.abs(q.reshape(heads, dim)[h]) for h in range(heads)]).reshape(-1)
    _assert_scaled(host(s), rs, sscale / np.sqrt(dim), "scores")
    # softmax of the oracle's scores on both sides: probabilities to 1e-5 relative
    p = ops.attn_softmax(dev(rs), heads, pos + 1)
    rp = oracle.attn_softmax(rs, heads, pos + 1)
    assert_f32_close(host(p), rp, what="softmax")
    out = ops.attn_values(dev(rp), dV, heads, kv, dim, pos)
    _assert_scaled(host(out), oracle.attn_values(rp, V, heads, kv, dim, pos),
                   _attn_scale(oracle, q, K, V, heads, kv, dim, pos), "values")
    # the chain on the GPU, gated, against the oracle's sequence
    s = ops.attn_scores(dq, dK, heads, kv, dim, pos)
    ops.attn_softmax(s, heads, pos + 1)
    o = ops.attn_values(s, dV, heads, kv, dim, pos)
    o = ops.attn_sigmoid_gate(o, dev(g), out=o)
    _assert_scaled(host(o), oracle.attn_decode(q, K, V, heads, kv, dim, pos, gate=g),
                   _attn_scale(oracle, q, K, V, heads, kv, dim, pos, g), "chain")


def test_attn_values_deterministic():
    """The values sum runs in a fixed order: the same call twice gives the same bits."""
    heads, kv, dim, pos = 16, 2, 256, 4095
    _, _, V, _ = _attn_inputs(rng(77), heads, kv, dim, pos + 1)
    p = rng(78).random(heads * (pos + 1)).astype(F32)
    dp, dV = dev(p), dev(V)
    a = host(ops.attn_values(dp, dV, heads, kv, dim, pos))
    b = host(ops.attn_values(dp, dV, heads, kv, dim, pos))
    assert_bits_equal(a, b)


@pytest.mark.parametrize("heads,kv,dim,pos,gated", [
    (16, 2, 256, 0, True), (16, 2, 256, 31, True), (16, 2, 256, 32, False), (16, 2, 256, 33, True),
    (16, 2, 256, 1000, True), (16, 2, 256, 4095, True), (8, 2, 128, 200, True), (32, 2, 64, 77, False),
    (6, 2, 256, 50, True), (16, 2, 100, 45, True), (4, 1, 512, 20, True),
    (32, 2, 256, 15, True), (32, 2, 256, 16, False), (32, 2, 256, 2047, True), (16, 1, 256, 700, True),
    (8, 1, 256, 63, True),
    # more splits than one pass of the combine's workgroup takes (128): 282 and 257 splits
    (16, 2, 256, 9000, True), (32, 2, 256, 4100, False)])
def test_attn_decode(oracle, heads, kv, dim, pos, gated):
    """Fused decode at the Qwen3.5 attention shape across split boundaries (32 keys per
    split), groups of 4 and 16, and the staged fallback (group 3, dim 100, dim 512)."""
    q, K, V, g = _attn_inputs(rng(heads * 7 + pos), heads, kv, dim, pos + 1)
    gate = g if gated else None
    got = host(ops.attn_decode(dev(q), dev(K), dev(V), heads, kv, dim, pos, gate=None if gate is None else dev(gate)))
    ref = oracle.attn_decode(q, K, V, heads, kv, dim, pos, gate=gate)
    _assert_scaled(got, ref, _attn_scale(oracle, q, K, V, heads, kv, dim, pos, gate), f"decode pos {pos}")


@pytest.mark.parametrize("heads,kv,dim,pos,rope,inplace", [(16, 2, 256, 2047, 64, False), (16, 2, 256, 0, 64, False),
                                                        (16, 2, 256, 31, 64, False), (16, 2, 256, 32, 64, False),
                                                        (16, 2, 256, 100, 64, False), (16, 1, 256, 47, 64, False),
                                                        (16, 2, 256, 40, 32, False), (8, 2, 128, 20, 64, False),
                                                        (16, 2, 256, 60, 64, True)])
def test_attn_decode_norm_rope_equals_front_end_then_decode(heads, kv, dim, pos, rope, inplace):
    """The attention front end folded into the decode (src/layer_attn.cpp:91-96 then
    :103-108) gives the bits of attn_qk_norm_rope_rows on a copy of q and on the
    cache row of pos followed by attn_decode: output, normalised q and the whole
    cache, on the one-pass form (8 and 16 query heads per kv head, key pos at the
    start, end and inside a 32-key split, one key only) and on the calls it falls
    back to (rope_dim 32, head dim 128, q normalised in place)."""
    r = rng(heads * 11 + pos + rope)
    q, K, V, g = _attn_inputs(r, heads, kv, dim, pos + 1)
    qw = (1 + 0.2 * r.standard_normal(dim)).astype(F32)
    kw = (1 + 0.2 * r.standard_normal(dim)).astype(F32)
    theta, eps = 1e7, 1e-6
    # reference: the front end on copies, then the decode
    q_ref, K_ref = dev(q), dev(K)
    ops.attn_qk_norm_rope_rows(q_ref.view(1, heads, dim), K_ref[pos].view(1, kv, dim), dev(qw), dev(kw), pos0=pos,
                               rope_dim=rope, theta=theta, eps=eps)
    out_ref = ops.attn_decode(q_ref, K_ref, dev(V), heads, kv, dim, pos, gate=dev(g))
    dq, dK = dev(q), dev(K)
    out, qn = ops.attn_decode_norm_rope(dq, dK, dev(V), heads, kv, dim, pos, dev(qw), dev(kw), rope, theta,
                                        gate=dev(g), q_normed=dq if inplace else None, eps=eps)
    assert_bits_equal(host(out), host(out_ref), what=f"out pos {pos}")
    assert_bits_equal(host(qn), host(q_ref), what="normalised q")
    assert_bits_equal(host(dK), host(K_ref), what="cache")
    if not inplace:
        assert_bits_equal(host(dq), q, what="q untouched")


def test_attn_decode_rejects_small_workspace():
    from qwen35_hip._lib import QwenError

    heads, kv, dim, pos = 16, 2, 256, 100
    x = torch.zeros(heads * dim * (pos + 1), device="cuda")
    need = ops.attn_decode_workspace_bytes(heads, kv, dim, pos)
    assert need > 0
    ws = torch.empty(need - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(QwenError, match="workspace"):
        ops.attn_decode(x, x, x, heads, kv, dim, pos, workspace=ws)
    assert ops.attn_decode_workspace_bytes(6, 4, 64, 3) == 0  # heads not a multiple of kv_heads


# ------------------------------------------------------------------ MoE routing
@pytest.mark.parametrize("rows,n,k", [(4096, 256, 8), (37, 100, 5), (3, 1024, 64), (5, 64, 1)])
def test_moe_topk_rows(oracle, rows, n, k):
    """Qwen3.5 routing (256 experts, top 8) over a token batch, plus ragged / wide /
    k = 64 / k = 1 shapes; ties (a 3-way tie at the top, an all-equal row) and a
    non-finite row that only writes idx[0] = -1, w[0] = NaN."""
    r = rng(rows * n + k)
    x = r.standard_normal((rows, n)).astype(F32)
    x[0, [n // 3, n - 1, 1]] = 7.0
    x[1, :] = 0.5
    x[2, n // 2] = np.nan if rows > 2 else x[2, n // 2]
    sent_i = np.full((rows, k), 1234, np.int32)
    sent_w = np.full((rows, k), 0.125, F32)
    di, dw = dev(sent_i), dev(sent_w)
    ops.moe_topk_rows(dev(x), k, idx=di, weights=dw)
    ri, rw = oracle.moe_topk_rows(x, k, idx=sent_i, w=sent_w)
    gi, gw = host(di), host(dw)
    assert np.array_equal(gi, ri), np.argwhere(gi != ri)[:5]
    assert_f32_close(gw, rw, what="weights")


@pytest.mark.parametrize("n,k,offset", [(256, 8, 0), (256, 8, 1), (1024, 64, 0), (200, 16, 0)])
def test_moe_topk_rows_many_ties(oracle, n, k, offset):
    """Logits on a coarse grid (a few distinct values per row), so the top k is
    decided by the lower-index rule between lanes and inside each lane's list;
    offset 1 starts every row 4 bytes past a 16-byte boundary (scalar loads)."""
    rows = 512
    r = rng(n * k + offset)
    x = (np.round(r.standard_normal((rows, n)) * 2.0) / 4.0).astype(F32)
    x[0, :] = 1.0                     # every logit tied
    x[1, ::7] = 9.0                   # a tie of many at the top, spread over lanes
    x[2, :] = -1.0                    # +0 and -0 compare equal (lower index first)
    x[2, 5::11] = -0.0
    x[2, 9::13] = 0.0
    x[3, :] = -3.0                    # negative logits only, ties among them
    x[3, ::5] = -2.5
    x[4, :] = np.float32(-3.4028235e38)   # the extremes of the finite range
    x[4, 3::9] = np.float32(3.4028235e38)
    buf = dev(np.concatenate([np.zeros(offset, F32), x.ravel()]))
    xin = buf[offset:].view(rows, n)
    ri, rw = oracle.moe_topk_rows(x, k)
    gi, gw = ops.moe_topk_rows(xin, k)
    gi, gw = host(gi), host(gw)
    assert np.array_equal(gi, ri), np.argwhere(gi != ri)[:5]
    assert_f32_close(gw, rw, what="weights")


def test_moe_add_and_weighted_sum(oracle):
    r = rng(8)
    rows, k, dim = 64, 8, 2048
    y = r.standard_normal((rows, k, dim)).astype(F32)
    w = r.uniform(0, 0.3, (rows, k)).astype(F32)
    out0 = r.standard_normal((rows, dim)).astype(F32)
    got = host(ops.moe_weighted_sum_rows(dev(out0), dev(y), dev(w)))
    assert_bits_equal(got, oracle.moe_weighted_sum_rows(out0, y, w), "weighted sum")
    a = float(np.float32(0.3719))
    assert_bits_equal(host(ops.moe_add(dev(out0[0]), dev(y[0, 0]), a)), oracle.moe_add(out0[0], y[0, 0], a), "moe_add")


@pytest.mark.parametrize("kind,M,K", [("Q4_K", 512, 2048), ("Q4_K", 2048, 512), ("Q6_K", 512, 2048), ("Q8_0", 96, 256)])
def test_moe_expert_matmul(oracle, kind, M, K):
    """Gate/up (512 x 2048) and down (2048 x 512, one input row per expert) projections
    of the selected experts with the ids on the device; an invalid id gives a NaN row."""
    import ggml_blocks

    t = ops.GGML_TYPES[kind]
    E = 12
    r = rng(M + K + t)
    n_el = E * M * K
    table = (synth.q4k_table(E * M, K, seed_tensor=3) if kind == "Q4_K" else
             synth.q6k_table(E * M, K, seed_tensor=3) if kind == "Q6_K" else
             ggml_blocks.random_blocks(r, t, n_el // ggml_blocks.BLOCK[t][0]))
    ids = np.array([7, 0, 11, 3, 12, 5, -1, 9], np.int32)
    xs = r.standard_normal((ids.size, K)).astype(F32)
    got = host(ops.moe_expert_matmul(dev(table), t, n_el, M * K, E, dev(ids), dev(xs), K, M, K))
    ref = oracle.moe_expert_gemv(table, t, ids, E, M * K, xs, K, M, K)
    bad = (ids < 0) | (ids >= E)
    assert np.isnan(got[bad]).all()
    assert_f32_close(got[~bad], ref[~bad], group=M, what=kind)
    # one shared input row for all experts (x_stride 0), as the gate / up projections use
    got0 = host(ops.moe_expert_matmul(dev(table), t, n_el, M * K, E, dev(ids[:3]), dev(xs[0]), 0, M, K))
    ref0 = oracle.moe_expert_gemv(table, t, ids[:3], E, M * K, xs[0], 0, M, K)
    assert_f32_close(got0, ref0, group=M, what=f"{kind} shared x")


@pytest.mark.parametrize("kind,M,K", [("Q4_K", 512, 2048), ("Q6_K", 512, 2048), ("Q4_K", 256, 4096),
                                      ("Q8_0", 96, 512)])
def test_moe_expert_gate_up_equals_two_expert_matmuls(kind, M, K):
    """The routed gate and up projections in one launch give the bits of two
    moe_expert_matmul calls (x_stride 0), invalid ids included (NaN rows); Q8_0
    takes the generic kernel inside the same entry point."""
    t = ops.GGML_TYPES[kind]
    E = 12
    r = rng(M + K + t + 1)
    tg, tu = (dev(_gemv_weight(kind, E * M, K, r)) for _ in range(2))
    n_el = E * M * K
    ids = dev(np.array([7, 0, 11, 3, 12, 5, -1, 9], np.int32))
    x = dev(r.standard_normal(K).astype(F32))
    g, u = ops.moe_expert_gate_up(tg, tu, t, n_el, M * K, E, ids, x, M, K)
    g_ref = ops.moe_expert_matmul(tg, t, n_el, M * K, E, ids, x, 0, M, K)
    u_ref = ops.moe_expert_matmul(tu, t, n_el, M * K, E, ids, x, 0, M, K)
    assert_bits_equal(host(g), host(g_ref), what=f"{kind} gate")
    assert_bits_equal(host(u), host(u_ref), what=f"{kind} up")
    assert np.isnan(host(g)[6]).all() and np.isnan(host(u)[6]).all()


@pytest.mark.parametrize("kind,skind,k,inter,S,K", [
    ("Q4_K", "Q4_K", 8, 512, 2048, 2048),    # the model's shapes: one launch
    ("Q4_K", "Q4_K", 3, 512, 4096, 1020),    # 3 experts (one per wave, one wave idle), 2-slice shared rows
    ("Q6_K", "Q4_K", 8, 512, 2048, 2048),    # shared expert of another type: two launches
    ("Q4_K", "Q4_K", 3, 768, 1024, 4096),    # two 8-block slices per row
    ("Q4_K", "Q4_K", 4, 512, 512, 512),      # K = 512: the separate kernels through the workspace
    ("Q8_0", "Q6_K", 2, 96, 2048, 2048),     # routed through the workspace, shared in one launch
])
def test_moe_expert_swiglu_equals_gemvs_then_silu_mul(kind, skind, k, inter, S, K):
    """The SwiGLU hidden rows of the routed experts and the shared expert give the
    bits of the separate calls (gate and up GEMVs, then moe_silu_mul), invalid ids
    included (NaN rows), on the one-launch kernel and on the workspace path."""
    r = rng(k * 100 + inter + S + K + ops.GGML_TYPES[kind])
    E = 12
    t, ts = ops.GGML_TYPES[kind], ops.GGML_TYPES[skind]
    wg, wu = dev(_gemv_weight(kind, E * inter, K, r)), dev(_gemv_weight(kind, E * inter, K, r))
    wsg, wsu = dev(_gemv_weight(skind, S, K, r)), dev(_gemv_weight(skind, S, K, r))
    ids = r.permutation(E)[:k].astype(np.int32)
    ids[-1] = -1 if k > 2 else ids[-1]
    ids = dev(ids)
    x = dev(r.standard_normal(K).astype(F32))
    n_el, stride = E * inter * K, inter * K
    h, sh = ops.moe_expert_swiglu(wg, wu, t, n_el, stride, E, ids, x, inter, K, wsg, wsu, ts, S * K, S)
    g_ref = ops.moe_expert_matmul(wg, t, n_el, stride, E, ids, x, 0, inter, K)
    u_ref = ops.moe_expert_matmul(wu, t, n_el, stride, E, ids, x, 0, inter, K)
    assert_bits_equal(host(h), host(ops.moe_silu_mul(g_ref, u_ref)), what=f"{kind} routed")
    sg = ops.matmul_dispatch(wsg, ts, S * K, x, S, K)
    su = ops.matmul_dispatch(wsu, ts, S * K, x, S, K)
    assert_bits_equal(host(sh), host(ops.moe_silu_mul(sg, su)), what=f"{skind} shared")
    if k > 2:
        assert np.isnan(host(h)[-1]).all()
    # routed experts only (no shared tensors)
    h2, none = ops.moe_expert_swiglu(wg, wu, t, n_el, stride, E, ids, x, inter, K)
    assert none is None
    assert_bits_equal(host(h2), host(h), what=f"{kind} routed only")


@pytest.mark.parametrize("kind,n,k,inter,S,K", [
    ("Q4_K", 256, 8, 512, 2048, 2048),     # the model's shapes: one launch, 4 logits per lane
    ("Q6_K", 128, 4, 256, 2048, 2048),     # 2 logits per lane
    ("Q4_K", 48, 6, 512, 0, 2048),         # 1 logit per lane, no shared expert
    ("Q4_K", 256, 8, 512, 512, 512),       # K = 512: top-k launch + the separate kernels
])
def test_moe_route_swiglu_equals_topk_then_swiglu(kind, n, k, inter, S, K):
    """Routing fused into the SwiGLU GEMV gives the ids, weights and hidden rows of
    moe_topk_rows followed by moe_expert_swiglu, bit for bit, with ties in the
    logits; a non-finite logit gives the top-k kernel's (-1, NaN) and a NaN row 0."""
    r = rng(n + k + inter + S + K)
    t = ops.GGML_TYPES[kind]
    wg, wu = dev(_gemv_weight(kind, n * inter, K, r)), dev(_gemv_weight(kind, n * inter, K, r))
    shared = {}
    if S:
        shared = dict(w_shared_gate=dev(_gemv_weight(kind, S, K, r)), w_shared_up=dev(_gemv_weight(kind, S, K, r)),
                      shared_type=t, shared_elements=S * K, shared_dim=S)
    x = dev(r.standard_normal(K).astype(F32))
    lg = r.standard_normal(n).astype(F32)
    lg[5] = lg[9] = lg.max() + 1          # a tie for the first pick
    logits = dev(lg)
    n_el, stride = n * inter * K, inter * K
    idx, w, h, sh = ops.moe_route_swiglu(logits, k, wg, wu, t, n_el, stride, x, inter, K, **shared)
    i_ref, w_ref = ops.moe_topk_rows(logits.view(1, n), k)
    h_ref, sh_ref = ops.moe_expert_swiglu(wg, wu, t, n_el, stride, n, i_ref.view(-1), x, inter, K,
                                          shared.get("w_shared_gate"), shared.get("w_shared_up"),
                                          shared.get("shared_type"), shared.get("shared_elements", 0), S)
    assert np.array_equal(host(idx), host(i_ref).reshape(-1)) and host(idx)[0] == 5
    assert_bits_equal(host(w), host(w_ref).reshape(-1), what="weights")
    assert_bits_equal(host(h), host(h_ref), what=f"{kind} routed")
    if S:
        assert_bits_equal(host(sh), host(sh_ref), what=f"{kind} shared")
    lg[3] = np.inf
    idx.fill_(7)
    _, _, h2, _ = ops.moe_route_swiglu(dev(lg), k, wg, wu, t, n_el, stride, x, inter, K, idx=idx, weights=w,
                                       **shared)
    assert host(idx)[0] == -1 and np.isnan(host(w)[0]) and (host(idx)[1:] == 7).all()
    assert np.isnan(host(h2)[0]).all()


def _down_combine_separate(wd, td, nd, stride, E, ids, wts, hid, inter, wsd, tsd, nsd, shid, logit, dm):
    """The separate calls the fused entry point replaces (src/layer_moe.cpp:135-147)."""
    k = ids.numel()
    eo = ops.moe_expert_matmul(wd, td, nd, stride, E, ids, hid, inter, dm, inter)
    so = ops.matmul_dispatch(wsd, tsd, nsd, shid, dm, shid.numel())
    out = torch.zeros(dm, device="cuda")
    ops.moe_weighted_sum_rows(out.view(1, dm), eo.view(1, k, dm), wts.view(1, k))
    ops.moe_shared_add_rows(out.view(1, dm), so.view(1, dm), logit)
    return out


@pytest.mark.parametrize("td,tsd,k,inter,S,dm", [
    ("Q4_K", "Q4_K", 8, 512, 2048, 2048),    # the model's shapes: one launch
    ("Q6_K", "Q4_K", 8, 512, 2048, 2048),
    ("Q4_K", "Q6_K", 5, 512, 4096, 1024),    # 5 experts (a partly idle wave), 2-slice shared rows
    ("Q6_K", "Q6_K", 3, 512, 2048, 512),
    ("Q4_K", "Q4_K", 8, 1024, 1024, 768),   # other shapes: separate launches through the workspace
    ("Q4_K", "Q6_K", 8, 512, 2048, 998),
])
def test_moe_down_combine_equals_separate_calls(td, tsd, k, inter, S, dm):
    """The routed down projections, the shared expert's and the weighted, gated
    combine in one entry point give the bits of the separate calls, for the fused
    kernel's shapes and for the fallback's."""
    r = rng(k * 1000 + inter + S + dm)
    E = 16
    stride = dm * inter
    wd = dev(_gemv_weight(td, E * dm, inter, r))
    wsd = dev(_gemv_weight(tsd, dm, S, r))
    nd, nsd = E * stride, dm * S
    ids = dev(r.permutation(E)[:k].astype(np.int32))
    w = r.uniform(0.1, 1, k).astype(F32)
    wts = dev(w / w.sum())
    hid = dev(r.standard_normal((k, inter)).astype(F32))
    shid = dev(r.standard_normal(S).astype(F32))
    logit = dev(np.array([0.3], F32))
    got = ops.moe_down_combine(wd, td, nd, stride, E, ids, wts, hid, inter, wsd, tsd, nsd, shid, logit, dm)
    ref = _down_combine_separate(wd, ops.GGML_TYPES[td], nd, stride, E, ids, wts, hid, inter, wsd,
                                 ops.GGML_TYPES[tsd], nsd, shid, logit, dm)
    assert_bits_equal(host(got), host(ref), what=f"{td}/{tsd} k={k} inter={inter} S={S} dm={dm}")
    # an invalid expert id makes the output NaN, as the separate calls' NaN row does
    bad = ids.clone()
    bad[k - 1] = E
    got = host(ops.moe_down_combine(wd, td, nd, stride, E, bad, wts, hid, inter, wsd, tsd, nsd, shid, logit, dm))
    assert np.isnan(got).all()


def test_moe_down_combine_rejects_small_workspace():
    from qwen35_hip._lib import QwenError

    t = dev(synth.q4k_table(16 * 2048, 512, seed_tensor=1))
    ts = dev(synth.q4k_table(2048, 2048, seed_tensor=2))
    z = torch.zeros(8 * 2048, device="cuda")
    ids = torch.zeros(8, dtype=torch.int32, device="cuda")
    ws = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(QwenError, match="workspace of 64 bytes"):
        ops.moe_down_combine(t, "Q4_K", t.numel() // 144 * 256, 2048 * 512, 16, ids, z[:8], z, 512, ts, "Q4_K",
                             2048 * 2048, z[:2048], z[:1], 2048, workspace=ws)


# ------------------------------------------------------------------ quantized GEMV
def _gemv_weight(kind: str, rows: int, cols: int, r) -> np.ndarray:
    """GGML bytes of a rows x cols tensor: the C5 table generators for Q4_K/Q6_K
    (fp16 d, dmin ~ U(0, 0.01)), random finite blocks or floats otherwise."""
    import ggml_blocks

    t = ops.GGML_TYPES[kind]
    if kind == "Q4_K" and cols % 256 == 0:
        return synth.q4k_table(rows, cols, seed_tensor=cols % 7)
    if kind == "Q6_K" and cols % 256 == 0:
        return synth.q6k_table(rows, cols, seed_tensor=cols % 5)
    if t in ggml_blocks.BLOCK:
        return ggml_blocks.random_blocks(r, t, rows * cols // ggml_blocks.BLOCK[t][0])
    dt = {"F32": np.float32, "F16": np.float16}.get(kind)
    if dt is not None:
        return r.standard_normal(rows * cols).astype(dt).view(np.uint8)
    return synth.to_bf16_bits(r.standard_normal(rows * cols).astype(np.float32)).view(np.uint8)


# (type, tensor rows, K, M, first row): fast-path launch shapes (8/4/2/1 units
# per wave, 2 slices per row, 2/4/8 rows per unit with ragged tails, an expert
# slice by element offset) and the generic path (K not a multiple of 2048 or a
# divisor of it, Q6_K offsets off the 8-block grid, the other GGML types).
GEMV_CASES = [
    ("Q4_K", 40000, 2048, 40000, 0), ("Q4_K", 20000, 2048, 20000, 0), ("Q4_K", 9000, 2048, 9000, 0),
    ("Q4_K", 2048, 4096, 2048, 0), ("Q4_K", 1001, 512, 1001, 0), ("Q4_K", 37, 256, 37, 0),
    ("Q4_K", 513, 1024, 513, 0), ("Q4_K", 4 * 512, 2048, 512, 2 * 512),
    ("Q6_K", 40000, 2048, 40000, 0), ("Q6_K", 4096, 4096, 4096, 0), ("Q6_K", 4 * 512, 512, 512, 3 * 512),
    ("Q6_K", 1008, 512, 1001, 0), ("Q6_K", 64, 256, 61, 0), ("Q6_K", 200, 1024, 100, 1),
    ("Q4_K", 64, 768, 64, 0), ("Q6_K", 64, 1280, 64, 0),
    ("Q8_0", 300, 2048, 300, 0), ("Q4_0", 100, 1024, 100, 0), ("Q5_0", 100, 512, 100, 0),
    ("Q5_K", 64, 2048, 64, 0), ("F32", 256, 2048, 256, 0), ("F16", 100, 1000, 100, 0), ("BF16", 77, 2048, 77, 0),
    ("Q8_0", 50, 96, 50, 0), ("F32", 33, 7, 33, 0),  # K < 256
    # persistent-grid shapes: 2 / 4 rows per tile, 2 slices held in VGPRs, x reloaded (K > 4096)
    ("Q4_K", 5000, 2048, 5000, 0), ("Q4_K", 9000, 4096, 9000, 0), ("Q4_K", 300, 8192, 300, 0),
    ("Q6_K", 5000, 2048, 5000, 0), ("Q6_K", 9000, 4096, 9000, 0), ("Q6_K", 300, 8192, 300, 0),
    # the MFMA path (Q6_K from 1024 tiles of 16 rows, Q4_K from 4096): k-slices of
    # 2 / 4 / 1 / 3 blocks, ragged last tiles, element offsets
    ("Q6_K", 16400, 2048, 16397, 0), ("Q6_K", 16420, 4096, 16401, 16), ("Q6_K", 20000, 512, 19999, 0),
    ("Q6_K", 16500, 768, 16500, 0), ("Q4_K", 65600, 2048, 65543, 40), ("Q4_K", 65600, 1024, 65600, 0),
    ("Q4_K", 65536, 3072, 65536, 0),
    # Q6_K direct form (rows of whole units): 2 rows per wave from 8192 rows, both slices of a
    # K = 4096 row at once with a row offset, three slices one at a time, a ragged last wave
    ("Q6_K", 8192, 2048, 8192, 0), ("Q6_K", 1100, 4096, 1000, 77), ("Q6_K", 301, 6144, 299, 1),
    ("Q6_K", 9001, 2048, 8999, 2),
]


def _gemv_audit(got, ref, M, what):
    """The GEMV bar is relative to the rms of the whole output vector (group M).
    Every error is held to half the bar against that rms (5e-6; measured up to
    1.6e-6 for the GEMVs, 3.1e-6 for the fp16-MFMA GEMM at K = 4096), so the
    outputs that pass only through the floor are near-zero outputs of cancelling
    sums, below 0.5 of the rms (measured: below 0.1). The count is printed with
    the audit: for N(0, 1)-like outputs it is about 0.8 x (error / rms) / 1e-5 of
    them."""
    got, ref = np.asarray(got, np.float32).reshape(-1), np.asarray(ref, np.float32).reshape(-1)
    fin = np.isfinite(ref)
    n = (fin.size // M) * M
    a = floor_audit(np.where(fin, got, 0)[:n], np.where(fin, ref, 0)[:n], M, what)
    assert a["max_err_over_rms"] <= 5e-6, a
    assert a["floor_only_max_abs_ref_over_rms"] < 0.5, a


@pytest.mark.parametrize("kind,rows,K,M,row0", GEMV_CASES)
def test_matmul_dispatch(oracle, kind, rows, K, M, row0):
    t = ops.GGML_TYPES[kind]
    r = rng(rows * 7 + K + M)
    w = _gemv_weight(kind, rows, K, r)
    x = r.standard_normal(K).astype(F32)
    n_el, off = rows * K, row0 * K
    got = host(ops.matmul_dispatch(dev(w), t, n_el, dev(x), M, K, element_offset=off))
    ref = oracle.gemv(w, t, x, M, K, element_offset=off, threads=THREADS)
    assert_f32_close(got, ref, group=M, what=f"{kind} {M}x{K} @ row {row0}")
    _gemv_audit(got, ref, M, f"GEMV {kind} {M}x{K} @ row {row0}")


def test_matmul_dispatch_reuses_x_and_checks_shapes(oracle):
    """Output rows past M stay untouched; bad shapes and types are rejected with
    the reference's conditions (src/cuda/matmul_q4.cu:187-195)."""
    from qwen35_hip._lib import QwenError

    rows, K = 48, 2048
    w = synth.q4k_table(rows, K)
    x = rng(3).standard_normal(K).astype(F32)
    out = torch.full((rows + 5,), 7.0, device="cuda")
    ops.matmul_dispatch(dev(w), "Q4_K", rows * K, dev(x), rows, K, out=out)
    got = host(out)
    assert_f32_close(got[:rows], oracle.gemv(w, 12, x, rows, K), group=rows)
    assert np.all(got[rows:] == 7.0)
    dw, dx = dev(w), dev(x)
    for kw in (dict(M=rows + 1), dict(M=0), dict(M=rows, element_offset=K)):
        with pytest.raises(QwenError):
            ops.matmul_dispatch(dw, "Q4_K", rows * K, dx, kw.get("M", rows), K, element_offset=kw.get("element_offset", 0))
    with pytest.raises(QwenError):
        ops.matmul_dispatch(dw, 3, rows * K, dx, rows, K)  # Q4_1: no path


@pytest.mark.parametrize("K", [2048, 4096, 512])
def test_matmul_dispatch_multi_equals_single_calls(oracle, K):
    """A layer's input projections in one call (qwen_matmul_dispatch_multi): the
    GDN layer's qkv / z / beta / alpha shapes, a row offset, a second type, a
    non-K-quant tensor (its own kernel) and more same-type matrices than one
    launch takes; every output bit-equal to its own matmul_dispatch call (the
    same per-row kernel, whose per-row sums do not depend on the launch), and
    one of them against the oracle."""
    import ggml_blocks

    r = rng(K)
    specs = [("Q4_K", 8192, 0), ("Q4_K", 4096, 0), ("Q8_0", 32, 0), ("Q6_K", 32, 0), ("Q4_K", 300, 7 * K),
             ("Q6_K", 2048, 8 * K)] + [("Q4_K", 64 + 16 * i, 0) for i in range(9)]
    jobs, single = [], []
    for kind, M, off in specs:
        t = ops.GGML_TYPES[kind]
        n_el = M * K + off
        w = dev(ggml_blocks.random_blocks(r, t, n_el // ggml_blocks.BLOCK[t][0]))
        jobs.append((w, kind, n_el, M, off, torch.full((M,), 3.0, device="cuda")))
    x = dev(r.standard_normal(K).astype(F32))
    outs = ops.matmul_dispatch_multi(jobs, x, K)
    for (w, kind, n_el, M, off, _), got in zip(jobs, outs):
        ref = ops.matmul_dispatch(w, kind, n_el, x, M, K, element_offset=off)
        assert_bits_equal(host(got), host(ref), f"{kind} {M}x{K} at {off}")
    w0, kind0, n0, M0, _, _ = jobs[1]
    assert_f32_close(host(outs[1]), oracle.gemv(host(w0), 12, host(x), M0, K), group=M0, what="multi vs oracle")


def test_matmul_dispatch_multi_rejects_before_launching():
    """A bad descriptor fails the whole call with matmul_dispatch's status and the
    descriptor's index, and no output is written."""
    from qwen35_hip._lib import QwenError, STATUS_OUT_OF_RANGE

    K = 2048
    w = dev(synth.q4k_table(64, K))
    x = dev(rng(1).standard_normal(K).astype(F32))
    a, b = torch.full((64,), 5.0, device="cuda"), torch.full((64,), 5.0, device="cuda")
    with pytest.raises(QwenError, match="descriptor 1") as e:
        ops.matmul_dispatch_multi([(w, "Q4_K", 64 * K, 64, 0, a), (w, "Q4_K", 64 * K, 64, K, b)], x, K)
    assert e.value.status == STATUS_OUT_OF_RANGE
    torch.cuda.synchronize()
    assert torch.all(a == 5.0) and torch.all(b == 5.0)
    assert ops.matmul_dispatch_multi([], x, K) == []


@pytest.mark.parametrize("kind,M", [("Q6_K", 16400), ("Q4_K", 65550)])
def test_matmul_dispatch_mfma_random_blocks(oracle, kind, M):
    """The MFMA path on GGML blocks with random fp16 fields of both signs
    (subnormals included) and every quant / scale byte value."""
    import ggml_blocks

    t, K = ops.GGML_TYPES[kind], 2048
    r = rng(M + 3)
    w = ggml_blocks.random_blocks(r, t, M * K // 256)
    x = r.standard_normal(K).astype(F32)
    got = host(ops.matmul_dispatch(dev(w), t, M * K, dev(x), M, K))
    ref = oracle.gemv(w, t, x, M, K, threads=THREADS)
    assert_f32_close(got, ref, group=M, what=kind)
    _gemv_audit(got, ref, M, f"GEMV MFMA random blocks {kind} {M}")


@pytest.mark.parametrize("case", ["nan", "inf", "zero", "tiny", "huge", "small", "large", "outlier"])
def test_matmul_dispatch_mfma_x_range(oracle, case):
    """x the integer-digit form covers (|x| from 2^-100 to 2^100 per k-slice,
    outliers) and x it hands to the per-element form (non-finite, beyond that
    range); zero x gives +0."""
    M, K = 16400, 2048
    w = synth.q6k_table(M, K, seed_tensor=2)
    x = rng(11).standard_normal(K).astype(F32)
    if case == "nan":
        x[777] = np.nan
    elif case == "inf":
        x[1500] = np.inf
    elif case == "zero":
        x[:] = 0
    else:
        x *= F32({"tiny": 1e-33, "huge": 1e33, "small": 1e-25, "large": 1e25, "outlier": 1.0}[case])
        if case == "outlier":
            x[5] = 1e4
    got = host(ops.matmul_dispatch(dev(w), "Q6_K", M * K, dev(x), M, K))
    ref = oracle.gemv(w, 14, x, M, K, threads=THREADS)
    if case == "nan":
        assert np.isnan(got).all()
    elif case == "inf":
        assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])
        assert np.isinf(ref).any()
    elif case == "zero":
        assert np.array_equal(got.view(np.uint32), np.zeros(M, np.uint32))
    else:
        assert_f32_close(got, ref, group=M, what=case)



# ------------------------------------------------------------------ batched GEMV (prefill GEMM)
GEMM_CASES = [   # kind, tokens, M, K, first row (element offset = row * K)
    ("Q4_K", 64, 512, 2048, 0), ("Q4_K", 100, 300, 2048, 0), ("Q4_K", 16, 256, 256, 0),
    ("Q4_K", 200, 1000, 4096, 3), ("Q6_K", 64, 512, 2048, 0), ("Q6_K", 77, 333, 2048, 5),
    ("Q6_K", 130, 256, 512, 0), ("Q6_K", 16, 17, 256, 0),
    ("Q4_K", 7, 512, 2048, 0), ("Q6_K", 15, 100, 768, 0), ("Q8_0", 20, 96, 512, 0), ("Q4_K", 40, 64, 320, 0),
    # the prep kernel's register form at K = 1024 and its two-pass form at K above 256 outside 512..4096
    ("Q4_K", 32, 256, 1024, 0), ("Q6_K", 32, 256, 1024, 0), ("Q6_K", 48, 100, 1536, 0), ("Q4_K", 20, 300, 3072, 1),
    # an odd number of blocks per row (the rings' block and half-block slots alternate unevenly), token
    # counts one past a 128-token tile and one short of two
    ("Q4_K", 129, 300, 1280, 2), ("Q6_K", 257, 260, 1280, 0), ("Q4_K", 255, 512, 768, 0), ("Q6_K", 129, 513, 768, 8),
]


@pytest.mark.parametrize("kind,T,M,K,row0", GEMM_CASES)
def test_matmul_rows(oracle, kind, T, M, K, row0):
    """matmul_rows (T tokens in one call) against the oracle's GEMV of each
    token (src/cuda/matmul_q4.cu:140-167): the matrix-core path for Q4_K / Q6_K
    at 16 tokens or more (ragged token and row tiles, a row offset), the
    per-token GEMV below 16 tokens, for K % 256 != 0 and for other types.
    Output rows past T stay untouched."""
    t = ops.GGML_TYPES[kind]
    r = rng(T * 31 + M + K)
    n_rows = M + row0
    w = _gemv_weight(kind, n_rows, K, r)
    x = r.standard_normal((T, K)).astype(F32)
    out = torch.full((T + 1, M), 5.0, device="cuda")
    ops.matmul_rows(dev(w), t, n_rows * K, dev(x), M, K, element_offset=row0 * K, out=out)
    got = host(out)
    ref = np.stack([oracle.gemv(w, t, x[i], M, K, element_offset=row0 * K, threads=THREADS) for i in range(T)])
    assert_f32_close(got[:T], ref, group=M, what=f"{kind} {T}x{M}x{K} @ row {row0}")
    _gemv_audit(got[:T], ref, M, f"GEMM {kind} {T}x{M}x{K} @ row {row0}")
    assert np.all(got[T:] == 5.0)


@pytest.mark.parametrize("kind,T,M,K", [("Q4_K", 4096, 8192, 2048), ("Q6_K", 1024, 2048, 4096)])
def test_matmul_rows_prefill_shapes(oracle, kind, T, M, K):
    """Prefill shapes (the GDN qkv projection over 4096 tokens; a Q6_K output
    projection over 1024): sampled tokens against the oracle's GEMV and against
    matmul_dispatch of the same token on the GPU, both within the fp32 bar;
    inputs with a wide dynamic range (per-token scales 2^-20 .. 2^20) keep it."""
    t = ops.GGML_TYPES[kind]
    r = rng(T + M + K)
    w = _gemv_weight(kind, M, K, r)
    x = r.standard_normal((T, K)).astype(F32)
    x *= np.exp2(r.integers(-20, 21, size=(T, 1))).astype(F32)
    dw, dx = dev(w), dev(x)
    got = host(ops.matmul_rows(dw, t, M * K, dx, M, K))
    for i in (0, 1, 63, 64, T // 2 + 5, T - 1):
        ref = oracle.gemv(w, t, x[i], M, K, threads=THREADS)
        assert_f32_close(got[i], ref, group=M, what=f"{kind} token {i} vs oracle")
        _gemv_audit(got[i], ref, M, f"GEMM prefill {kind} {T}x{M}x{K} token {i}")
        gv = host(ops.matmul_dispatch(dw, t, M * K, dx[i], M, K))
        assert_f32_close(got[i], gv, group=M, what=f"{kind} token {i} vs matmul_dispatch")


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_matmul_rows_extreme_block_scales(oracle, kind):
    """Block scales across fp16's range (zero, subnormal, 2^-14 .. 65504 for d and,
    in Q4_K, dmin) mixed within each row: the matrix-core path (its exact fp16
    operands, the min terms' two-part group sums, the per-block d and dmin
    products) against the oracle's GEMV, within the fp32 bar."""
    T, M, K = 64, 256, 2048
    t = ops.GGML_TYPES[kind]
    r = rng(91 + t)
    scales = np.array([0.0, 2.0 ** -24, 2.0 ** -20, 2.0 ** -14, 1e-3, 0.5, 3.0, 1000.0, 65504.0], dtype=np.float16)
    if kind == "Q4_K":
        w = synth.q4k_table(M, K, seed_tensor=3).reshape(-1, 144).copy()
        w[:, 0:2] = r.choice(scales, size=len(w)).view(np.uint8).reshape(-1, 2)
        w[:, 2:4] = r.choice(scales, size=len(w)).view(np.uint8).reshape(-1, 2)
    else:
        w = synth.q6k_table(M, K, seed_tensor=3).reshape(-1, 210).copy()
        w[:, 208:210] = r.choice(scales, size=len(w)).view(np.uint8).reshape(-1, 2)
    w = w.reshape(-1)
    x = r.standard_normal((T, K)).astype(F32)
    got = host(ops.matmul_rows(dev(w), t, M * K, dev(x), M, K))
    assert np.isfinite(got).all()
    for i in (0, 1, 17, 40, T - 1):
        assert_f32_close(got[i], oracle.gemv(w, t, x[i], M, K, threads=THREADS), group=M, what=f"{kind} token {i}")


@pytest.mark.parametrize("T", [16, 300])
def test_matmul_rows_multi_equals_single_calls(T):
    """Several matrices of one x in one call (one prep, one GEMM launch per K-quant
    type): the GDN layer's qkv / z / beta / alpha shapes, a Q6_K matrix, a row offset,
    a Q8_0 matrix and a block-misaligned offset (per-token path), and more Q4_K
    matrices than one launch takes; each output bit-equal to its own matmul_rows call."""
    import ggml_blocks

    r = rng(T + 77)
    K = 2048
    specs = [("Q4_K", 8192, 0), ("Q4_K", 4096, 0), ("Q4_K", 32, 0), ("Q4_K", 32, 0), ("Q6_K", 300, 0),
             ("Q4_K", 100, 5 * K), ("Q8_0", 64, 0), ("Q4_K", 48, 96 + K)] + \
        [("Q4_K", 64 + 16 * i, 0) for i in range(8)]
    jobs = []
    for kind, M, off in specs:
        t = ops.GGML_TYPES[kind]
        n_el = M * K + off + (256 if off % 256 else 0)
        n_el = -(-n_el // ggml_blocks.BLOCK[t][0]) * ggml_blocks.BLOCK[t][0]
        w = dev(ggml_blocks.random_blocks(r, t, n_el // ggml_blocks.BLOCK[t][0]))
        jobs.append((w, kind, n_el, M, off, torch.full((T, M), 3.0, device="cuda")))
    x = dev(r.standard_normal((T, K)).astype(F32))
    outs = ops.matmul_rows_multi(jobs, x, K)
    for (w, kind, n_el, M, off, _), got in zip(jobs, outs):
        ref = ops.matmul_rows(w, kind, n_el, x, M, K, element_offset=off)
        assert_bits_equal(host(got), host(ref), what=f"{kind} {M} rows @ {off}")


def test_matmul_rows_checks_shapes():
    """Statuses of matmul_dispatch (src/cuda/matmul_q4.cu:187-195) plus the token count."""
    from qwen35_hip._lib import QwenError

    rows, K = 48, 2048
    dw = dev(synth.q4k_table(rows, K))
    dx = torch.zeros(32, K, device="cuda")
    for M, off in ((rows + 1, 0), (0, 0), (rows, K)):
        with pytest.raises(QwenError, match="GEMV shape exceeds tensor"):
            ops.matmul_rows(dw, "Q4_K", rows * K, dx, M, K, element_offset=off)
    with pytest.raises(QwenError):
        ops.matmul_rows(dw, 3, rows * K, dx, rows, K)   # Q4_1: no path
    empty = ops.matmul_rows(dw, "Q4_K", rows * K, dx[:0], rows, K)
    assert empty.shape == (0, rows)
    need = ops.matmul_rows_workspace_bytes(32, K)
    assert need >= 32 * K * 4 and ops.matmul_rows_workspace_bytes(15, K) == 0
    with pytest.raises(QwenError, match="workspace"):
        ops.matmul_rows(dw, "Q4_K", rows * K, dx, rows, K, workspace=torch.empty(need - 16, dtype=torch.uint8,
                                                                                   device="cuda"))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_matmul_rows_nonfinite_and_zero_rows(oracle, kind):
    """Token rows holding infinities give the reference's pattern of +-inf and
    NaN (its per-element fp32 products: w * inf = +-inf, 0 * inf = NaN,
    +inf + -inf = NaN), a NaN row gives NaN, an all-zero row gives +0, and
    neighbouring rows are unaffected."""
    K, M, T = 2048, 256, 32
    t = ops.GGML_TYPES[kind]
    w = synth.q4k_table(M, K) if kind == "Q4_K" else synth.q6k_table(M, K)
    x = rng(11).standard_normal((T, K)).astype(F32)
    x[3, 100] = np.inf                      # one infinity
    x[7, 10], x[7, 2000] = np.inf, -np.inf  # both signs in one row
    x[9, 5] = np.nan
    x[9, 6] = np.inf                        # NaN beside an infinity
    x[5] = 0.0
    got = host(ops.matmul_rows(dev(w), kind, M * K, dev(x), M, K))
    for i in (3, 7, 9):
        ref = oracle.gemv(w, t, x[i], M, K)
        assert np.array_equal(np.isnan(got[i]), np.isnan(ref)), f"token {i}: NaN pattern"
        inf = np.isinf(ref)
        assert np.array_equal(got[i][inf], ref[inf]) and np.array_equal(np.isinf(got[i]), inf), f"token {i}: inf"
    assert np.isinf(oracle.gemv(w, t, x[3], M, K)).any()
    assert np.array_equal(got[5].view(np.uint32), np.zeros(M, np.uint32))
    for i in (0, 4, 6, 8, 10, T - 1):
        assert_f32_close(got[i], oracle.gemv(w, t, x[i], M, K), group=M, what=f"token {i}")
