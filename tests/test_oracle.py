"""Pins the CPU oracle (oracle/oracle.cpp) before it is trusted as the checker.

Every oracle function is checked against something other than its own formula:
the reference's known-answer fixtures (tests/kernel_tests.cu, frozen in
tests/golden/reference_fixtures.json), ggml's block-loop dequantizers
(tests/ggml_blocks.py), numpy / torch conversions, float64 evaluations and
closed-form special cases chosen so that a dropped term, a wrong sign or index,
or a transposed operand fails at least one test.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import ggml_blocks
from conftest import assert_bf16_close, assert_bits_equal, assert_f32_close

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "reference_fixtures.json").read_text())
F32 = np.float32


def silu64(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def sig64(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, dtype=np.float64)))


def bf16_of(x) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def f32_of_bf16(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("name", ["Q4_0", "Q5_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K"])
def test_reference_quant_fixture(oracle, name):
    fx = GOLDEN["quant"][name]
    raw = np.frombuffer(bytes.fromhex(fx["bytes_hex"]), dtype=np.uint8)
    exp = np.array(fx["expected"], dtype=F32)
    got = oracle.dequant_span(raw, fx["type"], 0, exp.size)
    # The fixture's expected values come from integer products
    # (tests/kernel_tests.cu:220), which carry no sign of zero, while the kernel's
    # float product (d * sc) * (q - 32) gives -0.0 for a negative scale. So values
    # are compared exactly (-0.0 == 0.0) and the zero signs are pinned separately
    # against ggml's float loop form below.
    assert np.array_equal(got, exp), name
    ggml = ggml_blocks.DEQUANT[fx["type"]](raw)
    assert np.array_equal(ggml, exp), f"ggml {name}"
    assert_bits_equal(got, ggml, f"{name} vs ggml")


@pytest.mark.parametrize("ggml_type", [2, 6, 8, 12, 13, 14])
def test_dequant_matches_ggml_loops(oracle, ggml_type):
    rng = np.random.default_rng(1000 + ggml_type)
    raw = ggml_blocks.random_blocks(rng, ggml_type, 512)
    elems = ggml_blocks.BLOCK[ggml_type][0] * 512
    got = oracle.dequant_span(raw, ggml_type, 0, elems)
    assert_bits_equal(got, ggml_blocks.DEQUANT[ggml_type](raw), f"type {ggml_type}")


def test_dequant_q6k_signed_zero(oracle):
    # (d * sc) * 0 with d * sc < 0 is -0.0 (src/cuda/matmul_q4.cu:125 association)
    raw = np.zeros(210, dtype=np.uint8)
    raw[192:208] = np.array([-3] * 16, dtype=np.int8).view(np.uint8)
    raw[0:128] = 0x00
    raw[128:192] = 0xAA  # hi bits 2 -> q = 32 in every quarter -> q - 32 = 0
    raw[208:210] = np.array([1.0], dtype=np.float16).view(np.uint8)
    got = oracle.dequant_span(raw, 14, 0, 256)
    assert np.all(got == 0) and np.all(np.signbit(got))
    assert_bits_equal(got, ggml_blocks.q6_k(raw))


def test_dequant_float_types(oracle):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got16 = oracle.dequant_span(h.view(np.uint8), 1, 0, h.size)
    ref16 = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref16)
    assert np.array_equal(np.isnan(got16), nan)
    assert_bits_equal(got16[~nan], ref16[~nan], "F16")
    gotb = oracle.dequant_span(h.view(np.uint8), 30, 0, h.size)
    assert_bits_equal(gotb[~np.isnan(gotb)], f32_of_bf16(h)[~np.isnan(gotb)], "BF16")
    x = np.random.default_rng(3).standard_normal(1000).astype(F32)
    assert_bits_equal(oracle.dequant_span(x.view(np.uint8), 0, 0, x.size), x, "F32")


@pytest.mark.parametrize("ggml_type", [12, 14, 8])
def test_dequant_gather_indexing(oracle, ggml_type):
    rng = np.random.default_rng(7)
    rows, cols = 64, 512
    elems, _ = ggml_blocks.BLOCK[ggml_type]
    raw = ggml_blocks.random_blocks(rng, ggml_type, rows * cols // elems)
    full = ggml_blocks.DEQUANT[ggml_type](raw).reshape(rows, cols)
    ids = rng.integers(0, rows, size=100).astype(np.int32)
    assert_bits_equal(oracle.dequant_gather(raw, ggml_type, ids, cols), full[ids], "gather")
    assert_bits_equal(oracle.dequant_gather(raw, ggml_type, ids, cols, threads=4), full[ids], "gather mt")


# ------------------------------------------------------------------ quantized GEMV
def _gemv_tensor(rng, ggml_type, n_el):
    """Raw GGML bytes of n_el elements and the same tensor dequantized by ggml's loops."""
    if ggml_type == 0:
        dense = rng.standard_normal(n_el).astype(F32)
        return dense.view(np.uint8), dense
    elems = ggml_blocks.BLOCK[ggml_type][0]
    raw = ggml_blocks.random_blocks(rng, ggml_type, n_el // elems)
    return raw, ggml_blocks.DEQUANT[ggml_type](raw)


@pytest.mark.parametrize("ggml_type", [12, 14, 8, 2, 0])
def test_gemv_matches_float64_matmul(oracle, ggml_type):
    """W (ggml block loops) @ x by numpy in float64: the oracle's single rounding
    of the exact sum must land within one float ulp of it."""
    rng = np.random.default_rng(100 + ggml_type)
    M, K = 24, 512
    raw, dense = _gemv_tensor(rng, ggml_type, M * K)
    x = rng.standard_normal(K).astype(F32)
    exact = dense.reshape(M, K).astype(np.float64) @ x.astype(np.float64)
    got = oracle.gemv(raw, ggml_type, x, M, K)
    ulp = np.spacing(np.abs(exact).astype(F32)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= ulp), ggml_type
    assert np.array_equal(oracle.gemv(raw, ggml_type, x, M, K, threads=4), got)


@pytest.mark.parametrize("ggml_type", [12, 14])
def test_gemv_one_hot_columns_and_offset(oracle, ggml_type):
    """x = e_j reads column j of W exactly; element_offset selects whole rows
    (src/layer_moe.cpp:131-138 slices experts by element offset)."""
    rng = np.random.default_rng(7 + ggml_type)
    E, M, K = 3, 8, 512
    raw, dense = _gemv_tensor(rng, ggml_type, E * M * K)
    W = dense.reshape(E, M, K)
    for j in (0, 1, 31, 32, 255, 256, 511):
        x = np.zeros(K, dtype=F32)
        x[j] = 1.0
        got = oracle.gemv(raw, ggml_type, x, E * M, K)
        assert np.array_equal(got, W.reshape(E * M, K)[:, j]), j
    x = rng.standard_normal(K).astype(F32)
    full = oracle.gemv(raw, ggml_type, x, E * M, K)
    for e in range(E):
        part = oracle.gemv(raw, ggml_type, x, M, K, element_offset=e * M * K)
        assert_bits_equal(part, full[e * M:(e + 1) * M], f"expert {e}")
    # linearity in x: W(2x) = 2 Wx exactly (scaling by 2 is exact throughout)
    assert_bits_equal(oracle.gemv(raw, ggml_type, 2 * x, E * M, K), 2 * full, "2x")


def test_type_supported(oracle):
    for t in range(40):
        assert oracle.type_supported(t) == (t in (0, 1, 2, 6, 8, 12, 13, 14, 30))


# ------------------------------------------------------------------ conversions
def test_half_to_float_all_values(oracle):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.half_to_float(h)
    ref = h.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert_bits_equal(got[ok], ref[ok])


def test_float_to_bf16_matches_torch(oracle):
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(20000).astype(F32) * 10.0,
        (rng.integers(0, 1 << 32, size=20000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.3895314e38], dtype=F32),
    ])
    x = x[~np.isnan(x)]
    assert np.array_equal(oracle.float_to_bf16(x), bf16_of(x))


# ------------------------------------------------------------------ RMSNorm
def test_rmsnorm_reference_fixture(oracle):
    fx = GOLDEN["rmsnorm"]
    got = oracle.rmsnorm_rows(np.array([fx["x"]], dtype=F32), np.array(fx["w"], dtype=F32), fx["eps"])
    assert np.max(np.abs(got[0] - np.array(fx["expected"], dtype=F32))) < fx["tol"]


def test_rmsnorm_float64(oracle):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((64, 2048)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(F32)
    got = oracle.rmsnorm_rows(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6) * w
    assert_f32_close(got, ref, rtol=1e-6)
    assert_bits_equal(oracle.rmsnorm_rows(x, w, 1e-6, threads=4), got, "threads")


def test_rmsnorm_invariants(oracle):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((8, 1000)).astype(F32)
    w = np.ones(1000, dtype=F32)
    a = oracle.rmsnorm_rows(x, w, 0.0)
    b = oracle.rmsnorm_rows(x * F(8.0), w, 0.0)  # exact scaling; eps 0 -> same output
    assert_f32_close(b, a, rtol=1e-6)
    assert np.allclose(np.mean(a.astype(np.float64) ** 2, axis=1), 1.0, rtol=1e-6)
    c = oracle.rmsnorm_rows(np.full((1, 16), -3.0, dtype=F32), np.arange(16, dtype=F32), 1e-6)
    assert_f32_close(c[0], -np.arange(16) * 3.0 / math.sqrt(9.0 + 1e-6), rtol=1e-6)


def F(v):
    return np.float32(v)


def test_rmsnorm_gated(oracle):
    rng = np.random.default_rng(13)
    x = rng.standard_normal((16, 256)).astype(F32)
    g = rng.standard_normal((16, 256)).astype(F32) * 3
    w = (1 + 0.1 * rng.standard_normal(256)).astype(F32)
    got = oracle.rmsnorm_gated_rows(x, g, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + 1e-6) * w * silu64(g)
    assert_f32_close(got, ref, rtol=2e-6)
    # gate 0 -> 0; gate large -> plain rmsnorm * gate
    assert np.all(oracle.rmsnorm_gated_rows(x, np.zeros_like(x), w) == 0)
    big = np.full_like(x, 40.0)
    assert_f32_close(oracle.rmsnorm_gated_rows(x, big, w), oracle.rmsnorm_rows(x, w) * 40.0, rtol=1e-6)


def test_residual_rmsnorm_f32_and_bf16(oracle):
    rng = np.random.default_rng(14)
    x = rng.standard_normal((32, 2048)).astype(F32)
    b = rng.standard_normal((32, 2048)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(F32)
    resid, normed = oracle.residual_rmsnorm_rows(x, b, w)
    assert_bits_equal(resid, x + b)
    assert_bits_equal(normed, oracle.rmsnorm_rows(x + b, w))
    xb, bb = bf16_of(x), bf16_of(b)
    r16, n16 = oracle.residual_rmsnorm_rows(xb, bb, w)
    s = bf16_of(f32_of_bf16(xb) + f32_of_bf16(bb))  # torch RNE of the fp32 sum
    assert np.array_equal(r16, s)
    s64 = f32_of_bf16(s).astype(np.float64)
    ref = s64 / np.sqrt(np.mean(s64 ** 2, axis=1, keepdims=True) + 1e-6) * w
    assert_bf16_close(n16, bf16_of(ref.astype(F32)))


def special_f32() -> np.ndarray:
    """Signed zeros, the smallest and largest subnormals, the smallest normal,
    values whose sum overflows or cancels exactly, infinities and NaNs."""
    tiny = np.finfo(F32).smallest_subnormal
    big = np.finfo(F32).max
    base = np.array([0.0, -0.0, tiny, -tiny, 2 * tiny, np.finfo(F32).smallest_normal - tiny,
                     np.finfo(F32).smallest_normal, -np.finfo(F32).smallest_normal, 1.0, -1.0, 1.5, big, -big,
                     np.inf, -np.inf, np.nan, 3.0e38, 1e-30, -1e-30], dtype=F32)
    return base


def test_residual_add_matches_numpy(oracle):
    """out = x1 + x2 (src/cuda/ops.cu:115-125) against numpy's float32 add: every
    pair of special values (signed zeros, subnormals, overflow to inf,
    inf - inf = NaN, NaN inputs) and random values across the exponent range."""
    s = special_f32()
    a = np.repeat(s, s.size)
    b = np.tile(s, s.size)
    got = oracle.residual_add(a, b)
    with np.errstate(all="ignore"):
        ref = (a + b).astype(F32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_bits_equal(got[~nan], ref[~nan], "special pairs")
    # signed zero rules and overflow, spelled out
    # (a list: as dict keys 0.0 and -0.0 would collide)
    pairs = [(0.0, -0.0, 0x00000000), (-0.0, -0.0, 0x80000000), (1.0, -1.0, 0x00000000)]
    for x, y, bits in pairs:
        assert oracle.residual_add(np.array([x], F32), np.array([y], F32)).view(np.uint32)[0] == bits
    big = np.finfo(F32).max
    assert oracle.residual_add(np.array([big], F32), np.array([big], F32))[0] == np.inf
    tiny = np.finfo(F32).smallest_subnormal
    assert oracle.residual_add(np.array([tiny], F32), np.array([tiny], F32))[0] == 2 * tiny  # no flush to zero
    rng = np.random.default_rng(71)
    bits = rng.integers(0, 1 << 32, size=(2, 100_003), dtype=np.uint64).astype(np.uint32)
    x, y = bits[0].view(F32), bits[1].view(F32)
    got = oracle.residual_add(x, y)
    with np.errstate(all="ignore"):
        ref = x + y
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_bits_equal(got[~nan], ref[~nan], "random bit patterns")


def test_encoder_rows_matches_table_indexing(oracle):
    """out[t] = table[ids[t]] (src/cuda/ops.cu:128-138) against numpy fancy
    indexing, bit for bit, with repeated ids, the first and last rows and rows
    holding NaN payloads and signed zeros (a copy, not arithmetic)."""
    rng = np.random.default_rng(72)
    table = rng.standard_normal((97, 40)).astype(F32)
    table[5, :3] = np.array([-0.0, np.inf, -np.inf], dtype=F32)
    table[7].view(np.uint32)[:] = 0x7FC01234  # NaN with a payload
    ids = np.array([0, 96, 5, 7, 5, 31, 0], dtype=np.int32)
    got = oracle.encoder_rows(ids, table)
    assert got.shape == (ids.size, 40)
    assert np.array_equal(got.view(np.uint32), table[ids].view(np.uint32))
    assert oracle.encoder_rows(np.zeros(0, np.int32), table).shape == (0, 40)


# ------------------------------------------------------------------ RoPE
def test_rope_reference_fixture(oracle):
    fx = GOLDEN["rope"]
    x = np.array(fx["x"], dtype=F32).reshape(1, fx["heads"], fx["head_dim"])
    got = oracle.rope_rows(x, pos0=fx["pos"], rope_dim=fx["rope_dim"], theta=fx["theta"])
    assert np.max(np.abs(got.ravel() - np.array(fx["expected"], dtype=F32))) < fx["tol"]


def test_rope_den_closed_forms(oracle):
    assert oracle.rope_den(0, 64, 1e7) == 1.0
    assert oracle.rope_den(1, 4, 1e4) == 100.0
    assert oracle.rope_den(16, 64, 1e7) == F(math.sqrt(1e7))  # exponent 16/32 = 1/2 exactly
    assert oracle.rope_den(8, 64, 1e7) == F(math.sqrt(math.sqrt(1e7)))
    d = [oracle.rope_den(i, 64, 1e7) for i in range(32)]
    assert all(a < b for a, b in zip(d, d[1:]))


def test_rope_properties(oracle):
    rng = np.random.default_rng(21)
    x = rng.standard_normal((32, 4, 256)).astype(F32)
    pos = rng.integers(0, 4096, size=32).astype(np.int32)
    # pos 0 is the identity, bit for bit
    assert_bits_equal(oracle.rope_rows(x, pos0=0, rope_dim=64, theta=1e7)[:1], x[:1])
    got = oracle.rope_rows(x, pos=pos, rope_dim=64, theta=1e7)
    # dims past rope_dim untouched; pair norms preserved
    assert_bits_equal(got[..., 64:], x[..., 64:])
    n_in = x[..., :32].astype(np.float64) ** 2 + x[..., 32:64].astype(np.float64) ** 2
    n_out = got[..., :32].astype(np.float64) ** 2 + got[..., 32:64].astype(np.float64) ** 2
    assert np.allclose(n_out, n_in, rtol=1e-6)
    # float64 rotation with the same (float) angles
    den = np.array([oracle.rope_den(i, 64, 1e7) for i in range(32)], dtype=F32)
    th = (pos.astype(F32)[:, None] / den[None, :]).astype(F32).astype(np.float64)
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    a, b = x[..., :32].astype(np.float64), x[..., 32:64].astype(np.float64)
    ref = x.astype(np.float64).copy()
    ref[..., :32] = a * c - b * s
    ref[..., 32:64] = b * c + a * s
    assert_f32_close(got, ref, group=256, rtol=1e-6)


def test_qk_norm_rope_composition(oracle):
    rng = np.random.default_rng(22)
    q = rng.standard_normal((16, 4, 256)).astype(F32)
    k = rng.standard_normal((16, 2, 256)).astype(F32)
    qw = (1 + 0.1 * rng.standard_normal(256)).astype(F32)
    kw = (1 + 0.1 * rng.standard_normal(256)).astype(F32)
    gq, gk = oracle.qk_norm_rope_rows(q, k, qw, kw, pos0=100, rope_dim=64, theta=1e7)
    for src, w, got in ((q, qw, gq), (k, kw, gk)):
        x64 = src.astype(np.float64)
        n = x64 / np.sqrt(np.mean(x64 ** 2, axis=-1, keepdims=True) + 1e-6) * w
        den = np.array([oracle.rope_den(i, 64, 1e7) for i in range(32)], dtype=F32)
        pos = np.arange(100, 116, dtype=F32)
        th = (pos[:, None] / den[None, :]).astype(F32).astype(np.float64)
        c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
        ref = n.copy()
        ref[..., :32] = n[..., :32] * c - n[..., 32:64] * s
        ref[..., 32:64] = n[..., 32:64] * c + n[..., :32] * s
        assert_f32_close(got, ref, group=256, rtol=2e-6)
    # norm-only equals head_norm; the attention norm uses x * (r * w)
    hn = oracle.head_norm_rows(q, qw)
    gq0, _ = oracle.qk_norm_rope_rows(q, k, qw, kw, pos0=0, rope_dim=0, theta=1e7)
    assert_bits_equal(gq0, hn)
    # ...and differs from the rmsnorm association (x * r) * w only by rounding
    assert_f32_close(hn, oracle.rmsnorm_rows(q, qw), rtol=2e-7)


# ------------------------------------------------------------------ GDN
def test_conv_special_cases(oracle):
    rng = np.random.default_rng(31)
    T, C = 10, 64
    x = rng.standard_normal((T, C)).astype(F32)
    hist = rng.standard_normal((C, 3)).astype(F32)
    w3 = np.zeros((C, 4), dtype=F32)
    w3[:, 3] = 1.0
    y, h = oracle.conv_rows(x, w3, hist)
    assert_f32_close(y, silu64(x), rtol=1e-6)
    assert_bits_equal(h, x[-3:].T.copy())
    w0 = np.zeros((C, 4), dtype=F32)
    w0[:, 0] = 1.0  # pure shift by 3, history first
    y0, _ = oracle.conv_rows(x, w0, hist)
    seq = np.concatenate([hist.T, x], axis=0)  # [T+3, C]
    assert_f32_close(y0, silu64(seq[:T]), rtol=1e-6)


def test_conv_chunking_and_steps(oracle):
    rng = np.random.default_rng(32)
    T, C = 37, 48
    x = rng.standard_normal((T, C)).astype(F32)
    w = (0.5 * rng.standard_normal((C, 4))).astype(F32)
    hist = rng.standard_normal((C, 3)).astype(F32)
    y, h = oracle.conv_rows(x, w, hist)
    y1, h1 = oracle.conv_rows(x[:20], w, hist)
    y2, h2 = oracle.conv_rows(x[20:], w, h1)
    assert_bits_equal(np.concatenate([y1, y2]), y)
    assert_bits_equal(h2, h)
    hs = hist
    for t in range(T):
        yt, hs = oracle.conv_rows(x[t:t + 1], w, hs)
        assert_bits_equal(yt[0], y[t])
    # float64 convolution
    seq = np.concatenate([hist.T, x], axis=0).astype(np.float64)
    s = sum(seq[j:j + T] * w[:, j].astype(np.float64) for j in range(4))
    assert_f32_close(y, silu64(s), group=C, rtol=1e-6)
    # short sequences (T < kernel - 1) shift the history
    _, hshort = oracle.conv_rows(x[:1], w, hist)
    assert_bits_equal(hshort, np.concatenate([hist[:, 1:], x[:1].T], axis=1))


def test_qk_l2_invariants(oracle):
    rng = np.random.default_rng(33)
    q = rng.standard_normal((8, 16, 128)).astype(F32)
    k = rng.standard_normal((8, 16, 128)).astype(F32)
    nq, nk = oracle.qk_l2_rows(q, k, 1e-6)
    sq = np.sum(q.astype(np.float64) ** 2, axis=-1)
    sk = np.sum(k.astype(np.float64) ** 2, axis=-1)
    assert np.allclose(np.sum(nk.astype(np.float64) ** 2, axis=-1), sk / (sk + 1e-6), rtol=2e-6)
    assert np.allclose(np.sum(nq.astype(np.float64) ** 2, axis=-1), sq / (sq + 1e-6) / 128.0, rtol=2e-6)
    cos = np.sum(nq.astype(np.float64) * q, axis=-1) / np.sqrt(np.sum(nq.astype(np.float64) ** 2, axis=-1) * sq)
    assert np.allclose(cos, 1.0, atol=1e-6)
    # eps sits on the sum: a tiny head is scaled by ~1/sqrt(eps), not normalised
    tiny = np.full((1, 1, 128), 1e-6, dtype=F32)
    _, tk = oracle.qk_l2_rows(tiny, tiny, 1e-6)
    assert np.allclose(tk, 1e-6 / math.sqrt(128e-12 + 1e-6), rtol=1e-5)


def test_gdn_frontend_composition(oracle):
    rng = np.random.default_rng(34)
    T, C, H, D = 12, 1024, 2, 128
    x = rng.standard_normal((T, C)).astype(F32)
    w = (0.5 * rng.standard_normal((C, 4))).astype(F32)
    hist = np.zeros((C, 3), dtype=F32)
    y, h = oracle.gdn_frontend_rows(x, w, hist, k_heads=H, key_dim=D)
    yc, hc = oracle.conv_rows(x, w, hist)
    assert_bits_equal(h, hc)
    assert_bits_equal(y[:, 2 * H * D:], yc[:, 2 * H * D:])  # v channels untouched by the norm
    q, k = yc[:, :H * D].reshape(T, H, D), yc[:, H * D:2 * H * D].reshape(T, H, D)
    q64, k64 = q.astype(np.float64), k.astype(np.float64)
    rq = q64 / np.sqrt(np.sum(q64 ** 2, -1, keepdims=True) + 1e-6) / math.sqrt(D)
    rk = k64 / np.sqrt(np.sum(k64 ** 2, -1, keepdims=True) + 1e-6)
    assert_f32_close(y[:, :H * D], rq.reshape(T, -1), rtol=1e-6)
    assert_f32_close(y[:, H * D:2 * H * D], rk.reshape(T, -1), rtol=1e-6)


def test_norm_gate(oracle):
    rng = np.random.default_rng(35)
    x = rng.standard_normal((16, 32, 128)).astype(F32)
    z = rng.standard_normal((16, 32, 128)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(128)).astype(F32)
    got = oracle.norm_gate_rows(x, z, w)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 ** 2, -1, keepdims=True) + 1e-6) * w * silu64(z)
    assert_f32_close(got, ref, rtol=2e-6)
    # z large -> silu(z) = z; z = 0 -> 0
    zb = np.full_like(z, 50.0)
    assert_f32_close(oracle.norm_gate_rows(x, zb, w), oracle.head_norm_rows(x, w) * 50.0, rtol=1e-6)
    assert np.all(oracle.norm_gate_rows(x, np.zeros_like(z), w) == 0)


def test_gdn_recurrent_reference_fixture(oracle):
    fx = GOLDEN["gdn_recurrent"]
    kh, vh, dk, dv = fx["key_heads"], fx["value_heads"], fx["key_dim"], fx["value_dim"]
    state = np.zeros(vh * dk * dv, dtype=F32)
    for st in fx["steps"]:
        out = oracle.gdn_recurrent_step(state, st["q"], st["k"], st["v"], st["beta"], st["decay"], kh, vh, dk, dv)
        assert np.max(np.abs(out - np.array(st["expected"], dtype=F32))) < fx["tol"]


def _delta_rule_f64(S, q, k, v, beta, decay, kh, vh, dk, dv):
    """The delta rule in matrix form, float64: S_h <- d S_h + k (beta (v - d S_h^T k))^T, out = S_h^T q."""
    S = S.reshape(vh, dk, dv)
    out = np.empty((vh, dv))
    for h in range(vh):
        src = h % kh
        kk, qq = k[src * dk:(src + 1) * dk], q[src * dk:(src + 1) * dk]
        Sd = decay[h] * S[h]
        delta = beta[h] * (v[h * dv:(h + 1) * dv] - Sd.T @ kk)
        S[h] = Sd + np.outer(kk, delta)
        out[h] = S[h].T @ qq
    return out.reshape(-1)


def test_gdn_recurrent_matches_matrix_form(oracle):
    """Independent float64 matrix form of the delta rule over 6 tokens, value heads
    tiling key heads as h % key_heads (kh=2, vh=6)."""
    kh, vh, dk, dv = 2, 6, 8, 5
    rng = np.random.default_rng(21)
    S32 = (0.3 * rng.standard_normal(vh * dk * dv)).astype(F32)
    S64 = S32.astype(np.float64)
    for _ in range(6):
        q = rng.standard_normal(kh * dk).astype(F32)
        k = (rng.standard_normal(kh * dk) / np.sqrt(dk)).astype(F32)
        v = rng.standard_normal(vh * dv).astype(F32)
        beta = rng.uniform(0.05, 0.95, vh).astype(F32)
        decay = rng.uniform(0.5, 1.0, vh).astype(F32)
        out = oracle.gdn_recurrent_step(S32, q, k, v, beta, decay, kh, vh, dk, dv)
        ref = _delta_rule_f64(S64, *(t.astype(np.float64) for t in (q, k, v, beta, decay)), kh, vh, dk, dv)
        assert_f32_close(out, ref, group=dv, rtol=1e-5, what="out")
        assert_f32_close(S32, S64, group=dv, rtol=1e-5, what="state")


def test_gdn_recurrent_rows_layout(oracle):
    """The multi-token form reads q | k | v out of one front-end row per token and
    equals the per-token calls."""
    kh, vh, dk, dv, T = 2, 4, 8, 6, 5
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((T, 2 * kh * dk + vh * dv + 3)).astype(F32)  # 3 spare columns: a real stride
    beta = rng.uniform(0.1, 0.9, (T, vh)).astype(F32)
    decay = rng.uniform(0.6, 1.0, (T, vh)).astype(F32)
    S0 = (0.2 * rng.standard_normal(vh * dk * dv)).astype(F32)
    S1 = S0.copy()
    out = oracle.gdn_recurrent_rows(S1, qkv, beta, decay, kh, vh, dk, dv)
    S2 = S0.copy()
    for t in range(T):
        q, k, v = qkv[t, :kh * dk], qkv[t, kh * dk:2 * kh * dk], qkv[t, 2 * kh * dk:2 * kh * dk + vh * dv]
        assert_bits_equal(out[t], oracle.gdn_recurrent_step(S2, q, k, v, beta[t], decay[t], kh, vh, dk, dv), f"t={t}")
    assert_bits_equal(S1, S2, "state")


def test_gdn_gate_values(oracle):
    b = np.array([0.0, 2.0, -3.0, 10.0], dtype=F32)
    alpha = np.array([0.0, 25.0, -1.0, 19.0], dtype=F32)
    a = np.array([-1.0, -0.5, -2.0, -0.1], dtype=F32)
    dt = np.array([0.5, 0.0, 0.25, 0.5], dtype=F32)
    beta, decay = oracle.gdn_gate_values(b, alpha, a, dt)
    assert beta[0] == 0.5
    assert_f32_close(beta, sig64(b), rtol=1e-6)
    xx = (alpha + dt).astype(np.float64)
    sp = np.where(xx > 20, xx, np.log1p(np.exp(xx)))
    assert_f32_close(decay, np.exp(a * sp), rtol=2e-6)


# ------------------------------------------------------------------ attention core (decode)
def _attn_f64(q, K, V, heads, kv_heads, dim, gate=None):
    """softmax(q K^T / sqrt(D)) V per head in float64, query head h reading kv head
    h // (heads / kv_heads) (consecutive query heads share a kv head)."""
    n = K.shape[0]
    Kh = K.reshape(n, kv_heads, dim).astype(np.float64)
    Vh = V.reshape(n, kv_heads, dim).astype(np.float64)
    out = np.empty((heads, dim))
    for h in range(heads):
        kv = h // (heads // kv_heads)
        s = Kh[:, kv] @ q.reshape(heads, dim)[h].astype(np.float64) / np.sqrt(dim)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ Vh[:, kv]
    out = out.reshape(-1)
    if gate is not None:
        out = out / (1.0 + np.exp(-gate.astype(np.float64)))
    return out


def test_attn_split_qg(oracle):
    qg = np.arange(3 * 2 * 5, dtype=F32)
    q, g = oracle.attn_split_qg(qg, 3, 5)
    assert np.array_equal(q, qg.reshape(3, 2, 5)[:, 0].reshape(-1))
    assert np.array_equal(g, qg.reshape(3, 2, 5)[:, 1].reshape(-1))


def test_attn_scores_softmax_values_float64(oracle):
    """Each stage against float64 numpy; 4 query heads over 2 kv heads, so mapping
    query head h to kv head h % 2 instead of h // 2 fails."""
    heads, kv_heads, dim, pos = 4, 2, 16, 9
    rng = np.random.default_rng(3)
    q = rng.standard_normal(heads * dim).astype(F32)
    K = rng.standard_normal((pos + 1, kv_heads * dim)).astype(F32)
    V = rng.standard_normal((pos + 1, kv_heads * dim)).astype(F32)
    s = oracle.attn_scores(q, K, heads, kv_heads, dim, pos)
    s64 = np.stack([K.reshape(pos + 1, kv_heads, dim)[:, h // 2].astype(np.float64) @ q.reshape(heads, dim)[h]
                    for h in range(heads)]) / np.sqrt(dim)
    assert_f32_close(s, s64.reshape(-1), rtol=1e-6, what="scores")
    p = oracle.attn_softmax(s, heads, pos + 1)
    e = np.exp(s.reshape(heads, -1).astype(np.float64) - s.reshape(heads, -1).max(axis=1, keepdims=True))
    assert_f32_close(p, (e / e.sum(axis=1, keepdims=True)).reshape(-1), rtol=1e-6, what="softmax")
    assert np.allclose(p.reshape(heads, -1).sum(axis=1), 1.0, atol=1e-6)
    out = oracle.attn_values(p, V, heads, kv_heads, dim, pos)
    ref = np.stack([p.reshape(heads, -1)[h].astype(np.float64) @ V.reshape(pos + 1, kv_heads, dim)[:, h // 2]
                    for h in range(heads)]).reshape(-1)
    assert_f32_close(out, ref, group=dim, what="values")


def test_attn_softmax_special_cases(oracle):
    """Shift invariance, a dominant score gives a one-hot row, equal scores a uniform row."""
    row = np.array([1.0, 2.0, 3.0, -5.0], dtype=F32)
    a = oracle.attn_softmax(row, 1, 4)
    b = oracle.attn_softmax(row + 100.0, 1, 4)
    assert_f32_close(a, b, rtol=2e-6, what="shift")
    assert np.array_equal(oracle.attn_softmax(np.array([0.0, 200.0, -3.0], dtype=F32), 1, 3), np.array([0, 1, 0], F32))
    assert np.array_equal(oracle.attn_softmax(np.full(8, 0.7, F32), 1, 8), np.full(8, 0.125, F32))


def test_attn_decode_end_to_end(oracle):
    heads, kv_heads, dim, pos = 16, 2, 256, 40
    rng = np.random.default_rng(4)
    q = rng.standard_normal(heads * dim).astype(F32)
    K = rng.standard_normal((pos + 1, kv_heads * dim)).astype(F32)
    V = rng.standard_normal((pos + 1, kv_heads * dim)).astype(F32)
    g = rng.standard_normal(heads * dim).astype(F32)
    got = oracle.attn_decode(q, K, V, heads, kv_heads, dim, pos, gate=g)
    assert_f32_close(got, _attn_f64(q, K, V, heads, kv_heads, dim, gate=g), group=dim, what="decode")
    assert_f32_close(oracle.attn_sigmoid_gate(q, g), q / (1 + np.exp(-g.astype(np.float64))), rtol=1e-6, what="gate")


# ------------------------------------------------------------------ MoE routing
def test_moe_topk_against_sort(oracle):
    """Top-k = the k largest in descending order, ties to the lower index (a stable
    sort of -x), then a float64 softmax over the picks."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((50, 256)).astype(F32)
    x[3, [10, 200, 57]] = 9.0          # a three-way tie at the top
    x[4, :] = 0.25                     # all equal: indices 0..k-1
    idx, w = oracle.moe_topk_rows(x, 8)
    order = np.argsort(-x, axis=1, kind="stable")[:, :8]
    assert np.array_equal(idx, order)
    assert list(idx[3, :3]) == [10, 57, 200]
    assert list(idx[4]) == list(range(8))
    sel = np.take_along_axis(x, order, axis=1).astype(np.float64)
    e = np.exp(sel - sel.max(axis=1, keepdims=True))
    assert_f32_close(w, e / e.sum(axis=1, keepdims=True), rtol=1e-6, what="weights")
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_moe_topk_non_finite(oracle):
    x = np.zeros((2, 16), F32)
    x[1, 5] = np.inf
    idx, w = oracle.moe_topk_rows(x, 4, idx=np.full((2, 4), 7, np.int32), w=np.full((2, 4), 0.5, F32))
    assert idx[1, 0] == -1 and np.isnan(w[1, 0])
    assert list(idx[1, 1:]) == [7, 7, 7] and list(w[1, 1:]) == [0.5] * 3  # untouched, as the reference
    assert list(idx[0]) == [0, 1, 2, 3]


def test_moe_weighted_sum_and_expert_gemv(oracle):
    rng = np.random.default_rng(12)
    rows, k, dim = 3, 4, 10
    y = rng.standard_normal((rows, k, dim)).astype(F32)
    w = rng.uniform(0, 1, (rows, k)).astype(F32)
    out0 = rng.standard_normal((rows, dim)).astype(F32)
    got = oracle.moe_weighted_sum_rows(out0, y, w)
    ref = out0.astype(np.float64) + np.einsum("tk,tkd->td", w.astype(np.float64), y.astype(np.float64))
    assert_f32_close(got, ref, group=dim, what="weighted sum")
    assert_bits_equal(oracle.moe_add(out0[0], y[0, 0], 0.5), out0[0] + np.float32(0.5) * y[0, 0], "moe_add")
    # expert GEMV = matmul_dispatch at element offset e * stride, per selected expert
    E, M, K = 5, 8, 512
    raw = ggml_blocks.random_blocks(rng, 12, E * M * K // 256)
    xs = rng.standard_normal((3, K)).astype(F32)
    ids = np.array([4, 0, 9], np.int32)  # 9: no such expert -> NaN row
    yy = oracle.moe_expert_gemv(raw, 12, ids, E, M * K, xs, K, M, K)
    for j, e in enumerate(ids[:2]):
        assert_bits_equal(yy[j], oracle.gemv(raw, 12, xs[j], M, K, element_offset=int(e) * M * K), f"expert {e}")
    assert np.isnan(yy[2]).all()


# ------------------------------------------------------------------ MoE
def test_silu_scalars(oracle):
    assert oracle.silu(0.0) == 0.0
    assert oracle.sigmoid(0.0) == 0.5
    assert oracle.silu(100.0) == 100.0
    assert oracle.silu(-100.0) == 0.0


def test_swiglu_bf16_exhaustive(oracle):
    g = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    gf = f32_of_bf16(g)
    keep = ~np.isnan(gf)
    one = np.full(g.shape, 0x3F80, dtype=np.uint16)  # bf16 1.0
    got = oracle.swiglu_bf16(g[keep], one[keep])
    # Where expf(-g) is finite the float formula is within 1 bf16 ulp of the exact
    # SiLU; below g = -88.72 expf(-g) overflows and the reference's formula
    # g / (1 + inf) gives -0.0, which the oracle must reproduce.
    finite = gf[keep] > -88.72
    ref = bf16_of(silu64(gf[keep]).astype(F32))
    assert_bf16_close(got[finite], ref[finite])
    assert np.mean(got[finite] == ref[finite]) > 0.999
    tail = ~finite & np.isfinite(gf[keep])
    assert tail.sum() > 0 and np.all(got[tail] == 0x8000)
    # g = -inf: -inf / (1 + inf) is NaN
    assert np.isnan(f32_of_bf16(got[np.isneginf(gf[keep])])).all()


def test_swiglu_and_shared(oracle):
    rng = np.random.default_rng(41)
    g = bf16_of(2 * rng.standard_normal((64, 512)).astype(F32))
    u = bf16_of(2 * rng.standard_normal((64, 512)).astype(F32))
    lg = rng.standard_normal(64).astype(F32)
    h = oracle.swiglu_bf16(g, u)
    ref = silu64(f32_of_bf16(g)) * f32_of_bf16(u)
    assert_bf16_close(h, bf16_of(ref.astype(F32)))
    hs = oracle.shared_swiglu_sigmoid_bf16(g, u, lg)
    assert_bf16_close(hs, bf16_of((ref * sig64(lg)[:, None]).astype(F32)))
    hf = oracle.silu_mul(f32_of_bf16(g), f32_of_bf16(u))
    assert_f32_close(hf, ref, rtol=1e-6)
    acc = rng.standard_normal((64, 512)).astype(F32)
    x = rng.standard_normal((64, 512)).astype(F32)
    got = oracle.shared_add_rows(acc, x, lg)
    assert_f32_close(got, acc + x * sig64(lg)[:, None], group=512, rtol=1e-6)


# ------------------------------------------------------------------ timed CPU baseline build
def test_fp32_math_build_computes_the_same_functions(oracle):
    """liboracle_fp32.so (float math and float sums: what bench.py times as the
    reference CPU path) computes the step's functions within the parity bars of
    the checker build, so the timed baseline does the same work."""
    from qwen35_hip import synth

    c1, c2, c3, c4 = synth.c1_rmsnorm(rows=8), synth.c2_qk_rope(rows=16), synth.c3_residual(rows=8), synth.c4_norm_gate(rows=8)
    fe = synth.c4_frontend(rows=40, channels=1024, random_history=True)
    fe["k_heads"], fe["key_dim"] = 2, 128
    sw, sh = synth.c3_swiglu(rows=8), synth.c3_shared(rows=8)

    def run():
        return {
            "rms": oracle.rmsnorm_rows(c1["x"], c1["w"]),
            "rope": oracle.qk_norm_rope_rows(c2["q"], c2["k"], c2["qw"], c2["kw"], pos=c2["pos"], rope_dim=64,
                                             theta=1e7),
            "res": oracle.residual_rmsnorm_rows(c3["x"], c3["branch"], c3["w"]),
            "fe": oracle.gdn_frontend_rows(fe["x"], fe["w"], fe["hist"], 2, 128),
            "ng": oracle.norm_gate_rows(c4["x"], c4["z"], c4["w"]),
            "sw": oracle.swiglu_bf16(sw["g"], sw["u"]),
            "sh": oracle.shared_swiglu_sigmoid_bf16(sh["g"], sh["u"], sh["logits"]),
        }

    exact = run()
    with oracle.fp32_math():
        f32 = run()
    assert_f32_close(f32["rms"], exact["rms"], what="rmsnorm")
    for a, b in zip(f32["rope"], exact["rope"]):
        assert_f32_close(a, b, group=256, what="qk_norm_rope")
    assert np.array_equal(f32["res"][0], exact["res"][0])
    assert_bf16_close(f32["res"][1], exact["res"][1], what="residual_rmsnorm")
    assert_f32_close(f32["fe"][0], exact["fe"][0], group=128, what="gdn_frontend")
    assert_bits_equal(f32["fe"][1], exact["fe"][1], "history")
    assert_f32_close(f32["ng"], exact["ng"], what="norm_gate")
    assert_bf16_close(f32["sw"], exact["sw"], what="swiglu")
    assert_bf16_close(f32["sh"], exact["sh"], what="shared swiglu")
    assert oracle.lib() is not None and oracle._variant == "exact"
