"""numpy front end of liboracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker (or the timed CPU baseline). It computes
on the CPU and is never part of the product path.

Every function takes and returns numpy arrays (bf16 as uint16 bit patterns) and
mirrors one function of oracle.h.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64

_SIGS = {
    "or_silu": ([_F], _F),
    "or_sigmoid": ([_F], _F),
    "or_rsqrt": ([_F], _F),
    "or_half_to_float": ([ctypes.c_uint16], _F),
    "or_bf16_to_float": ([ctypes.c_uint16], _F),
    "or_float_to_bf16": ([_F], ctypes.c_uint16),
    "or_dequant": ([_P, _I, _U64], _F),
    "or_rmsnorm_rows": ([_P, _P, _P, _I, _I, _F, _I], None),
    "or_rmsnorm_gated_rows": ([_P, _P, _P, _P, _I, _I, _F, _I], None),
    "or_residual_add": ([_P, _P, _P, _I64], None),
    "or_encoder_rows": ([_P, _I, _P, _P, _I], None),
    "or_residual_rmsnorm_rows_f32": ([_P, _P, _P, _P, _P, _I, _I, _F, _I], None),
    "or_residual_rmsnorm_rows_bf16": ([_P, _P, _P, _P, _P, _I, _I, _F, _I], None),
    "or_head_norm_rows": ([_P, _P, _I, _I, _I, _F, _I], None),
    "or_rope_den": ([_I, _I, _F], _F),
    "or_rope_rows": ([_P, _P, _I, _I, _I, _I, _I, _F, _I], None),
    "or_qk_norm_rope_rows": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _I], None),
    "or_conv_rows": ([_P, _P, _P, _P, _P, _I, _I, _I, _I], None),
    "or_qk_l2_rows": ([_P, _P, _I64, _I, _I, _I, _F, _I], None),
    "or_gdn_frontend_rows": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I], None),
    "or_norm_gate_rows": ([_P, _P, _P, _P, _I, _I, _I, _F, _I], None),
    "or_gdn_gate_values": ([_P, _P, _P, _P, _P, _P, _I], None),
    "or_gdn_recurrent_step": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I], None),
    "or_gdn_recurrent_rows": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I64, _I64], None),
    "or_silu_mul_f32": ([_P, _P, _P, _I64, _I], None),
    "or_swiglu_bf16": ([_P, _P, _P, _I64, _I], None),
    "or_shared_swiglu_sigmoid_bf16": ([_P, _P, _P, _P, _I, _I, _I], None),
    "or_shared_add_rows": ([_P, _P, _P, _I, _I], None),
    "or_type_supported": ([_I], _I),
    "or_dequant_gather": ([_P, _I, _P, _I, _I, _P, _I], None),
    "or_dequant_span": ([_P, _I, _U64, _I, _P], None),
    "or_gemv": ([_P, _I, _P, _P, _I, _I, _U64, _I], None),
    "or_attn_split_qg": ([_P, _P, _P, _I, _I], None),
    "or_moe_topk_rows": ([_P, _P, _P, _I, _I, _I], None),
    "or_moe_add": ([_P, _P, ctypes.c_float, _I64], None),
    "or_moe_weighted_sum_rows": ([_P, _P, _P, _I, _I, _I], None),
    "or_moe_expert_gemv": ([_P, _I, _P, _I, _I, _U64, _P, _I64, _P, _I, _I], None),
    "or_attn_scores": ([_P, _P, _P, _I, _I, _I, _I], None),
    "or_attn_softmax": ([_P, _I, _I], None),
    "or_attn_values": ([_P, _P, _P, _I, _I, _I, _I], None),
    "or_attn_sigmoid_gate": ([_P, _P, _P, _I64], None),
    "or_attn_decode": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I], None),
}

_libs: dict[str, ctypes.CDLL] = {}
_variant = "exact"
_PATHS = {"exact": LIB_PATH, "fp32": HERE / "liboracle_fp32.so"}


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    """The checker build (double-evaluated math), or inside `fp32_math()` the
    float-math build that bench.py times as the CPU baseline."""
    if _variant not in _libs:
        path = _PATHS[_variant]
        if not path.exists():
            build()
        l = ctypes.CDLL(str(path))
        for name, (args, res) in _SIGS.items():
            f = getattr(l, name)
            f.argtypes = args
            f.restype = res
        _libs[_variant] = l
    return _libs[_variant]


class fp32_math:
    """Context: the wrappers call liboracle_fp32.so (float math, float sums of
    squares, as the reference's host loops) -- the timed CPU baseline only."""

    def __enter__(self):
        global _variant
        self._prev, _variant = _variant, "fp32"
        return self

    def __exit__(self, *exc):
        global _variant
        _variant = self._prev
        return False


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


F32, U16, I32, U8 = np.float32, np.uint16, np.int32, np.uint8


# ---------------------------------------------------------------- scalars
def silu(x: float) -> float: return lib().or_silu(x)
def sigmoid(x: float) -> float: return lib().or_sigmoid(x)
def rsqrt(x: float) -> float: return lib().or_rsqrt(x)
def rope_den(i: int, rope_dim: int, theta: float) -> float: return lib().or_rope_den(i, rope_dim, theta)


def half_to_float(bits: np.ndarray) -> np.ndarray:
    f = lib().or_half_to_float
    return np.array([f(int(b)) for b in np.asarray(bits).ravel()], dtype=F32).reshape(np.shape(bits))


def float_to_bf16(x: np.ndarray) -> np.ndarray:
    f = lib().or_float_to_bf16
    return np.array([f(float(v)) for v in np.asarray(x, dtype=F32).ravel()], dtype=U16).reshape(np.shape(x))


# ---------------------------------------------------------------- norms
def rmsnorm_rows(x, w, eps=1e-6, threads=1):
    x = _c(x, F32)
    w = _c(w, F32)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().or_rmsnorm_rows(_p(x), _p(w), _p(out), x.size // n, n, eps, threads)
    return out


def rmsnorm_gated_rows(x, gate, w, eps=1e-6, threads=1):
    x, gate, w = _c(x, F32), _c(gate, F32), _c(w, F32)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().or_rmsnorm_gated_rows(_p(x), _p(gate), _p(w), _p(out), x.size // n, n, eps, threads)
    return out


def residual_add(a, b):
    a, b = _c(a, F32), _c(b, F32)
    out = np.empty_like(a)
    lib().or_residual_add(_p(a), _p(b), _p(out), a.size)
    return out


def encoder_rows(ids, table):
    ids, table = _c(ids, I32), _c(table, F32)
    out = np.empty((ids.size, table.shape[1]), dtype=F32)
    lib().or_encoder_rows(_p(ids), ids.size, _p(table), _p(out), table.shape[1])
    return out


def residual_rmsnorm_rows(x, branch, w, eps=1e-6, threads=1):
    """fp32 (float32 arrays) or bf16 (uint16 bit-pattern arrays)."""
    bf16 = np.asarray(x).dtype == U16
    dt = U16 if bf16 else F32
    x, branch, w = _c(x, dt), _c(branch, dt), _c(w, F32)
    n = x.shape[-1]
    resid, normed = np.empty_like(x), np.empty_like(x)
    fn = lib().or_residual_rmsnorm_rows_bf16 if bf16 else lib().or_residual_rmsnorm_rows_f32
    fn(_p(x), _p(branch), _p(w), _p(resid), _p(normed), x.size // n, n, eps, threads)
    return resid, normed


# ---------------------------------------------------------------- attention
def head_norm_rows(x, w, eps=1e-6, threads=1):
    x = _c(x, F32).copy()
    d = x.shape[-1]
    lib().or_head_norm_rows(_p(x), _p(_c(w, F32)), 1, x.size // d, d, eps, threads)
    return x


def rope_rows(x, pos=None, pos0=0, rope_dim=64, theta=1e6, threads=1):
    """x [rows, heads, head_dim] -> rotated copy."""
    x = _c(x, F32).copy()
    rows, heads, hd = x.shape
    p = None if pos is None else _c(pos, I32)
    lib().or_rope_rows(_p(x), _p(p), pos0, rows, heads, hd, rope_dim, theta, threads)
    return x


def qk_norm_rope_rows(q, k, qw, kw, pos=None, pos0=0, rope_dim=64, theta=1e7, eps=1e-6, threads=1):
    q, k = _c(q, F32).copy(), _c(k, F32).copy()
    rows, qh, hd = q.shape
    kh = k.shape[1]
    p = None if pos is None else _c(pos, I32)
    lib().or_qk_norm_rope_rows(_p(q), _p(k), _p(_c(qw, F32)), _p(_c(kw, F32)), _p(p), pos0, rows, qh, kh, hd,
                               rope_dim, theta, eps, threads)
    return q, k


# ---------------------------------------------------------------- Gated DeltaNet
def conv_rows(x, w, hist, threads=1):
    x, w, hist = _c(x, F32), _c(w, F32), _c(hist, F32)
    rows, c = x.shape
    k = w.shape[1]
    y = np.empty_like(x)
    hist_out = np.empty_like(hist)
    lib().or_conv_rows(_p(x), _p(w), _p(hist), _p(hist_out), _p(y), rows, c, k, threads)
    return y, hist_out


def qk_l2_rows(q, k, eps=1e-6, threads=1):
    """q, k [rows, heads, dim] -> normalised copies."""
    q, k = _c(q, F32).copy(), _c(k, F32).copy()
    rows, heads, dim = q.shape
    lib().or_qk_l2_rows(_p(q), _p(k), heads * dim, rows, heads, dim, eps, threads)
    return q, k


def gdn_frontend_rows(x, w, hist, k_heads=16, key_dim=128, eps=1e-6, threads=1):
    x, w, hist = _c(x, F32), _c(w, F32), _c(hist, F32)
    rows, c = x.shape
    k = w.shape[1]
    y = np.empty_like(x)
    hist_out = np.empty_like(hist)
    lib().or_gdn_frontend_rows(_p(x), _p(w), _p(hist), _p(hist_out), _p(y), rows, c, k, k_heads, key_dim, eps,
                               threads)
    return y, hist_out


def norm_gate_rows(x, z, w, eps=1e-6, threads=1):
    x, z, w = _c(x, F32), _c(z, F32), _c(w, F32)
    d = x.shape[-1]
    out = np.empty_like(x)
    lib().or_norm_gate_rows(_p(x), _p(z), _p(w), _p(out), 1, x.size // d, d, eps, threads)
    return out


def gdn_gate_values(b, alpha, a, dt):
    b, alpha, a, dt = (_c(v, F32) for v in (b, alpha, a, dt))
    beta, decay = np.empty_like(b), np.empty_like(b)
    lib().or_gdn_gate_values(_p(b), _p(alpha), _p(a), _p(dt), _p(beta), _p(decay), b.size)
    return beta, decay


def gdn_recurrent_step(state, q, k, v, beta, decay, key_heads, value_heads, key_dim, value_dim):
    """Updates `state` (float32, contiguous) in place; returns out [value_heads * value_dim]."""
    assert state.dtype == F32 and state.flags.c_contiguous
    q, k, v, beta, decay = (_c(t, F32) for t in (q, k, v, beta, decay))
    out = np.empty(value_heads * value_dim, dtype=F32)
    lib().or_gdn_recurrent_step(_p(state), _p(q), _p(k), _p(v), _p(beta), _p(decay), _p(out), key_heads,
                                value_heads, key_dim, value_dim)
    return out


def gdn_gate_values_rows(b, alpha, a, dt):
    """b, alpha [rows, heads]; a, dt [heads] -> beta, decay [rows, heads]."""
    b, alpha = _c(b, F32), _c(alpha, F32)
    rows, heads = b.shape
    beta, decay = gdn_gate_values(b.reshape(-1), alpha.reshape(-1), np.tile(_c(a, F32), rows), np.tile(_c(dt, F32), rows))
    return beta.reshape(rows, heads), decay.reshape(rows, heads)


def gdn_recurrent_rows(state, qkv, beta, decay, key_heads, value_heads, key_dim, value_dim):
    """qkv [rows, 2*key_heads*key_dim + value_heads*value_dim] (q | k | v per token, the
    GDN front end's output layout); beta, decay [rows, value_heads]. Updates `state` in
    place; returns out [rows, value_heads * value_dim]."""
    assert state.dtype == F32 and state.flags.c_contiguous
    qkv, beta, decay = _c(qkv, F32), _c(beta, F32), _c(decay, F32)
    rows, stride = qkv.shape
    kd = key_heads * key_dim
    out = np.empty((rows, value_heads * value_dim), dtype=F32)
    base = qkv.ctypes.data
    lib().or_gdn_recurrent_rows(_p(state), ctypes.c_void_p(base), ctypes.c_void_p(base + 4 * kd),
                                ctypes.c_void_p(base + 8 * kd), _p(beta), _p(decay), _p(out), rows, key_heads,
                                value_heads, key_dim, value_dim, stride, value_heads * value_dim)
    return out


# ---------------------------------------------------------------- MoE
def silu_mul(g, u, threads=1):
    g, u = _c(g, F32), _c(u, F32)
    h = np.empty_like(g)
    lib().or_silu_mul_f32(_p(g), _p(u), _p(h), g.size, threads)
    return h


def swiglu_bf16(g, u, threads=1):
    g, u = _c(g, U16), _c(u, U16)
    h = np.empty_like(g)
    lib().or_swiglu_bf16(_p(g), _p(u), _p(h), g.size, threads)
    return h


def shared_swiglu_sigmoid_bf16(g, u, logits, threads=1):
    g, u, logits = _c(g, U16), _c(u, U16), _c(logits, F32)
    dim = g.shape[-1]
    h = np.empty_like(g)
    lib().or_shared_swiglu_sigmoid_bf16(_p(g), _p(u), _p(logits), _p(h), g.size // dim, dim, threads)
    return h


def shared_add_rows(accum, x, gate):
    accum = _c(accum, F32).copy()
    x, gate = _c(x, F32), _c(gate, F32)
    dim = accum.shape[-1]
    lib().or_shared_add_rows(_p(accum), _p(x), _p(gate), accum.size // dim, dim)
    return accum


# ---------------------------------------------------------------- dequant
def type_supported(t: int) -> bool:
    return bool(lib().or_type_supported(t))


def dequant_gather(table, ggml_type: int, ids, cols: int, threads=1):
    table, ids = _c(table, U8), _c(ids, I32)
    out = np.empty((ids.size, cols), dtype=F32)
    lib().or_dequant_gather(_p(table), ggml_type, _p(ids), ids.size, cols, _p(out), threads)
    return out


def dequant_span(data, ggml_type: int, start: int, count: int):
    data = _c(data, U8)
    out = np.empty(count, dtype=F32)
    lib().or_dequant_span(_p(data), ggml_type, start, count, _p(out))
    return out


# ---------------------------------------------------------------- quantized GEMV
def gemv(weight, ggml_type: int, x, M: int, K: int, element_offset: int = 0, threads=1):
    """y[m] = sum_k W[element_offset + m*K + k] * x[k] (exact products, double sum)."""
    weight, x = _c(weight, U8), _c(x, F32)
    assert x.size >= K
    y = np.empty(M, dtype=F32)
    lib().or_gemv(_p(weight), ggml_type, _p(x), _p(y), M, K, element_offset, threads)
    return y


# ---------------------------------------------------------------- attention core (decode)
def attn_split_qg(qg, heads, dim):
    qg = _c(qg, F32)
    q, g = np.empty(heads * dim, F32), np.empty(heads * dim, F32)
    lib().or_attn_split_qg(_p(qg), _p(q), _p(g), heads, dim)
    return q, g


def attn_scores(q, k_cache, heads, kv_heads, dim, pos):
    q, k_cache = _c(q, F32), _c(k_cache, F32)
    s = np.empty(heads * (pos + 1), F32)
    lib().or_attn_scores(_p(q), _p(k_cache), _p(s), heads, kv_heads, dim, pos)
    return s


def attn_softmax(scores, heads, n):
    s = _c(scores, F32).copy()
    lib().or_attn_softmax(_p(s), heads, n)
    return s


def attn_values(scores, v_cache, heads, kv_heads, dim, pos):
    scores, v_cache = _c(scores, F32), _c(v_cache, F32)
    out = np.empty(heads * dim, F32)
    lib().or_attn_values(_p(scores), _p(v_cache), _p(out), heads, kv_heads, dim, pos)
    return out


def attn_sigmoid_gate(x, g):
    x, g = _c(x, F32), _c(g, F32)
    out = np.empty_like(x)
    lib().or_attn_sigmoid_gate(_p(x), _p(g), _p(out), x.size)
    return out


def attn_decode(q, k_cache, v_cache, heads, kv_heads, dim, pos, gate=None):
    q, k_cache, v_cache = _c(q, F32), _c(k_cache, F32), _c(v_cache, F32)
    g = None if gate is None else _c(gate, F32)
    out = np.empty(heads * dim, F32)
    scratch = np.empty(heads * (pos + 1), F32)
    lib().or_attn_decode(_p(q), _p(k_cache), _p(v_cache), _p(g), _p(out), _p(scratch), heads, kv_heads, dim, pos)
    return out


# ---------------------------------------------------------------- MoE routing
def moe_topk_rows(x, k, idx=None, w=None):
    """x [rows, n] -> idx int32 [rows, k], w [rows, k] (inputs idx / w give the
    untouched entries of a non-finite row)."""
    x = _c(x, F32)
    rows, n = x.shape
    idx = np.zeros((rows, k), np.int32) if idx is None else _c(idx, I32).copy()
    w = np.zeros((rows, k), F32) if w is None else _c(w, F32).copy()
    lib().or_moe_topk_rows(_p(x), _p(idx), _p(w), rows, n, k)
    return idx, w


def moe_add(out, x, a):
    out = _c(out, F32).copy()
    lib().or_moe_add(_p(out), _p(_c(x, F32)), a, out.size)
    return out


def moe_weighted_sum_rows(out, y, w):
    """out [rows, dim] += sum_j w[rows, k] * y[rows, k, dim]."""
    out = _c(out, F32).copy()
    y, w = _c(y, F32), _c(w, F32)
    rows, k, dim = y.shape
    lib().or_moe_weighted_sum_rows(_p(out), _p(y), _p(w), rows, k, dim)
    return out


def moe_expert_gemv(weight, ggml_type, idx, n_experts, expert_stride, x, x_stride, M, K):
    weight, idx, x = _c(weight, U8), _c(idx, I32), _c(x, F32)
    y = np.empty((idx.size, M), F32)
    lib().or_moe_expert_gemv(_p(weight), ggml_type, _p(idx), idx.size, n_experts, expert_stride, _p(x), x_stride,
                             _p(y), M, K)
    return y
