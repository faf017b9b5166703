"""Tensor-level entry points over the C ABI.

Each function checks on the host that every tensor is a contiguous device
tensor of the dtype and shape the kernel assumes (the C ABI can only check
sizes, not buffer extents), then enqueues the kernel on `stream` (default: the
current torch stream) and returns the output tensor(s). Nothing here computes on
the CPU: the work is done by libqwen35_hip.so or not at all.

torch is used for device memory and streams only.
"""

from __future__ import annotations

import ctypes

import torch

from ._lib import check, load

BF16 = torch.bfloat16  # bf16 storage (fp32 math inside the kernels)

GGML_TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "BF16": 30}


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _dev(*ts: torch.Tensor, dtype=None) -> None:
    for t in ts:
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("expected a device tensor")
        if not t.is_contiguous():
            raise ValueError("expected a contiguous tensor")
        if dtype is not None and t.dtype != dtype:
            raise ValueError(f"expected dtype {dtype}, got {t.dtype}")


def _same(shape, *ts: torch.Tensor) -> None:
    for t in ts:
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"shape {tuple(t.shape)} != {tuple(shape)}")


def _rows(x: torch.Tensor) -> tuple[int, int]:
    if x.dim() < 1:
        raise ValueError("expected at least one dimension")
    n = x.shape[-1]
    return (x.numel() // n if n else 0), n


# ------------------------------------------------------------------ norms
def rmsnorm_rows(x, weight, out=None, eps=1e-6, stream=None):
    _dev(x, weight, dtype=torch.float32)
    rows, n = _rows(x)
    _same((n,), weight)
    out = torch.empty_like(x) if out is None else out
    _dev(out, dtype=torch.float32)
    _same(x.shape, out)
    check(load().qwen_rmsnorm_rows(_p(x), _p(weight), _p(out), rows, n, eps, _stream(stream)))
    return out


def rmsnorm_gated_rows(x, gate, weight, out=None, eps=1e-6, stream=None):
    _dev(x, gate, weight, dtype=torch.float32)
    rows, n = _rows(x)
    _same(x.shape, gate)
    _same((n,), weight)
    out = torch.empty_like(x) if out is None else out
    _dev(out, dtype=torch.float32)
    _same(x.shape, out)
    check(load().qwen_rmsnorm_gated_rows(_p(x), _p(gate), _p(weight), _p(out), rows, n, eps, _stream(stream)))
    return out


def residual_add(x1, x2, out=None, stream=None):
    _dev(x1, x2, dtype=torch.float32)
    _same(x1.shape, x2)
    out = torch.empty_like(x1) if out is None else out
    _dev(out, dtype=torch.float32)
    _same(x1.shape, out)
    check(load().qwen_residual_add(_p(x1), _p(x2), _p(out), x1.numel(), _stream(stream)))
    return out


def residual_rmsnorm_rows(x, branch, weight, resid=None, normed=None, eps=1e-6, stream=None):
    """resid = x + branch; normed = rmsnorm(resid) * weight. fp32 or bf16 storage."""
    dt = x.dtype
    if dt not in (torch.float32, BF16):
        raise ValueError("x must be float32 or bfloat16")
    _dev(x, branch, dtype=dt)
    _dev(weight, dtype=torch.float32)
    rows, n = _rows(x)
    _same(x.shape, branch)
    _same((n,), weight)
    resid = torch.empty_like(x) if resid is None else resid
    normed = torch.empty_like(x) if normed is None else normed
    _dev(resid, normed, dtype=dt)
    _same(x.shape, resid, normed)
    fn = load().qwen_residual_rmsnorm_rows_f32 if dt == torch.float32 else load().qwen_residual_rmsnorm_rows_bf16
    check(fn(_p(x), _p(branch), _p(weight), _p(resid), _p(normed), rows, n, eps, _stream(stream)))
    return resid, normed


def encoder_forward(token_id: int, table, out=None, stream=None):
    _dev(table, dtype=torch.float32)
    vocab, d = table.shape
    if not 0 <= token_id < vocab:
        raise ValueError(f"token {token_id} outside the table of {vocab} rows")
    out = torch.empty(d, dtype=torch.float32, device=table.device) if out is None else out
    _dev(out, dtype=torch.float32)
    _same((d,), out)
    check(load().qwen_encoder_forward(token_id, _p(table), _p(out), d, _stream(stream)))
    return out


# ------------------------------------------------------------------ attention
def attn_head_norm(x, weight, eps=1e-6, stream=None):
    """In place on x [..., heads, dim]."""
    _dev(x, weight, dtype=torch.float32)
    heads, dim = _rows(x)
    _same((dim,), weight)
    check(load().qwen_attn_head_norm(_p(x), _p(weight), heads, dim, eps, _stream(stream)))
    return x


def rope_forward(x, pos: int, rope_dim=64, theta=1e6, stream=None):
    """In place on x [heads, head_dim] (one token)."""
    _dev(x, dtype=torch.float32)
    heads, hd = _rows(x)
    check(load().qwen_rope_forward(_p(x), pos, heads, hd, rope_dim, theta, _stream(stream)))
    return x


def attn_qk_norm_rope_rows(q, k, q_weight, k_weight, pos=None, pos0=0, rope_dim=64, theta=1e7, eps=1e-6,
                           stream=None):
    """In place: q [rows, q_heads, hd], k [rows, k_heads, hd]; pos int32 [rows] or None."""
    _dev(q, k, q_weight, k_weight, dtype=torch.float32)
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q, k must be [rows, heads, head_dim] with equal rows and head_dim")
    rows, qh, hd = q.shape
    kh = k.shape[1]
    _same((hd,), q_weight, k_weight)
    if pos is not None:
        _dev(pos, dtype=torch.int32)
        _same((rows,), pos)
    check(load().qwen_attn_qk_norm_rope_rows(_p(q), _p(k), _p(q_weight), _p(k_weight), _p(pos), pos0, rows, qh, kh,
                                             hd, rope_dim, theta, eps, _stream(stream)))
    return q, k


# ------------------------------------------------------------------ Gated DeltaNet
def gdn_frontend_rows(x, weight, hist_in, hist_out=None, y=None, k_heads=16, key_dim=128, eps=1e-6, stream=None):
    """x [rows, C], weight [C, K], hist [C, K-1] -> (y [rows, C], hist_out)."""
    _dev(x, weight, hist_in, dtype=torch.float32)
    rows, c = _rows(x)
    if weight.dim() != 2 or weight.shape[0] != c:
        raise ValueError("weight must be [channels, kernel]")
    kernel = weight.shape[1]
    _same((c, kernel - 1), hist_in)
    hist_out = torch.empty_like(hist_in) if hist_out is None else hist_out
    y = torch.empty_like(x) if y is None else y
    _dev(hist_out, y, dtype=torch.float32)
    _same(hist_in.shape, hist_out)
    _same(x.shape, y)
    check(load().qwen_gdn_frontend_rows(_p(x), _p(weight), _p(hist_in), _p(hist_out), _p(y), rows, c, kernel, k_heads,
                                        key_dim, eps, _stream(stream)))
    return y, hist_out


def gdn_conv_step(x, weight, history, y=None, stream=None):
    """One token: x [C], weight [C, K], history [C, K-1] (updated in place)."""
    _dev(x, weight, history, dtype=torch.float32)
    c = x.numel()
    kernel = weight.shape[1]
    _same((c, kernel), weight)
    _same((c, kernel - 1), history)
    y = torch.empty_like(x) if y is None else y
    _dev(y, dtype=torch.float32)
    _same(x.shape, y)
    check(load().qwen_gdn_conv_step(_p(x), _p(weight), _p(history), _p(y), c, kernel, _stream(stream)))
    return y


def gdn_qk_normalize(q, k, eps=1e-6, stream=None):
    """In place on q, k [heads, dim]."""
    _dev(q, k, dtype=torch.float32)
    heads, dim = _rows(q)
    _same(q.shape, k)
    check(load().qwen_gdn_qk_normalize(_p(q), _p(k), heads, dim, eps, _stream(stream)))
    return q, k


def gdn_norm_gate_rows(x, z, weight, out=None, eps=1e-6, stream=None):
    """x, z [..., heads, dim]; weight [dim]."""
    _dev(x, z, weight, dtype=torch.float32)
    heads_total, dim = _rows(x)
    _same(x.shape, z)
    _same((dim,), weight)
    out = torch.empty_like(x) if out is None else out
    _dev(out, dtype=torch.float32)
    _same(x.shape, out)
    check(load().qwen_gdn_norm_gate_rows(_p(x), _p(z), _p(weight), _p(out), heads_total, 1, dim, eps,
                                         _stream(stream)))
    return out


def gdn_norm_gate_matmul(x, z, norm_weight, weight, ggml_type, num_elements: int, M: int, element_offset: int = 0,
                         normed=None, out=None, eps=1e-6, stream=None):
    """x, z [heads, dim]; norm_weight [dim] -> normed [heads, dim] (the gated norm) and
    out [M] = W[element_offset ..] @ normed, in one launch where the library can
    (src/layer_gdn.cpp:109-112)."""
    _dev(x, z, norm_weight, dtype=torch.float32)
    _dev(weight, dtype=torch.uint8)
    heads, dim = _rows(x)
    _same(x.shape, z)
    _same((dim,), norm_weight)
    normed = torch.empty_like(x) if normed is None else normed
    _dev(normed, dtype=torch.float32)
    _same(x.shape, normed)
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    out = torch.empty(M, dtype=torch.float32, device=x.device) if out is None else out
    _dev(out, dtype=torch.float32)
    if out.numel() < M:
        raise ValueError(f"out has {out.numel()} elements, M = {M}")
    check(load().qwen_gdn_norm_gate_matmul(_p(x), _p(z), _p(norm_weight), _p(normed), heads, dim, eps, _p(weight), t,
                                           num_elements, _p(out), M, element_offset, _stream(stream)))
    return normed, out


def gdn_gate_values_rows(beta_raw, alpha_raw, a, dt_bias, beta=None, decay=None, stream=None):
    """beta_raw, alpha_raw [rows, heads] (or [heads]); a, dt_bias [heads] -> beta, decay."""
    _dev(beta_raw, alpha_raw, a, dt_bias, dtype=torch.float32)
    heads = a.numel()
    _same((heads,), dt_bias)
    _same(beta_raw.shape, alpha_raw)
    if beta_raw.numel() % max(heads, 1):
        raise ValueError("beta_raw must hold whole rows of `heads` values")
    rows = beta_raw.numel() // max(heads, 1)
    beta = torch.empty_like(beta_raw) if beta is None else beta
    decay = torch.empty_like(beta_raw) if decay is None else decay
    _dev(beta, decay, dtype=torch.float32)
    _same(beta_raw.shape, beta, decay)
    check(load().qwen_gdn_gate_values_rows(_p(beta_raw), _p(alpha_raw), _p(a), _p(dt_bias), _p(beta), _p(decay), rows,
                                           heads, _stream(stream)))
    return beta, decay


def gdn_recurrent_step(state, q, k, v, beta, decay, key_heads, value_heads, key_dim, value_dim, out=None,
                       stream=None):
    """state [value_heads, key_dim, value_dim] updated in place; q, k [key_heads * key_dim];
    v [value_heads * value_dim]; beta, decay [value_heads] -> out [value_heads * value_dim]."""
    _dev(state, q, k, v, beta, decay, dtype=torch.float32)
    if state.numel() != value_heads * key_dim * value_dim:
        raise ValueError("state shape does not match the head sizes")
    for t, n in ((q, key_heads * key_dim), (k, key_heads * key_dim), (v, value_heads * value_dim),
                 (beta, value_heads), (decay, value_heads)):
        if t.numel() < n:
            raise ValueError(f"input of {t.numel()} elements, need {n}")
    out = torch.empty(value_heads * value_dim, dtype=torch.float32, device=state.device) if out is None else out
    _dev(out, dtype=torch.float32)
    check(load().qwen_gdn_recurrent_step(_p(state), _p(q), _p(k), _p(v), _p(beta), _p(decay), _p(out), key_heads,
                                         value_heads, key_dim, value_dim, _stream(stream)))
    return out


def gdn_recurrent_rows(state, qkv, beta, decay, key_heads, value_heads, key_dim, value_dim, out=None, stream=None):
    """qkv [rows, 2*key_heads*key_dim + value_heads*value_dim] (q | k | v per token, the GDN
    front end's output rows); beta, decay [rows, value_heads]; state updated in place
    -> out [rows, value_heads * value_dim]."""
    _dev(state, qkv, beta, decay, dtype=torch.float32)
    rows, stride = qkv.shape
    kd = key_heads * key_dim
    if stride < 2 * kd + value_heads * value_dim:
        raise ValueError("qkv rows too short for q | k | v")
    if state.numel() != value_heads * key_dim * value_dim:
        raise ValueError("state shape does not match the head sizes")
    _same((rows, value_heads), beta, decay)
    out = torch.empty((rows, value_heads * value_dim), dtype=torch.float32, device=qkv.device) if out is None else out
    _dev(out, dtype=torch.float32)
    _same((rows, value_heads * value_dim), out)
    base = qkv.data_ptr()
    check(load().qwen_gdn_recurrent_rows(_p(state), ctypes.c_void_p(base), ctypes.c_void_p(base + 4 * kd),
                                         ctypes.c_void_p(base + 8 * kd), _p(beta), _p(decay), _p(out), rows,
                                         key_heads, value_heads, key_dim, value_dim, stride, value_heads * value_dim,
                                         _stream(stream)))
    return out


def gdn_gated_recurrent_rows(state, qkv, beta_raw, alpha_raw, a, dt_bias, key_heads, value_heads, key_dim,
                             value_dim, out=None, stream=None):
    """gdn_gate_values_rows fused into gdn_recurrent_rows: beta_raw, alpha_raw [rows, value_heads],
    a, dt_bias [value_heads]; other arguments as gdn_recurrent_rows."""
    _dev(state, qkv, beta_raw, alpha_raw, a, dt_bias, dtype=torch.float32)
    rows, stride = qkv.shape
    kd = key_heads * key_dim
    if stride < 2 * kd + value_heads * value_dim:
        raise ValueError("qkv rows too short for q | k | v")
    if state.numel() != value_heads * key_dim * value_dim:
        raise ValueError("state shape does not match the head sizes")
    _same((rows, value_heads), beta_raw, alpha_raw)
    _same((value_heads,), a, dt_bias)
    out = torch.empty((rows, value_heads * value_dim), dtype=torch.float32, device=qkv.device) if out is None else out
    _dev(out, dtype=torch.float32)
    _same((rows, value_heads * value_dim), out)
    base = qkv.data_ptr()
    check(load().qwen_gdn_gated_recurrent_rows(_p(state), ctypes.c_void_p(base), ctypes.c_void_p(base + 4 * kd),
                                               ctypes.c_void_p(base + 8 * kd), _p(beta_raw), _p(alpha_raw), _p(a),
                                               _p(dt_bias), _p(out), rows, key_heads, value_heads, key_dim, value_dim,
                                               stride, value_heads * value_dim, _stream(stream)))
    return out


def gdn_decode_step(x, conv_w, hist_in, hist_out, state, beta_raw, alpha_raw, a, dt_bias, key_heads, value_heads,
                    key_dim, value_dim, y=None, out=None, eps=1e-6, stream=None):
    """One decode token after the projections: gdn_frontend_rows on x [C] (hist_in -> hist_out, y [C]),
    then gdn_gated_recurrent_rows on y (state in place, out [value_heads * value_dim])."""
    _dev(x, conv_w, hist_in, hist_out, state, beta_raw, alpha_raw, a, dt_bias, dtype=torch.float32)
    C = 2 * key_heads * key_dim + value_heads * value_dim
    K = conv_w.shape[-1]
    if x.numel() != C or conv_w.numel() != C * K or hist_in.numel() != C * (K - 1) or hist_out.numel() != C * (K - 1):
        raise ValueError("x, conv weights or history do not match the channel count")
    if state.numel() != value_heads * key_dim * value_dim:
        raise ValueError("state must be [value_heads, key_dim, value_dim]")
    _same((value_heads,), beta_raw, alpha_raw, a, dt_bias)
    y = torch.empty(C, dtype=torch.float32, device=x.device) if y is None else y
    out = torch.empty(value_heads * value_dim, dtype=torch.float32, device=x.device) if out is None else out
    _dev(y, out, dtype=torch.float32)
    if y.numel() != C or out.numel() != value_heads * value_dim:
        raise ValueError("y or out of the wrong size")
    check(load().qwen_gdn_decode_step(_p(x), _p(conv_w), _p(hist_in), _p(hist_out), _p(y), _p(state), _p(beta_raw),
                                      _p(alpha_raw), _p(a), _p(dt_bias), _p(out), key_heads, value_heads, key_dim,
                                      value_dim, K, eps, _stream(stream)))
    return out


def gdn_recurrent_chunked(state, qkv, beta, decay, key_heads, value_heads, key_dim, value_dim, out=None,
                          workspace=None, stream=None):
    """qwen_gdn_recurrent_rows' chunked form (prefill): same arguments; `workspace` a
    uint8 device tensor of at least the required bytes (allocated here if None)."""
    _dev(state, qkv, beta, decay, dtype=torch.float32)
    rows, stride = qkv.shape
    kd = key_heads * key_dim
    if stride < 2 * kd + value_heads * value_dim:
        raise ValueError("qkv rows too short for q | k | v")
    if state.numel() != value_heads * key_dim * value_dim:
        raise ValueError("state shape does not match the head sizes")
    _same((rows, value_heads), beta, decay)
    out = torch.empty((rows, value_heads * value_dim), dtype=torch.float32, device=qkv.device) if out is None else out
    _dev(out, dtype=torch.float32)
    _same((rows, value_heads * value_dim), out)
    need = load().qwen_gdn_recurrent_chunked_workspace_bytes(rows, value_heads)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=qkv.device)
    _dev(workspace, dtype=torch.uint8)
    base = qkv.data_ptr()
    check(load().qwen_gdn_recurrent_chunked(_p(state), ctypes.c_void_p(base), ctypes.c_void_p(base + 4 * kd),
                                            ctypes.c_void_p(base + 8 * kd), _p(beta), _p(decay), _p(out), rows,
                                            key_heads, value_heads, key_dim, value_dim, stride,
                                            value_heads * value_dim, _p(workspace), workspace.numel(),
                                            _stream(stream)))
    return out


# ------------------------------------------------------------------ attention core (decode)
def attn_split_qg(qg, heads, dim, q=None, g=None, stream=None):
    _dev(qg, dtype=torch.float32)
    if qg.numel() != 2 * heads * dim:
        raise ValueError("qg must hold heads x 2 x dim values")
    q = torch.empty(heads * dim, dtype=torch.float32, device=qg.device) if q is None else q
    g = torch.empty_like(q) if g is None else g
    _dev(q, g, dtype=torch.float32)
    if q.numel() < heads * dim or g.numel() < heads * dim:
        raise ValueError("q / g outputs smaller than heads x dim")
    check(load().qwen_attn_split_qg(_p(qg), _p(q), _p(g), heads, dim, _stream(stream)))
    return q, g


def _attn_check(q, cache, heads, kv_heads, dim, pos):
    if q.numel() < heads * dim or cache.numel() < (pos + 1) * kv_heads * dim:
        raise ValueError("q or cache too small for the shape")


def attn_scores(q, k_cache, heads, kv_heads, dim, pos, out=None, stream=None):
    _dev(q, k_cache, dtype=torch.float32)
    _attn_check(q, k_cache, heads, kv_heads, dim, pos)
    out = torch.empty(heads * (pos + 1), dtype=torch.float32, device=q.device) if out is None else out
    _dev(out, dtype=torch.float32)
    if out.numel() < heads * (pos + 1):
        raise ValueError("scores output too small for the shape")
    check(load().qwen_attn_scores(_p(q), _p(k_cache), _p(out), heads, kv_heads, dim, pos, _stream(stream)))
    return out


def attn_softmax(scores, heads, valid_len, stream=None):
    _dev(scores, dtype=torch.float32)
    if scores.numel() < heads * valid_len:
        raise ValueError("scores too small")
    check(load().qwen_attn_softmax(_p(scores), heads, valid_len, _stream(stream)))
    return scores


def attn_values(scores, v_cache, heads, kv_heads, dim, pos, out=None, stream=None):
    _dev(scores, v_cache, dtype=torch.float32)
    if scores.numel() < heads * (pos + 1) or v_cache.numel() < (pos + 1) * kv_heads * dim:
        raise ValueError("scores or cache too small for the shape")
    out = torch.empty(heads * dim, dtype=torch.float32, device=scores.device) if out is None else out
    _dev(out, dtype=torch.float32)
    if out.numel() < heads * dim:
        raise ValueError("values output too small for the shape")
    check(load().qwen_attn_values(_p(scores), _p(v_cache), _p(out), heads, kv_heads, dim, pos, _stream(stream)))
    return out


def attn_sigmoid_gate(x, gate, out=None, stream=None):
    _dev(x, gate, dtype=torch.float32)
    _same(x.shape, gate)
    out = torch.empty_like(x) if out is None else out
    check(load().qwen_attn_sigmoid_gate(_p(x), _p(gate), _p(out), x.numel(), _stream(stream)))
    return out


def attn_kv_store(k, v, k_cache, v_cache, pos, max_seq_len, stream=None):
    _dev(k, v, k_cache, v_cache, dtype=torch.float32)
    _same(k.shape, v)
    if k_cache.numel() < max_seq_len * k.numel() or v_cache.numel() < max_seq_len * k.numel():
        raise ValueError("caches smaller than max_seq_len rows")
    check(load().qwen_attn_kv_store(_p(k), _p(v), _p(k_cache), _p(v_cache), pos, k.numel(), max_seq_len,
                                    _stream(stream)))


def attn_decode_workspace_bytes(heads, kv_heads, dim, pos) -> int:
    return int(load().qwen_attn_decode_workspace_bytes(heads, kv_heads, dim, pos))


def attn_decode(q, k_cache, v_cache, heads, kv_heads, dim, pos, gate=None, workspace=None, out=None, stream=None):
    """One query per head against cache rows 0..pos -> out [heads * dim] (x sigmoid(gate))."""
    _dev(q, k_cache, v_cache, dtype=torch.float32)
    _attn_check(q, k_cache, heads, kv_heads, dim, pos)
    _attn_check(q, v_cache, heads, kv_heads, dim, pos)
    if gate is not None:
        _dev(gate, dtype=torch.float32)
    nbytes = attn_decode_workspace_bytes(heads, kv_heads, dim, pos)
    if workspace is None:
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    _dev(workspace)
    out = torch.empty(heads * dim, dtype=torch.float32, device=q.device) if out is None else out
    _dev(out, dtype=torch.float32)
    check(load().qwen_attn_decode(_p(q), _p(k_cache), _p(v_cache), _p(gate), _p(out), heads, kv_heads, dim, pos,
                                  _p(workspace), workspace.numel() * workspace.element_size(), _stream(stream)))
    return out


def attn_decode_norm_rope(q, k_cache, v_cache, heads, kv_heads, dim, pos, q_weight, k_weight, rope_dim, theta,
                          gate=None, workspace=None, q_normed=None, out=None, eps=1e-6, stream=None):
    """attn_qk_norm_rope_rows on a copy of q (-> q_normed) and on the cache row of pos
    (in place), then attn_decode of q_normed, in one split pass where the library can
    (src/layer_attn.cpp:91-96, 103-108). Returns (out, q_normed)."""
    _dev(q, k_cache, v_cache, q_weight, k_weight, dtype=torch.float32)
    _attn_check(q, k_cache, heads, kv_heads, dim, pos)
    _attn_check(q, v_cache, heads, kv_heads, dim, pos)
    _same((dim,), q_weight)
    _same((dim,), k_weight)
    if gate is not None:
        _dev(gate, dtype=torch.float32)
    nbytes = attn_decode_workspace_bytes(heads, kv_heads, dim, pos)
    if workspace is None:
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    _dev(workspace)
    q_normed = torch.empty(heads * dim, dtype=torch.float32, device=q.device) if q_normed is None else q_normed
    _dev(q_normed, dtype=torch.float32)
    if q_normed.numel() < heads * dim:
        raise ValueError(f"q_normed has {q_normed.numel()} elements, need {heads * dim}")
    out = torch.empty(heads * dim, dtype=torch.float32, device=q.device) if out is None else out
    _dev(out, dtype=torch.float32)
    check(load().qwen_attn_decode_norm_rope(_p(q), _p(q_normed), _p(k_cache), _p(v_cache), _p(gate), _p(out), heads,
                                            kv_heads, dim, pos, _p(q_weight), _p(k_weight), rope_dim, theta, eps,
                                            _p(workspace), workspace.numel() * workspace.element_size(),
                                            _stream(stream)))
    return out, q_normed


def attn_decode_noalloc(q, k_cache, v_cache, heads, kv_heads, dim, pos, gate=None, out=None, stream=None):
    """attn_decode with the library's fixed device scratch instead of a workspace
    (no device allocation in the call when `out` is given)."""
    _dev(q, k_cache, v_cache, dtype=torch.float32)
    _attn_check(q, k_cache, heads, kv_heads, dim, pos)
    _attn_check(q, v_cache, heads, kv_heads, dim, pos)
    if gate is not None:
        _dev(gate, dtype=torch.float32)
    out = torch.empty(heads * dim, dtype=torch.float32, device=q.device) if out is None else out
    _dev(out, dtype=torch.float32)
    check(load().qwen_attn_decode_noalloc(_p(q), _p(k_cache), _p(v_cache), _p(gate), _p(out), heads, kv_heads, dim,
                                          pos, _stream(stream)))
    return out


# ------------------------------------------------------------------ MoE routing
def moe_topk_rows(logits, k, idx=None, weights=None, stream=None):
    """logits [rows, n] (or [n]) -> idx int32, weights float32 [rows, k]."""
    _dev(logits, dtype=torch.float32)
    n = logits.shape[-1]
    rows = logits.numel() // n
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device) if idx is None else idx
    weights = torch.empty((rows, k), dtype=torch.float32, device=logits.device) if weights is None else weights
    _dev(idx, dtype=torch.int32)
    _dev(weights, dtype=torch.float32)
    _same((rows, k), idx, weights)
    check(load().qwen_moe_topk_rows(_p(logits), _p(idx), _p(weights), rows, n, k, _stream(stream)))
    return idx, weights


def moe_add(out, x, a: float, stream=None):
    _dev(out, x, dtype=torch.float32)
    _same(out.shape, x)
    check(load().qwen_moe_add(_p(out), _p(x), a, out.numel(), _stream(stream)))
    return out


def moe_weighted_sum_rows(out, expert_out, weights, stream=None):
    """out [rows, dim] += sum_j weights[rows, k] * expert_out[rows, k, dim]."""
    _dev(out, expert_out, weights, dtype=torch.float32)
    rows, k, dim = expert_out.shape
    _same((rows, dim), out)
    _same((rows, k), weights)
    check(load().qwen_moe_weighted_sum_rows(_p(out), _p(expert_out), _p(weights), rows, k, dim, _stream(stream)))
    return out


def moe_expert_matmul(weight, ggml_type, num_elements, expert_stride, n_experts, idx, x, x_stride, M, K, out=None,
                      stream=None):
    """y[j] = W_{idx[j]} x[j * x_stride : + K] for the n_sel = idx.numel() ids (device int32)."""
    _dev(weight, dtype=torch.uint8)
    _dev(idx, dtype=torch.int32)
    _dev(x, dtype=torch.float32)
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    n_sel = idx.numel()
    if n_sel and x.numel() < (n_sel - 1) * x_stride + K:
        raise ValueError("x too small for n_sel inputs")
    out = torch.empty((n_sel, M), dtype=torch.float32, device=x.device) if out is None else out
    _dev(out, dtype=torch.float32)
    check(load().qwen_moe_expert_matmul(_p(weight), t, num_elements, expert_stride, n_experts, _p(idx), n_sel, _p(x),
                                        x_stride, _p(out), M, K, _stream(stream)))
    return out


def moe_expert_gate_up(w_gate, w_up, ggml_type, num_elements, expert_stride, n_experts, idx, x, M, K, gate_out=None,
                       up_out=None, stream=None):
    """gate_out[j] = Wg_{idx[j]} x, up_out[j] = Wu_{idx[j]} x in one launch; [n_sel, M] each."""
    _dev(w_gate, w_up, dtype=torch.uint8)
    _dev(idx, dtype=torch.int32)
    _dev(x, dtype=torch.float32)
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    n_sel = idx.numel()
    if x.numel() < K:
        raise ValueError(f"x has {x.numel()} elements, K = {K}")
    gate_out = torch.empty((n_sel, M), dtype=torch.float32, device=x.device) if gate_out is None else gate_out
    up_out = torch.empty((n_sel, M), dtype=torch.float32, device=x.device) if up_out is None else up_out
    _dev(gate_out, up_out, dtype=torch.float32)
    if gate_out.numel() < n_sel * M or up_out.numel() < n_sel * M:
        raise ValueError("outputs smaller than n_sel x M")
    check(load().qwen_moe_expert_gate_up(_p(w_gate), _p(w_up), t, num_elements, expert_stride, n_experts, _p(idx),
                                         n_sel, _p(x), _p(gate_out), _p(up_out), M, K, _stream(stream)))
    return gate_out, up_out


def moe_expert_swiglu_workspace_bytes(n_sel, inter, shared_dim) -> int:
    return int(load().qwen_moe_expert_swiglu_workspace_bytes(n_sel, inter, shared_dim))


def moe_expert_swiglu(w_gate, w_up, ggml_type, num_elements, expert_stride, n_experts, idx, x, inter, K,
                      w_shared_gate=None, w_shared_up=None, shared_type=None, shared_elements=0, shared_dim=0,
                      hidden=None, shared_hidden=None, workspace=None, stream=None):
    """hidden[j] = SiLU(Wg_{idx[j]} x) * (Wu_{idx[j]} x) [n_sel, inter]; with the shared tensors also
    shared_hidden = SiLU(Wsg x) * (Wsu x) [shared_dim]. Returns (hidden, shared_hidden or None)."""
    _dev(w_gate, w_up, dtype=torch.uint8)
    _dev(idx, dtype=torch.int32)
    _dev(x, dtype=torch.float32)
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    n_sel = idx.numel()
    if x.numel() < K:
        raise ValueError(f"x has {x.numel()} elements, K = {K}")
    has_shared = w_shared_gate is not None
    if has_shared:
        _dev(w_shared_gate, w_shared_up, dtype=torch.uint8)
        ts = GGML_TYPES[shared_type] if isinstance(shared_type, str) else int(shared_type)
    else:
        ts, shared_dim = 0, 0
    hidden = torch.empty((n_sel, inter), dtype=torch.float32, device=x.device) if hidden is None else hidden
    _dev(hidden, dtype=torch.float32)
    if hidden.numel() < n_sel * inter:
        raise ValueError("hidden smaller than n_sel x inter")
    if has_shared:
        shared_hidden = (torch.empty(shared_dim, dtype=torch.float32, device=x.device) if shared_hidden is None
                         else shared_hidden)
        _dev(shared_hidden, dtype=torch.float32)
        if shared_hidden.numel() < shared_dim:
            raise ValueError("shared_hidden smaller than shared_dim")
    nbytes = moe_expert_swiglu_workspace_bytes(n_sel, inter, shared_dim)
    if workspace is None:
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    _dev(workspace)
    check(load().qwen_moe_expert_swiglu(_p(w_gate), _p(w_up), t, num_elements, expert_stride, n_experts, _p(idx),
                                        n_sel, inter, _p(w_shared_gate) if has_shared else None,
                                        _p(w_shared_up) if has_shared else None, ts, shared_elements, shared_dim,
                                        _p(x), K, _p(hidden), _p(shared_hidden) if has_shared else None,
                                        _p(workspace), workspace.numel() * workspace.element_size(),
                                        _stream(stream)))
    return hidden, (shared_hidden if has_shared else None)


def moe_route_swiglu(logits, k, w_gate, w_up, ggml_type, num_elements, expert_stride, x, inter, K,
                     w_shared_gate=None, w_shared_up=None, shared_type=None, shared_elements=0, shared_dim=0,
                     idx=None, weights=None, hidden=None, shared_hidden=None, workspace=None, stream=None):
    """moe_topk_rows on the router logits [n_experts] fused into moe_expert_swiglu.
    Returns (idx int32 [k], weights [k], hidden [k, inter], shared_hidden or None)."""
    _dev(logits, dtype=torch.float32)
    _dev(w_gate, w_up, dtype=torch.uint8)
    _dev(x, dtype=torch.float32)
    n_experts = logits.numel()
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    if x.numel() < K:
        raise ValueError(f"x has {x.numel()} elements, K = {K}")
    idx = torch.empty(k, dtype=torch.int32, device=x.device) if idx is None else idx
    weights = torch.empty(k, dtype=torch.float32, device=x.device) if weights is None else weights
    _dev(idx, dtype=torch.int32)
    _dev(weights, dtype=torch.float32)
    _same((k,), idx, weights)
    has_shared = w_shared_gate is not None
    if has_shared:
        _dev(w_shared_gate, w_shared_up, dtype=torch.uint8)
        ts = GGML_TYPES[shared_type] if isinstance(shared_type, str) else int(shared_type)
    else:
        ts, shared_dim = 0, 0
    hidden = torch.empty((k, inter), dtype=torch.float32, device=x.device) if hidden is None else hidden
    _dev(hidden, dtype=torch.float32)
    if hidden.numel() < k * inter:
        raise ValueError("hidden smaller than k x inter")
    if has_shared:
        shared_hidden = (torch.empty(shared_dim, dtype=torch.float32, device=x.device) if shared_hidden is None
                         else shared_hidden)
        _dev(shared_hidden, dtype=torch.float32)
        if shared_hidden.numel() < shared_dim:
            raise ValueError("shared_hidden smaller than shared_dim")
    nbytes = moe_expert_swiglu_workspace_bytes(k, inter, shared_dim)
    if workspace is None:
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    _dev(workspace)
    check(load().qwen_moe_route_swiglu(_p(logits), _p(idx), _p(weights), k, _p(w_gate), _p(w_up), t, num_elements,
                                       expert_stride, n_experts, inter, _p(w_shared_gate) if has_shared else None,
                                       _p(w_shared_up) if has_shared else None, ts, shared_elements, shared_dim,
                                       _p(x), K, _p(hidden), _p(shared_hidden) if has_shared else None,
                                       _p(workspace), workspace.numel() * workspace.element_size(),
                                       _stream(stream)))
    return idx, weights, hidden, (shared_hidden if has_shared else None)


def moe_down_combine_workspace_bytes(n_sel, d_model) -> int:
    return int(load().qwen_moe_down_combine_workspace_bytes(n_sel, d_model))


def moe_down_combine(w_down, down_type, down_elements, expert_stride, n_experts, idx, weights, hidden, inter,
                     w_shared_down, shared_type, shared_elements, shared_hidden, shared_logit, d_model, out=None,
                     workspace=None, stream=None):
    """out [d_model] = sum_j weights[j] Wd_{idx[j]} hidden[j] + sigmoid(shared_logit[0]) Wsd shared_hidden."""
    _dev(w_down, w_shared_down, dtype=torch.uint8)
    _dev(idx, dtype=torch.int32)
    _dev(weights, hidden, shared_hidden, shared_logit, dtype=torch.float32)
    n_sel = idx.numel()
    _same((n_sel,), weights)
    if hidden.numel() < n_sel * inter:
        raise ValueError("hidden smaller than n_sel x inter")
    shared_dim = shared_hidden.numel()
    if shared_logit.numel() < 1:
        raise ValueError("shared_logit is empty")
    td = GGML_TYPES[down_type] if isinstance(down_type, str) else int(down_type)
    ts = GGML_TYPES[shared_type] if isinstance(shared_type, str) else int(shared_type)
    nbytes = moe_down_combine_workspace_bytes(n_sel, d_model)
    if workspace is None:
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=hidden.device)
    _dev(workspace)
    out = torch.empty(d_model, dtype=torch.float32, device=hidden.device) if out is None else out
    _dev(out, dtype=torch.float32)
    if out.numel() < d_model:
        raise ValueError("out smaller than d_model")
    check(load().qwen_moe_down_combine(_p(w_down), td, down_elements, expert_stride, n_experts, _p(idx), _p(weights),
                                       n_sel, _p(hidden), inter, _p(w_shared_down), ts, shared_elements,
                                       _p(shared_hidden), shared_dim, _p(shared_logit), _p(out), d_model,
                                       _p(workspace), workspace.numel() * workspace.element_size(), _stream(stream)))
    return out


# ------------------------------------------------------------------ MoE
def moe_silu_mul(g, u, out=None, stream=None):
    _dev(g, u, dtype=torch.float32)
    _same(g.shape, u)
    out = torch.empty_like(g) if out is None else out
    _dev(out, dtype=torch.float32)
    _same(g.shape, out)
    check(load().qwen_moe_silu_mul(_p(g), _p(u), _p(out), g.numel(), _stream(stream)))
    return out


def moe_shared_add_rows(accum, shared_out, gate, stream=None):
    """accum [rows, n] += shared_out * sigmoid(gate[rows]) in place."""
    _dev(accum, shared_out, gate, dtype=torch.float32)
    rows, n = _rows(accum)
    _same(accum.shape, shared_out)
    _same((rows,), gate)
    check(load().qwen_moe_shared_add_rows(_p(accum), _p(shared_out), _p(gate), rows, n, _stream(stream)))
    return accum


def swiglu_bf16(g, u, out=None, stream=None):
    _dev(g, u, dtype=BF16)
    _same(g.shape, u)
    out = torch.empty_like(g) if out is None else out
    _dev(out, dtype=BF16)
    _same(g.shape, out)
    check(load().qwen_swiglu_bf16(_p(g), _p(u), _p(out), g.numel(), _stream(stream)))
    return out


def shared_swiglu_sigmoid_rows_bf16(g, u, logits, out=None, stream=None):
    _dev(g, u, dtype=BF16)
    _dev(logits, dtype=torch.float32)
    rows, dim = _rows(g)
    _same(g.shape, u)
    _same((rows,), logits)
    out = torch.empty_like(g) if out is None else out
    _dev(out, dtype=BF16)
    _same(g.shape, out)
    check(load().qwen_shared_swiglu_sigmoid_rows_bf16(_p(g), _p(u), _p(logits), _p(out), rows, dim, _stream(stream)))
    return out


def swiglu_routed_shared_bf16(g, u, sg, su, logits, out=None, shared_out=None, stream=None):
    """Routed SwiGLU over g, u (any shape) and the shared expert's gated SwiGLU
    over sg, su [rows x dim] with logits [rows], in one launch; returns
    (out, shared_out)."""
    _dev(g, u, sg, su, dtype=BF16)
    _dev(logits, dtype=torch.float32)
    _same(g.shape, u)
    rows, dim = _rows(sg)
    _same(sg.shape, su)
    _same((rows,), logits)
    out = torch.empty_like(g) if out is None else out
    shared_out = torch.empty_like(sg) if shared_out is None else shared_out
    _dev(out, shared_out, dtype=BF16)
    _same(g.shape, out)
    _same(sg.shape, shared_out)
    check(load().qwen_swiglu_routed_shared_bf16(_p(g), _p(u), _p(out), g.numel(), _p(sg), _p(su), _p(logits),
                                                _p(shared_out), rows, dim, _stream(stream)))
    return out, shared_out


# ------------------------------------------------------------------ dequant
def dequant_gather_rows(table, ggml_type, num_elements: int, ids, cols: int, out=None, stream=None):
    """table: uint8 device tensor of GGML blocks; ids int32 [n]; -> float32 [n, cols]."""
    _dev(table, dtype=torch.uint8)
    _dev(ids, dtype=torch.int32)
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    n = ids.numel()
    out = torch.empty((n, cols), dtype=torch.float32, device=table.device) if out is None else out
    _dev(out, dtype=torch.float32)
    _same((n, cols), out)
    check(load().qwen_dequant_gather_rows(_p(table), t, num_elements, _p(ids), n, cols, _p(out), _stream(stream)))
    return out


def dequantize_row(table, ggml_type, num_elements: int, row: int, cols: int, out=None, stream=None):
    _dev(table, dtype=torch.uint8)
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    out = torch.empty(cols, dtype=torch.float32, device=table.device) if out is None else out
    _dev(out, dtype=torch.float32)
    _same((cols,), out)
    check(load().qwen_dequantize_row(_p(table), t, num_elements, _p(out), row, cols, _stream(stream)))
    return out


# ------------------------------------------------------------------ quantized GEMV
class GemvDesc(ctypes.Structure):
    """qwen_gemv_desc (include/qwen35_hip.h)."""
    _fields_ = [("weight", ctypes.c_void_p), ("type", ctypes.c_int), ("M", ctypes.c_int),
                ("num_elements", ctypes.c_uint64), ("element_offset", ctypes.c_uint64), ("y", ctypes.c_void_p),
                ("split", ctypes.c_int)]


def matmul_dispatch_multi(jobs, x, K: int, stream=None):
    """jobs: (weight uint8 tensor, ggml type, num_elements, M, element_offset, out float32 [M] or None
    [, split]); y_j = W_j x for every job, all from one x [K]. split s > 0 writes the rows in the
    attn_split_qg layout (pairs of s-row halves: first halves to out[:M/2], second to out[M/2:]).
    Returns the outputs."""
    _dev(x, dtype=torch.float32)
    if x.numel() < K:
        raise ValueError(f"x has {x.numel()} elements, K = {K}")
    descs = (GemvDesc * max(1, len(jobs)))()
    outs = []
    for j, job in enumerate(jobs):
        w, t, ne, M, off, out = job[:6]
        split = job[6] if len(job) > 6 else 0
        _dev(w, dtype=torch.uint8)
        out = torch.empty(M, dtype=torch.float32, device=x.device) if out is None else out
        _dev(out, dtype=torch.float32)
        if out.numel() < M:
            raise ValueError(f"job {j}: out has {out.numel()} elements, M = {M}")
        descs[j] = GemvDesc(w.data_ptr(), GGML_TYPES[t] if isinstance(t, str) else int(t), M, ne, off, out.data_ptr(),
                            split)
        outs.append(out)
    check(load().qwen_matmul_dispatch_multi(ctypes.cast(descs, ctypes.c_void_p), len(jobs), _p(x), K,
                                            _stream(stream)))
    return outs


def matmul_rows_workspace_bytes(rows: int, K: int) -> int:
    return load().qwen_matmul_rows_workspace_bytes(rows, K)


def matmul_rows(weight, ggml_type, num_elements: int, x, M: int, K: int, element_offset: int = 0, out=None,
                workspace=None, stream=None):
    """matmul_dispatch for every row of x: x float32 [rows, K] -> y float32 [rows, M],
    y[t, m] = sum_k W[element_offset + m*K + k] * x[t, k] (one call; matrix cores for
    Q4_K / Q6_K at 16 rows or more, with a workspace allocated here unless given)."""
    _dev(weight, dtype=torch.uint8)
    _dev(x, dtype=torch.float32)
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [rows, {K}], got {tuple(x.shape)}")
    rows = x.shape[0]
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    out = torch.empty(rows, M, dtype=torch.float32, device=x.device) if out is None else out
    _dev(out, dtype=torch.float32)
    if out.numel() < rows * M:
        raise ValueError(f"out has {out.numel()} elements, rows * M = {rows * M}")
    if workspace is None:
        workspace = torch.empty(max(1, matmul_rows_workspace_bytes(rows, K)), dtype=torch.uint8, device=x.device)
    _dev(workspace, dtype=torch.uint8)
    check(load().qwen_matmul_rows(_p(weight), t, num_elements, _p(x), _p(out), rows, M, K, element_offset,
                                  _p(workspace), workspace.numel(), _stream(stream)))
    return out


def matmul_rows_multi(jobs, x, K: int, workspace=None, stream=None):
    """jobs: (weight uint8 tensor, ggml type, num_elements, M, element_offset, out float32 [rows, M]
    or None); y_j = x W_j^T for every job from one x [rows, K] (one prep, one GEMM launch per
    K-quant type). Returns the outputs."""
    _dev(x, dtype=torch.float32)
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [rows, {K}], got {tuple(x.shape)}")
    rows = x.shape[0]
    descs = (GemvDesc * max(1, len(jobs)))()
    outs = []
    for j, (w, t, ne, M, off, out) in enumerate(jobs):
        _dev(w, dtype=torch.uint8)
        out = torch.empty(rows, M, dtype=torch.float32, device=x.device) if out is None else out
        _dev(out, dtype=torch.float32)
        if out.numel() < rows * M:
            raise ValueError(f"job {j}: out has {out.numel()} elements, rows * M = {rows * M}")
        descs[j] = GemvDesc(w.data_ptr(), GGML_TYPES[t] if isinstance(t, str) else int(t), M, ne, off, out.data_ptr(), 0)
        outs.append(out)
    if workspace is None:
        workspace = torch.empty(max(1, matmul_rows_workspace_bytes(rows, K)), dtype=torch.uint8, device=x.device)
    _dev(workspace, dtype=torch.uint8)
    check(load().qwen_matmul_rows_multi(ctypes.cast(descs, ctypes.c_void_p), len(jobs), _p(x), rows, K,
                                        _p(workspace), workspace.numel(), _stream(stream)))
    return outs


def matmul_dispatch(weight, ggml_type, num_elements: int, x, M: int, K: int, element_offset: int = 0, out=None,
                    stream=None):
    """weight: uint8 device tensor of GGML blocks; x float32 [K] -> y float32 [M],
    y[m] = sum_k W[element_offset + m*K + k] * x[k]."""
    _dev(weight, dtype=torch.uint8)
    _dev(x, dtype=torch.float32)
    if x.numel() < K:
        raise ValueError(f"x has {x.numel()} elements, K = {K}")
    t = GGML_TYPES[ggml_type] if isinstance(ggml_type, str) else int(ggml_type)
    out = torch.empty(M, dtype=torch.float32, device=x.device) if out is None else out
    _dev(out, dtype=torch.float32)
    if out.numel() < M:
        raise ValueError(f"out has {out.numel()} elements, M = {M}")
    check(load().qwen_matmul_dispatch(_p(weight), t, num_elements, _p(x), _p(out), M, K, element_offset,
                                      _stream(stream)))
    return out
