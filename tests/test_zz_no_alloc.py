"""qwen_attn_decode_noalloc: the decode attention entry point that allocates
nothing (its split-K partials in the library's fixed device scratch).

Called through the C ABI and compared bit for bit with qwen_attn_decode (the
existing entry point, with a caller workspace) on the same inputs, over
consecutive calls whose shapes shrink, so a call that read the previous call's
partials would differ; plus the oracle's decode at the fp32 bar.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from qwen35_hip import _lib

pytestmark = pytest.mark.gpu
F32 = np.float32
P = ctypes.c_void_p


def _inputs(seed, heads, kv_heads, dim, n_keys):
    r = np.random.default_rng(seed)
    q = r.standard_normal(heads * dim).astype(F32)
    K = r.standard_normal((n_keys, kv_heads * dim)).astype(F32)
    V = r.standard_normal((n_keys, kv_heads * dim)).astype(F32)
    g = (2 * r.standard_normal(heads * dim)).astype(F32)
    return q, K, V, g


def _decode_both(lib, heads, kv_heads, dim, pos, seed):
    q, K, V, g = (torch.from_numpy(a).cuda() for a in _inputs(seed, heads, kv_heads, dim, pos + 1))
    stream = P(torch.cuda.current_stream().cuda_stream)
    need = lib.qwen_attn_decode_workspace_bytes(heads, kv_heads, dim, pos)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
    ref = torch.full((heads * dim,), 7.0, device="cuda")
    got = torch.full((heads * dim,), -7.0, device="cuda")
    ptrs = [P(t.data_ptr()) for t in (q, K, V, g)]
    assert lib.qwen_attn_decode(*ptrs, P(ref.data_ptr()), heads, kv_heads, dim, pos, P(ws.data_ptr()), ws.numel(),
                                stream) == 0, lib.qwen_last_error()
    assert lib.qwen_attn_decode_noalloc(*ptrs, P(got.data_ptr()), heads, kv_heads, dim, pos, stream) == 0, \
        lib.qwen_last_error()
    torch.cuda.synchronize()
    return got.cpu().numpy(), ref.cpu().numpy(), (q, K, V, g)


def test_noalloc_decode_equals_workspace_decode_on_consecutive_calls(oracle):
    lib = _lib.load()
    assert lib.qwen_attn_decode_noalloc_max_scratch_bytes() == 8 << 20
    # model shape at the full context, then smaller calls on the same scratch: a
    # shorter context, 16 query heads per kv head, and the staged path (dim 128)
    for heads, kv, dim, pos, seed in [(16, 2, 256, 4095, 1), (16, 2, 256, 100, 2), (16, 1, 256, 40, 3),
                                      (4, 2, 128, 9, 4)]:
        got, ref, (q, K, V, g) = _decode_both(lib, heads, kv, dim, pos, seed)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (heads, kv, dim, pos)
        qh, Kh, Vh, gh = (t.cpu().numpy() for t in (q, K, V, g))
        want = oracle.attn_decode(qh, Kh, Vh, heads, kv, dim, pos, gate=gh)
        # fp32 bar relative to each output's condition scale sum_t p_t |v_tj| x sigmoid(gate)
        p = oracle.attn_softmax(oracle.attn_scores(qh, Kh, heads, kv, dim, pos), heads, pos + 1).reshape(heads, -1)
        Va = np.abs(Vh.reshape(pos + 1, kv, dim).astype(np.float64))
        scale = np.stack([p[h].astype(np.float64) @ Va[:, h // (heads // kv)] for h in range(heads)]).reshape(-1)
        scale = scale / (1.0 + np.exp(-gh.astype(np.float64)))
        err = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), scale)
        assert err.max() <= 1e-5, (heads, kv, dim, pos, err.max())


def test_noalloc_decode_rejects_shapes_beyond_its_scratch():
    lib = _lib.load()
    x = torch.zeros(16, device="cuda")
    px = P(x.data_ptr())
    # 64 query / 8 kv heads of 256 at 20,000 keys needs ~41 MB of partials
    need = lib.qwen_attn_decode_workspace_bytes(64, 8, 256, 19999)
    assert need > lib.qwen_attn_decode_noalloc_max_scratch_bytes()
    st = lib.qwen_attn_decode_noalloc(px, px, px, px, px, 64, 8, 256, 19999, P(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.STATUS_INVALID_ARGUMENT
    assert b"scratch" in lib.qwen_last_error()


_CAPTURE_CHILD = r"""
import ctypes, sys
import numpy as np, torch
from qwen35_hip import _lib
lib = _lib.load()
P = ctypes.c_void_p
torch.cuda.set_device(0)
H, KV, D, pos = 16, 2, 256, 1000
r = np.random.default_rng(11)
q, K, V, g = (torch.from_numpy(a).cuda() for a in (
    r.standard_normal(H * D).astype(np.float32), r.standard_normal((pos + 1, KV * D)).astype(np.float32),
    r.standard_normal((pos + 1, KV * D)).astype(np.float32), r.standard_normal(H * D).astype(np.float32)))
ptrs = [P(t.data_ptr()) for t in (q, K, V, g)]
out = torch.zeros(H * D, device="cuda")
ref = torch.zeros(H * D, device="cuda")
need = lib.qwen_attn_decode_workspace_bytes(H, KV, D, pos)
ws = torch.empty(need, dtype=torch.uint8, device="cuda")
torch.cuda.synchronize()
s = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):   # the first noalloc call of this process
    rc = lib.qwen_attn_decode_noalloc(*ptrs, P(out.data_ptr()), H, KV, D, pos, P(s.cuda_stream))
assert rc == 0, lib.qwen_last_error()
cur = P(torch.cuda.current_stream().cuda_stream)
assert lib.qwen_attn_decode(*ptrs, P(ref.data_ptr()), H, KV, D, pos, P(ws.data_ptr()), need, cur) == 0
for i in range(3):
    out.fill_(float(i))                    # eager work between the replays
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {i}"
print("noalloc capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """The scratch array's address is looked up at the first call on a device: that
    first call may itself be under HIP graph capture (a fresh process captures it,
    replays the graph three times with eager work between, and every replay equals
    qwen_attn_decode with a workspace bit for bit)."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    pkg = Path(_lib.__file__).resolve().parents[1]
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(pkg), os.environ.get("PYTHONPATH", "")]))
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD], env=env, capture_output=True, text=True, timeout=110)
    assert res.returncode == 0 and "noalloc capture ok" in res.stdout, res.stdout + res.stderr
