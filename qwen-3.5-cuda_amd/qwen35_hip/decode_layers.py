"""A layer's decode step composed from the library's entry points, for each of the
three layer kinds of the reference's decoder (GDN, full attention, MoE).

Each class holds the layer's weights and per-layer state as the reference's
layer object does and runs its decode forward in two ways: one library call per
reference call (`forward_reference_launches`) and through the fused entry points
(`forward`). Weights are GGML tensors (uint8 device tensors of blocks) of one
K-quant type.

`GdnLayerDecode` follows the reference's GdnLayer (src/layer_gdn.cpp:37-57: conv
history, recurrent state, per-token buffers; forward src/layer_gdn.cpp:78-113):

* `forward_reference_launches(x)`: four projections (:83-86), conv step (:89),
  Q/K normalize (:97), gates (:100), recurrent step (:103-106), gated norm
  (:109), output projection (:112): ten launches;
* `forward(x)`: the four projections in one `matmul_dispatch_multi`, conv + SiLU
  + Q/K L2 + gates + recurrence in `gdn_decode_step` (the bits of
  `gdn_frontend_rows` followed by `gdn_gated_recurrent_rows`), then the gated
  norm and the output projection in `gdn_norm_gate_matmul` (the bits of
  `gdn_norm_gate_rows` followed by `matmul_dispatch`): three launches.

Both update the layer's conv history and recurrent state (the fused step writes
the new history into a second buffer and the two are swapped, since the
one-launch step cannot update it in place).

`GdnLayerDecode.prefill(xs)` runs a prompt of T tokens through the same layer
in one pass, where the reference runs its decode forward T times: the four
input projections in one `matmul_rows_multi` (one prep, one GEMM launch) and the
output projection in `matmul_rows`, the front
end over all rows (`gdn_frontend_rows`, history carried), the gates of all
rows, the chunked recurrence (`gdn_recurrent_chunked`) and the gated norm. It
leaves the history and state where T decode steps leave them.
"""

from __future__ import annotations

import math

import torch

from . import ops


class GdnLayerDecode:
    def __init__(self, w_qkv, w_z, w_beta, w_alpha, w_out, conv_w, a, dt_bias, norm_w, *, wtype="Q4_K",
                 d_model=2048, key_heads=16, value_heads=32, key_dim=128, value_dim=128, eps=1e-6):
        self.kh, self.vh, self.dk, self.dv, self.dm, self.eps = key_heads, value_heads, key_dim, value_dim, d_model, eps
        self.kd, self.vd = key_heads * key_dim, value_heads * value_dim
        self.cd = 2 * self.kd + self.vd
        self.wtype = wtype
        self.w = {"qkv": (w_qkv, self.cd), "z": (w_z, self.vd), "beta": (w_beta, value_heads),
                  "alpha": (w_alpha, value_heads), "out": (w_out, d_model)}
        self.conv_w, self.a, self.dt, self.norm_w = conv_w, a, dt_bias, norm_w
        dev = conv_w.device
        f = dict(dtype=torch.float32, device=dev)
        self.history = torch.zeros((self.cd, conv_w.shape[1] - 1), **f)      # layer_gdn.cpp:42-44
        self._history_next = torch.empty_like(self.history)   # the fused step writes the new history here
        self.state = torch.zeros((value_heads, key_dim, value_dim), **f)     # layer_gdn.cpp:38
        self.qkv = torch.empty(self.cd, **f)
        self.z = torch.empty(self.vd, **f)
        self.beta_raw = torch.empty(value_heads, **f)
        self.alpha_raw = torch.empty(value_heads, **f)
        self.conv = torch.empty(self.cd, **f)
        self.beta = torch.empty(value_heads, **f)
        self.decay = torch.empty(value_heads, **f)
        self.core = torch.empty(self.vd, **f)
        self.normed = torch.empty(self.vd, **f)

    def _proj(self, name, x, y, K):
        w, M = self.w[name]
        ops.matmul_dispatch(w, self.wtype, M * K, x, M, K, out=y)

    def forward_reference_launches(self, x, out):
        kd = self.kd
        self._proj("qkv", x, self.qkv, self.dm)
        self._proj("z", x, self.z, self.dm)
        self._proj("beta", x, self.beta_raw, self.dm)
        self._proj("alpha", x, self.alpha_raw, self.dm)
        ops.gdn_conv_step(self.qkv, self.conv_w, self.history, y=self.conv)
        ops.gdn_qk_normalize(self.conv[:kd].view(self.kh, self.dk), self.conv[kd:2 * kd].view(self.kh, self.dk),
                             eps=self.eps)
        ops.gdn_gate_values_rows(self.beta_raw, self.alpha_raw, self.a, self.dt, beta=self.beta, decay=self.decay)
        ops.gdn_recurrent_step(self.state, self.conv[:kd], self.conv[kd:2 * kd], self.conv[2 * kd:], self.beta,
                               self.decay, self.kh, self.vh, self.dk, self.dv, out=self.core)
        ops.gdn_norm_gate_rows(self.core.view(self.vh, self.dv), self.z.view(self.vh, self.dv), self.norm_w,
                               out=self.normed.view(self.vh, self.dv), eps=self.eps)
        self._proj("out", self.normed, out, self.vd)
        return out

    def forward(self, x, out):
        jobs = [(self.w[n][0], self.wtype, self.w[n][1] * self.dm, self.w[n][1], 0, y)
                for n, y in (("qkv", self.qkv), ("z", self.z), ("beta", self.beta_raw), ("alpha", self.alpha_raw))]
        ops.matmul_dispatch_multi(jobs, x, self.dm)
        ops.gdn_decode_step(self.qkv, self.conv_w, self.history, self._history_next, self.state, self.beta_raw,
                            self.alpha_raw, self.a, self.dt, self.kh, self.vh, self.dk, self.dv, y=self.conv,
                            out=self.core, eps=self.eps)
        self.history, self._history_next = self._history_next, self.history
        w, M = self.w["out"]
        ops.gdn_norm_gate_matmul(self.core.view(self.vh, self.dv), self.z.view(self.vh, self.dv), self.norm_w, w,
                                 self.wtype, M * self.vd, M, normed=self.normed.view(self.vh, self.dv), out=out,
                                 eps=self.eps)
        return out


    def prefill(self, xs, out=None):
        """xs [T, d_model] -> out [T, d_model]: T tokens of this layer in one pass
        (src/layer_gdn.cpp:78-113 applied token by token in the reference)."""
        T = xs.shape[0]
        f = dict(dtype=torch.float32, device=xs.device)
        out = torch.empty((T, self.dm), **f) if out is None else out
        ws = torch.empty(max(1, ops.matmul_rows_workspace_bytes(T, self.dm), ops.matmul_rows_workspace_bytes(T, self.vd)),
                         dtype=torch.uint8, device=xs.device)
        names = ("qkv", "z", "beta", "alpha")
        outs = ops.matmul_rows_multi([(self.w[n][0], self.wtype, self.w[n][1] * self.dm, self.w[n][1], 0, None)
                                      for n in names], xs, self.dm, workspace=ws)
        proj = dict(zip(names, outs))
        conv = torch.empty((T, self.cd), **f)
        ops.gdn_frontend_rows(proj["qkv"], self.conv_w, self.history, self._history_next, y=conv, k_heads=self.kh,
                              key_dim=self.dk, eps=self.eps)
        self.history, self._history_next = self._history_next, self.history
        beta, decay = torch.empty((T, self.vh), **f), torch.empty((T, self.vh), **f)
        ops.gdn_gate_values_rows(proj["beta"], proj["alpha"], self.a, self.dt, beta=beta, decay=decay)
        core = torch.empty((T, self.vd), **f)
        ops.gdn_recurrent_chunked(self.state, conv, beta, decay, self.kh, self.vh, self.dk, self.dv, out=core)
        normed = torch.empty_like(core)
        ops.gdn_norm_gate_rows(core.view(T, self.vh, self.dv), proj["z"].view(T, self.vh, self.dv), self.norm_w,
                               out=normed.view(T, self.vh, self.dv), eps=self.eps)
        w, M = self.w["out"]
        ops.matmul_rows(w, self.wtype, M * self.vd, normed, M, self.vd, out=out, workspace=ws)
        return out


class AttnLayerDecode:
    """A full-attention layer's decode step (src/layer_attn.cpp:63-111) with its
    KV cache (src/layer_attn.cpp:44-46: max_seq_len rows of kv_heads x head_dim
    floats per cache) and per-token buffers.

    * `forward_reference_launches(x, pos, out)`: the reference's sequence — three
      projections (:85-87), split (:90), two head norms (:91-92), two RoPE calls
      (:95-96), two cache copies (:99-100), scores / softmax / values (:103-105),
      sigmoid gate (:108), output projection (:109): fifteen launches;
    * `forward(x, pos, out)`: the three projections in one `matmul_dispatch_multi`
      whose query | gate output is written already split (q, then the gate) and
      whose K and V outputs are the cache rows at `pos` (no split launch, no cache
      copies), Q/K head norm + partial RoPE folded into the decode
      (`attn_decode_norm_rope`: the bits of `attn_qk_norm_rope_rows`, K normalized
      in place in the cache row, followed by `attn_decode` with its scores,
      softmax, values and sigmoid gate), output projection: three calls.
    """

    def __init__(self, w_qg, w_k, w_v, w_out, q_norm, k_norm, *, wtype="Q4_K", d_model=2048, heads=16, kv_heads=2,
                 head_dim=256, rope_dim=64, theta=1e7, eps=1e-6, max_seq_len=4096):
        self.h, self.kvh, self.hd, self.dm = heads, kv_heads, head_dim, d_model
        self.rope_dim, self.theta, self.eps, self.max_seq_len = rope_dim, theta, eps, max_seq_len
        self.qd, self.kd = heads * head_dim, kv_heads * head_dim
        self.wtype = wtype
        self.w = {"qg": (w_qg, 2 * self.qd), "k": (w_k, self.kd), "v": (w_v, self.kd), "out": (w_out, d_model)}
        self.q_norm, self.k_norm = q_norm, k_norm
        f = dict(dtype=torch.float32, device=q_norm.device)
        self.k_cache = torch.zeros((max_seq_len, self.kd), **f)      # layer_attn.cpp:44-46
        self.v_cache = torch.zeros((max_seq_len, self.kd), **f)
        self.qg = torch.empty(2 * self.qd, **f)
        self.q = torch.empty(self.qd, **f)
        self.gate = torch.empty(self.qd, **f)
        self.k = torch.empty(self.kd, **f)
        self.v = torch.empty(self.kd, **f)
        self.scores = torch.empty(heads * max_seq_len, **f)
        self.attn = torch.empty(self.qd, **f)
        self.gated = torch.empty(self.qd, **f)
        nbytes = max(ops.attn_decode_workspace_bytes(heads, kv_heads, head_dim, p) for p in range(max_seq_len))
        self.workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q_norm.device)

    def _check_pos(self, pos):
        if pos < 0 or pos >= self.max_seq_len:                        # layer_attn.cpp:75-77
            raise ValueError("attention position exceeds configured context")

    def _proj(self, name, x, y, K):
        w, M = self.w[name]
        ops.matmul_dispatch(w, self.wtype, M * K, x, M, K, out=y)

    def forward_reference_launches(self, x, pos, out):
        self._check_pos(pos)
        h, kvh, hd = self.h, self.kvh, self.hd
        self._proj("qg", x, self.qg, self.dm)
        self._proj("k", x, self.k, self.dm)
        self._proj("v", x, self.v, self.dm)
        ops.attn_split_qg(self.qg, h, hd, q=self.q, g=self.gate)
        ops.attn_head_norm(self.q.view(h, hd), self.q_norm, eps=self.eps)
        ops.attn_head_norm(self.k.view(kvh, hd), self.k_norm, eps=self.eps)
        ops.rope_forward(self.q.view(h, hd), pos, self.rope_dim, self.theta)
        ops.rope_forward(self.k.view(kvh, hd), pos, self.rope_dim, self.theta)
        self.k_cache[pos].copy_(self.k)
        self.v_cache[pos].copy_(self.v)
        ops.attn_scores(self.q, self.k_cache, h, kvh, hd, pos, out=self.scores)
        ops.attn_softmax(self.scores, h, pos + 1)
        ops.attn_values(self.scores, self.v_cache, h, kvh, hd, pos, out=self.attn)
        ops.attn_sigmoid_gate(self.attn, self.gate, out=self.gated)
        self._proj("out", self.gated, out, self.qd)
        return out

    def forward(self, x, pos, out):
        self._check_pos(pos)
        h, kvh, hd = self.h, self.kvh, self.hd
        jobs = [(self.w[n][0], self.wtype, self.w[n][1] * self.dm, self.w[n][1], 0, y, s)
                for n, y, s in (("qg", self.qg, hd), ("k", self.k_cache[pos], 0), ("v", self.v_cache[pos], 0))]
        ops.matmul_dispatch_multi(jobs, x, self.dm)        # qg = [q | gate] (the split layout)
        q, gate = self.qg[:self.qd], self.qg[self.qd:]
        ops.attn_decode_norm_rope(q, self.k_cache, self.v_cache, h, kvh, hd, pos, self.q_norm, self.k_norm,
                                  self.rope_dim, self.theta, gate=gate, workspace=self.workspace, q_normed=self.q,
                                  out=self.gated, eps=self.eps)
        self._proj("out", self.gated, out, self.qd)
        return out


class MoeLayerDecode:
    """A MoE layer's decode step (src/layer_moe.cpp:80-159): router, top-k,
    k routed experts (gate, up, SiLU x up, down, weighted add) and the gated
    shared expert.

    * `forward_reference_launches(x, out)`: the reference's sequence — router
      projection and top-k (:95-96), the ids and weights copied to the host with a
      stream synchronisation and checked there (:99-117), a zero fill (:104), five
      launches per routed expert (:120-135), shared expert gate / gate / up
      projections, SiLU x up, down projection, gated add (:138-146) and the copy
      out (:147): 8 + 5k launches and a host round trip;
    * `forward(x, out)`: the router and the shared-expert gate logit in one
      `matmul_dispatch_multi`, then `moe_route_swiglu` (the top-k of the router
      logits, and the k routed experts' and the shared expert's gate and up
      projections with SiLU x up) and `moe_down_combine` (the routed and shared
      down projections and the weighted, gated combine): three launches, no host
      round trip. The host-side routing check is the one part this path leaves
      out (the top-k weights are a softmax, finite and normalised by
      construction; a non-finite router logit makes the output NaN).
    """

    def __init__(self, w_router, w_gate, w_up, w_down, w_sgate, w_sg, w_su, w_sd, *, wtype="Q4_K", d_model=2048,
                 experts=256, k=8, inter=512, shared=2048):
        self.dm, self.E, self.k, self.I, self.S = d_model, experts, k, inter, shared
        self.wtype = wtype
        self.w = {"router": (w_router, experts), "sgate": (w_sgate, 1), "sg": (w_sg, shared), "su": (w_su, shared),
                  "sd": (w_sd, d_model)}
        self.experts_w = {"gate": w_gate, "up": w_up, "down": w_down}
        f = dict(dtype=torch.float32, device=w_router.device)
        self.router = torch.empty(experts, **f)
        self.top_idx = torch.empty(k, dtype=torch.int32, device=w_router.device)
        self.top_w = torch.empty(k, **f)
        # routed rows [k, inter] followed by the shared expert's [shared] row, so one
        # SiLU x up launch covers both
        self.gate_all = torch.empty(k * inter + shared, **f)
        self.up_all = torch.empty(k * inter + shared, **f)
        self.hidden_all = torch.empty(k * inter + shared, **f)
        self.expert_out = torch.empty((k, d_model), **f)
        self.sgate = torch.empty(1, **f)
        self.shared_out = torch.empty(d_model, **f)
        self.accum = torch.empty(d_model, **f)
        self.workspace = torch.empty(max(16, ops.moe_down_combine_workspace_bytes(k, d_model)),
                                     dtype=torch.uint8, device=w_router.device)
        self.ws_swiglu = torch.empty(max(16, ops.moe_expert_swiglu_workspace_bytes(k, inter, shared)),
                                     dtype=torch.uint8, device=w_router.device)
        self.h_idx = torch.empty(k, dtype=torch.int32).pin_memory()
        self.h_w = torch.empty(k, dtype=torch.float32).pin_memory()

    def _proj(self, name, x, y, K):
        w, M = self.w[name]
        ops.matmul_dispatch(w, self.wtype, M * K, x, M, K, out=y)

    def _expert_proj(self, name, e, x, y, M, K):
        ops.matmul_dispatch(self.experts_w[name], self.wtype, self.E * M * K, x, M, K, element_offset=e * M * K, out=y)

    def forward_reference_launches(self, x, out):
        k, I, S, dm = self.k, self.I, self.S, self.dm
        self._proj("router", x, self.router, dm)
        ops.moe_topk_rows(self.router.view(1, self.E), k, idx=self.top_idx.view(1, k), weights=self.top_w.view(1, k))
        self.h_idx.copy_(self.top_idx, non_blocking=True)
        self.h_w.copy_(self.top_w, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        self.accum.zero_()
        ids, wts = self.h_idx.tolist(), self.h_w.tolist()
        if any(e < 0 or e >= self.E or not math.isfinite(w) or w < 0 for e, w in zip(ids, wts)):
            raise RuntimeError("invalid/non-finite MoE routing result")
        if not math.isfinite(sum(wts)) or abs(sum(wts) - 1.0) > 1e-4:
            raise RuntimeError("MoE routing weights are not normalized")
        g, u, hdn = self.gate_all[:I], self.up_all[:I], self.hidden_all[:I]
        for e, wt in zip(ids, wts):
            self._expert_proj("gate", e, x, g, I, dm)
            self._expert_proj("up", e, x, u, I, dm)
            ops.moe_silu_mul(g, u, out=hdn)
            self._expert_proj("down", e, hdn, self.expert_out[0], dm, I)
            ops.moe_add(self.accum, self.expert_out[0], wt)
        self._proj("sgate", x, self.sgate, dm)
        sg, su, sh = self.gate_all[k * I:], self.up_all[k * I:], self.hidden_all[k * I:]
        self._proj("sg", x, sg, dm)
        self._proj("su", x, su, dm)
        ops.moe_silu_mul(sg, su, out=sh)
        self._proj("sd", sh, self.shared_out, S)
        ops.moe_shared_add_rows(self.accum.view(1, dm), self.shared_out.view(1, dm), self.sgate)
        out.copy_(self.accum)
        return out

    def forward(self, x, out):
        k, I, S, dm, E = self.k, self.I, self.S, self.dm, self.E
        jobs = [(self.w[n][0], self.wtype, self.w[n][1] * dm, self.w[n][1], 0, y)
                for n, y in (("router", self.router), ("sgate", self.sgate))]
        ops.matmul_dispatch_multi(jobs, x, dm)
        ops.moe_route_swiglu(self.router, k, self.experts_w["gate"], self.experts_w["up"], self.wtype, E * I * dm,
                             I * dm, x, I, dm, self.w["sg"][0], self.w["su"][0], self.wtype, S * dm, S,
                             idx=self.top_idx, weights=self.top_w, hidden=self.hidden_all[:k * I],
                             shared_hidden=self.hidden_all[k * I:], workspace=self.ws_swiglu)
        ops.moe_down_combine(self.experts_w["down"], self.wtype, E * dm * I, dm * I, E, self.top_idx, self.top_w,
                             self.hidden_all, I, self.w["sd"][0], self.wtype, dm * S, self.hidden_all[k * I:],
                             self.sgate, dm, out=out, workspace=self.workspace)
        return out
