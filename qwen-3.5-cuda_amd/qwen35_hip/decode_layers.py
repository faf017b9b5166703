"""One Gated DeltaNet layer's decode step composed from the library's entry points.

`GdnLayerDecode` holds a GDN layer's weights and per-layer state as the
reference's GdnLayer does (src/layer_gdn.cpp:37-57: conv history, recurrent
state, per-token buffers) and runs the decode step of its forward
(src/layer_gdn.cpp:78-113) in two ways:

* `forward_reference_launches(x)`: the reference's sequence, one library call per
  reference call — four projections (:83-86), conv step (:89), Q/K normalize
  (:97), gates (:100), recurrent step (:103-106), gated norm (:109), output
  projection (:112): ten launches;
* `forward(x)`: the fused entry points — the four projections in one
  `matmul_dispatch_multi`, conv + SiLU + Q/K L2 in `gdn_frontend_rows`, gates +
  recurrence in `gdn_gated_recurrent_rows`, then the gated norm and the output
  projection: five launches.

Both update the layer's conv history and recurrent state in place. Weights are
GGML tensors (uint8 device tensors of blocks) of one K-quant type.
"""

from __future__ import annotations

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
        ops.gdn_frontend_rows(self.qkv.view(1, self.cd), self.conv_w, self.history, hist_out=self.history,
                              y=self.conv.view(1, self.cd), k_heads=self.kh, key_dim=self.dk, eps=self.eps)
        ops.gdn_gated_recurrent_rows(self.state, self.conv.view(1, self.cd), self.beta_raw.view(1, self.vh),
                                     self.alpha_raw.view(1, self.vh), self.a, self.dt, self.kh, self.vh, self.dk,
                                     self.dv, out=self.core.view(1, self.vd))
        ops.gdn_norm_gate_rows(self.core.view(self.vh, self.dv), self.z.view(self.vh, self.dv), self.norm_w,
                               out=self.normed.view(self.vh, self.dv), eps=self.eps)
        self._proj("out", self.normed, out, self.vd)
        return out
