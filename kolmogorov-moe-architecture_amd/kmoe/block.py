"""The FFN half of the reference's TransformerBlock, with its boundary fused into
the MoE kernels.

TransformerBlock.forward (moe_arch/model/layers.py:142-191) computes, around the
MoE layer,

    residual = h;  out = residual + residual_dropout(ffn(ffn_norm(h)))

with ffn_norm an RMSNorm (embeddings.py:167-195, get_norm_layer at :196-212).
MoEFFNBlock owns the same two submodules (state-dict keys ``ffn_norm.weight`` and
``ffn.*``, as in a TransformerBlock) and, for a token-choice bf16 layer without
gradients, runs the whole expression on the layer's kernels with no extra pass:

* RMSNorm(x) = w_norm * x * r(x), r = 1/sqrt(mean(x^2) + eps).  w_norm is folded
  into the columns of the router's first weight and the rows of w1 / w2 (once per
  parameter version); r is a per-token scale, which commutes with both products:
  the router kernel computes it from the x rows it reads and applies it to its
  hidden pre-activation, the gate/up GEMM applies it to the gate and up values
  before the SiLU.  The normalised activations are never written.
* The residual add happens in the combine (one f32 add before the one rounding).

Other configurations (layernorm, expert choice, fp8, balanced routing, gradients
wanted, active residual dropout) run the unfused composition: the reference's
RMSNorm / LayerNorm in torch, the kmoe MoE layer (with its HIP backward where it
has one) and a torch add.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops
from .moe import MoELayer


class RMSNorm(nn.Module):
    """RMSNorm of moe_arch/model/embeddings.py:167-195: weight * x / sqrt(mean(x^2) + eps)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rms = torch.sqrt(torch.mean(x ** 2, dim=-1, keepdim=True) + self.eps)
        return self.weight * (x / rms)


def get_norm_layer(config) -> nn.Module:
    """Norm layer of the config (embeddings.py:196-212)."""
    norm_type = getattr(config, "norm_type", "rmsnorm")
    eps = getattr(config, "norm_eps", 1e-5)
    if norm_type == "rmsnorm":
        return RMSNorm(config.d_model, eps=eps)
    if norm_type == "layernorm":
        return nn.LayerNorm(config.d_model, eps=eps)
    raise ValueError(f"Unknown norm type: {norm_type}")


class MoEFFNBlock(nn.Module):
    """out = h + residual_dropout(MoE(ffn_norm(h))): the FFN half of
    TransformerBlock.forward (layers.py:142-147 pre-norm, 184-191 residual and aux)."""

    def __init__(self, config, layer_idx: int = 0, ffn: MoELayer = None):
        super().__init__()
        self.config = config
        self.ffn_norm = get_norm_layer(config)
        # an existing MoE layer can be wrapped (its parameters are shared, not copied)
        self.ffn = ffn if ffn is not None else MoELayer(config, layer_idx)
        self.residual_dropout = nn.Dropout(getattr(config, "residual_dropout", 0.1))
        self.aux_loss = 0.0
        self._fused_cache = None
        # which path the last forward took ("fused" or "unfused")
        self.last_path = None

    def _fusable(self, h: torch.Tensor) -> bool:
        ffn = self.ffn
        if not isinstance(self.ffn_norm, RMSNorm) or ffn.routing_type == "expert_choice":
            return False
        if ffn.grouped_experts.use_fp8 or ffn.router.balanced_routing:
            return False
        if self.training and self.residual_dropout.p > 0:
            return False
        if torch.is_grad_enabled() and (h.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        return torch.promote_types(h.dtype, self.ffn_norm.weight.dtype) in (torch.bfloat16, torch.float32)

    def _fused_weights(self):
        """Router w_in and packed w1/w2/w3 with the norm weight folded in (cached per version)."""
        ge = self.ffn.grouped_experts
        w_in, w_out = self.ffn.router.router[0].weight, self.ffn.router.router[2].weight
        g = self.ffn_norm.weight
        key = tuple((t.data_ptr(), t._version, t.device) for t in (g, w_in, w_out, ge.w1, ge.w2, ge.w3))
        if self._fused_cache is None or self._fused_cache[0] != key:
            with torch.no_grad():
                gf = g.detach().float()
                w_in_g = (w_in.detach().float() * gf[None, :]).to(torch.bfloat16).contiguous()
                w_out_b = w_out.detach().to(torch.bfloat16).contiguous()
                # folded in f32, rounded to bf16 once by the pack
                w1g = ge.w1.detach().float() * gf[None, :, None]
                w2g = ge.w2.detach().float() * gf[None, :, None]
                pw = ops.pack_weights(w1g, w2g, ge.w3.detach(), fp8=False)
                del w1g, w2g
            self._fused_cache = (key, w_in_g, w_out_b, pw)
        return self._fused_cache[1:]

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if self._fusable(hidden_states):
            out = self._forward_fused(hidden_states)
            self.last_path = "fused"
        else:
            residual = hidden_states
            ffn_output = self.residual_dropout(self.ffn(self.ffn_norm(hidden_states)))
            out = residual + ffn_output
            self.last_path = "unfused"
        self.aux_loss = self.ffn.aux_loss if self.training else 0.0
        return out

    def _forward_fused(self, h: torch.Tensor) -> torch.Tensor:
        ffn = self.ffn
        B, S, d = h.shape
        T, k, E = B * S, ffn.top_k, ffn.n_experts
        out_dtype = torch.promote_types(h.dtype, self.ffn_norm.weight.dtype)
        x2d = h.reshape(T, d)
        xb = x2d.to(torch.bfloat16).contiguous()
        w_in_g, w_out, pw = self._fused_weights()
        router = ffn.router
        bias = None
        if router.logit_bias is not None:
            if router.logit_bias.device != h.device:
                router.logit_bias = router.logit_bias.to(h.device)
            bias = router.logit_bias
        r = ops.router(xb, w_in_g, w_out, k, bias=bias, rms_eps=self.ffn_norm.eps)
        cap = ops.capacity_of(ffn.capacity_factor, T, k, E) if ffn.drop_overflow else 0
        disp = ops.dispatch(xb, r.idx, r.w, E, capacity=cap, materialize=False)
        hbuf = ops.gemm_gate_up_rows(xb, None, disp.row_token, disp.offsets, pw, T * k, rscale=r.rscale)
        yperm = ops.gemm_down(hbuf, None, disp.offsets, pw, T * k)
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k), T, out_dtype=out_dtype,
                        residual=x2d)
        ffn._set_token_choice_aux(r, disp, T)
        return y.view(B, S, d)
