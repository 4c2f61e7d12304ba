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

With gradients (training) and an RMSNorm and a token-choice bf16 layer, the block
runs _BlockTrainFn: kmoe_rmsnorm writes the normalised
rows once (the saved activation the weight gradients need; folding the norm weight
into the expert weights would cost a re-fold of both weight packs every step), the
layer's training forward (MoD-gated when the block has a MoD router and is in
training mode, layers.py:148-177) adds the residual in its combine, and the backward
is the layer's (or the MoD composition's) HIP backward followed by kmoe_rmsnorm_bwd,
which also adds the residual's gradient.

With residual dropout active (training, p > 0) the keep mask is one Bernoulli(1-p)
draw per call (the block's keep_mask_fn) and is applied in the combine, before the
residual add; its backward scales the MoE's output gradient by the same mask.
Other configurations (layernorm, expert choice, fp8) run the unfused composition:
the reference's RMSNorm / LayerNorm in torch, the kmoe MoE layer (MoD-gated in training mode, with its HIP backward where it has one) and a
torch add.  In training mode the MoD router's auxiliary BCE loss (mod.py:114-171) is
added to aux_loss on the fused path as on the unfused one (MoDRouter.aux).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import backward as _bwd
from . import ops
from .mod import MoDRouter, mod_ffn
from .moe import MoELayer, _once


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


def _bernoulli_keep(shape, device, p):
    """Keep mask of nn.Dropout(p): True with probability 1-p (torch's generator)."""
    return torch.empty(shape, device=device, dtype=torch.bool).bernoulli_(1.0 - p)


class MoEFFNBlock(nn.Module):
    """out = h + residual_dropout(MoE(ffn_norm(h))): the FFN half of
    TransformerBlock.forward (layers.py:142-147 pre-norm, 184-191 residual and aux)."""

    def __init__(self, config, layer_idx: int = 0, ffn: MoELayer = None):
        super().__init__()
        self.config = config
        self.ffn_norm = get_norm_layer(config)
        # an existing MoE layer can be wrapped (its parameters are shared, not copied)
        self.ffn = ffn if ffn is not None else MoELayer(config, layer_idx)
        # the MoD router of the FFN (layers.py:84-88), used in training mode only
        self.ffn_mod_router = MoDRouter(config) if getattr(config, "mod_enabled", False) else None
        self.residual_dropout = nn.Dropout(getattr(config, "residual_dropout", 0.1))
        # keep-mask source of the fused paths' residual dropout: (shape, device, p) -> bool
        # tensor, True where kept (replaceable, e.g. by a test that fixes the mask)
        self.keep_mask_fn = _bernoulli_keep
        self.aux_loss = 0.0
        self._fused_cache = None
        # which path the last forward took ("fused" or "unfused")
        self.last_path = None

    def _fusable(self, h: torch.Tensor) -> bool:
        ffn = self.ffn
        if not isinstance(self.ffn_norm, RMSNorm) or ffn.routing_type == "expert_choice":
            return False
        if ffn.grouped_experts.use_fp8 or ffn.router.balanced_routing or not ffn.grouped_experts.gated:
            return False
        if torch.is_grad_enabled() and (h.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        return torch.promote_types(h.dtype, self.ffn_norm.weight.dtype) in (torch.bfloat16, torch.float32)

    def _dropout_keep(self, T, d, device):
        """(keep mask or None, 1/(1-p)) of this forward's residual dropout."""
        p = float(self.residual_dropout.p)
        if not self.training or p <= 0.0:
            return None, 1.0
        if p >= 1.0:
            return torch.zeros(T, d, device=device, dtype=torch.bool), 1.0
        return self.keep_mask_fn((T, d), device, p), 1.0 / (1.0 - p)

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

    def _train_fusable(self, h: torch.Tensor) -> bool:
        """Whether the forward records the fused training backward (_BlockTrainFn)."""
        ffn = self.ffn
        if not torch.is_grad_enabled():
            return False
        params = tuple(self.parameters())
        if not (h.requires_grad or any(p.requires_grad for p in params)):
            return False
        if not isinstance(self.ffn_norm, RMSNorm) or ffn.routing_type == "expert_choice":
            return False
        if not ffn._trainable_experts():
            return False
        return h.dtype in (torch.bfloat16, torch.float32) and self.ffn_norm.weight.dtype in (torch.bfloat16,
                                                                                               torch.float32)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        use_mod = self.ffn_mod_router is not None and self.training
        if self._train_fusable(hidden_states):
            ffn, ge = self.ffn, self.ffn.grouped_experts
            w_mod = self.ffn_mod_router.router.weight if use_mod else None
            out, aux, n, rows = _BlockTrainFn.apply(hidden_states, self.ffn_norm.weight, w_mod,
                                                    ffn.router.router[0].weight, ffn.router.router[2].weight, ge.w1,
                                                    ge.w2, ge.w3, self, use_mod)
            ffn.aux_loss = aux if ffn.training else 0.0
            if use_mod:
                self.ffn_mod_router.aux(n, rows)
            self.last_path = "fused_train"
        elif not use_mod and self._fusable(hidden_states):
            out = self._forward_fused(hidden_states)
            self.last_path = "fused"
        else:
            residual = hidden_states
            xn = self.ffn_norm(hidden_states)
            ffn_output = mod_ffn(self.ffn, self.ffn_mod_router, xn) if use_mod else self.ffn(xn)
            out = residual + self.residual_dropout(ffn_output)
            self.last_path = "unfused"
        self.aux_loss = self.ffn.aux_loss if self.training else 0.0
        if use_mod:
            self.aux_loss = self.aux_loss + self.ffn_mod_router.aux_loss
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
        keep, keep_scale = self._dropout_keep(T, d, h.device)
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k), T, out_dtype=out_dtype,
                        residual=x2d, keep_mask=keep, keep_scale=keep_scale)
        ffn._set_token_choice_aux(r, disp, T)
        return y.view(B, S, d)


class _BlockTrainFn(torch.autograd.Function):
    """out = h + residual_dropout(MoE(RMSNorm(h))) (MoD-gated when use_mod,
    layers.py:142-190) with its backward on the HIP kernels.  Outputs (out, aux)."""

    @staticmethod
    def forward(ctx, h, g, w_mod, w_in, w_out, w1, w2, w3, blk, use_mod):
        B, S, d = h.shape
        T = B * S
        ffn = blk.ffn
        h2d = h.detach().reshape(T, d).contiguous()
        w_mod = blk.ffn_mod_router.router.weight if use_mod else None
        # the norm kernel also writes the MoD logits of the normalised rows
        n, rrms, mod_logits = ops.rmsnorm(h2d, g, blk.ffn_norm.eps, w_mod=w_mod)
        out_dtype = torch.promote_types(h.dtype, g.dtype)
        sel = None
        keep = 0
        kmask, kscale = blk._dropout_keep(T, d, h.device)
        if use_mod:
            sel = blk.ffn_mod_router.select(n.view(B, S, d), logits=mod_logits)
            keep = sel.sel_idx.shape[1]
            x_sel, _ = ops.gather_rows(n, sel.token_rows, B * keep)
            y, aux, sv = ffn._train_forward(x_sel, B * keep, out_dtype, out_map=sel.out_map,
                                            scale=sel.sel_w.reshape(-1), residual=h2d, T_out=T, keep_mask=kmask,
                                            keep_scale=kscale)
        else:
            y, aux, sv = ffn._train_forward(n, T, out_dtype, residual=h2d, keep_mask=kmask, keep_scale=kscale)
        ctx.sv = (sv, sel, h2d, rrms, kmask, kscale)
        ctx.blk = blk
        ctx.meta = (B, S, d, keep, h.dtype, aux is not None, use_mod)
        aux_t = aux if aux is not None else torch.zeros((), device=h.device, dtype=torch.float32)
        # the normalised rows and the kept rows, for the MoD auxiliary router's loss
        rows = sel.token_rows if use_mod else torch.zeros(0, device=h.device, dtype=torch.int32)
        ctx.mark_non_differentiable(n, rows)
        return y.view(B, S, d), aux_t, n, rows

    @staticmethod
    def backward(ctx, dy, daux, dn, drows):
        sv, sel, h2d, rrms, kmask, kscale = _once(ctx)
        blk = ctx.blk
        B, S, d, keep, h_dtype, has_aux, use_mod = ctx.meta
        T = B * S
        ffn, ge = blk.ffn, blk.ffn.grouped_experts
        w_in, w_out = ffn.router.router[0].weight, ffn.router.router[2].weight
        g = blk.ffn_norm.weight
        need_w = any(ctx.needs_input_grad[2:8])
        dy2 = dy.reshape(T, d)
        ga = daux if has_aux else None
        # the MoE output's gradient through the residual dropout; the residual's own
        # gradient (dres below) is dy
        dffn = dy2 if kmask is None else (dy2 * kmask.to(dy2.dtype)) * kscale
        dw_mod = None
        if use_mod:
            w_mod = blk.ffn_mod_router.router.weight
            mg = _bwd.mod_backward(sv, sel, B, keep, dffn, ga, w_out, w_mod, ffn._bwd_weights(), ffn.n_experts,
                                   ge.d_ff, ffn.load_balance_loss_weight, ffn.router_z_loss_weight,
                                   need_weights=need_w)
            dn, lg = mg.dx, mg.layer
            if need_w:
                dw_mod = mg.dw_mod.view_as(w_mod).to(w_mod.dtype)
        else:
            lg = _bwd.moe_backward(sv, dffn, ga, w_out, ffn._bwd_weights(), ffn.n_experts, ge.d_ff,
                                   ffn.load_balance_loss_weight, ffn.router_z_loss_weight, need_weights=need_w)
            dn = lg.dx
        # the norm's backward, plus the residual's gradient dy
        dh, dg = ops.rmsnorm_bwd(dn, h2d, g, rrms, dres=dy2)
        dh = dh.view(B, S, d).to(h_dtype)
        if not need_w:
            return dh, dg, None, None, None, None, None, None, None, None
        return (dh, dg, dw_mod, lg.dw_in.to(w_in.dtype), lg.dw_out.to(w_out.dtype),
                *ge.cast_grads(lg.dw1, lg.dw2, lg.dw3), None, None)
