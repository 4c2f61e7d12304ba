"""Mixture-of-Depths token selection around the MoE layer.

MoDRouter mirrors moe_arch/model/mod.py:18-122 (same parameters: ``router``
Linear(d,1) and the unused-here ``aux_router`` MLP).  MoDMoE is the FFN half of
TransformerBlock.forward with MoD in training mode (layers.py:148-185):
select the top ``int(S*cf)`` tokens per sequence, run the MoE on them, weight
by the softmax over the kept router logits and scatter back, zeros elsewhere.
Without gradients the gather is fused into the router/dispatch reads (row
indirection) and the weighted scatter into the combine, so no (B,k,d) copy is
materialised.  With gradients (mod_ffn's training function) the kept rows are
gathered once (they are the saved activation of the router's and the experts'
weight gradients), the weighted scatter stays in the combine, and the backward
runs on the HIP kernels: the combine backward reads dy at the kept rows and
yields the MoD weights' gradient, kmoe_mod_bwd the kept logits' and W_mod's,
and one gather writes the input gradient of every token.
In training the MoD router's auxiliary loss (mod.py:114-171: an MLP on the detached
input predicting the selection, binary cross-entropy) runs on the router MLP kernels.
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from . import _lib
from . import backward as _bwd
from . import ops
from .config import AdvancedMoEConfig
from .moe import MoELayer, _forward_only, _once


class MoDRouter(nn.Module):
    def __init__(self, config: AdvancedMoEConfig):
        super().__init__()
        self.config = config
        self.d_model = config.d_model
        self.capacity_factor = config.mod_capacity_factor
        self.router = nn.Linear(config.d_model, 1, bias=False)
        aux_hidden = getattr(config, "mod_router_hidden_dim", 128)
        self.aux_router = nn.Sequential(
            nn.Linear(config.d_model, aux_hidden, bias=False),
            nn.SiLU(),
            nn.Linear(aux_hidden, 1, bias=False),
        )
        self.aux_loss_weight = config.mod_load_balance_loss_weight
        self.aux_loss = 0.0

    def aux(self, x2d: torch.Tensor, token_rows: torch.Tensor):
        """Sets and returns aux_loss for the selection token_rows (the kept rows of the
        flattened input x2d): in training the auxiliary router's loss (mod.py:114-118,
        141-171), else 0.0."""
        if not self.training:
            self.aux_loss = 0.0
            return self.aux_loss
        w_a, w_b = self.aux_router[0].weight, self.aux_router[2].weight
        if w_a.shape[0] != _lib.ROUTER_HIDDEN:
            raise NotImplementedError(f"kmoe: the MoD auxiliary router runs on the router kernels, hidden size "
                                      f"{_lib.ROUTER_HIDDEN} (mod_router_hidden_dim={w_a.shape[0]})")
        weight = float(self.aux_loss_weight)
        if torch.is_grad_enabled() and (w_a.requires_grad or w_b.requires_grad):
            self.aux_loss = _ModAuxFn.apply(x2d.detach(), w_a, w_b, token_rows, weight)
            return self.aux_loss
        # forward only: the same kernels without an autograd record, in order on the
        # caller's stream
        self.aux_loss = ops.mod_aux_bce(ops.router(x2d.detach(), w_a, w_b, 0, partials=False, stage="mod_aux_router").logits,
                                        token_rows, weight)
        return self.aux_loss

    def keep_count(self, seq_len: int) -> int:
        return max(1, min(seq_len, int(seq_len * self.capacity_factor)))  # mod.py:97

    def select(self, hidden_states: torch.Tensor, logits: torch.Tensor = None) -> ops.ModSelectOut:
        """The selection of mod.py:93-112; `logits` ((B, S) f32) when already computed
        (the block's RMSNorm kernel writes them)."""
        B, S, _ = hidden_states.shape
        w = self.router.weight.detach()
        return ops.mod_select(hidden_states, w, self.keep_count(S), logits=logits)

    def forward(self, hidden_states: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        """(sorted_indices, router_weights, router_logits, topk_indices) as mod.py:122.

        topk_indices is returned in ascending order (the same set as the reference's
        unsorted top-k)."""
        sel = self.select(hidden_states)
        B, S, d = hidden_states.shape
        self.aux(hidden_states.reshape(B * S, d), sel.token_rows)
        dt = hidden_states.dtype
        return sel.sel_idx, sel.sel_w.to(dt), sel.logits.to(dt), sel.sel_idx


class _ModAuxFn(torch.autograd.Function):
    """weight * mean over the B*S tokens of BCE-with-logits(aux_router(x), selected)
    (mod.py:141-171) with aux_router = Linear(d, 128), SiLU, Linear(128, 1): the router
    MLP kernel with one output, then kmoe_mod_aux_bce.  x enters detached (mod.py:155),
    so only the two weights get gradients, from the router MLP backward kernels with
    dl = weight (sigmoid(l) - t) / T."""

    @staticmethod
    def forward(ctx, x2d, w_a, w_b, token_rows, weight):
        T = x2d.shape[0]
        r = ops.router(x2d, w_a, w_b, 0, save_hidden=True, partials=False, stage="mod_aux_router")
        ctx.save_for_backward(x2d, r.hidden, r.logits, token_rows)
        ctx.w_b = w_b
        ctx.dtypes = (w_a.dtype, w_b.dtype)
        ctx.weight = weight
        return ops.mod_aux_bce(r.logits, token_rows, weight)

    @staticmethod
    def backward(ctx, g):
        x2d, hidden, lg, token_rows = ctx.saved_tensors
        T = x2d.shape[0]
        t = torch.zeros(T, 1, device=x2d.device, dtype=torch.float32)
        t[token_rows.long()] = 1.0
        dl = ((g.float() * (ctx.weight / T)) * (torch.sigmoid(lg) - t)).contiguous()
        dw_a, dw_b = _bwd.router_weight_grads(x2d, hidden, ctx.w_b, dl)
        del ctx.w_b
        return None, dw_a.to(ctx.dtypes[0]), dw_b.to(ctx.dtypes[1]), None, None


class _MoDTrainFn(torch.autograd.Function):
    """ffn_output (+ residual) of layers.py:148-187 for a normalised input x, with its
    backward on the HIP kernels (mod_backward).  Outputs (y, aux)."""

    @staticmethod
    def forward(ctx, x, residual, w_mod, w_in, w_out, w1, w2, w3, ffn, mod_router, xb, sel):
        B, S, d = x.shape
        keep = sel.sel_idx.shape[1]
        T = B * keep
        x_sel, _ = ops.gather_rows(xb.view(B * S, d), sel.token_rows, T)
        out_dtype = torch.float32 if x.dtype == torch.float32 else torch.bfloat16
        res2d = None if residual is None else residual.detach().reshape(B * S, d)
        y, aux, sv = ffn._train_forward(x_sel, T, out_dtype, out_map=sel.out_map, scale=sel.sel_w.reshape(-1),
                                        residual=res2d, T_out=B * S)
        ctx.sv = (sv, sel)
        ctx.mods = (ffn, mod_router)
        ctx.meta = (B, S, d, keep, x.dtype, None if residual is None else residual.dtype, aux is not None)
        aux_t = aux if aux is not None else torch.zeros((), device=x.device, dtype=torch.float32)
        return y.view(B, S, d).to(x.dtype), aux_t

    @staticmethod
    def backward(ctx, dy, daux):
        sv, sel = _once(ctx)
        ffn, mod_router = ctx.mods
        B, S, d, keep, x_dtype, r_dtype, has_aux = ctx.meta
        ge = ffn.grouped_experts
        w_in, w_out = ffn.router.router[0].weight, ffn.router.router[2].weight
        w_mod = mod_router.router.weight
        need_w = any(ctx.needs_input_grad[2:8])
        g = _bwd.mod_backward(sv, sel, B, keep, dy.reshape(B * S, d), daux if has_aux else None, w_out, w_mod,
                              ffn._bwd_weights(), ffn.n_experts, ge.d_ff, ffn.load_balance_loss_weight,
                              ffn.router_z_loss_weight, need_weights=need_w)
        dx = g.dx.view(B, S, d).to(x_dtype)
        dres = None if r_dtype is None else dy.to(r_dtype)
        if not need_w:
            return dx, dres, None, None, None, None, None, None, None, None, None, None
        lg = g.layer
        return (dx, dres, g.dw_mod.view_as(w_mod).to(w_mod.dtype), lg.dw_in.to(w_in.dtype), lg.dw_out.to(w_out.dtype),
                *ge.cast_grads(lg.dw1, lg.dw2, lg.dw3), None, None, None, None)


def mod_trainable(ffn: MoELayer, mod_router: MoDRouter, *inputs) -> bool:
    """Whether the MoD composition records a backward through the HIP kernels."""
    if not torch.is_grad_enabled():
        return False
    params = tuple(ffn.parameters()) + (mod_router.router.weight,)
    if not any(isinstance(t, torch.Tensor) and t.requires_grad for t in inputs + params):
        return False
    return ffn.routing_type != "expert_choice" and ffn._trainable_experts()


def mod_ffn(ffn: MoELayer, mod_router: MoDRouter, hidden_states: torch.Tensor,
            residual: torch.Tensor = None) -> torch.Tensor:
    """ffn_output of layers.py:148-177 for the normalised input (residual + it with
    `residual`), setting ffn.aux_loss; trains through the HIP backward when gradients
    are wanted."""
    return _mod_ffn(ffn, mod_router, hidden_states, residual)


def _mod_ffn(ffn: MoELayer, mod_router: MoDRouter, hidden_states: torch.Tensor,
             residual: torch.Tensor = None) -> torch.Tensor:
    B, S, d = hidden_states.shape
    x = hidden_states.detach().to(torch.bfloat16).contiguous()
    sel = mod_router.select(x)
    mod_router.aux(x.view(B * S, d), sel.token_rows)
    if ffn.routing_type == "expert_choice":
        return _mod_expert_choice(ffn, mod_router, hidden_states, residual, sel)
    if mod_trainable(ffn, mod_router, hidden_states, residual):
        ge = ffn.grouped_experts
        y, aux = _MoDTrainFn.apply(hidden_states, residual, mod_router.router.weight, ffn.router.router[0].weight,
                                   ffn.router.router[2].weight, ge.w1, ge.w2, ge.w3, ffn, mod_router, x, sel)
        ffn.aux_loss = aux if ffn.training else 0.0
        return y
    keep = sel.sel_idx.shape[1]
    out_dtype = torch.float32 if hidden_states.dtype == torch.float32 else torch.bfloat16
    res2d = None if residual is None else residual.reshape(B * S, d)
    y, r, disp = ffn.forward_rows(x.reshape(B * S, d), T=B * keep, row_index=sel.token_rows, T_out=B * S,
                                  out_map=sel.out_map, scale=sel.sel_w.reshape(-1), out_dtype=out_dtype,
                                  residual=res2d)
    ffn._set_token_choice_aux(r, disp, B * keep)
    ins = (hidden_states,) if residual is None else (hidden_states, residual)
    return _forward_only(y.view(B, S, d).to(hidden_states.dtype), *ins, *ffn.parameters(),
                         *mod_router.parameters())


def _mod_expert_choice(ffn: MoELayer, mod_router: MoDRouter, hidden_states: torch.Tensor,
                       residual: torch.Tensor, sel: ops.ModSelectOut) -> torch.Tensor:
    """MoD around an expert-choice MoELayer (layers.py:148-187 with moe_routing
    "expert_choice"): at the MoD selection sel, the kept rows (B, keep, d) through
    the expert-choice layer (its capacity from the kept length, moe.py:494-530; it trains
    through its own HIP backward and sets ffn.aux_loss), then the rows weighted by the
    softmax over the kept logits (mod.py:112) and scattered back (layers.py:175-184).
    The expert-choice combine sums each token's rows from its own fan-in tables, so the
    gather, the kept logits' softmax and the weighted scatter around it are tensor ops
    on the GPU, differentiable: autograd takes the gradients of x, the residual and
    w_mod through them."""
    B, S, d = hidden_states.shape
    x = hidden_states
    gidx = sel.sel_idx.long().unsqueeze(-1).expand(-1, -1, d)
    xs = torch.gather(x, 1, gidx)
    ys = ffn(xs)
    w_mod = mod_router.router.weight
    p = torch.softmax((xs.float() @ w_mod.float().t()).squeeze(-1), dim=-1)
    out = torch.zeros(B, S, d, device=x.device, dtype=torch.float32).scatter_add(1, gidx,
                                                                                 p.unsqueeze(-1) * ys.float())
    if residual is not None:
        out = out + residual.float()
    return out.to(x.dtype)


class MoDMoE(nn.Module):
    """MoD-gated MoE FFN: ffn_output of layers.py:148-185 for a normalised input."""

    def __init__(self, config: AdvancedMoEConfig, layer_idx: int = 0):
        super().__init__()
        self.ffn_mod_router = MoDRouter(config)
        self.ffn = MoELayer(config, layer_idx)
        self.aux_loss = 0.0

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor = None) -> torch.Tensor:
        """ffn_output; with `residual` (B, S, d), residual + ffn_output (layers.py:187) from the same
        combine: unselected tokens get the residual row, selected ones residual + weighted output."""
        y = mod_ffn(self.ffn, self.ffn_mod_router, hidden_states, residual)
        self.aux_loss = self.ffn.aux_loss + self.ffn_mod_router.aux_loss
        return y
