"""Mixture-of-Depths token selection around the MoE layer.

MoDRouter mirrors moe_arch/model/mod.py:18-122 (same parameters: ``router``
Linear(d,1) and the unused-here ``aux_router`` MLP).  MoDMoE is the FFN half of
TransformerBlock.forward with MoD in training mode (layers.py:148-185):
select the top ``int(S*cf)`` tokens per sequence, run the MoE on them, weight
by the softmax over the kept router logits and scatter back, zeros elsewhere.
Here the gather is fused into the router/dispatch reads (row indirection) and
the weighted scatter into the combine, so no (B,k,d) copy is materialised.
The MoD auxiliary BCE loss is out of scope.
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from . import ops
from .config import AdvancedMoEConfig
from .moe import MoELayer, _forward_only


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
        self.aux_loss = 0.0

    def keep_count(self, seq_len: int) -> int:
        return max(1, min(seq_len, int(seq_len * self.capacity_factor)))  # mod.py:97

    def select(self, hidden_states: torch.Tensor) -> ops.ModSelectOut:
        B, S, _ = hidden_states.shape
        w = self.router.weight.detach()
        return ops.mod_select(hidden_states, w, self.keep_count(S))

    def forward(self, hidden_states: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        """(sorted_indices, router_weights, router_logits, topk_indices) as mod.py:122.

        topk_indices is returned in ascending order (the same set as the reference's
        unsorted top-k)."""
        sel = self.select(hidden_states)
        dt = hidden_states.dtype
        return sel.sel_idx, sel.sel_w.to(dt), sel.logits.to(dt), sel.sel_idx


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
        B, S, d = hidden_states.shape
        x = hidden_states if hidden_states.dtype == torch.bfloat16 else hidden_states.to(torch.bfloat16)
        sel = self.ffn_mod_router.select(x)
        keep = sel.sel_idx.shape[1]
        out_dtype = torch.float32 if hidden_states.dtype == torch.float32 else torch.bfloat16
        res2d = None if residual is None else residual.reshape(B * S, d)
        y, r, disp = self.ffn.forward_rows(x.reshape(B * S, d), T=B * keep, row_index=sel.token_rows,
                                           T_out=B * S, out_map=sel.out_map, scale=sel.sel_w.reshape(-1),
                                           out_dtype=out_dtype, residual=res2d)
        self.ffn._set_token_choice_aux(r, disp, B * keep)
        self.aux_loss = self.ffn.aux_loss
        ins = (hidden_states,) if residual is None else (hidden_states, residual)
        return _forward_only(y.view(B, S, d).to(hidden_states.dtype), *ins, *self.parameters())
