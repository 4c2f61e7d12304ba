"""Drop-in MoE modules with the reference's Python API, running on the HIP kernels.

Same constructor signatures, attribute names, parameter names/shapes and
return contracts as moe_arch/model/moe.py:
  Router                      moe.py:327-462   (router(h) -> (w, idx, logits))
  ExpertChoiceRouter          moe.py:465-530   (router(h) -> (w, idx, logits, C))
  GroupedExperts              moe.py:161-294   (forward(x, idx, w) -> y)
  GroupedExpertsExpertChoice  moe.py:533-673   (forward(x, w, idx) -> y)
  MoELayer                    moe.py:676-950   (forward(h) -> y, sets .aux_loss)

Numerics: the router accumulates in fp32 and ranks experts by fp32 logit
(equal logits -> lowest expert index); expert GEMMs run bf16 (or fp8 e4m3)
MFMA with fp32 accumulation; the combine accumulates in fp32 in a fixed order.
Backward: the token-choice bf16 layer (MoELayer with top-k routing, optional
capacity drop) trains through the HIP backward kernels (kmoe.backward); the
other paths (expert choice, fp8, balanced routing, MoD, GroupedExperts called
directly) are forward-only and raise in backward.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import backward as _bwd
from . import ops
from .config import AdvancedMoEConfig

ROUTER_HIDDEN = 128  # moe.py:346


class _ForwardOnly(torch.autograd.Function):
    """Marks kernel outputs so that a backward through them fails loudly."""

    @staticmethod
    def forward(ctx, y, *inputs):
        return y

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("kmoe: the MoE backward pass is not implemented (forward-only kernels)")


def _forward_only(y, *inputs):
    needs = torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in inputs)
    return _ForwardOnly.apply(y, *inputs) if needs else y


def _init_expert_weights(*ws):
    """Per-expert kaiming-uniform bound 1/sqrt(fan_in) (moe.py:194-211)."""
    for w in ws:
        if w is not None:
            fan_in = w.shape[1]
            bound = math.sqrt(3.0) * math.sqrt(1.0 / 3.0) / math.sqrt(fan_in)
            nn.init.uniform_(w, -bound, bound)


class _RouterMLP(nn.Module):
    """d -> 128 -> E MLP shared by both routers; param names router.0/2.weight."""

    def __init__(self, d_model: int, n_experts: int):
        super().__init__()
        self.router = nn.Sequential(
            nn.Linear(d_model, ROUTER_HIDDEN, bias=False),
            nn.SiLU(),
            nn.Linear(ROUTER_HIDDEN, n_experts, bias=False),
        )
        self._bf16_cache = None

    def _kernel_weights(self):
        w_in, w_out = self.router[0].weight, self.router[2].weight
        if w_in.dtype == torch.bfloat16:
            return w_in.detach(), w_out.detach()
        key = (w_in.data_ptr(), w_in._version, w_out.data_ptr(), w_out._version)
        if self._bf16_cache is None or self._bf16_cache[0] != key:
            self._bf16_cache = (key, w_in.detach().to(torch.bfloat16).contiguous(),
                                w_out.detach().to(torch.bfloat16).contiguous())
        return self._bf16_cache[1], self._bf16_cache[2]


class Router(_RouterMLP):
    """Token-choice top-k router (moe.py:327-462)."""

    def __init__(self, config: AdvancedMoEConfig):
        super().__init__(config.d_model, config.n_experts)
        self.d_model = config.d_model
        self.n_experts = config.n_experts
        self.top_k = config.moe_top_k
        self.balanced_routing = getattr(config, "moe_balanced_routing", False)
        bias = getattr(config, "moe_router_bias", None)
        # fp32 per-expert logit bias (kept out of the state dict and of dtype casts)
        self.logit_bias = None if bias is None else torch.tensor(list(bias), dtype=torch.float32)

    def route(self, x2d: torch.Tensor, row_index: Optional[torch.Tensor] = None,
              T: Optional[int] = None, save_hidden: bool = False) -> ops.RouterOut:
        """Kernel-level routing of flattened tokens: fp32 logits, int64 idx, f32 weights.
        With moe_balanced_routing the picks are the capacity-balanced assignment
        (moe.py:443-451) over all the tokens of the call."""
        w_in, w_out = self._kernel_weights()
        bias = None
        if self.logit_bias is not None:
            if self.logit_bias.device != x2d.device:
                self.logit_bias = self.logit_bias.to(x2d.device)
            bias = self.logit_bias
        if self.balanced_routing:
            if save_hidden:
                raise NotImplementedError("kmoe: backward through balanced routing is not implemented")
            r = ops.router(x2d, w_in, w_out, 0, bias=bias, row_index=row_index, T=T)
            idx, w = ops.balanced_topk(r.logits, self.top_k)
            return ops.RouterOut(r.logits, idx, w, r.partials)
        return ops.router(x2d, w_in, w_out, self.top_k, bias=bias, row_index=row_index, T=T, save_hidden=save_hidden)

    def forward(self, hidden_states: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        B, S, d = hidden_states.shape
        r = self.route(hidden_states.reshape(B * S, d))
        dt = hidden_states.dtype
        return (r.w.view(B, S, self.top_k).to(dt), r.idx.view(B, S, self.top_k),
                r.logits.view(B, S, self.n_experts).to(dt))


class ExpertChoiceRouter(_RouterMLP):
    """Expert-choice router (moe.py:465-530)."""

    def __init__(self, config: AdvancedMoEConfig):
        super().__init__(config.d_model, config.n_experts)
        self.d_model = config.d_model
        self.n_experts = config.n_experts
        self.capacity_factor = config.moe_capacity_factor

    def capacity(self, seq_len: int) -> int:
        return int(math.ceil(seq_len * self.capacity_factor / self.n_experts))  # moe.py:511

    def route(self, hidden_states: torch.Tensor, descending: bool = True):
        B, S, d = hidden_states.shape
        C = min(self.capacity(S), S)
        w_in, w_out = self._kernel_weights()
        r = ops.router(hidden_states.reshape(B * S, d), w_in, w_out, 0)
        sel = ops.ec_select(r.logits, B, S, self.n_experts, C, descending=descending)
        return r, sel, C

    def forward(self, hidden_states: torch.Tensor):
        B, S, _ = hidden_states.shape
        r, sel, C = self.route(hidden_states)
        dt = hidden_states.dtype
        return sel.w.to(dt), sel.idx, r.logits.view(B, S, self.n_experts).to(dt), C


class _PackedExperts(nn.Module):
    """Holds w1,w2 (E,d,F), w3 (E,F,d) and their packed kernel layout (derived cache)."""

    def __init__(self, n_experts: int, d_model: int, d_ff: int, activation: str = "swiglu"):
        super().__init__()
        if activation != "swiglu":
            raise NotImplementedError(f"kmoe: expert activation {activation!r} (only swiglu is implemented)")
        self.n_experts = n_experts
        self.d_model = d_model
        self.d_ff = d_ff
        self.activation = activation
        self.w1 = nn.Parameter(torch.empty(n_experts, d_model, d_ff))
        self.w2 = nn.Parameter(torch.empty(n_experts, d_model, d_ff))
        self.w3 = nn.Parameter(torch.empty(n_experts, d_ff, d_model))
        _init_expert_weights(self.w1, self.w2, self.w3)
        self._packed = None
        self.use_fp8 = False

    def _packed_key(self):
        return tuple((w.data_ptr(), w._version, w.device) for w in (self.w1, self.w2, self.w3)) + (self.use_fp8,)

    def install_packed(self, pw: ops.PackedWeights) -> None:
        """Use `pw` (packed from exactly the current w1/w2/w3, e.g. read back from disk)
        until a parameter changes."""
        if (pw.E, pw.d, pw.F, pw.fp8) != (self.n_experts, self.d_model, self.d_ff, self.use_fp8):
            raise ValueError("kmoe: packed weights do not match the experts' shapes / fp8 mode")
        self._packed = (self._packed_key(), pw)

    def packed(self) -> ops.PackedWeights:
        """Packed weights, rebuilt only when a parameter changed (version counters)."""
        key = self._packed_key()
        if self._packed is None or self._packed[0] != key:
            with torch.no_grad():
                pw = ops.pack_weights(self.w1.detach(), self.w2.detach(), self.w3.detach(), fp8=self.use_fp8)
            self._packed = (key, pw)
        return self._packed[1]


class GroupedExperts(_PackedExperts):
    """Token-choice grouped SwiGLU experts (moe.py:161-294)."""

    def run(self, x2d, expert_indices, expert_weights, row_index=None, T_out=None, out_map=None, scale=None,
            out_dtype=torch.bfloat16, residual=None, capacity=0, block_counts=None):
        """dispatch -> grouped GEMMs -> combine (+ residual, added in the combine); returns (y, DispatchOut).
        capacity > 0 drops each expert's assignments past the first `capacity` (MoELayer's
        drop_overflow rule); 0, the default and what forward() uses, drops nothing (the
        reference's GroupedExperts never drops).  block_counts: the router's per-block
        histograms of expert_indices (RouterOut.block_counts), if it wrote them."""
        E = self.n_experts
        pw = self.packed()
        T, k = expert_indices.shape
        if pw.fp8:
            disp = ops.dispatch(x2d, expert_indices, expert_weights, E, capacity=capacity, fp8=True,
                                row_index=row_index, block_counts=block_counts)
            yperm = ops.grouped_ffn(disp.xperm, disp.xscale, disp.offsets, pw, T * k)
        else:
            # bf16: the gate/up GEMM gathers the token rows itself (no permuted copy of x)
            disp = ops.dispatch(x2d, expert_indices, expert_weights, E, capacity=capacity,
                                row_index=row_index, materialize=False, block_counts=block_counts)
            h = ops.gemm_gate_up_rows(x2d, row_index, disp.row_token, disp.offsets, pw, T * k)
            yperm = ops.gemm_down(h, None, disp.offsets, pw, T * k)
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k),
                        T if T_out is None else T_out, out_map=out_map, scale=scale, out_dtype=out_dtype,
                        residual=residual)
        return y, disp

    def forward(self, x: torch.Tensor, expert_indices: torch.Tensor, expert_weights: torch.Tensor) -> torch.Tensor:
        out_dtype = torch.float32 if x.dtype == torch.float32 else torch.bfloat16
        y, _ = self.run(x, expert_indices, expert_weights, out_dtype=out_dtype)
        return _forward_only(y.to(x.dtype), x, self.w1, self.w2, self.w3, expert_weights)


class GroupedExpertsExpertChoice(_PackedExperts):
    """Expert-choice grouped experts (moe.py:533-673)."""

    def run(self, x2d, sel: ops.ECSelectOut, B, S, C, out_dtype=torch.bfloat16):
        pw = self.packed()
        n_rows = self.n_experts * B * C
        xperm, xscale = ops.gather_rows(x2d, sel.row_token, n_rows, fp8=pw.fp8)
        yperm = ops.grouped_ffn(xperm, xscale, sel.offsets, pw, n_rows)
        return ops.combine(yperm, sel.src_row, sel.src_w, B * S, out_dtype=out_dtype)

    def forward(self, x: torch.Tensor, expert_weights: torch.Tensor, token_indices: torch.Tensor) -> torch.Tensor:
        B, S, d = x.shape
        _, E, C = token_indices.shape
        # Tables from caller-provided indices (host-built; the fused path uses ec_select's tables).
        dev = x.device
        b_idx = torch.arange(B, device=dev).view(B, 1, 1)
        e_idx = torch.arange(E, device=dev).view(1, E, 1)
        c_idx = torch.arange(C, device=dev).view(1, 1, C)
        rows = (e_idx * (B * C) + b_idx * C + c_idx).reshape(-1)
        toks = (b_idx * S + token_indices).reshape(-1)
        row_token = torch.empty(E * B * C, device=dev, dtype=torch.int32)
        row_token[rows] = toks.to(torch.int32)
        src_row = torch.full((B * S, E), -1, device=dev, dtype=torch.int32)
        src_w = torch.zeros(B * S, E, device=dev, dtype=torch.float32)
        ee = e_idx.expand(B, E, C).reshape(-1)
        src_row[toks, ee] = rows.to(torch.int32)
        src_w[toks, ee] = expert_weights.reshape(-1).float()
        offsets = (torch.arange(E + 1, device=dev, dtype=torch.int32) * (B * C))
        sel = ops.ECSelectOut(token_indices, expert_weights, row_token, offsets, src_row, src_w)
        out_dtype = torch.float32 if x.dtype == torch.float32 else torch.bfloat16
        y = self.run(x.reshape(B * S, d), sel, B, S, C, out_dtype=out_dtype)
        return _forward_only(y.view(B, S, d).to(x.dtype), x, self.w1, self.w2, self.w3, expert_weights)


class _MoETrainFn(torch.autograd.Function):
    """Token-choice MoE layer whose backward runs on the HIP backward kernels.

    Inputs are the layer input and the parameters (so autograd routes their
    gradients); outputs are y and the aux loss (a 0-dim tensor, 0 in eval)."""

    @staticmethod
    def forward(ctx, x, w_in, w_out, w1, w2, w3, layer):
        B, S, d = x.shape
        T = B * S
        x2d = x.reshape(T, d).to(torch.bfloat16).contiguous()
        y2d, aux, sv = layer._train_forward(x2d, T, layer._out_dtype(x))
        ctx.layer = layer
        ctx.sv = sv
        ctx.meta = (B, S, d, x.dtype, aux is not None)
        aux_t = aux if aux is not None else torch.zeros((), device=x.device, dtype=torch.float32)
        return y2d.view(B, S, d).to(x.dtype), aux_t

    @staticmethod
    def backward(ctx, dy, daux):
        if ctx.sv is None:
            raise RuntimeError("kmoe: backward through the MoE layer can run once per forward; "
                               "retain_graph=True with a second backward is not supported")
        B, S, d, x_dtype, has_aux = ctx.meta
        layer = ctx.layer
        ge = layer.grouped_experts
        w_in, w_out = layer.router.router[0].weight, layer.router.router[2].weight
        need_w = any(ctx.needs_input_grad[1:6])
        g = _bwd.moe_backward(ctx.sv, dy, daux if has_aux else None, w_out, layer._bwd_weights(), layer.n_experts,
                              ge.d_ff, layer.load_balance_loss_weight, layer.router_z_loss_weight, need_weights=need_w)
        ctx.sv = None
        dx = g.dx.view(B, S, d).to(x_dtype)
        if not need_w:
            return dx, None, None, None, None, None, None
        return (dx, g.dw_in.to(w_in.dtype), g.dw_out.to(w_out.dtype), g.dw1.to(ge.w1.dtype), g.dw2.to(ge.w2.dtype),
                g.dw3.to(ge.w3.dtype), None)


class MoELayer(nn.Module):
    """MoE feed-forward layer (moe.py:676-950) on the HIP kernels."""

    def __init__(self, config: AdvancedMoEConfig, layer_idx: int = 0, process_group=None):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.n_experts = config.n_experts
        self.top_k = config.moe_top_k
        self.capacity_factor = config.moe_capacity_factor
        self.routing_type = getattr(config, "moe_routing", "token_choice")
        self.implementation = getattr(config, "moe_implementation", "batched")
        if self.implementation == "expert_parallel" or process_group is not None:
            raise NotImplementedError("kmoe: expert-parallel MoE is out of scope (single-GPU build)")
        self._use_expert_parallel = False
        self.expert_parallel_layer = None
        self.drop_overflow = bool(getattr(config, "moe_drop_overflow", False))
        use_fp8 = bool(getattr(config, "moe_fp8", False))
        if self.routing_type == "expert_choice":
            self.router = ExpertChoiceRouter(config)
            self.grouped_experts = None
            self.grouped_experts_ec = GroupedExpertsExpertChoice(config.n_experts, config.d_model,
                                                                 config.d_ff_expert, config.ffn_activation)
            self.grouped_experts_ec.use_fp8 = use_fp8
        else:
            self.router = Router(config)
            self.grouped_experts_ec = None
            self.grouped_experts = GroupedExperts(config.n_experts, config.d_model, config.d_ff_expert,
                                                 config.ffn_activation)
            self.grouped_experts.use_fp8 = use_fp8
        self.experts = None
        self.load_balance_loss_weight = config.moe_load_balance_loss_weight
        self.router_z_loss_weight = config.moe_router_z_loss_weight
        self.aux_loss = 0.0
        # last forward's router statistics (per-expert routed counts, int32)
        self.last_expert_counts: Optional[torch.Tensor] = None

    # ---------------------------------------------------------------- forward
    def forward(self, hidden_states: torch.Tensor, return_aux: bool = False):
        if self.routing_type == "expert_choice":
            y = self._forward_expert_choice(hidden_states)
        else:
            y = self._forward_token_choice(hidden_states)
        return (y, self.aux_loss) if return_aux else y

    def _out_dtype(self, x):
        return torch.float32 if x.dtype == torch.float32 else torch.bfloat16

    def _trainable(self, x) -> bool:
        """Whether this forward records a backward through the HIP kernels."""
        if not torch.is_grad_enabled():
            return False
        if not (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        ge = self.grouped_experts
        # the weight-gradient stores write rows of 8 bf16 (d_ff_expert a multiple of 8)
        return not (ge.use_fp8 or self.router.balanced_routing or ge.d_ff % 8)

    def _bwd_weights(self) -> _bwd.BwdWeights:
        """Backward packed weights, rebuilt only when a parameter changed."""
        ge = self.grouped_experts
        w_in = self.router.router[0].weight
        key = tuple((w.data_ptr(), w._version) for w in (ge.w1, ge.w2, ge.w3, w_in))
        cache = getattr(self, "_bwd_cache", None)
        if cache is None or cache[0] != key:
            with torch.no_grad():
                cache = (key, _bwd.pack_bwd_weights(ge.w1, ge.w2, ge.w3, w_in))
            self._bwd_cache = cache
        return cache[1]

    def _train_forward(self, x2d, T, out_dtype):
        """Token-choice forward keeping what the backward needs: (y, aux or None, Saved)."""
        r = self.router.route(x2d, T=T, save_hidden=True)
        ge = self.grouped_experts
        k, E = self.top_k, self.n_experts
        cap = ops.capacity_of(self.capacity_factor, T, k, E) if self.drop_overflow else 0
        pw = ge.packed()
        # the permuted x rows are kept for the weight gradient (the gate/up GEMM still
        # gathers its own A rows from x)
        disp = ops.dispatch(x2d, r.idx, r.w, E, capacity=cap, materialize=True, block_counts=r.block_counts)
        h, gu = ops.gemm_gate_up_rows(x2d, None, disp.row_token, disp.offsets, pw, T * k, save_gu=True)
        yperm = ops.gemm_down(h, None, disp.offsets, pw, T * k)
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k), T, out_dtype=out_dtype)
        self.last_expert_counts = disp.counts
        aux = None
        if self.training:
            aux = ops.aux_loss(r.partials, T, E, disp.counts, k, self.load_balance_loss_weight,
                               self.router_z_loss_weight)[0]
        sv = _bwd.Saved(x2d, r.logits, r.idx, r.w, r.hidden, disp, h, gu, yperm, disp.xperm)
        return y, aux, sv

    def _forward_token_choice(self, hidden_states: torch.Tensor) -> torch.Tensor:
        B, S, d = hidden_states.shape
        if self._trainable(hidden_states):
            ge = self.grouped_experts
            y, aux = _MoETrainFn.apply(hidden_states, self.router.router[0].weight, self.router.router[2].weight,
                                       ge.w1, ge.w2, ge.w3, self)
            self.aux_loss = aux if self.training else 0.0
            return y
        x2d = hidden_states.reshape(B * S, d)
        y, r, disp = self.forward_rows(x2d, T=B * S, out_dtype=self._out_dtype(hidden_states))
        self._set_token_choice_aux(r, disp, B * S)
        return _forward_only(y.view(B, S, d).to(hidden_states.dtype), hidden_states, *self.parameters())

    def forward_rows(self, x2d, T, row_index=None, T_out=None, out_map=None, scale=None,
                     out_dtype=torch.bfloat16, residual=None):
        """Token-choice MoE over rows row_index[t] (t < T) of x2d; kernel-level entry
        used by the MoD composition.  Returns (y, RouterOut, DispatchOut)."""
        if x2d.dtype != torch.bfloat16:
            x2d = x2d.to(torch.bfloat16)
        r = self.router.route(x2d, row_index=row_index, T=T)
        cap = ops.capacity_of(self.capacity_factor, T, self.top_k, self.n_experts) if self.drop_overflow else 0
        y, disp = self.grouped_experts.run(x2d, r.idx, r.w, row_index=row_index, T_out=T_out, out_map=out_map,
                                           scale=scale, out_dtype=out_dtype, residual=residual, capacity=cap,
                                           block_counts=r.block_counts)
        return y, r, disp

    def _set_token_choice_aux(self, r, disp, T):
        self.last_expert_counts = disp.counts
        if self.training:
            out = ops.aux_loss(r.partials, T, self.n_experts, disp.counts, self.top_k,
                               self.load_balance_loss_weight, self.router_z_loss_weight)
            self.aux_loss = out[0]
        else:
            self.aux_loss = 0.0

    def _forward_expert_choice(self, hidden_states: torch.Tensor) -> torch.Tensor:
        B, S, d = hidden_states.shape
        x = hidden_states if hidden_states.dtype == torch.bfloat16 else hidden_states.to(torch.bfloat16)
        # the layer output does not depend on the order of an expert's C slots: take
        # them in token order (no sort)
        r, sel, C = self.router.route(x, descending=False)
        y = self.grouped_experts_ec.run(x.reshape(B * S, d), sel, B, S, C, out_dtype=self._out_dtype(hidden_states))
        if self.training and self.router_z_loss_weight > 0:
            out = ops.aux_loss(r.partials, B * S, self.n_experts, None, 1, 0.0, self.router_z_loss_weight)
            self.aux_loss = out[0]
        else:
            self.aux_loss = 0.0
        return _forward_only(y.view(B, S, d).to(hidden_states.dtype), hidden_states, *self.parameters())

    def get_expert_utilization(self):
        """Per-expert routed-token fractions of the last forward (moe.py:941-950 returns {})."""
        if self.last_expert_counts is None:
            return {}
        c = self.last_expert_counts.float()
        tot = float(c.sum().item()) or 1.0
        return {f"expert_{i}": float(v) / tot for i, v in enumerate(c.tolist())}
