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
Backward (bf16 weights and activations) runs on the HIP backward kernels
(kmoe.backward) for: the token-choice MoELayer (top-k routing, optional capacity
drop), the expert-choice MoELayer, and Router / ExpertChoiceRouter /
GroupedExperts / GroupedExpertsExpertChoice called on their own (the reference's
distillation code trains them so, distill.py:289-314), balanced routing included (its
weights' backward is the top-k renormalisation's, without the + 1e-9 of moe.py:411,
a relative difference below 1e-8).  fp8 experts train straight-through on their bf16
master weights: the gradients pass the e4m3 quantisers unchanged and multiply by the
dequantised operands the fp8 GEMMs took.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
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
        raise NotImplementedError("kmoe: no HIP backward for this configuration (d_ff_expert not a multiple of 8)")


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
        self._bwd_cache = None

    def _bwd_weights(self):
        """Backward packed w_in (rebuilt only when it changed)."""
        w_in = self.router[0].weight
        key = (w_in.data_ptr(), w_in._version)
        if self._bwd_cache is None or self._bwd_cache[0] != key:
            with torch.no_grad():
                self._bwd_cache = (key, _bwd.pack_bwd_weights(None, None, None, w_in))
        return self._bwd_cache[1]

    def _trainable(self, x) -> bool:
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

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
              T: Optional[int] = None, save_hidden: bool = False, hist: bool = True) -> ops.RouterOut:
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
            r = ops.router(x2d, w_in, w_out, 0, bias=bias, row_index=row_index, T=T, save_hidden=save_hidden)
            idx, w = ops.balanced_topk(r.logits, self.top_k)
            return ops.RouterOut(r.logits, idx, w, r.partials, r.hidden)
        return ops.router(x2d, w_in, w_out, self.top_k, bias=bias, row_index=row_index, T=T, save_hidden=save_hidden,
                          hist=hist)

    def forward(self, hidden_states: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        B, S, d = hidden_states.shape
        dt = hidden_states.dtype
        if self._trainable(hidden_states):
            w, idx, logits = _RouterFn.apply(hidden_states.reshape(B * S, d), self.router[0].weight,
                                             self.router[2].weight, self)
            return (w.view(B, S, self.top_k).to(dt), idx.view(B, S, self.top_k),
                    logits.view(B, S, self.n_experts).to(dt))
        r = self.route(hidden_states.reshape(B * S, d), hist=False)
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

    def route(self, hidden_states: torch.Tensor, descending: bool = True, save_hidden: bool = False):
        B, S, d = hidden_states.shape
        C = min(self.capacity(S), S)
        w_in, w_out = self._kernel_weights()
        r = ops.router(hidden_states.reshape(B * S, d), w_in, w_out, 0, save_hidden=save_hidden)
        sel = ops.ec_select(r.logits, B, S, self.n_experts, C, descending=descending)
        return r, sel, C

    def forward(self, hidden_states: torch.Tensor):
        B, S, _ = hidden_states.shape
        dt = hidden_states.dtype
        if self._trainable(hidden_states):
            C = min(self.capacity(S), S)
            w, idx, logits = _ECRouterFn.apply(hidden_states, self.router[0].weight, self.router[2].weight, self)
            return w.to(dt), idx, logits.to(dt), C
        r, sel, C = self.route(hidden_states)
        return sel.w.to(dt), sel.idx, r.logits.view(B, S, self.n_experts).to(dt), C


class _PackedExperts(nn.Module):
    """Holds w1,w2 (E,d,F), w3 (E,F,d) and their packed kernel layout (derived cache)."""

    def __init__(self, n_experts: int, d_model: int, d_ff: int, activation: str = "swiglu"):
        super().__init__()
        self.n_experts = n_experts
        self.d_model = d_model
        self.d_ff = d_ff
        self.activation = activation
        # swiglu: (silu(x w1) * (x w2)) w3; any other activation string: silu(x w1) w2, with
        # w2 (E, F, d) and no w3 (moe.py:180-191, 275-283)
        self.gated = activation == "swiglu"
        self.w1 = nn.Parameter(torch.empty(n_experts, d_model, d_ff))
        if self.gated:
            self.w2 = nn.Parameter(torch.empty(n_experts, d_model, d_ff))
            self.w3 = nn.Parameter(torch.empty(n_experts, d_ff, d_model))
        else:
            self.w2 = nn.Parameter(torch.empty(n_experts, d_ff, d_model))
            self.register_parameter("w3", None)
        _init_expert_weights(self.w1, self.w2, self.w3)
        self._packed = None
        self.use_fp8 = False

    def _weights(self):
        return tuple(w for w in (self.w1, self.w2, self.w3) if w is not None)

    def _packed_key(self):
        return tuple((w.data_ptr(), w._version, w.device) for w in self._weights()) + (self.use_fp8,)

    def cast_grads(self, dw1, dw2, dw3):
        """The weight gradients in the parameters' dtypes (dw3 None for non-gated experts)."""
        if dw1 is None:
            return None, None, None
        return (dw1.to(self.w1.dtype), dw2.to(self.w2.dtype), None if self.w3 is None else dw3.to(self.w3.dtype))

    def expert_rows(self, x2d, row_token, offsets, A, xperm=None, save=False, xscale=None):
        """The experts on A routed rows: (yperm (A, d), h, pre-activations or None, the
        permuted input rows the weight gradient reads).  Gated bf16: the gate/up GEMM
        gathers x2d[row_token[r]] itself (with save, the pre-activation gate/up values
        for the backward); non-gated: from the permuted rows xperm (the pre-activation
        x w1 is always returned); fp8: from the e4m3 rows xperm with row scales xscale,
        with save h and the input rows dequantised (bf16, the values the fp8 GEMMs
        took: the straight-through backward's operands) and the descaled gate/up values."""
        pw = self.packed()
        if self.use_fp8:
            if not save:
                return ops.grouped_ffn(xperm, xscale, offsets, pw, A), None, None, None
            h, gu = ops.gemm_gate_up(xperm, xscale, offsets, pw, A, save_gu=True)
            n_dev = offsets[self.n_experts:]
            hq, hs = ops.quant_rows_fp8(h, n_dev)
            yperm = ops.gemm_down(hq, hs, offsets, pw, A)
            return yperm, ops.dequant_rows_fp8(hq, hs, n_dev), gu, ops.dequant_rows_fp8(xperm, xscale, n_dev)
        if not self.gated:
            return (*ops.plain_ffn(xperm, offsets, pw, A), xperm)
        if save:
            h, gu = ops.gemm_gate_up_rows(x2d, None, row_token, offsets, pw, A, save_gu=True)
        else:
            h, gu = ops.gemm_gate_up_rows(x2d, None, row_token, offsets, pw, A), None
        return ops.gemm_down(h, None, offsets, pw, A), h, gu, xperm

    def bwd_source_weights(self):
        """The expert weights the backward multiplies by: the parameters, or for fp8
        experts the fake-quantised ones the fp8 GEMMs used (straight-through: their
        gradients go to the parameters unchanged)."""
        if not self.use_fp8:
            return self.w1, self.w2, self.w3
        return tuple(ops.fake_quant_cols_e4m3(w) for w in (self.w1, self.w2, self.w3))

    def install_packed(self, pw: ops.PackedWeights) -> None:
        """Use `pw` (packed from exactly the current w1/w2/w3, e.g. read back from disk)
        until a parameter changes."""
        if not self.gated:
            raise ValueError("kmoe: packed-weight files hold gated (swiglu) experts only")
        if (pw.E, pw.d, pw.F, pw.fp8) != (self.n_experts, self.d_model, self.d_ff, self.use_fp8):
            raise ValueError("kmoe: packed weights do not match the experts' shapes / fp8 mode")
        self._packed = (self._packed_key(), pw)

    def bwd_packed(self) -> _bwd.BwdWeights:
        """Backward packed weights (no router part), rebuilt only when a parameter changed."""
        key = tuple((w.data_ptr(), w._version) for w in self._weights()) + (self.use_fp8,)
        cache = getattr(self, "_bwd_cache", None)
        if cache is None or cache[0] != key:
            with torch.no_grad():
                cache = (key, _bwd.pack_bwd_weights(*self.bwd_source_weights(), None))
            self._bwd_cache = cache
        return cache[1]

    def _trainable(self, *inputs) -> bool:
        """Whether a direct call records a backward through the HIP kernels."""
        if not torch.is_grad_enabled():
            return False
        if not any(isinstance(t, torch.Tensor) and t.requires_grad for t in inputs + tuple(self.parameters())):
            return False
        return not self.d_ff % 8

    def packed(self) -> ops.PackedWeights:
        """Packed weights, rebuilt only when a parameter changed (version counters)."""
        key = self._packed_key()
        if self._packed is None or self._packed[0] != key:
            with torch.no_grad():
                if not self.gated:
                    if self.use_fp8:
                        raise NotImplementedError("kmoe: fp8 non-gated experts are not implemented")
                    pw = ops.pack_weights_plain(self.w1.detach(), self.w2.detach())
                else:
                    pw = ops.pack_weights(self.w1.detach(), self.w2.detach(), self.w3.detach(), fp8=self.use_fp8)
            self._packed = (key, pw)
        return self._packed[1]


class GroupedExperts(_PackedExperts):
    """Token-choice grouped SwiGLU experts (moe.py:161-294)."""

    def run(self, x2d, expert_indices, expert_weights, row_index=None, T_out=None, out_map=None, scale=None,
            out_dtype=torch.bfloat16, residual=None, capacity=0, block_counts=None, aux=None):
        """dispatch -> grouped GEMMs -> combine (+ residual, added in the combine); returns (y, DispatchOut).
        capacity > 0 drops each expert's assignments past the first `capacity` (MoELayer's
        drop_overflow rule); 0, the default and what forward() uses, drops nothing (the
        reference's GroupedExperts never drops).  block_counts: the router's per-block
        histograms of expert_indices (RouterOut.block_counts), if it wrote them.
        aux = (partials, w_lb, w_z): the dispatch also computes the aux losses
        (DispatchOut.aux; needs block_counts)."""
        E = self.n_experts
        pw = self.packed()
        T, k = expert_indices.shape
        if pw.fp8:
            disp = ops.dispatch(x2d, expert_indices, expert_weights, E, capacity=capacity, fp8=True,
                                row_index=row_index, block_counts=block_counts, aux=aux)
            yperm = ops.grouped_ffn(disp.xperm, disp.xscale, disp.offsets, pw, T * k)
        elif not self.gated:
            # non-gated experts run on the permuted rows (materialised by the dispatch)
            disp = ops.dispatch(x2d, expert_indices, expert_weights, E, capacity=capacity, row_index=row_index,
                                materialize=True, block_counts=block_counts, aux=aux)
            yperm = ops.plain_ffn(disp.xperm, disp.offsets, pw, T * k)[0]
        else:
            # bf16: the gate/up GEMM gathers the token rows itself (no permuted copy of x)
            disp = ops.dispatch(x2d, expert_indices, expert_weights, E, capacity=capacity,
                                row_index=row_index, materialize=False, block_counts=block_counts, aux=aux)
            h = ops.gemm_gate_up_rows(x2d, row_index, disp.row_token, disp.offsets, pw, T * k)
            yperm = ops.gemm_down(h, None, disp.offsets, pw, T * k)
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k),
                        T if T_out is None else T_out, out_map=out_map, scale=scale, out_dtype=out_dtype,
                        residual=residual)
        return y, disp

    def forward(self, x: torch.Tensor, expert_indices: torch.Tensor, expert_weights: torch.Tensor) -> torch.Tensor:
        if self._trainable(x, expert_weights):
            return _ExpertsFn.apply(x, expert_weights, self.w1, self.w2, self.w3, self, expert_indices)
        out_dtype = torch.float32 if x.dtype == torch.float32 else torch.bfloat16
        y, _ = self.run(x, expert_indices, expert_weights, out_dtype=out_dtype)
        return _forward_only(y.to(x.dtype), x, self.w1, self.w2, self.w3, expert_weights)


class GroupedExpertsExpertChoice(_PackedExperts):
    """Expert-choice grouped experts (moe.py:533-673)."""

    def run(self, x2d, sel: ops.ECSelectOut, B, S, C, out_dtype=torch.bfloat16):
        pw = self.packed()
        n_rows = self.n_experts * B * C
        if isinstance(pw, ops.PackedWeights) and not pw.fp8:
            # bf16 SwiGLU: the gate/up GEMM gathers the selected token rows itself (no
            # permuted copy of x; a -1 entry of row_token reads as a zero row, as gather_rows
            # writes it)
            h = ops.gemm_gate_up_rows(x2d, None, sel.row_token, sel.offsets, pw, n_rows)
            yperm = ops.gemm_down(h, None, sel.offsets, pw, n_rows)
        else:
            xperm, xscale = ops.gather_rows(x2d, sel.row_token, n_rows, fp8=pw.fp8)
            yperm = ops.grouped_ffn(xperm, xscale, sel.offsets, pw, n_rows)
        return ops.combine(yperm, sel.src_row, sel.src_w, B * S, out_dtype=out_dtype)

    def forward(self, x: torch.Tensor, expert_weights: torch.Tensor, token_indices: torch.Tensor) -> torch.Tensor:
        if self._trainable(x, expert_weights):
            return _ExpertsECFn.apply(x, expert_weights, self.w1, self.w2, self.w3, self, token_indices)
        B, S, d = x.shape
        _, E, C = token_indices.shape
        sel = self.tables(token_indices, expert_weights, S)
        out_dtype = torch.float32 if x.dtype == torch.float32 else torch.bfloat16
        y = self.run(x.reshape(B * S, d), sel, B, S, C, out_dtype=out_dtype)
        return _forward_only(y.view(B, S, d).to(x.dtype), x, self.w1, self.w2, self.w3, expert_weights)

    def tables(self, token_indices: torch.Tensor, expert_weights: torch.Tensor, S: int) -> ops.ECSelectOut:
        """Expert-major rows (row = e*B*C + b*C + c) and per-token combine tables from
        caller-provided (B, E, C) token indices and weights (moe.py:649-671)."""
        B, E, C = token_indices.shape
        dev = token_indices.device
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
        src_w[toks, ee] = expert_weights.detach().reshape(-1).float()
        offsets = (torch.arange(E + 1, device=dev, dtype=torch.int32) * (B * C))
        return ops.ECSelectOut(token_indices, expert_weights, row_token, offsets, src_row, src_w)


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
        sv = _once(ctx)
        B, S, d, x_dtype, has_aux = ctx.meta
        layer = ctx.layer
        ge = layer.grouped_experts
        w_in, w_out = layer.router.router[0].weight, layer.router.router[2].weight
        need_w = any(ctx.needs_input_grad[1:6])
        g = _bwd.moe_backward(sv, dy, daux if has_aux else None, w_out, layer._bwd_weights(), layer.n_experts,
                              ge.d_ff, layer.load_balance_loss_weight, layer.router_z_loss_weight, need_weights=need_w)
        dx = g.dx.view(B, S, d).to(x_dtype)
        if not need_w:
            return dx, None, None, None, None, None, None
        return (dx, g.dw_in.to(w_in.dtype), g.dw_out.to(w_out.dtype), *ge.cast_grads(g.dw1, g.dw2, g.dw3), None)


def _once(ctx):
    if ctx.sv is None:
        raise RuntimeError("kmoe: backward through an MoE module can run once per forward; "
                           "retain_graph=True with a second backward is not supported")
    sv = ctx.sv
    ctx.sv = None
    return sv


class _RouterFn(torch.autograd.Function):
    """Router.forward (moe.py:423-462) with its backward on the HIP kernels: from the
    gradients of the top-k weights and of the logits to x, w_in and w_out."""

    @staticmethod
    def forward(ctx, x2d, w_in, w_out, router):
        r = router.route(x2d.detach().to(torch.bfloat16).contiguous(), save_hidden=True, hist=False)
        ctx.sv = (x2d, r)
        ctx.router = router
        ctx.mark_non_differentiable(r.idx)
        return r.w, r.idx, r.logits

    @staticmethod
    def backward(ctx, dw, didx, dlogits):
        x2d, r = _once(ctx)
        router = ctx.router
        xb = x2d.detach().to(torch.bfloat16).contiguous()
        T = xb.shape[0]
        dw = torch.zeros(T, router.top_k, device=xb.device) if dw is None else dw.float().contiguous()
        need_w = any(ctx.needs_input_grad[1:3])
        dx, dw_in, dw_out = _bwd.router_backward(xb, r.logits, r.idx, r.w, r.hidden, dw, dlogits,
                                                 router.router[2].weight, router._bwd_weights(), need_weights=need_w)
        w_in, w_out = router.router[0].weight, router.router[2].weight
        return (dx.to(x2d.dtype), None if dw_in is None else dw_in.to(w_in.dtype), dw_out.to(w_out.dtype), None)


class _ECRouterFn(torch.autograd.Function):
    """ExpertChoiceRouter.forward (moe.py:494-530) with its backward on the HIP kernels:
    from the gradients of the (B, E, C) weights and of the logits to x, w_in, w_out."""

    @staticmethod
    def forward(ctx, x3d, w_in, w_out, router):
        B, S, d = x3d.shape
        r, sel, C = router.route(x3d.detach().to(torch.bfloat16).contiguous(), save_hidden=True)
        ctx.sv = (x3d, r, sel)
        ctx.router = router
        ctx.mark_non_differentiable(sel.idx)
        return sel.w, sel.idx, r.logits.view(B, S, router.n_experts)

    @staticmethod
    def backward(ctx, dw, didx, dlogits):
        x3d, r, sel = _once(ctx)
        router = ctx.router
        B, S, d = x3d.shape
        E = router.n_experts
        xb = x3d.detach().reshape(B * S, d).to(torch.bfloat16).contiguous()
        # the weights' gradient in the per-token (B*S, E) layout of the combine tables
        dw_te = torch.zeros(B * S, E, device=xb.device, dtype=torch.float32)
        if dw is not None:
            tok = (torch.arange(B, device=xb.device).view(B, 1, 1) * S + sel.idx).reshape(-1)
            ex = torch.arange(E, device=xb.device).view(1, E, 1).expand_as(sel.idx).reshape(-1)
            dw_te[tok, ex] = dw.float().reshape(-1)
        dl = torch.zeros(B * S, E, device=xb.device, dtype=torch.float32)
        ops.ec_dlogits(r.logits, B, S, E, sel.src_row, sel.src_w, dw_te, dl)
        if dlogits is not None:
            dl += dlogits.reshape(B * S, E).float()
        need_w = any(ctx.needs_input_grad[1:3])
        dx = torch.empty(B * S, d, device=xb.device, dtype=torch.bfloat16)
        dw_in, dw_out = _bwd._router_core(xb, r.hidden, router.router[2].weight, router._bwd_weights(), dl, dx,
                                          need_w)
        w_in, w_out = router.router[0].weight, router.router[2].weight
        return (dx.view(B, S, d).to(x3d.dtype), None if dw_in is None else dw_in.to(w_in.dtype),
                dw_out.to(w_out.dtype), None)


class _ExpertsFn(torch.autograd.Function):
    """GroupedExperts.forward (moe.py:213-294) with its backward on the HIP kernels:
    gradients of x, of the routing weights and of w1 / w2 / w3."""

    @staticmethod
    def forward(ctx, x2d, w, w1, w2, w3, experts, idx):
        T, k = idx.shape
        E = experts.n_experts
        xb = x2d.detach().to(torch.bfloat16).contiguous()
        disp = ops.dispatch(xb, idx, w.detach(), E, materialize=True, fp8=experts.use_fp8)
        yperm, h, gu, xrows = experts.expert_rows(xb, disp.row_token, disp.offsets, T * k, xperm=disp.xperm,
                                                  xscale=disp.xscale, save=True)
        out_dtype = torch.float32 if x2d.dtype == torch.float32 else torch.bfloat16
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k), T, out_dtype=out_dtype)
        ctx.sv = (disp, h, gu, yperm, xrows)
        ctx.experts = experts
        ctx.meta = (x2d.dtype, w.dtype, T, k)
        return y.to(x2d.dtype)

    @staticmethod
    def backward(ctx, dy):
        disp, h, gu, yperm, xrows = _once(ctx)
        ge = ctx.experts
        x_dtype, w_dtype, T, k = ctx.meta
        need_w = any(ctx.needs_input_grad[2:5])
        dy = dy.reshape(T, -1).to(torch.bfloat16).contiguous()
        dx, dw, dw1, dw2, dw3 = _bwd.experts_backward(dy, yperm, gu, h, xrows, disp.slot_row.view(T, k),
                                                      disp.slot_w.view(T, k), disp.offsets, T * k, ge.bwd_packed(),
                                                      ge.n_experts, ge.d_ff, need_weights=need_w)
        wg = ge.cast_grads(dw1, dw2, dw3)
        return (dx.to(x_dtype), dw.to(w_dtype), *wg, None, None)


class _ExpertsECFn(torch.autograd.Function):
    """GroupedExpertsExpertChoice.forward (moe.py:588-673) with its backward on the HIP
    kernels: gradients of x, of the (B, E, C) weights and of w1 / w2 / w3."""

    @staticmethod
    def forward(ctx, x3d, w, w1, w2, w3, experts, token_indices):
        B, S, d = x3d.shape
        _, E, C = token_indices.shape
        sel = experts.tables(token_indices, w, S)
        xb = x3d.detach().reshape(B * S, d).to(torch.bfloat16).contiguous()
        A = E * B * C
        xperm, xscale = ops.gather_rows(xb, sel.row_token, A, fp8=experts.use_fp8)
        yperm, h, gu, xperm = experts.expert_rows(xb, sel.row_token, sel.offsets, A, xperm=xperm, xscale=xscale,
                                                  save=True)
        out_dtype = torch.float32 if x3d.dtype == torch.float32 else torch.bfloat16
        y = ops.combine(yperm, sel.src_row, sel.src_w, B * S, out_dtype=out_dtype)
        ctx.sv = (sel, h, gu, yperm, xperm)
        ctx.experts = experts
        ctx.meta = (x3d.dtype, w.dtype, B, S, d)
        return y.view(B, S, d).to(x3d.dtype)

    @staticmethod
    def backward(ctx, dy):
        sel, h, gu, yperm, xperm = _once(ctx)
        ge = ctx.experts
        x_dtype, w_dtype, B, S, d = ctx.meta
        E = ge.n_experts
        need_w = any(ctx.needs_input_grad[2:5])
        dy = dy.reshape(B * S, d).to(torch.bfloat16).contiguous()
        dx, dw_te, dw1, dw2, dw3 = _bwd.experts_backward(dy, yperm, gu, h, xperm, sel.src_row, sel.src_w, sel.offsets,
                                                         h.shape[0], ge.bwd_packed(), E, ge.d_ff, need_weights=need_w)
        tok = (torch.arange(B, device=dy.device).view(B, 1, 1) * S + sel.idx).reshape(-1)
        ex = torch.arange(E, device=dy.device).view(1, E, 1).expand_as(sel.idx).reshape(-1)
        dw = dw_te[tok, ex].view(sel.idx.shape)
        wg = ge.cast_grads(dw1, dw2, dw3)
        return (dx.view(B, S, d).to(x_dtype), dw.to(w_dtype), *wg, None, None)


class _MoEECTrainFn(torch.autograd.Function):
    """Expert-choice MoE layer (moe.py:494-530, 588-673, 815-838) whose backward runs on
    the HIP kernels; outputs y and the z-loss (0-dim, 0 in eval)."""

    @staticmethod
    def forward(ctx, x, w_in, w_out, w1, w2, w3, layer):
        B, S, d = x.shape
        T = B * S
        E = layer.n_experts
        ge = layer.grouped_experts_ec
        xb = x.detach().to(torch.bfloat16).contiguous()
        r, sel, C = layer.router.route(xb, descending=False, save_hidden=True)
        x2d = xb.reshape(T, d)
        A = E * B * C
        xperm, xscale = ops.gather_rows(x2d, sel.row_token, A, fp8=ge.use_fp8)
        yperm, h, gu, xperm = ge.expert_rows(x2d, sel.row_token, sel.offsets, A, xperm=xperm, xscale=xscale,
                                             save=True)
        y = ops.combine(yperm, sel.src_row, sel.src_w, T, out_dtype=layer._out_dtype(x))
        has_aux = layer.training and layer.router_z_loss_weight > 0
        aux = (ops.aux_loss(r.partials, T, E, None, 1, 0.0, layer.router_z_loss_weight)[0] if has_aux
               else torch.zeros((), device=x.device, dtype=torch.float32))
        ctx.sv = _bwd.SavedEC(x2d, r.logits, r.hidden, sel, h, gu, yperm, xperm, B, S)
        ctx.layer = layer
        ctx.meta = (x.dtype, has_aux)
        return y.view(B, S, d).to(x.dtype), aux

    @staticmethod
    def backward(ctx, dy, daux):
        sv = _once(ctx)
        layer = ctx.layer
        ge = layer.grouped_experts_ec
        x_dtype, has_aux = ctx.meta
        w_in, w_out = layer.router.router[0].weight, layer.router.router[2].weight
        need_w = any(ctx.needs_input_grad[1:6])
        g = _bwd.ec_backward(sv, dy, daux if has_aux else None, w_out, layer._bwd_weights(), layer.n_experts,
                             ge.d_ff, layer.router_z_loss_weight, need_weights=need_w)
        dx = g.dx.view(sv.B, sv.S, -1).to(x_dtype)
        if not need_w:
            return dx, None, g.dw_out.to(w_out.dtype), None, None, None, None
        return (dx, g.dw_in.to(w_in.dtype), g.dw_out.to(w_out.dtype), *ge.cast_grads(g.dw1, g.dw2, g.dw3), None)


def check_supported(config: AdvancedMoEConfig) -> None:
    """Raises ValueError, at construction, for shapes the HIP kernels do not take: more
    than MAX_EXPERTS experts (dispatch, router and GEMM slot tables hold one expert per
    wave lane), d_model not a multiple of 64 (the GEMMs' K-steps and the row kernels'
    16-byte vectors), top-k outside [1, min(8, n_experts)] for token choice (the router
    keeps its picks in registers).  The reference takes any of these
    (moe.py:183-185, configs/1b_150m_active.yaml: 164 experts, d_model 1512)."""
    E, d = int(config.n_experts), int(config.d_model)
    routing = getattr(config, "moe_routing", "token_choice")
    problems = []
    if not 1 <= E <= _lib.MAX_EXPERTS:
        problems.append(f"n_experts={E} (supported: 1..{_lib.MAX_EXPERTS})")
    if d <= 0 or d % 64:
        problems.append(f"d_model={d} (supported: a positive multiple of 64)")
    if routing != "expert_choice":
        k = int(config.moe_top_k)
        if not 1 <= k <= min(8, E):
            problems.append(f"moe_top_k={k} (supported: 1..min(8, n_experts))")
    if problems:
        raise ValueError("kmoe.MoELayer: configuration outside the HIP kernels' range: " + "; ".join(problems))


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
        if use_fp8 and getattr(config, "ffn_activation", "swiglu") != "swiglu":
            raise NotImplementedError("kmoe: fp8 experts are implemented for swiglu only")
        check_supported(config)
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
        return self._trainable_experts()

    def _trainable_experts(self) -> bool:
        """Whether the experts have a HIP backward: d_ff_expert a multiple of 8 (the
        weight-gradient stores write rows of 8 bf16).  fp8 experts train straight-through:
        the gradients pass the e4m3 quantisations unchanged and multiply by the
        dequantised operands the fp8 GEMMs took (bf16 master weights)."""
        ge = self.grouped_experts if self.grouped_experts is not None else self.grouped_experts_ec
        return not ge.d_ff % 8

    def _bwd_weights(self) -> _bwd.BwdWeights:
        """Backward packed weights, rebuilt only when a parameter changed."""
        ge = self.grouped_experts if self.grouped_experts is not None else self.grouped_experts_ec
        w_in = self.router.router[0].weight
        key = tuple((w.data_ptr(), w._version) for w in ge._weights() + (w_in,)) + (ge.use_fp8,)
        cache = getattr(self, "_bwd_cache", None)
        if cache is None or cache[0] != key:
            with torch.no_grad():
                cache = (key, _bwd.pack_bwd_weights(*ge.bwd_source_weights(), w_in))
            self._bwd_cache = cache
        return cache[1]

    def _train_forward(self, x2d, T, out_dtype, out_map=None, scale=None, residual=None, T_out=None,
                       keep_mask=None, keep_scale=1.0):
        """Token-choice forward keeping what the backward needs: (y, aux or None, Saved).
        out_map / scale / residual / T_out / keep_mask go to the combine (the MoD scatter,
        the block's residual add and residual dropout): y[o] = residual[o] +
        keep[o] keep_scale scale[t] MoE(x)[t] for t = out_map[o]."""
        r = self.router.route(x2d, T=T, save_hidden=True)
        ge = self.grouped_experts
        k, E = self.top_k, self.n_experts
        cap = ops.capacity_of(self.capacity_factor, T, k, E) if self.drop_overflow else 0
        # the permuted x rows are kept for the weight gradient (the gated gate/up GEMM still
        # gathers its own A rows from x; fp8: the rows are the dispatch's e4m3 codes, kept
        # dequantised)
        aux_in = self._aux_args(r, T)
        disp = ops.dispatch(x2d, r.idx, r.w, E, capacity=cap, materialize=True, fp8=ge.use_fp8,
                            block_counts=r.block_counts, aux=aux_in)
        yperm, h, gu, xrows = ge.expert_rows(x2d, disp.row_token, disp.offsets, T * k, xperm=disp.xperm,
                                             xscale=disp.xscale, save=True)
        y = ops.combine(yperm, disp.slot_row.view(T, k), disp.slot_w.view(T, k), T if T_out is None else T_out,
                        out_map=out_map, scale=scale, out_dtype=out_dtype, residual=residual, keep_mask=keep_mask,
                        keep_scale=keep_scale)
        self.last_expert_counts = disp.counts
        aux = None
        if self.training:
            aux = (disp.aux if disp.aux is not None else
                   ops.aux_loss(r.partials, T, E, disp.counts, k, self.load_balance_loss_weight,
                                self.router_z_loss_weight))[0]
        sv = _bwd.Saved(x2d, r.logits, r.idx, r.w, r.hidden, disp, h, gu, yperm, xrows)
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
                                           block_counts=r.block_counts, aux=self._aux_args(r, T))
        return y, r, disp

    def _aux_args(self, r, T):
        """(partials, w_lb, w_z) for a dispatch that computes the aux losses too (training
        mode, router block histograms present), else None."""
        if self.training and T > 0 and r.block_counts is not None and r.partials is not None:
            return (r.partials, self.load_balance_loss_weight, self.router_z_loss_weight)
        return None

    def _set_token_choice_aux(self, r, disp, T):
        self.last_expert_counts = disp.counts
        if self.training:
            out = disp.aux if disp.aux is not None else ops.aux_loss(
                r.partials, T, self.n_experts, disp.counts, self.top_k, self.load_balance_loss_weight,
                self.router_z_loss_weight)
            self.aux_loss = out[0]
        else:
            self.aux_loss = 0.0

    def _forward_expert_choice(self, hidden_states: torch.Tensor) -> torch.Tensor:
        B, S, d = hidden_states.shape
        if self._trainable(hidden_states):
            ge = self.grouped_experts_ec
            y, aux = _MoEECTrainFn.apply(hidden_states, self.router.router[0].weight, self.router.router[2].weight,
                                         ge.w1, ge.w2, ge.w3, self)
            self.aux_loss = aux if (self.training and self.router_z_loss_weight > 0) else 0.0
            return y
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
