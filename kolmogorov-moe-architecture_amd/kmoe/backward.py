"""Backward pass of the token-choice MoE layer on the HIP kernels.

Gradients of MoELayer.forward's token-choice path (moe.py:759-838): the router
MLP and top-k renormalisation (moe.py:423-462), the grouped SwiGLU experts and
combine (moe.py:213-294, ffn.py:17-64) and the load-balance / z losses
(moe.py:840-939).  The reference gets these from autograd through its eager ops;
its native grouped kernel has no backward at all (moe_arch/kernels/__init__.py:
167-244 is unused, sparse_moe.py:362-368).

Data flow (A = routed rows, grouped by expert):
  dy --combine_bwd--> dyperm (A,d), dw (T,k)
  dh  = dyperm . w3^T            grouped GEMM (packed w3n)
  dgu = swiglu_bwd(dh, g, u)     g, u saved by the forward's gate/up GEMM
  dxp = dgu . [w1|w2]^T          grouped GEMM (packed w13t)
  dx  = sum_j dxp[slot(t,j)] + (da . w_in)[t]   (one unit-weight gather of both)
  dW3 = h^T dyperm, dW1|dW2 = xperm^T dgu       per-expert GEMMs on the row buffers (LDS transpose reads)
  dlogits = topk-renorm backward(dw) + aux backward;  da, dW_out (router MLP);  dW_in = da^T x
"""
from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from . import _lib, ops
from ._lib import ptr

_BF16 = torch.bfloat16
WG_SPLIT = 512  # token rows per split-K segment of the router's weight gradient


def _ru(a: int, b: int) -> int:
    return (a + b - 1) // b * b


class BwdWeights(NamedTuple):
    w3n: torch.Tensor    # (E, round_up(F,256), d) packed rows of w3 (non-gated: of w2)
    w13t: torch.Tensor   # (E, round_up(d,256), 2*F_pad) packed rows of w1|w2 (non-gated: rows of w1, F_pad)
    w_in_t: torch.Tensor  # (round_up(d,256), 128) packed rows of w_in^T
    plain: bool = False  # non-gated experts (silu(x w1) w2)


def pack_bwd_weights(w1, w2, w3, w_in) -> BwdWeights:
    """Backward packed layouts of the expert weights (w1/w2/w3; w1 None: skipped; w3 None:
    the non-gated experts' w1 (E,d,F), w2 (E,F,d)) and of the router's w_in (None: skipped)."""
    lib = _lib.load()
    w3n = w13t = wit = None
    plain = False
    if w1 is not None and w3 is None:
        E, d, F = w1.shape
        dt = w1.dtype if w1.dtype in (torch.float32, _BF16) else torch.float32
        w1, w2 = (w.detach().to(dt).contiguous() for w in (w1, w2))
        w3n = torch.empty(lib.kmoe_packed_w3n_bytes(E, d, F), device=w1.device, dtype=torch.uint8)
        w13t = torch.empty(lib.kmoe_packed_w1n_bytes(E, d, F), device=w1.device, dtype=torch.uint8)
        _lib.call("kmoe_pack_weights_plain_bwd", ptr(w1), ptr(w2),
                  _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16, E, d, F, ptr(w3n), ptr(w13t),
                  ops._stream(w1))
        plain = True
        w1 = None
    if w1 is not None:
        E, d, F = w1.shape
        dt = w1.dtype
        if dt not in (torch.float32, _BF16):
            raise ValueError(f"kmoe backward: unsupported weight dtype {dt}")
        w1, w2, w3 = (w.detach().contiguous() for w in (w1, w2, w3))
        wdt = _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16
        dev = w1.device
        w3n = torch.empty(lib.kmoe_packed_w3n_bytes(E, d, F), device=dev, dtype=torch.uint8)
        w13t = torch.empty(lib.kmoe_packed_w13t_bytes(E, d, F), device=dev, dtype=torch.uint8)
        _lib.call("kmoe_pack_weights_bwd", ptr(w1), ptr(w2), ptr(w3), wdt, E, d, F, ptr(w3n), ptr(w13t),
                  ops._stream(w1))
    if w_in is not None:
        dt = w_in.dtype if w_in.dtype in (torch.float32, _BF16) else torch.float32
        w_in = w_in.detach().to(dt).contiguous()
        d = w_in.shape[1]
        wdt = _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16
        wit = torch.empty(lib.kmoe_packed_w_in_t_bytes(d), device=w_in.device, dtype=torch.uint8)
        _lib.call("kmoe_pack_w_in_t", ptr(w_in), wdt, d, ptr(wit), ops._stream(w_in))
    return BwdWeights(w3n, w13t, wit, plain)


class Saved(NamedTuple):
    """What the training forward keeps for the backward."""
    x2d: torch.Tensor        # (T, d) bf16 layer input
    logits: torch.Tensor     # (T, E) f32
    idx: torch.Tensor        # (T, k) int64
    w: torch.Tensor          # (T, k) f32
    hidden: torch.Tensor     # (T, 128) f32 router pre-activation
    disp: ops.DispatchOut    # routing tables
    h: torch.Tensor          # (A, F_pad) bf16 (fp8 experts: dequantised from the down GEMM's e4m3 rows)
    gu: torch.Tensor         # (A, 2 F_pad) bf16 pre-activation gate / up
    yperm: torch.Tensor      # (A, d) bf16 expert outputs
    xperm: torch.Tensor      # (A, d) bf16 permuted input rows (fp8: dequantised e4m3 rows)


class Grads(NamedTuple):
    dx: torch.Tensor
    dw_in: torch.Tensor
    dw_out: torch.Tensor
    dw1: torch.Tensor
    dw2: torch.Tensor
    dw3: torch.Tensor


def _stage(name):
    return ops._Stage(name)


_INDEX_CACHE: dict = {}


def _index_tensors(T: int, k: int, dev):
    """Small constant index tensors of a backward of T tokens (cached per shape and
    device, so that a step makes no host-to-device copies): the one-segment offsets
    [0, T], the split-K token segments of the router weight gradient, the unit
    weights and the router-row column of the dx gather."""
    key = (T, k, str(dev))
    hit = _INDEX_CACHE.get(key)
    if hit is None:
        split = max(WG_SPLIT, _ru(-(-T // _lib.MAX_EXPERTS), 64))  # at most MAX_EXPERTS segments
        nseg = max(1, -(-T // split))
        segs = torch.clamp(torch.arange(nseg + 1, dtype=torch.int64) * split, max=T).to(torch.int32).to(dev)
        one_seg = torch.tensor([0, T], dtype=torch.int32).to(dev)
        ones = torch.ones(T, k + 1, device=dev, dtype=torch.float32)
        extra = torch.arange(T * k, T * k + T, dtype=torch.int32).to(dev)[:, None]
        hit = (one_seg, segs, nseg, ones, extra)
        if len(_INDEX_CACHE) > 16:
            _INDEX_CACHE.clear()
        _INDEX_CACHE[key] = hit
    return hit


def _experts_core(dy, yperm, gu, slot_row, slot_w, kk, offsets, A, bw: BwdWeights, E, F, extra_rows=0,
                  row_index=None, scale=None):
    """Expert-path backward shared by every layer form: from dy through the combine
    (routing-weight gradients dw (T, kk), dyperm), the down GEMM (dh), the SwiGLU and the
    gate/up GEMM (dgu, dxp rows [0, A)).  dxp has `extra_rows` more rows after the A
    expert rows for the caller (the router's dx contribution).  T = slot_row.shape[0];
    token t's output row is dy[row_index[t]] (or dy[t]), scaled by scale[t] (or 1).
    Returns (dxp, dw, dyperm, dgu, dscale) (dscale (T,): gradient of the scale, or None)."""
    T = slot_row.shape[0]
    d = dy.shape[1]
    Fp = _ru(F, 128)
    dev = dy.device
    s = ops._stream(dy)
    dyperm = torch.empty(max(A, 1), d, device=dev, dtype=_BF16)
    dw = torch.empty(T, kk, device=dev, dtype=torch.float32)
    dscale = None
    with _stage("bwd_combine"):
        if row_index is None and scale is None:
            _lib.call("kmoe_combine_bwd", ptr(dy), ptr(yperm), ptr(slot_row), ptr(slot_w), kk, d, T, ptr(dyperm),
                      ptr(dw), s)
        else:
            dscale = torch.empty(T, device=dev, dtype=torch.float32) if scale is not None else None
            _lib.call("kmoe_combine_bwd_rows", ptr(dy), ptr(yperm), ptr(slot_row), ptr(slot_w), kk, d, T,
                      ptr(row_index), ptr(scale), ptr(dyperm), ptr(dw), ptr(dscale), s)
    dh = torch.empty(max(A, 1), Fp, device=dev, dtype=_BF16)
    with _stage("bwd_gemm_dh"):
        _lib.call("kmoe_gemm_grouped", ptr(dyperm), ptr(offsets), E, d, A, ptr(bw.w3n), _ru(F, 256), Fp,
                  ptr(dh), Fp, Fp, s)
    # gated: [dg | du] from the saved gate / up values; non-gated: dp from the saved p
    kk2 = 1 if bw.plain else 2
    dgu = torch.empty(max(A, 1), kk2 * Fp, device=dev, dtype=_BF16)
    with _stage("bwd_swiglu"):
        if bw.plain:
            _lib.call("kmoe_silu_bwd", ptr(dh), ptr(gu), A, ptr(offsets[E:]), F, ptr(dgu), s)
        else:
            _lib.call("kmoe_swiglu_bwd", ptr(dh), ptr(gu), A, ptr(offsets[E:]), F, ptr(dgu), s)
    dxp = torch.empty(A + extra_rows, d, device=dev, dtype=_BF16)
    with _stage("bwd_gemm_dx"):
        _lib.call("kmoe_gemm_grouped", ptr(dgu), ptr(offsets), E, kk2 * Fp, A, ptr(bw.w13t), _ru(d, 256), d,
                  ptr(dxp), d, d, s)
    return dxp, dw, dyperm, dgu, dscale


def _expert_weight_grads(h, dyperm, xperm, dgu, offsets, A, E, d, F, plain=False):
    """dW3 = h^T dyperm and dW1 | dW2 = xperm^T dgu per expert, straight from the row
    buffers (transpose reads in LDS).  Non-gated experts: (dW1 = xperm^T dp, dW2 = h^T
    dyperm, None)."""
    Fp = _ru(F, 128)
    dev = h.device
    s = ops._stream(h)
    dpad = _ru(d, 256)
    dw3 = torch.empty(E, F, d, device=dev, dtype=_BF16)
    with _stage("bwd_wgrad_w3"):
        _lib.call("kmoe_gemm_wgrad_rows", ptr(h), Fp, ptr(dyperm), d, A, ptr(offsets), E, F, dpad, ptr(dw3),
                  None, _lib.DTYPE_BF16, d, d, s)
    if plain:
        dw1 = torch.empty(E, d, F, device=dev, dtype=_BF16)
        with _stage("bwd_wgrad_w13"):
            _lib.call("kmoe_gemm_wgrad_rows", ptr(xperm), d, ptr(dgu), Fp, A, ptr(offsets), E, d, _ru(F, 256),
                      ptr(dw1), None, _lib.DTYPE_BF16, F, F, s)
        return dw1, dw3, None
    dw1 = torch.empty(E, d, F, device=dev, dtype=_BF16)
    dw2 = torch.empty(E, d, F, device=dev, dtype=_BF16)
    with _stage("bwd_wgrad_w13"):
        _lib.call("kmoe_gemm_wgrad_rows", ptr(xperm), d, ptr(dgu), 2 * Fp, A, ptr(offsets), E, d, 2 * Fp,
                  ptr(dw1), ptr(dw2), _lib.DTYPE_BF16, F, F, s)
    return dw1, dw2, dw3


def _router_core(x2d, hidden, w_out, bw: BwdWeights, dl, dx_rows, need_weights):
    """Router MLP backward from the logit gradient dl (T, E): da and dW_out
    (kmoe_router_mlp_bwd), the dx contribution da . w_in written to dx_rows (T, d) bf16
    (dx_rows None: no input gradient), and dW_in = da^T x (split-K over token segments, reduced in order).  Returns
    (dw_in or None, dw_out)."""
    lib = _lib.load()
    T, d = x2d.shape
    E = dl.shape[1]
    dev = x2d.device
    s = ops._stream(x2d)
    one_seg, segs, nseg, _, _ = _index_tensors(T, 1, dev)
    with _stage("bwd_router"):
        da = torch.empty(T, _lib.ROUTER_HIDDEN, device=dev, dtype=_BF16)
        wdt = w_out.dtype
        dw_out = torch.empty(E, _lib.ROUTER_HIDDEN, device=dev, dtype=wdt)
        wsb = lib.kmoe_router_bwd_workspace_bytes(T, E)
        ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
        w_out_b = w_out.detach().to(_BF16).contiguous()
        _lib.call("kmoe_router_mlp_bwd", ptr(dl), ptr(hidden), T, E, ptr(w_out_b), ptr(da), ptr(dw_out),
                  _lib.DTYPE_F32 if wdt == torch.float32 else _lib.DTYPE_BF16, ptr(ws), wsb, s)
        if dx_rows is not None:
            _lib.call("kmoe_gemm_grouped", ptr(da), ptr(one_seg), 1, _lib.ROUTER_HIDDEN, T, ptr(bw.w_in_t),
                      _ru(d, 256), d, ptr(dx_rows), d, d, s)
    if not need_weights:
        return None, dw_out
    # dW_in = da^T x: a 128 x d output (few tiles) over K = T, split into token
    # segments of WG_SPLIT rows whose fp32 partial sums are then reduced in order
    dw_in = torch.empty(_lib.ROUTER_HIDDEN, d, device=dev, dtype=_BF16)
    with _stage("bwd_wgrad_router"):
        part = torch.empty(nseg, _lib.ROUTER_HIDDEN, d, device=dev, dtype=torch.float32)
        _lib.call("kmoe_gemm_wgrad_rows", ptr(da), _lib.ROUTER_HIDDEN, ptr(x2d), d, T, ptr(segs), nseg,
                  _lib.ROUTER_HIDDEN, _ru(d, 256), ptr(part), None, _lib.DTYPE_F32, d, d, s)
        _lib.call("kmoe_reduce_f32", ptr(part), nseg, _lib.ROUTER_HIDDEN * d, ptr(dw_in), _lib.DTYPE_BF16, s)
    return dw_in, dw_out


def router_weight_grads(x2d, hidden, w_out, dl):
    """(dW_in, dW_out) of a router MLP (Linear(d, 128), SiLU, Linear(128, E)) from the
    logit gradient dl (T, E) f32, for an input that takes no gradient (the MoD
    auxiliary router's detached input, mod.py:155)."""
    return _router_core(x2d, hidden, w_out, None, dl, None, True)


def _gather_dx(dxp, src, T, d, residual=None):
    """dx[t] = (residual[t] +) sum of the token's rows src[t, :] of dxp (unit weights,
    f32 in a fixed order, one bf16 rounding); rows -1 contribute nothing."""
    fan = src.shape[1]
    ones = _ones(T, fan, dxp.device)
    dx = torch.empty(T, d, device=dxp.device, dtype=_BF16)
    with _stage("bwd_gather_dx"):
        if residual is None:
            _lib.call("kmoe_combine", ptr(dxp), d, ptr(src), ptr(ones), fan, None, None, T, ptr(dx), _lib.DTYPE_BF16,
                      ops._stream(dxp))
        else:
            _lib.call("kmoe_combine_residual", ptr(dxp), d, ptr(src), ptr(ones), fan, None, None, ptr(residual), T,
                      ptr(dx), _lib.DTYPE_BF16, ops._stream(dxp))
    return dx


_ONES: dict = {}


def _ones(T, fan, dev):
    key = (T, fan, str(dev))
    t = _ONES.get(key)
    if t is None:
        if len(_ONES) > 16:
            _ONES.clear()
        t = _ONES[key] = torch.ones(T, fan, device=dev, dtype=torch.float32)
    return t


def _token_choice_core(sv: Saved, dy, grad_aux, w_out, bw: BwdWeights, E, F, w_lb, w_z, need_weights,
                       extra_rows=0, row_index=None, scale=None):
    """Expert path and router of a token-choice layer backward: dxp (A + T + extra_rows, d)
    holds the expert rows' dx in [0, A) and the router's in [A, A + T); returns
    (dxp, dscale, dw_in, dw_out, dyperm, dgu)."""
    x2d = sv.x2d
    T, d = x2d.shape
    k = sv.idx.shape[1]
    A = T * k
    dev = x2d.device
    s = ops._stream(x2d)
    disp = sv.disp
    dxp, dw, dyperm, dgu, dscale = _experts_core(dy, sv.yperm, sv.gu, disp.slot_row.view(T, k), disp.slot_w, k,
                                                 disp.offsets, A, bw, E, F, extra_rows=T + extra_rows,
                                                 row_index=row_index, scale=scale)
    # router: logit gradient (top-k renormalisation + aux), MLP backward, dx rows, dW_in
    dl = torch.empty(T, E, device=dev, dtype=torch.float32)
    ga = None if grad_aux is None else grad_aux.reshape(1).to(torch.float32).contiguous()
    with _stage("bwd_router"):
        _lib.call("kmoe_router_dlogits", ptr(sv.logits), T, E, ptr(sv.idx), ptr(sv.w), ptr(dw), k,
                  ptr(disp.counts), ptr(ga), float(w_lb), float(w_z), ptr(dl), s)
    dw_in, dw_out = _router_core(x2d, sv.hidden, w_out, bw, dl, dxp[A:A + T], need_weights)
    return dxp, dscale, dw_in, dw_out, dyperm, dgu


def moe_backward(sv: Saved, dy: torch.Tensor, grad_aux: Optional[torch.Tensor], w_out: torch.Tensor,
                 bw: BwdWeights, E: int, F: int, w_lb: float, w_z: float, need_weights: bool = True) -> Grads:
    """All gradients of one token-choice MoE layer forward (bf16 compute)."""
    x2d = sv.x2d
    T, d = x2d.shape
    k = sv.idx.shape[1]
    A = T * k
    disp = sv.disp
    dy = dy.reshape(T, d).to(_BF16).contiguous()
    _, _, _, _, extra = _index_tensors(T, k, x2d.device)
    # the router's dx contribution goes to rows [A, A + T) of dxp and one unit-weight
    # gather sums both per token
    dxp, _, dw_in, dw_out, dyperm, dgu = _token_choice_core(sv, dy, grad_aux, w_out, bw, E, F, w_lb, w_z,
                                                            need_weights)
    src = torch.cat([disp.slot_row.view(T, k), extra], 1)
    dx = _gather_dx(dxp, src, T, d)
    if not need_weights:
        return Grads(dx, None, dw_out, None, None, None)
    dw1, dw2, dw3 = _expert_weight_grads(sv.h, dyperm, sv.xperm, dgu, disp.offsets, A, E, d, F, bw.plain)
    return Grads(dx, dw_in, dw_out, dw1, dw2, dw3)


class ModGrads(NamedTuple):
    dx: torch.Tensor          # (B*S, d) bf16: gradient of the MoD input (0 on unkept tokens)
    dw_mod: Optional[torch.Tensor]
    layer: Grads              # the inner layer's weight gradients (its dx field unused: None)


def mod_backward(sv: Saved, sel: "ops.ModSelectOut", B: int, keep: int, dy: torch.Tensor,
                 grad_aux: Optional[torch.Tensor], w_out, w_mod, bw: BwdWeights, E: int, F: int, w_lb: float,
                 w_z: float, need_weights: bool = True) -> ModGrads:
    """All gradients of the MoD composition of layers.py:148-184 (gather the kept rows,
    MoE, weight by the MoD softmax, scatter) with the layer run on the kept rows sv.x2d
    (B*keep, d).  dy (B*S, d) is the gradient of the scattered output.

    One pass per stage: the combine backward reads dy at the kept rows and returns the
    MoD weights' gradient; kmoe_mod_bwd turns it into the kept logits' gradient (written
    into the dx gather's weight table) and dW_mod; one gather then writes the input
    gradient of every token, sum of its expert rows, its router row and dlog * w_mod."""
    x_sel = sv.x2d
    T, d = x_sel.shape
    k = sv.idx.shape[1]
    A = T * k
    T_out = dy.shape[0]
    dev = x_sel.device
    s = ops._stream(x_sel)
    disp = sv.disp
    dy = dy.to(_BF16).contiguous()
    sel_w = sel.sel_w.reshape(-1)
    dxp, dsel, dw_in, dw_out, dyperm, dgu = _token_choice_core(sv, dy, grad_aux, w_out, bw, E, F, w_lb, w_z,
                                                               need_weights, extra_rows=1,
                                                               row_index=sel.token_rows, scale=sel_w)
    # gather table: the k expert rows and the router row with weight 1, w_mod with dlog
    src, gw = _mod_tables(T, k, dev)
    lib = _lib.load()
    dw_mod = None
    wsb = 0
    if need_weights:
        dw_mod = torch.empty(d, device=dev, dtype=w_mod.dtype if w_mod.dtype in (torch.float32, _BF16) else _BF16)
        wsb = lib.kmoe_mod_bwd_workspace_bytes(T, d)
    ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
    with _stage("bwd_mod"):
        _lib.call("kmoe_mod_bwd", ptr(sel_w), ptr(dsel), B, keep, ptr(x_sel), d, ptr(gw[:, k + 1:]), k + 2,
                  ptr(dw_mod), _lib.DTYPE_F32 if dw_mod is not None and dw_mod.dtype == torch.float32
                  else _lib.DTYPE_BF16, ptr(ws), wsb, s)
        dxp[A + T].copy_(w_mod.detach().reshape(-1))
    src[:, :k].copy_(disp.slot_row.view(T, k))
    dx = ops.combine(dxp, src, gw, T_out, out_map=sel.out_map, out_dtype=_BF16)
    if not need_weights:
        return ModGrads(dx, None, Grads(None, None, dw_out, None, None, None))
    dw1, dw2, dw3 = _expert_weight_grads(sv.h, dyperm, sv.xperm, dgu, disp.offsets, A, E, d, F, bw.plain)
    return ModGrads(dx, dw_mod, Grads(None, dw_in, dw_out, dw1, dw2, dw3))


def _mod_tables(T, k, dev):
    """Fresh (src (T, k+2) int32, weights (T, k+2) f32) of the MoD dx gather: columns
    k and k+1 of src hold the router row A + t and the w_mod row A + T (A = T k); the
    weights are 1 except column k+1 (filled by kmoe_mod_bwd)."""
    A = T * k
    src = torch.empty(T, k + 2, device=dev, dtype=torch.int32)
    src[:, k] = torch.arange(A, A + T, device=dev, dtype=torch.int32)
    src[:, k + 1] = A + T
    gw = torch.ones(T, k + 2, device=dev, dtype=torch.float32)
    return src, gw


class SavedEC(NamedTuple):
    """What the expert-choice training forward keeps for the backward."""
    x2d: torch.Tensor        # (B*S, d) bf16 layer input
    logits: torch.Tensor     # (B*S, E) f32
    hidden: torch.Tensor     # (B*S, 128) f32 router pre-activation
    sel: "ops.ECSelectOut"   # selection and combine tables (src_row / src_w (B*S, E))
    h: torch.Tensor          # (A, F_pad) bf16, A = E*B*C
    gu: torch.Tensor         # (A, 2 F_pad) bf16
    yperm: torch.Tensor      # (A, d) bf16
    xperm: torch.Tensor      # (A, d) bf16 gathered rows
    B: int
    S: int


def ec_backward(sv: SavedEC, dy: torch.Tensor, grad_aux: Optional[torch.Tensor], w_out: torch.Tensor,
                bw: BwdWeights, E: int, F: int, w_z: float, need_weights: bool = True) -> Grads:
    """All gradients of one expert-choice MoE layer forward (moe.py:494-530, 588-673,
    132-158 and the z-loss of moe.py:833-836)."""
    x2d = sv.x2d
    T, d = x2d.shape
    sel = sv.sel
    A = sv.h.shape[0]
    dev = x2d.device
    s = ops._stream(x2d)
    dy = dy.reshape(T, d).to(_BF16).contiguous()
    dxp, dw, dyperm, dgu, _ = _experts_core(dy, sv.yperm, sv.gu, sel.src_row, sel.src_w, E, sel.offsets, A, bw,
                                            E, F, extra_rows=T)
    dl = torch.empty(T, E, device=dev, dtype=torch.float32)
    ga = None if grad_aux is None else grad_aux.reshape(1).to(torch.float32).contiguous()
    with _stage("bwd_router"):
        # the z-loss part (zero without an aux gradient), then the selection's part
        _lib.call("kmoe_router_dlogits", ptr(sv.logits), T, E, None, None, None, 0, None, ptr(ga), 0.0, float(w_z),
                  ptr(dl), s)
        _lib.call("kmoe_ec_dlogits", ptr(sv.logits), sv.B, sv.S, E, ptr(sel.src_row), ptr(sel.src_w), ptr(dw),
                  ptr(dl), s)
    dw_in, dw_out = _router_core(x2d, sv.hidden, w_out, bw, dl, dxp[A:], need_weights)
    # dx: the token's expert rows (fan up to E) plus its router row, summed once
    dx = _gather_dx(dxp, sel.src_row, T, d, residual=dxp[A:])
    if not need_weights:
        return Grads(dx, None, dw_out, None, None, None)
    dw1, dw2, dw3 = _expert_weight_grads(sv.h, dyperm, sv.xperm, dgu, sel.offsets, A, E, d, F, bw.plain)
    return Grads(dx, dw_in, dw_out, dw1, dw2, dw3)


def experts_backward(dy, yperm, gu, h, xperm, slot_row, slot_w, offsets, A, bw: BwdWeights, E, F,
                     need_weights=True):
    """Backward of the experts alone (GroupedExperts / GroupedExpertsExpertChoice called
    directly, moe.py:213-294 / 626-673): returns (dx (T, d), dw (T, kk) gradient of each
    slot's routing weight, dw1, dw2, dw3)."""
    T, d = dy.shape
    kk = slot_row.shape[1]
    dxp, dw, dyperm, dgu, _ = _experts_core(dy, yperm, gu, slot_row, slot_w, kk, offsets, A, bw, E, F)
    dx = _gather_dx(dxp, slot_row, T, d)
    if not need_weights:
        return dx, dw, None, None, None
    dw1, dw2, dw3 = _expert_weight_grads(h, dyperm, xperm, dgu, offsets, A, E, d, F, bw.plain)
    return dx, dw, dw1, dw2, dw3


def router_backward(x2d, logits, idx, w, hidden, dw, dlogits_in, w_out, bw: BwdWeights, need_weights=True):
    """Backward of Router.forward alone (moe.py:423-462): from the gradients of its top-k
    weights dw (T, k) and of its logits (T, E, nullable) to (dx, dw_in, dw_out)."""
    T, d = x2d.shape
    E = logits.shape[1]
    k = idx.shape[1]
    dev = x2d.device
    s = ops._stream(x2d)
    dl = torch.empty(T, E, device=dev, dtype=torch.float32)
    with _stage("bwd_router"):
        _lib.call("kmoe_router_dlogits", ptr(logits), T, E, ptr(idx), ptr(w), ptr(dw), k, None, None, 0.0, 0.0,
                  ptr(dl), s)
    if dlogits_in is not None:
        dl += dlogits_in.reshape(T, E).to(torch.float32)
    dx = torch.empty(T, d, device=dev, dtype=_BF16)
    dw_in, dw_out = _router_core(x2d, hidden, w_out, bw, dl, dx, need_weights)
    return dx, dw_in, dw_out
