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
    w3n: torch.Tensor    # (E, round_up(F,256), d) packed rows of w3
    w13t: torch.Tensor   # (E, round_up(d,256), 2*F_pad) packed rows of w1|w2
    w_in_t: torch.Tensor  # (round_up(d,256), 128) packed rows of w_in^T


def pack_bwd_weights(w1, w2, w3, w_in) -> BwdWeights:
    E, d, F = w1.shape
    dt = w1.dtype
    if dt not in (torch.float32, _BF16):
        raise ValueError(f"kmoe backward: unsupported weight dtype {dt}")
    w1, w2, w3 = (w.detach().contiguous() for w in (w1, w2, w3))
    w_in = w_in.detach().to(dt).contiguous()
    lib = _lib.load()
    wdt = _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16
    dev = w1.device
    w3n = torch.empty(lib.kmoe_packed_w3n_bytes(E, d, F), device=dev, dtype=torch.uint8)
    w13t = torch.empty(lib.kmoe_packed_w13t_bytes(E, d, F), device=dev, dtype=torch.uint8)
    wit = torch.empty(lib.kmoe_packed_w_in_t_bytes(d), device=dev, dtype=torch.uint8)
    s = ops._stream(w1)
    _lib.call("kmoe_pack_weights_bwd", ptr(w1), ptr(w2), ptr(w3), wdt, E, d, F, ptr(w3n), ptr(w13t), s)
    _lib.call("kmoe_pack_w_in_t", ptr(w_in), wdt, d, ptr(wit), s)
    return BwdWeights(w3n, w13t, wit)


class Saved(NamedTuple):
    """What the training forward keeps for the backward."""
    x2d: torch.Tensor        # (T, d) bf16 layer input
    logits: torch.Tensor     # (T, E) f32
    idx: torch.Tensor        # (T, k) int64
    w: torch.Tensor          # (T, k) f32
    hidden: torch.Tensor     # (T, 128) f32 router pre-activation
    disp: ops.DispatchOut    # routing tables
    h: torch.Tensor          # (A, F_pad) bf16
    gu: torch.Tensor         # (A, 2 F_pad) bf16 pre-activation gate / up
    yperm: torch.Tensor      # (A, d) bf16 expert outputs
    xperm: torch.Tensor      # (A, d) bf16 permuted input rows (the dispatch's gather)


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


def moe_backward(sv: Saved, dy: torch.Tensor, grad_aux: Optional[torch.Tensor], w_out: torch.Tensor,
                 bw: BwdWeights, E: int, F: int, w_lb: float, w_z: float, need_weights: bool = True) -> Grads:
    """All gradients of one token-choice MoE layer forward (bf16 compute)."""
    lib = _lib.load()
    x2d = sv.x2d
    T, d = x2d.shape
    k = sv.idx.shape[1]
    A = T * k
    Fp = _ru(F, 128)
    dev = x2d.device
    s = ops._stream(x2d)
    disp = sv.disp
    dy = dy.reshape(T, d).to(_BF16).contiguous()
    one_seg, segs, nseg, ones, extra = _index_tensors(T, k, dev)

    # ---- combine backward: dyperm, dw
    dyperm = torch.empty(max(A, 1), d, device=dev, dtype=_BF16)
    dw = torch.empty(T, k, device=dev, dtype=torch.float32)
    with _stage("bwd_combine"):
        _lib.call("kmoe_combine_bwd", ptr(dy), ptr(sv.yperm), ptr(disp.slot_row), ptr(disp.slot_w), k, d, T,
                  ptr(dyperm), ptr(dw), s)
    # ---- dh = dyperm . w3^T (fused nothing: plain grouped GEMM), SwiGLU backward
    dh = torch.empty(max(A, 1), Fp, device=dev, dtype=_BF16)
    with _stage("bwd_gemm_dh"):
        _lib.call("kmoe_gemm_grouped", ptr(dyperm), ptr(disp.offsets), E, d, A, ptr(bw.w3n), _ru(F, 256), Fp,
                  ptr(dh), Fp, Fp, s)
    dgu = torch.empty(max(A, 1), 2 * Fp, device=dev, dtype=_BF16)
    with _stage("bwd_swiglu"):
        _lib.call("kmoe_swiglu_bwd", ptr(dh), ptr(sv.gu), A, ptr(disp.offsets[E:]), F, ptr(dgu), s)
    # ---- dxperm = dgu . [w1|w2]^T (rows [0, A)); the router's dx contribution goes to
    # rows [A, A + T) and one unit-weight gather sums both per token
    dxp = torch.empty(A + T, d, device=dev, dtype=_BF16)
    with _stage("bwd_gemm_dx"):
        _lib.call("kmoe_gemm_grouped", ptr(dgu), ptr(disp.offsets), E, 2 * Fp, A, ptr(bw.w13t), _ru(d, 256), d,
                  ptr(dxp), d, d, s)

    # ---- router: logit gradient, MLP backward, dx contribution, dW_in
    dl = torch.empty(T, E, device=dev, dtype=torch.float32)
    ga = None if grad_aux is None else grad_aux.reshape(1).to(torch.float32).contiguous()
    with _stage("bwd_router"):
        _lib.call("kmoe_router_dlogits", ptr(sv.logits), T, E, ptr(sv.idx), ptr(sv.w), ptr(dw), k,
                  ptr(disp.counts), ptr(ga), float(w_lb), float(w_z), ptr(dl), s)
        da = torch.empty(T, _lib.ROUTER_HIDDEN, device=dev, dtype=_BF16)
        wdt = w_out.dtype
        dw_out = torch.empty(E, _lib.ROUTER_HIDDEN, device=dev, dtype=wdt)
        wsb = lib.kmoe_router_bwd_workspace_bytes(T, E)
        ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
        w_out_b = w_out.detach().to(_BF16).contiguous()
        _lib.call("kmoe_router_mlp_bwd", ptr(dl), ptr(sv.hidden), T, E, ptr(w_out_b), ptr(da), ptr(dw_out),
                  _lib.DTYPE_F32 if wdt == torch.float32 else _lib.DTYPE_BF16, ptr(ws), wsb, s)
        _lib.call("kmoe_gemm_grouped", ptr(da), ptr(one_seg), 1, _lib.ROUTER_HIDDEN, T, ptr(bw.w_in_t), _ru(d, 256),
                  d, ptr(dxp[A:]), d, d, s)
    src = torch.cat([disp.slot_row.view(T, k), extra], 1)
    dx = torch.empty(T, d, device=dev, dtype=_BF16)
    with _stage("bwd_gather_dx"):
        _lib.call("kmoe_combine", ptr(dxp), d, ptr(src), ptr(ones), k + 1, None, None, T, ptr(dx), _lib.DTYPE_BF16, s)
    if not need_weights:
        return Grads(dx, None, dw_out, None, None, None)

    # ---- weight gradients, straight from the row-major buffers (transpose reads in LDS)
    dpad = _ru(d, 256)
    # dW_in = da^T x: a 128 x d output (few tiles) over K = T, split into token
    # segments of WG_SPLIT rows whose fp32 partial sums are then reduced in order
    dw_in = torch.empty(_lib.ROUTER_HIDDEN, d, device=dev, dtype=_BF16)
    with _stage("bwd_wgrad_router"):
        part = torch.empty(nseg, _lib.ROUTER_HIDDEN, d, device=dev, dtype=torch.float32)
        _lib.call("kmoe_gemm_wgrad_rows", ptr(da), _lib.ROUTER_HIDDEN, ptr(x2d), d, T, ptr(segs), nseg,
                  _lib.ROUTER_HIDDEN, dpad, ptr(part), None, _lib.DTYPE_F32, d, d, s)
        _lib.call("kmoe_reduce_f32", ptr(part), nseg, _lib.ROUTER_HIDDEN * d, ptr(dw_in), _lib.DTYPE_BF16, s)
    del part
    # expert weight gradients straight from the row buffers (transpose reads in LDS)
    dw3 = torch.empty(E, F, d, device=dev, dtype=_BF16)
    with _stage("bwd_wgrad_w3"):
        _lib.call("kmoe_gemm_wgrad_rows", ptr(sv.h), Fp, ptr(dyperm), d, A, ptr(disp.offsets), E, F, dpad, ptr(dw3),
                  None, _lib.DTYPE_BF16, d, d, s)
    dw1 = torch.empty(E, d, F, device=dev, dtype=_BF16)
    dw2 = torch.empty(E, d, F, device=dev, dtype=_BF16)
    with _stage("bwd_wgrad_w13"):
        _lib.call("kmoe_gemm_wgrad_rows", ptr(sv.xperm), d, ptr(dgu), 2 * Fp, A, ptr(disp.offsets), E, d, 2 * Fp,
                  ptr(dw1), ptr(dw2), _lib.DTYPE_BF16, F, F, s)
    return Grads(dx, dw_in, dw_out, dw1, dw2, dw3)
