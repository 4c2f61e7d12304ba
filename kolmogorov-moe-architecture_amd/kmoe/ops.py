"""Tensor-level wrappers over the kmoe C ABI (one function per entry point).

Every wrapper validates shapes/dtypes/devices on the host, allocates its
outputs with torch (the C ABI itself never allocates), and launches on
torch's current HIP stream.  There is no CPU path: inputs must live on a GPU.
"""
from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch

from . import _lib
from ._lib import ptr

_BF16 = torch.bfloat16


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("kmoe: tensors must be on a GPU (the HIP kernels are the only implementation)")


def _contig(t, dtype=None):
    if t is None:
        return None
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _stream(t):
    return _lib.stream_ptr(t.device)


# ---------------------------------------------------------------- stage timing
# When a list is installed here (bench.py does), every stage records a pair of
# HIP events on the launch stream: (name, start, end).  Off by default.
_STAGE_EVENTS: Optional[list] = None


class _Stage:
    def __init__(self, name):
        self.name = name
        self.on = _STAGE_EVENTS is not None and (_STAGE_ONLY is None or name in _STAGE_ONLY)

    def __enter__(self):
        if self.on:
            self.start = torch.cuda.Event(enable_timing=True)
            self.start.record()
        return self

    def __exit__(self, *exc):
        if self.on:
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            _STAGE_EVENTS.append((self.name, self.start, end))
        return False


_STAGE_ONLY: Optional[set] = None


def set_stage_timing(events: Optional[list], only: Optional[set] = None):
    """Install (a list) or remove (None) the per-stage event recorder; `only`
    restricts it to the named stages."""
    global _STAGE_EVENTS, _STAGE_ONLY
    _STAGE_EVENTS = events
    _STAGE_ONLY = set(only) if only is not None else None


class RouterOut(NamedTuple):
    logits: torch.Tensor          # (T, E) f32
    idx: Optional[torch.Tensor]   # (T, k) int64
    w: Optional[torch.Tensor]     # (T, k) f32
    partials: Optional[torch.Tensor]  # per-block aux partial sums (None: router(partials=False))
    hidden: Optional[torch.Tensor] = None  # (T, 128) f32 pre-activation (training router)
    rscale: Optional[torch.Tensor] = None  # (T,) f32 RMSNorm scale 1/sqrt(mean(x^2)+eps) (rms router)
    block_counts: Optional[torch.Tensor] = None  # (ceil(T/b), E) int32 per-block routed counts, b = router_block_tokens(T)


def router(x2d, w_in, w_out, k, bias=None, row_index=None, T=None, save_hidden=False,
           rms_eps=None, hist=True, partials=True, stage="router") -> RouterOut:
    """logits/top-k of the reference Router (moe.py:423-462) on the HIP kernel.

    x2d: (rows, d) bf16; w_in: (128, d); w_out: (E, 128); row_index: optional
    int32 (T,) selecting the rows of x2d that are the tokens.
    rms_eps: route RMSNorm(x) (embeddings.py:167-195) with the norm weight already
    folded into w_in's columns; the result carries the per-token scale (rscale).
    hist (k > 0, not rms): also return each router block's per-expert routed counts
    (blocks of router_block_tokens(T) tokens), which dispatch(block_counts=...) takes
    instead of counting them again.
    partials: write the per-block aux partial sums (aux_loss's input); False for a router
    that only needs its logits (like the MoD auxiliary router).
    stage: the name the per-stage timing records the launch under.
    """
    _need_gpu(x2d, w_in, w_out)
    x2d = _contig(x2d, _BF16)
    w_in = _contig(w_in, _BF16)
    w_out = _contig(w_out, _BF16)
    d = x2d.shape[1]
    E = w_out.shape[0]
    if w_in.shape != (_lib.ROUTER_HIDDEN, d) or w_out.shape[1] != _lib.ROUTER_HIDDEN:
        raise ValueError(f"kmoe.router: weight shapes {tuple(w_in.shape)}, {tuple(w_out.shape)} "
                         f"do not match d={d}, hidden={_lib.ROUTER_HIDDEN}")
    if T is None:
        T = row_index.shape[0] if row_index is not None else x2d.shape[0]
    dev = x2d.device
    logits = torch.empty(T, E, device=dev, dtype=torch.float32)
    idx = torch.empty(T, k, device=dev, dtype=torch.int64) if k > 0 else None
    w = torch.empty(T, k, device=dev, dtype=torch.float32) if k > 0 else None
    if partials:
        partials = torch.empty(max(_lib.load().kmoe_router_partials_len(T, E), 1), device=dev, dtype=torch.float32)
    else:
        partials = None
    bias = _contig(bias, torch.float32)
    hidden = torch.empty(T, _lib.ROUTER_HIDDEN, device=dev, dtype=torch.float32) if save_hidden else None
    if rms_eps is not None:
        if save_hidden:
            raise ValueError("kmoe.router: rms_eps is a forward-only (inference) path")
        rscale = torch.empty(max(T, 1), device=dev, dtype=torch.float32)
        with _Stage(stage):
            _lib.call("kmoe_router_rms", ptr(x2d), ptr(row_index), T, d, ptr(w_in), ptr(w_out), E, ptr(bias), k,
                      ptr(logits), ptr(idx), ptr(w), ptr(partials), float(rms_eps), ptr(rscale), _stream(x2d))
        return RouterOut(logits, idx, w, partials, None, rscale)
    if hist and k > 0 and T > 0:
        bc = torch.empty(-(-T // router_block_tokens(T)), E, device=dev, dtype=torch.int32)
        with _Stage(stage):
            _lib.call("kmoe_router_hist", ptr(x2d), ptr(row_index), T, d, ptr(w_in), ptr(w_out), E, ptr(bias), k,
                      ptr(logits), ptr(idx), ptr(w), ptr(partials), ptr(hidden), ptr(bc), _stream(x2d))
        return RouterOut(logits, idx, w, partials, hidden, None, bc)
    with _Stage(stage):
        _lib.call("kmoe_router_train", ptr(x2d), ptr(row_index), T, d, ptr(w_in), ptr(w_out), E, ptr(bias), k,
                  ptr(logits), ptr(idx), ptr(w), ptr(partials), ptr(hidden), _stream(x2d))
    return RouterOut(logits, idx, w, partials, hidden)


def router_block_tokens(T: int) -> int:
    """Tokens per router workgroup for a call over T tokens on the current device (32 when
    32-token tiles fit the device in one wave of workgroups, else 64): the token span of
    one row of the router's aux partials and block histograms."""
    return int(_lib.load().kmoe_router_block_tokens(T))


def balanced_topk(logits, k):
    """Capacity-balanced top-k of Router._balanced_topk_assignment (moe.py:353-421)
    from fp32 logits (T, E): returns (idx (T,k) int64, w (T,k) f32)."""
    _need_gpu(logits)
    logits = _contig(logits, torch.float32)
    T, E = logits.shape
    dev = logits.device
    idx = torch.empty(T, k, device=dev, dtype=torch.int64)
    w = torch.empty(T, k, device=dev, dtype=torch.float32)
    lib = _lib.load()
    wsb = lib.kmoe_balanced_workspace_bytes(E, k)
    ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
    with _Stage("router"):
        _lib.call("kmoe_balanced_topk", ptr(logits), T, E, k, ptr(idx), ptr(w), ptr(ws), wsb, _stream(logits))
    return idx, w


def aux_loss(partials, T, E, counts, k, w_lb, w_z):
    """(aux, load_balance, z) of MoELayer._compute_auxiliary_losses (moe.py:840-939)."""
    out = torch.empty(3, device=partials.device, dtype=torch.float32)
    with _Stage("aux"):
        _lib.call("kmoe_aux_loss", ptr(partials), T, E, ptr(counts), k, float(w_lb), float(w_z), ptr(out),
              _stream(partials))
    return out


def mod_aux_bce(logits, rows, weight):
    """The MoD auxiliary router's loss (mod.py:141-171) from its logits (T,) or (T, 1)
    f32 and the kept rows (int32): weight * mean BCE-with-logits, targets 1 at rows."""
    _need_gpu(logits, rows)
    logits = _contig(logits, torch.float32)
    rows = _contig(rows, torch.int32)
    out = torch.empty(1, device=logits.device, dtype=torch.float32)
    _lib.call("kmoe_mod_aux_bce", ptr(logits), logits.numel(), ptr(rows), rows.numel(), float(weight), ptr(out),
              _stream(logits))
    return out[0]


class DispatchOut(NamedTuple):
    counts: torch.Tensor     # (E,) int32 routed counts
    offsets: torch.Tensor    # (E+1,) int32 kept-row offsets
    row_token: torch.Tensor  # (T*k,) int32
    slot_row: torch.Tensor   # (T*k,) int32, -1 = dropped
    slot_w: torch.Tensor     # (T*k,) f32
    xperm: torch.Tensor      # (T*k, d) bf16 or uint8 (fp8 e4m3)
    xscale: Optional[torch.Tensor]  # (T*k,) f32 for fp8
    aux: Optional[torch.Tensor] = None  # (3,) f32 aux losses, when asked for (aux_loss's output)


def capacity_of(cf: float, T: int, k: int, E: int) -> int:
    """Per-expert capacity ceil(cf*T*k/E) of the token-choice drop rule."""
    return int(math.ceil(cf * T * k / E))


def dispatch(x2d, idx, w, E, capacity=0, fp8=False, row_index=None, materialize=True,
             no_alloc=False, block_counts=None, aux=None) -> DispatchOut:
    """Stable counting-sort dispatch (moe.py:238-272) + optional capacity drop.

    materialize=False (bf16 only) writes the routing tables but not the permuted
    rows: gemm_gate_up_rows gathers them itself (xperm is then None).
    no_alloc=True calls kmoe_dispatch_noalloc, whose histograms live in the library's
    own device scratch (no workspace allocation; calls on one GPU must not overlap).
    block_counts: the router's per-block histograms of idx (RouterOut.block_counts);
    kmoe_dispatch_counted then skips counting them.
    aux = (partials, w_lb, w_z) (with block_counts): the aux losses of aux_loss(partials, T,
    E, counts, k, w_lb, w_z) come back in DispatchOut.aux, computed inside the dispatch's
    table launch (kmoe_dispatch_counted_aux) instead of a launch of their own."""
    if not materialize and fp8:
        raise ValueError("kmoe.dispatch: the fp8 path needs the quantised permuted rows (materialize=True)")
    _need_gpu(x2d, idx, w)
    x2d = _contig(x2d, _BF16)
    idx = _contig(idx, torch.int64)
    if w.dtype not in (torch.float32, _BF16):
        w = w.float()
    w = w.contiguous()
    T, k = idx.shape
    d = x2d.shape[1]
    A = T * k
    dev = x2d.device
    lib = _lib.load()
    counts = torch.empty(E, device=dev, dtype=torch.int32)
    offsets = torch.empty(E + 1, device=dev, dtype=torch.int32)
    row_token = torch.empty(max(A, 1), device=dev, dtype=torch.int32)
    slot_row = torch.empty(max(A, 1), device=dev, dtype=torch.int32)
    slot_w = torch.empty(max(A, 1), device=dev, dtype=torch.float32)
    xperm = torch.empty(max(A, 1), d, device=dev, dtype=torch.uint8 if fp8 else _BF16) if materialize else None
    xscale = torch.empty(max(A, 1), device=dev, dtype=torch.float32) if fp8 else None
    wdt = _lib.DTYPE_F32 if w.dtype == torch.float32 else _lib.DTYPE_BF16
    if no_alloc:
        with _Stage("dispatch"):
            _lib.call("kmoe_dispatch_noalloc", ptr(x2d), ptr(row_index), T, d, ptr(idx), ptr(w), wdt, k, E,
                      int(capacity), ptr(counts), ptr(offsets), ptr(row_token), ptr(slot_row), ptr(slot_w), ptr(xperm),
                      _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16, ptr(xscale), _stream(x2d))
        return DispatchOut(counts, offsets, row_token, slot_row, slot_w, xperm, xscale)
    wsb = lib.kmoe_dispatch_workspace_bytes(T, k, E)
    ws = torch.empty(wsb, device=dev, dtype=torch.uint8)
    if aux is not None and (block_counts is None or no_alloc or T == 0):
        raise ValueError("kmoe.dispatch: aux needs block_counts (and T > 0, not no_alloc)")
    if block_counts is not None:
        hb = router_block_tokens(T)
        if block_counts.dtype != torch.int32 or block_counts.numel() != -(-T // hb) * E:
            raise ValueError(f"kmoe.dispatch: block_counts must be int32 (ceil(T/{hb}), E) "
                             f"(router_block_tokens)")
        if aux is not None:
            partials, w_lb, w_z = aux
            aux_out = torch.empty(3, device=dev, dtype=torch.float32)
            with _Stage("dispatch"):
                _lib.call("kmoe_dispatch_counted_aux", ptr(x2d), ptr(row_index), T, d, ptr(idx), ptr(w), wdt, k, E,
                          int(capacity), ptr(block_counts), ptr(counts), ptr(offsets), ptr(row_token), ptr(slot_row),
                          ptr(slot_w), ptr(xperm), _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16, ptr(xscale),
                          ptr(ws), wsb, ptr(partials), float(w_lb), float(w_z), ptr(aux_out), _stream(x2d))
            return DispatchOut(counts, offsets, row_token, slot_row, slot_w, xperm, xscale, aux_out)
        with _Stage("dispatch"):
            _lib.call("kmoe_dispatch_counted", ptr(x2d), ptr(row_index), T, d, ptr(idx), ptr(w), wdt, k, E,
                      int(capacity), ptr(block_counts), ptr(counts), ptr(offsets), ptr(row_token), ptr(slot_row),
                      ptr(slot_w), ptr(xperm), _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16, ptr(xscale),
                      ptr(ws), wsb, _stream(x2d))
        return DispatchOut(counts, offsets, row_token, slot_row, slot_w, xperm, xscale)
    with _Stage("dispatch"):
        _lib.call("kmoe_dispatch", ptr(x2d), ptr(row_index), T, d, ptr(idx), ptr(w), wdt, k, E, int(capacity),
              ptr(counts), ptr(offsets), ptr(row_token), ptr(slot_row), ptr(slot_w), ptr(xperm),
              _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16, ptr(xscale), ptr(ws), wsb, _stream(x2d))
    return DispatchOut(counts, offsets, row_token, slot_row, slot_w, xperm, xscale)


def gather_rows(x2d, row_token, n_rows, fp8=False, n_rows_dev=None):
    _need_gpu(x2d, row_token)
    x2d = _contig(x2d, _BF16)
    d = x2d.shape[1]
    out = torch.empty(max(n_rows, 1), d, device=x2d.device, dtype=torch.uint8 if fp8 else _BF16)
    scale = torch.empty(max(n_rows, 1), device=x2d.device, dtype=torch.float32) if fp8 else None
    with _Stage("gather"):
        _lib.call("kmoe_gather_rows", ptr(x2d), ptr(row_token), n_rows, ptr(n_rows_dev), d, ptr(out),
              _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16, ptr(scale), _stream(x2d))
    return out, scale


class PackedWeights(NamedTuple):
    w13: torch.Tensor
    w3: torch.Tensor
    s13: Optional[torch.Tensor]
    s3: Optional[torch.Tensor]
    E: int
    d: int
    F: int
    fp8: bool


def pack_weights(w1, w2, w3, fp8=False) -> PackedWeights:
    """Derived kernel layout of the reference expert weights w1,w2 (E,d,F), w3 (E,F,d)."""
    _need_gpu(w1, w2, w3)
    E, d, F = w1.shape
    if w2.shape != (E, d, F) or w3.shape != (E, F, d):
        raise ValueError("kmoe.pack_weights: w1/w2 must be (E,d,F) and w3 (E,F,d)")
    if w1.dtype not in (torch.float32, _BF16):
        raise ValueError(f"kmoe.pack_weights: unsupported weight dtype {w1.dtype}")
    dt = w1.dtype
    w1, w2, w3 = _contig(w1, dt), _contig(w2, dt), _contig(w3, dt)
    lib = _lib.load()
    pdt = _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16
    wdt = _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16
    Fp = lib.kmoe_padded_ff(F)
    dp = (d + 255) // 256 * 256
    dev = w1.device
    w13p = torch.empty(lib.kmoe_packed_w13_bytes(E, d, F, pdt), device=dev, dtype=torch.uint8)
    w3p = torch.empty(lib.kmoe_packed_w3_bytes(E, d, F, pdt), device=dev, dtype=torch.uint8)
    s13 = torch.empty(E * 2 * Fp, device=dev, dtype=torch.float32) if fp8 else None
    s3 = torch.empty(E * dp, device=dev, dtype=torch.float32) if fp8 else None
    _lib.call("kmoe_pack_weights", ptr(w1), ptr(w2), ptr(w3), wdt, E, d, F, pdt, ptr(w13p), ptr(s13), ptr(w3p),
              ptr(s3), _stream(w1))
    return PackedWeights(w13p, w3p, s13, s3, E, d, F, fp8)


def gemm_gate_up(xperm, xscale, offsets, pw: PackedWeights, max_rows, save_gu=False):
    """h = SwiGLU gate/up of the permuted rows.  save_gu (fp8 training forward) also
    returns the descaled pre-activation gate/up values (max_rows, 2*F_pad) bf16 in the
    packed order: returns (h, gu)."""
    lib = _lib.load()
    Fp = lib.kmoe_padded_ff(pw.F)
    h = torch.empty(max(max_rows, 1), Fp, device=xperm.device, dtype=_BF16)
    if save_gu:
        if not pw.fp8:
            raise ValueError("kmoe.gemm_gate_up: save_gu is for fp8 rows (bf16: gemm_gate_up_rows)")
        gu = torch.empty(max(max_rows, 1), 2 * Fp, device=xperm.device, dtype=_BF16)
        with _Stage("gemm_gate_up"):
            _lib.call("kmoe_gemm_gate_up_fp8_gu", ptr(xperm), ptr(xscale), ptr(offsets), pw.E, pw.d, pw.F, max_rows,
                      ptr(pw.w13), ptr(pw.s13), ptr(h), ptr(gu), _stream(xperm))
        return h, gu
    with _Stage("gemm_gate_up"):
        _lib.call("kmoe_gemm_gate_up", ptr(xperm), ptr(xscale),
              _lib.DTYPE_FP8_E4M3 if pw.fp8 else _lib.DTYPE_BF16, ptr(offsets), pw.E, pw.d, pw.F, max_rows,
              ptr(pw.w13), ptr(pw.s13), ptr(h), _stream(xperm))
    return h


def gemm_gate_up_rows(x2d, row_index, row_token, offsets, pw: PackedWeights, max_rows, save_gu=False,
                      rscale=None):
    """gate_up GEMM whose A rows are x2d[row_index[row_token[r]]] (x2d[row_token[r]]
    without row_index): the dispatch gather fused into the GEMM's loads (bf16).
    save_gu (training) also returns the pre-activation gate/up values (max_rows,
    2*F_pad) in the packed order: returns (h, gu).
    rscale (T,) f32: row r's gate/up values are scaled by rscale[row_token[r]] (the
    RMSNorm scale; pw packed from norm-folded w1/w2)."""
    if pw.fp8:
        raise ValueError("kmoe.gemm_gate_up_rows: bf16 weights only (fp8 reads quantised permuted rows)")
    _need_gpu(x2d, row_token, offsets)
    x2d = _contig(x2d, _BF16)
    lib = _lib.load()
    Fp = lib.kmoe_padded_ff(pw.F)
    h = torch.empty(max(max_rows, 1), Fp, device=x2d.device, dtype=_BF16)
    if rscale is not None:
        if save_gu:
            raise ValueError("kmoe.gemm_gate_up_rows: rscale is a forward-only (inference) path")
        with _Stage("gemm_gate_up"):
            _lib.call("kmoe_gemm_gate_up_rows_scaled", ptr(x2d), ptr(row_index), x2d.shape[0], ptr(row_token),
                      ptr(offsets), pw.E, pw.d, pw.F, max_rows, ptr(pw.w13), ptr(rscale), ptr(h), _stream(x2d))
        return h
    if save_gu:
        gu = torch.empty(max(max_rows, 1), 2 * Fp, device=x2d.device, dtype=_BF16)
        with _Stage("gemm_gate_up"):
            _lib.call("kmoe_gemm_gate_up_rows_gu", ptr(x2d), ptr(row_index), x2d.shape[0], ptr(row_token),
                      ptr(offsets), pw.E, pw.d, pw.F, max_rows, ptr(pw.w13), ptr(h), ptr(gu), _stream(x2d))
        return h, gu
    with _Stage("gemm_gate_up"):
        _lib.call("kmoe_gemm_gate_up_rows", ptr(x2d), ptr(row_index), x2d.shape[0], ptr(row_token), ptr(offsets),
                  pw.E, pw.d, pw.F, max_rows, ptr(pw.w13), ptr(h), _stream(x2d))
    return h


def gemm_down(h, hscale, offsets, pw: PackedWeights, max_rows):
    y = torch.empty(max(max_rows, 1), pw.d, device=h.device, dtype=_BF16)
    with _Stage("gemm_down"):
        _lib.call("kmoe_gemm_down", ptr(h), ptr(hscale), _lib.DTYPE_FP8_E4M3 if pw.fp8 else _lib.DTYPE_BF16,
              ptr(offsets), pw.E, pw.d, pw.F, max_rows, ptr(pw.w3), ptr(pw.s3), ptr(y), _stream(h))
    return y


def quant_rows_fp8(m, n_rows_dev=None):
    rows, cols = m.shape
    q = torch.empty(rows, cols, device=m.device, dtype=torch.uint8)
    s = torch.empty(rows, device=m.device, dtype=torch.float32)
    with _Stage("quant_h"):
        _lib.call("kmoe_quant_rows_fp8", ptr(m), rows, ptr(n_rows_dev), cols, ptr(q), ptr(s), _stream(m))
    return q, s


def dequant_rows_fp8(q, scale, n_rows_dev=None):
    """bf16(e4m3(q) * scale[:, None]) of fp8 rows (rows past *n_rows_dev not written):
    the operand the fp8 GEMM took, for the straight-through backward."""
    _need_gpu(q, scale)
    rows, cols = q.shape
    out = torch.empty(rows, cols, device=q.device, dtype=_BF16)
    with _Stage("fp8_dequant"):
        _lib.call("kmoe_dequant_rows_fp8", ptr(q), ptr(scale), rows, ptr(n_rows_dev), cols, ptr(out), _stream(q))
    return out


def fake_quant_cols_e4m3(w):
    """w (E, K, N) fake-quantised per output column of each expert exactly as the fp8
    weight packing quantises it, dequantised to bf16 (the weights the fp8 GEMMs
    multiplied)."""
    _need_gpu(w)
    if w.dtype not in (torch.float32, _BF16):
        raise ValueError(f"kmoe.fake_quant_cols_e4m3: unsupported weight dtype {w.dtype}")
    w = _contig(w.detach(), w.dtype)
    E, K, N = w.shape
    out = torch.empty(E, K, N, device=w.device, dtype=_BF16)
    _lib.call("kmoe_fake_quant_e4m3_cols", ptr(w), _lib.DTYPE_F32 if w.dtype == torch.float32 else _lib.DTYPE_BF16,
              E, K, N, ptr(out), _stream(w))
    return out


class PlainPacked(NamedTuple):
    """Packed weights of non-gated experts (silu(x w1) w2): w1t (rows f of w1^T), w2t (rows n of w2^T)."""
    w1t: torch.Tensor
    w2t: torch.Tensor
    E: int
    d: int
    F: int
    fp8: bool = False


def pack_weights_plain(w1, w2) -> PlainPacked:
    """Derived kernel layout of non-gated expert weights w1 (E,d,F), w2 (E,F,d) (moe.py:187-191)."""
    _need_gpu(w1, w2)
    E, d, F = w1.shape
    if w2.shape != (E, F, d):
        raise ValueError("kmoe.pack_weights_plain: w1 must be (E,d,F) and w2 (E,F,d)")
    if w1.dtype not in (torch.float32, _BF16):
        raise ValueError(f"kmoe.pack_weights_plain: unsupported weight dtype {w1.dtype}")
    dt = w1.dtype
    w1, w2 = _contig(w1, dt), _contig(w2, dt)
    lib = _lib.load()
    dev = w1.device
    w1t = torch.empty(lib.kmoe_packed_w1t_bytes(E, d, F), device=dev, dtype=torch.uint8)
    w2t = torch.empty(lib.kmoe_packed_w3_bytes(E, d, F, _lib.DTYPE_BF16), device=dev, dtype=torch.uint8)
    _lib.call("kmoe_pack_weights_plain", ptr(w1), ptr(w2), _lib.DTYPE_F32 if dt == torch.float32 else _lib.DTYPE_BF16,
              E, d, F, ptr(w1t), ptr(w2t), _stream(w1))
    return PlainPacked(w1t, w2t, E, d, F)


def plain_ffn(xperm, offsets, pp: PlainPacked, max_rows):
    """Non-gated experts on the permuted rows (moe.py:281-283): p = x w1, h = silu(p),
    y = h w2.  Returns (yperm (max_rows, d), h, p) bf16."""
    E, d, F = pp.E, pp.d, pp.F
    lib = _lib.load()
    Fp = lib.kmoe_padded_ff(F)
    dev = xperm.device
    s = _stream(xperm)
    rows = max(max_rows, 1)
    p = torch.empty(rows, Fp, device=dev, dtype=_BF16)
    h = torch.empty(rows, Fp, device=dev, dtype=_BF16)
    y = torch.empty(rows, d, device=dev, dtype=_BF16)
    with _Stage("gemm_gate_up"):
        _lib.call("kmoe_gemm_grouped", ptr(xperm), ptr(offsets), E, d, max_rows, ptr(pp.w1t), (F + 255) // 256 * 256,
                  Fp, ptr(p), Fp, Fp, s)
    with _Stage("silu"):
        _lib.call("kmoe_silu_rows", ptr(p), max_rows, ptr(offsets[E:]), F, ptr(h), s)
    with _Stage("gemm_down"):
        _lib.call("kmoe_gemm_grouped", ptr(h), ptr(offsets), E, Fp, max_rows, ptr(pp.w2t), (d + 255) // 256 * 256, d,
                  ptr(y), d, d, s)
    return y, h, p


def grouped_ffn(xperm, xscale, offsets, pw: PackedWeights, max_rows):
    """gate_up -> (fp8: per-row requant of h) -> down.  Returns yperm (max_rows, d) bf16."""
    if isinstance(pw, PlainPacked):
        return plain_ffn(xperm, offsets, pw, max_rows)[0]
    h = gemm_gate_up(xperm, xscale, offsets, pw, max_rows)
    if pw.fp8:
        hq, hs = quant_rows_fp8(h, offsets[pw.E:])
        return gemm_down(hq, hs, offsets, pw, max_rows)
    return gemm_down(h, None, offsets, pw, max_rows)


def combine(yperm, src_row, src_w, T_out, out_map=None, scale=None, out_dtype=_BF16, residual=None,
            keep_mask=None, keep_scale=1.0):
    """y[o] = scale[s] * sum_j src_w[s,j] * yperm[src_row[s,j]] (moe.py:285-292, 132-158),
    plus residual[o] ((T_out, d), cast to out_dtype) when given (layers.py:187).
    keep_mask ((T_out, d) bool, with a residual): the residual dropout, the sum times
    keep_scale = 1/(1-p) where kept and 0 elsewhere (layers.py:190)."""
    fan = src_row.shape[1]
    d = yperm.shape[1]
    y = torch.empty(T_out, d, device=yperm.device, dtype=out_dtype)
    ydt = _lib.DTYPE_F32 if out_dtype == torch.float32 else _lib.DTYPE_BF16
    if residual is not None:
        residual = _contig(residual, out_dtype)
        if residual.shape != (T_out, d):
            raise ValueError(f"kmoe.combine: residual shape {tuple(residual.shape)} != {(T_out, d)}")
    if keep_mask is not None:
        if residual is None:
            raise ValueError("kmoe.combine: a dropout keep mask needs the residual")
        if keep_mask.shape != (T_out, d) or keep_mask.dtype not in (torch.bool, torch.uint8):
            raise ValueError(f"kmoe.combine: keep_mask must be bool/uint8 {(T_out, d)}, got "
                             f"{keep_mask.dtype} {tuple(keep_mask.shape)}")
        keep_mask = keep_mask.contiguous()
        with _Stage("combine"):
            _lib.call("kmoe_combine_residual_dropout", ptr(yperm), d, ptr(src_row), ptr(src_w), fan, ptr(out_map),
                      ptr(scale), ptr(residual), ptr(keep_mask), float(keep_scale), T_out, ptr(y), ydt,
                      _stream(yperm))
        return y
    with _Stage("combine"):
        _lib.call("kmoe_combine_residual", ptr(yperm), d, ptr(src_row), ptr(src_w), fan, ptr(out_map), ptr(scale),
                  ptr(residual), T_out, ptr(y), ydt, _stream(yperm))
    return y


class ECSelectOut(NamedTuple):
    idx: torch.Tensor        # (B,E,C) int64
    w: torch.Tensor          # (B,E,C) f32
    row_token: torch.Tensor  # (E*B*C,) int32
    offsets: torch.Tensor    # (E+1,) int32
    src_row: torch.Tensor    # (B*S, E) int32
    src_w: torch.Tensor      # (B*S, E) f32


def ec_select(logits, B, S, E, C, descending=True) -> ECSelectOut:
    """Expert-choice top-C per (sequence, expert) (moe.py:494-530).

    descending=True gives the reference's topk order; False the same selection in
    ascending token order (no sort: enough for a layer forward)."""
    _need_gpu(logits)
    logits = _contig(logits, torch.float32)
    dev = logits.device
    idx = torch.empty(B, E, C, device=dev, dtype=torch.int64)
    w = torch.empty(B, E, C, device=dev, dtype=torch.float32)
    row_token = torch.empty(E * B * C, device=dev, dtype=torch.int32)
    offsets = torch.empty(E + 1, device=dev, dtype=torch.int32)
    src_row = torch.empty(B * S, E, device=dev, dtype=torch.int32)
    src_w = torch.empty(B * S, E, device=dev, dtype=torch.float32)
    ws_bytes = _lib.load().kmoe_ec_workspace_bytes(B, S, E)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)  # the logits transposed per expert
    with _Stage("ec_select"):
        _lib.call("kmoe_ec_select", ptr(logits), B, S, E, C, 1 if descending else 0, ptr(idx), ptr(w),
                  ptr(row_token), ptr(offsets), ptr(src_row), ptr(src_w), ptr(ws), ws_bytes, _stream(logits))
    return ECSelectOut(idx, w, row_token, offsets, src_row, src_w)


def ec_dlogits(logits, B, S, E, src_row, src_w, dw, dl):
    """Adds the expert-choice selection's logit gradient (kmoe_ec_dlogits) to dl (B*S, E)."""
    _need_gpu(logits, src_row, src_w, dw, dl)
    with _Stage("bwd_router"):
        _lib.call("kmoe_ec_dlogits", ptr(_contig(logits, torch.float32)), B, S, E, ptr(src_row), ptr(src_w),
                  ptr(_contig(dw, torch.float32)), ptr(dl), _stream(logits))
    return dl


class ModSelectOut(NamedTuple):
    logits: torch.Tensor      # (B,S) f32
    sel_idx: torch.Tensor     # (B,keep) int64 ascending
    sel_w: torch.Tensor       # (B,keep) f32 softmax over kept
    token_rows: torch.Tensor  # (B*keep,) int32
    out_map: torch.Tensor     # (B*S,) int32


def mod_select(x3d, w_mod, keep, logits=None) -> ModSelectOut:
    """Mixture-of-Depths top-keep per sequence (mod.py:67-122).  With `logits` ((B, S)
    f32, e.g. rmsnorm's mod_logits) the selection runs on them and x3d is not read."""
    _need_gpu(x3d, w_mod)
    B, S, d = x3d.shape
    dev = x3d.device
    stream = _stream(x3d)
    if logits is not None:
        logits = _contig(logits, torch.float32).view(B, S)
        x3d = w_mod = None
    else:
        x3d = _contig(x3d, _BF16)
        w_mod = _contig(w_mod, _BF16).reshape(-1)
        logits = torch.empty(B, S, device=dev, dtype=torch.float32)
    sel_idx = torch.empty(B, keep, device=dev, dtype=torch.int64)
    sel_w = torch.empty(B, keep, device=dev, dtype=torch.float32)
    token_rows = torch.empty(B * keep, device=dev, dtype=torch.int32)
    out_map = torch.empty(B * S, device=dev, dtype=torch.int32)
    with _Stage("mod_select"):
        _lib.call("kmoe_mod_select", ptr(x3d), B, S, d, ptr(w_mod), keep, ptr(logits), ptr(sel_idx), ptr(sel_w),
              ptr(token_rows), ptr(out_map), None, 0, stream)
    return ModSelectOut(logits, sel_idx, sel_w, token_rows, out_map)


def _fdt(t):
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    if t.dtype == _BF16:
        return _lib.DTYPE_BF16
    raise ValueError(f"kmoe: unsupported dtype {t.dtype}")


class NormOut(NamedTuple):
    n: torch.Tensor                       # (T, d) bf16 normalised rows
    rrms: torch.Tensor                    # (T,) f32 1/sqrt(mean(x^2) + eps)
    mod_logits: Optional[torch.Tensor]    # (T,) f32 n . w_mod (with w_mod)


def rmsnorm(x2d, weight, eps, w_mod=None) -> NormOut:
    """RMSNorm (embeddings.py:167-195) of the rows of x2d (bf16 or f32) with weight (d,);
    with w_mod (d,) also the MoD router logits of the normalised rows (mod.py:93)."""
    _need_gpu(x2d, weight)
    if x2d.dtype not in (torch.float32, _BF16):
        x2d = x2d.float()
    x2d = x2d.contiguous()
    weight = weight.detach()
    if weight.dtype not in (torch.float32, _BF16):
        weight = weight.float()
    weight = weight.contiguous()
    T, d = x2d.shape
    n = torch.empty(T, d, device=x2d.device, dtype=_BF16)
    rrms = torch.empty(T, device=x2d.device, dtype=torch.float32)
    ml = None
    if w_mod is not None:
        w_mod = _contig(w_mod.detach(), _BF16).reshape(-1)
        ml = torch.empty(T, device=x2d.device, dtype=torch.float32)
    with _Stage("rmsnorm"):
        _lib.call("kmoe_rmsnorm", ptr(x2d), _fdt(x2d), ptr(weight), _fdt(weight), float(eps), T, d, ptr(n), ptr(rrms),
                  ptr(w_mod), ptr(ml), _stream(x2d))
    return NormOut(n, rrms, ml)


def rmsnorm_bwd(dn, x2d, weight, rrms, dres=None, dw_dtype=None):
    """Backward of rmsnorm: (dx in x2d's dtype (+ dres), dweight (d,))."""
    T, d = x2d.shape
    dn = _contig(dn, _BF16)
    weight = weight.detach().contiguous()
    if dres is not None:
        dres = _contig(dres, x2d.dtype)
    dw_dtype = weight.dtype if dw_dtype is None else dw_dtype
    dx = torch.empty(T, d, device=x2d.device, dtype=x2d.dtype)
    dwt = torch.empty(d, device=x2d.device, dtype=dw_dtype)
    lib = _lib.load()
    wsb = lib.kmoe_rmsnorm_bwd_workspace_bytes(T, d)
    ws = torch.empty(max(wsb, 4), device=x2d.device, dtype=torch.uint8)
    with _Stage("bwd_rmsnorm"):
        _lib.call("kmoe_rmsnorm_bwd", ptr(dn), ptr(x2d), _fdt(x2d), ptr(weight), _fdt(weight), ptr(rrms), ptr(dres), T,
                  d, ptr(dx), ptr(dwt), _fdt(dwt), ptr(ws), wsb, _stream(x2d))
    return dx, dwt
