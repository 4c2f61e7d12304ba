"""torch-CPU restatement of the reference's default PyTorch MoE path
(TEST INFRASTRUCTURE ONLY; the timed CPU baseline of bench.py).

It runs the same sequence of ATen ops as the reference's `batched`
implementation, so its CPU time is the reference's CPU time:
  token choice  Router.forward (moe.py:423-462) then GroupedExperts.forward
                (moe.py:213-294): stable argsort, bincount, cumsum, gather,
                .item() max count, zero-padded (E, max, d) buffer, 3 x bmm,
                gather back, weight multiply, index_add_
  aux losses    moe.py:840-939 (one_hot counts, softmax mean, logsumexp^2)
  expert choice ExpertChoiceRouter.forward (moe.py:494-530) then
                GroupedExpertsExpertChoice.forward (moe.py:626-673) with the
                weight repeat and scatter_add_ (moe.py:132-158)
The code is this build's own; only the op sequence follows the reference.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def router_tc(x3d, w_in, w_out, k):
    """(weights, experts, logits) as Router.forward."""
    logits = F.linear(F.silu(F.linear(x3d, w_in)), w_out)
    probs = F.softmax(logits, dim=-1)
    w, idx = torch.topk(probs, k, dim=-1)
    return w / w.sum(dim=-1, keepdim=True), idx, logits


def balanced_topk_tc(probs, k):
    """Router._balanced_topk_assignment's op sequence (moe.py:353-421) on (T, E)
    probabilities: per round, capacity-masked max, fallback to the unmasked
    max, gather of the original probability, count update, own-pick masking."""
    T, E = probs.shape
    cap = max((T * k) // E, 1)
    sel = torch.zeros(T, k, dtype=torch.long)
    wts = torch.zeros(T, k, dtype=probs.dtype)
    work = probs.clone()
    counts = torch.zeros(E, dtype=torch.long)
    for r in range(k):
        m = work.clone()
        m[:, counts >= cap] = float("-inf")
        best_p, best = m.max(dim=-1)
        reset = best_p == float("-inf")
        if reset.any():
            best[reset] = work[reset].argmax(dim=-1)
        sel[:, r] = best
        wts[:, r] = probs.gather(1, best.unsqueeze(-1)).squeeze(-1)
        counts.scatter_add_(0, best, torch.ones_like(best))
        work.scatter_(1, best.unsqueeze(-1), float("-inf"))
    return wts / (wts.sum(dim=-1, keepdim=True) + 1e-9), sel


def _expert_bmm(padded, w1, w2, w3):
    """The experts' batched products (moe.py:275-283): swiglu (silu(x w1) * (x w2)) w3, or,
    with w3 None, the non-gated silu(x w1) w2."""
    if w3 is None:
        return torch.bmm(F.silu(torch.bmm(padded, w1)), w2)
    return torch.bmm(F.silu(torch.bmm(padded, w1)) * torch.bmm(padded, w2), w3)


def ste(fq, t):
    """Straight-through fake quantisation: the value fq(t), the gradient of t."""
    return t + (fq(t) - t).detach()


def _expert_bmm_fp8_ste(padded, w1, w2, w3, quant_h=True):
    """_expert_bmm with config 5's e4m3 fake quantisation (per-row scales of the input
    rows, per-output-column scales of each expert's weights, h rounded to bf16 and
    re-quantised per row: moe_layer_fp8_mod's scheme), each quantisation
    straight-through: the gradients multiply by the dequantised operands and pass the
    quantisers unchanged to the bf16 master values (the reference's fp8 experts,
    fp8_moe.py:179-279, are differentiated by autograd through their scaled operands)."""
    fqw = lambda w: _fake_e4m3_rows(w.transpose(1, 2)).transpose(1, 2)
    xq = ste(_fake_e4m3_rows, padded)
    w1q, w2q, w3q = ste(fqw, w1), ste(fqw, w2), ste(fqw, w3)
    h = F.silu(torch.bmm(xq, w1q)) * torch.bmm(xq, w2q)
    if quant_h:
        h = ste(lambda t: _fake_e4m3_rows(t.to(torch.bfloat16).to(t.dtype)), h)
    return torch.bmm(h, w3q)


def grouped_experts_tc(x, idx, w, w1, w2, w3, fp8=False):
    """GroupedExperts.forward's padded-bmm formulation (fp8: the experts fake-quantised
    straight-through, _expert_bmm_fp8_ste)."""
    n_tok, k = idx.shape
    E = w1.shape[0]
    flat_e = idx.reshape(-1)
    flat_w = w.reshape(-1)
    tok = torch.arange(n_tok).unsqueeze(1).expand(-1, k).reshape(-1)
    order = torch.argsort(flat_e, stable=True)
    s_tok, s_e, s_w = tok[order], flat_e[order], flat_w[order]
    counts = torch.bincount(flat_e, minlength=E)
    ends = torch.cumsum(counts, 0)
    starts = ends - counts
    rows = x[s_tok]
    m = int(counts.max().item())
    if m == 0:
        return torch.zeros_like(x)
    pos = torch.arange(s_tok.numel()) - starts[s_e]
    padded = x.new_zeros(E, m, x.shape[1])
    padded[s_e, pos] = rows
    out = _expert_bmm_fp8_ste(padded, w1, w2, w3) if fp8 else _expert_bmm(padded, w1, w2, w3)
    contrib = out[s_e, pos] * s_w.unsqueeze(1)
    y = x.new_zeros(x.shape)
    y.index_add_(0, s_tok, contrib)
    return y


def aux_tc(logits, idx, E, w_lb=0.01, w_z=0.001):
    P = F.softmax(logits, dim=-1).mean(dim=[0, 1])
    B, S, k = idx.shape
    f = F.one_hot(idx, num_classes=E).float().sum(dim=[0, 1, 2]) / (B * S * k)
    lb = E * (f * P).sum()
    z = (torch.logsumexp(logits, dim=-1) ** 2).mean()
    return w_lb * lb + w_z * z


def moe_layer_tc(x3d, w_in, w_out, w1, w2, w3, k, training=True):
    """MoELayer token-choice forward (moe.py:782-813): returns (y, aux)."""
    B, S, d = x3d.shape
    w, idx, logits = router_tc(x3d, w_in, w_out, k)
    y = grouped_experts_tc(x3d.reshape(-1, d), idx.reshape(-1, k), w.reshape(-1, k), w1, w2, w3)
    aux = aux_tc(logits, idx, w_out.shape[0]) if training else 0.0
    return y.view(B, S, d), aux


def moe_loss_tc_routed(x2d, w_in, w_out, w1, w2, w3, idx, dy, capacity=0, bias=None, training=True, w_lb=0.01,
                       w_z=0.001, fp8=False):
    """Scalar loss sum(y * dy) (+ aux in training) of MoELayer's token-choice forward with
    the routing fixed to `idx` (T, k): Router.forward's logits / softmax and its top-k
    values gathered at idx and renormalised (moe.py:423-462), GroupedExperts.forward's
    stable-argsort / padded-bmm / index_add_ experts (moe.py:213-294), the load-balance
    and z losses with one-hot counts of idx (moe.py:840-939).  For autograd: at a fixed
    routing the layer is smooth, so the gradients of this loss are the reference's
    backward.  capacity > 0 keeps the first `capacity` assignments of each expert in
    assignment order (the build's drop rule); bias (E,) is added to the logits.
    fp8: the experts fake-quantised straight-through (_expert_bmm_fp8_ste)."""
    y, aux = moe_tc_routed(x2d, w_in, w_out, w1, w2, w3, idx, capacity, bias, training, w_lb, w_z, fp8=fp8)
    return (y * dy).sum() + aux


def moe_tc_routed(x2d, w_in, w_out, w1, w2, w3, idx, capacity=0, bias=None, training=True, w_lb=0.01, w_z=0.001,
                  fp8=False):
    """(y, aux) of moe_loss_tc_routed's layer (aux 0 when not training)."""
    T, d = x2d.shape
    k = idx.shape[1]
    E = w1.shape[0]
    logits = F.linear(F.silu(F.linear(x2d, w_in)), w_out)
    if bias is not None:
        logits = logits + bias
    probs = F.softmax(logits, dim=-1)
    v = probs.gather(1, idx)
    w = v / v.sum(dim=-1, keepdim=True)
    flat_e = idx.reshape(-1)
    tok = torch.arange(T).unsqueeze(1).expand(-1, k).reshape(-1)
    order = torch.argsort(flat_e, stable=True)
    s_tok, s_e, s_w = tok[order], flat_e[order], w.reshape(-1)[order]
    counts = torch.bincount(flat_e, minlength=E)
    starts = torch.cumsum(counts, 0) - counts
    pos = torch.arange(s_tok.numel()) - starts[s_e]
    if capacity > 0:
        keep = pos < capacity
        s_tok, s_e, s_w, pos = s_tok[keep], s_e[keep], s_w[keep], pos[keep]
    y = x2d.new_zeros(x2d.shape)
    if s_tok.numel():
        m = int(pos.max().item()) + 1
        padded = x2d.new_zeros(E, m, d)
        padded = padded.index_put((s_e, pos), x2d[s_tok])
        out = _expert_bmm_fp8_ste(padded, w1, w2, w3) if fp8 else _expert_bmm(padded, w1, w2, w3)
        y = y.index_add(0, s_tok, out[s_e, pos] * s_w.unsqueeze(1))
    aux = x2d.new_zeros(())
    if training:
        f = counts.to(x2d.dtype) / (T * k)
        lb = E * (f * probs.mean(dim=0)).sum()
        z = (torch.logsumexp(logits, dim=-1) ** 2).mean()
        aux = w_lb * lb + w_z * z
    return y, aux


def ffn_half_loss_routed(h3d, w_in, w_out, w1, w2, w3, idx, dy, norm_w=None, eps=1e-5, w_mod=None, sel_idx=None,
                         residual=None, capacity=0, training=True, w_lb=0.01, w_z=0.001, return_out=False,
                         drop_keep=None, p_drop=0.0, fp8=False):
    """Scalar loss sum(out * dy) (+ the MoE aux in training) of the FFN half of
    TransformerBlock.forward (layers.py:142-190) at a fixed MoD selection, routing and
    residual-dropout mask (drop_keep (B, S, d) bool, nn.Dropout's output = input *
    drop_keep * (1 / (1 - p_drop)); None: no dropout):
      x = RMSNorm(h) (embeddings.py:182-195) when norm_w is given, else h
      MoD (w_mod and sel_idx (B, keep) ascending given; layers.py:148-184): router
        logits x . w_mod (mod.py:93), the kept logits in ascending token order
        (mod.py:100-109), their softmax (mod.py:112); gather the kept rows
        (layers.py:160-165), the MoE on them with routing idx (B*keep, k), weight by
        the softmax (layers.py:175), scatter_add_ into zeros (layers.py:180-184)
      no MoD: the MoE on all rows with routing idx (B*S, k)
      out = h + dropout(ffn_output) with a norm (layers.py:187-190), else
        residual + dropout(ffn_output) (residual optional).
    At a fixed selection and routing the composition is smooth: autograd of this loss
    is the reference's backward.  return_out: (loss, out).  fp8: the experts
    fake-quantised straight-through (_expert_bmm_fp8_ste)."""
    B, S, d = h3d.shape
    x = h3d
    if norm_w is not None:
        rms = torch.sqrt(torch.mean(h3d ** 2, dim=-1, keepdim=True) + eps)
        x = norm_w * (h3d / rms)
    if fp8:
        # the layer's activations are bf16 and the e4m3 codes of a row follow from its
        # bf16 values (rounded straight-through, as every bf16 activation is here)
        x = ste(lambda t: t.to(torch.bfloat16).to(t.dtype), x)
    if w_mod is not None:
        keep = sel_idx.shape[1]

        def moe(xs):
            y, aux = moe_tc_routed(xs.reshape(B * keep, d), w_in, w_out, w1, w2, w3, idx, capacity, None, training,
                                   w_lb, w_z, fp8=fp8)
            return y.view(B, keep, d), aux

        ffn_out, aux = mod_apply(x, w_mod, sel_idx, moe)
    else:
        y, aux = moe_tc_routed(x.reshape(B * S, d), w_in, w_out, w1, w2, w3, idx, capacity, None, training, w_lb,
                               w_z, fp8=fp8)
        ffn_out = y.view(B, S, d)
    if drop_keep is not None:
        ffn_out = ffn_out * drop_keep.to(ffn_out.dtype) * (1.0 / (1.0 - p_drop))
    base = h3d if norm_w is not None else residual
    out = ffn_out if base is None else base + ffn_out
    loss = (out * dy).sum() + aux
    return (loss, out) if return_out else loss


def mod_apply(x, w_mod, sel_idx, f):
    """The MoD composition of layers.py:148-184 around f at a fixed selection sel_idx
    (B, keep), ascending: the router logits x . w_mod (mod.py:93), the softmax over the
    kept ones (mod.py:112), f on the gathered rows (B, keep, d) -> (y, aux), the rows
    weighted by the softmax and scatter_add_-ed into zeros.  Returns (ffn_out, aux)."""
    d = x.shape[-1]
    r = (x @ w_mod.reshape(-1, 1)).squeeze(-1)
    p = F.softmax(r.gather(1, sel_idx), dim=-1)
    gidx = sel_idx.unsqueeze(-1).expand(-1, -1, d)
    y, aux = f(torch.gather(x, 1, gidx))
    return torch.zeros_like(x).scatter_add(1, gidx, p.unsqueeze(-1) * y), aux


def mod_aux_loss(x3d, w_a, w_b, sel_idx, weight=0.001):
    """The MoD router's auxiliary loss (mod.py:141-171): weight * mean over (B, S) of
    binary cross-entropy with logits aux_router(x) = Linear(d, h) -> SiLU -> Linear(h, 1)
    (mod.py:44-50) and targets 1 at the selected positions sel_idx (B, keep), 0 elsewhere."""
    a = F.linear(F.silu(F.linear(x3d, w_a)), w_b).squeeze(-1)
    t = torch.zeros_like(a).scatter(1, sel_idx, 1.0)
    return weight * (F.softplus(a) - t * a).mean()


def grouped_experts_ec_tc(x3d, ew, ti, w1, w2, w3, fp8=False):
    """GroupedExpertsExpertChoice.forward (moe.py:626-673): gather the selected tokens,
    bmm SwiGLU with the weights repeated per sequence, weight, scatter_add_ back (fp8:
    the experts fake-quantised straight-through, _expert_bmm_fp8_ste)."""
    B, S, d = x3d.shape
    _, E, C = ti.shape
    gi = ti.unsqueeze(-1).expand(-1, -1, -1, d)
    xin = torch.gather(x3d.unsqueeze(1).expand(-1, E, -1, -1), 2, gi).reshape(B * E, C, d)
    W1, W2 = w1.repeat(B, 1, 1), w2.repeat(B, 1, 1)
    W3 = None if w3 is None else w3.repeat(B, 1, 1)
    out = (_expert_bmm_fp8_ste(xin, W1, W2, W3) if fp8 else _expert_bmm(xin, W1, W2, W3)).view(B, E, C, d)
    wout = out * ew.unsqueeze(-1)
    y = x3d.new_zeros(B, S, d)
    return y.scatter_add(1, ti.reshape(B, E * C).unsqueeze(-1).expand(-1, -1, d), wout.reshape(B, E * C, d))


def ec_weights_routed(logits, ti):
    """ExpertChoiceRouter.forward's weights at a fixed selection ti (B, E, C): softmax of
    the logits over each sequence's tokens, gathered at ti, normalised per expert with
    the + 1e-9 of moe.py:528."""
    probs = F.softmax(logits.transpose(1, 2), dim=-1)
    ew = probs.gather(2, ti)
    return ew / (ew.sum(dim=-1, keepdim=True) + 1e-9)


def moe_layer_ec(x3d, w_in, w_out, w1, w2, w3, cf):
    """MoELayer expert-choice forward (moe.py:815-838) without torch.compile."""
    B, S, d = x3d.shape
    E = w_out.shape[0]
    C = int(math.ceil(S * cf / E))
    logits = F.linear(F.silu(F.linear(x3d, w_in)), w_out)
    probs = F.softmax(logits.transpose(1, 2), dim=-1)
    ew, ti = torch.topk(probs, C, dim=-1)
    ew = ew / (ew.sum(dim=-1, keepdim=True) + 1e-9)
    return grouped_experts_ec_tc(x3d, ew, ti, w1, w2, w3)


def moe_loss_ec_routed(x3d, w_in, w_out, w1, w2, w3, ti, dy, training=True, w_z=0.001, fp8=False):
    """Scalar loss sum(y * dy) (+ w_z * z-loss in training, moe.py:833-836) of MoELayer's
    expert-choice forward with the selection fixed to ti (B, E, C): at a fixed selection
    the layer is smooth, so the autograd gradients of this loss are the reference's."""
    y, aux = ec_layer_routed(x3d, w_in, w_out, w1, w2, w3, ti, training, w_z, fp8=fp8)
    return (y * dy).sum() + aux


def ec_layer_routed(x3d, w_in, w_out, w1, w2, w3, ti, training=True, w_z=0.001, fp8=False):
    """(y, aux) of MoELayer's expert-choice forward (moe.py:815-838) with the selection
    fixed to ti (B, E, C); aux = w_z * z-loss in training (moe.py:833-836), else 0."""
    logits = F.linear(F.silu(F.linear(x3d, w_in)), w_out)
    y = grouped_experts_ec_tc(x3d, ec_weights_routed(logits, ti), ti, w1, w2, w3, fp8=fp8)
    aux = w_z * (torch.logsumexp(logits, dim=-1) ** 2).mean() if training else 0.0
    return y, aux


def ffn_half_loss_ec_routed(x3d, w_in, w_out, w1, w2, w3, ti, dy, w_mod, sel_idx, residual=None, training=True,
                            w_z=0.001, return_out=False):
    """Scalar loss sum(out * dy) (+ the layer's z-loss in training) of the FFN half of
    TransformerBlock.forward with MoD (layers.py:148-187) around an expert-choice
    MoELayer: mod_apply with the expert-choice layer on the kept rows (B, keep, d), its
    selection fixed to ti (B, E, C) over the kept positions; out = residual + ffn_output
    (residual optional).  return_out: (loss, out)."""
    ffn_out, aux = mod_apply(x3d, w_mod, sel_idx,
                             lambda xs: ec_layer_routed(xs, w_in, w_out, w1, w2, w3, ti, training, w_z))
    out = ffn_out if residual is None else residual + ffn_out
    loss = (out * dy).sum() + aux
    return (loss, out) if return_out else loss


def router_loss_routed(x2d, w_in, w_out, idx, gw, gl):
    """sum(w * gw) + sum(logits * gl) of Router.forward (moe.py:423-462) with the top-k
    experts fixed to idx: for the gradients of the router alone."""
    logits = F.linear(F.silu(F.linear(x2d, w_in)), w_out)
    v = F.softmax(logits, dim=-1).gather(1, idx)
    w = v / v.sum(dim=-1, keepdim=True)
    return (w * gw).sum() + (logits * gl).sum()


def _fake_e4m3_rows(m):
    """Per-row e4m3 fake quantisation in fp32 (config 5's scheme, cast mechanics as
    fp8_moe.py:112-125): scale = amax/448, clamp to +-448, float8_e4m3fn cast, back to
    fp32 times the scale."""
    amax = m.abs().amax(dim=-1, keepdim=True)
    inv = torch.where(amax > 0, 448.0 / amax, torch.zeros_like(amax))
    q = (m * inv).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.float32)
    return q * (amax / 448.0)


def fake_quant_expert_weights(w1, w2, w3):
    """Expert weights with per-expert per-output-column e4m3 scales (the columns of w
    (E, K, N) are the output rows of x @ w), dequantised to fp32."""
    fq = lambda w: _fake_e4m3_rows(w.transpose(1, 2)).transpose(1, 2).contiguous()
    return fq(w1), fq(w2), fq(w3)


def moe_layer_fp8_mod(x3d, w_mod, w_in, w_out, w1q, w2q, w3q, k, keep):
    """Config 5 forward: MoD selection of `keep` tokens per sequence (mod.py:93-112:
    r = x w_mod, top-k over the sequence, indices sorted ascending, softmax over the kept
    logits), the token-choice MoE on the gathered rows (moe.py:423-462 routing, the
    padded-bmm experts of moe.py:213-294) with e4m3 fake quantisation (per-token scales
    of x, per-output-row scales of the weights, pre-quantised in w1q/w2q/w3q, h
    held in bf16 and re-quantised per row before the down product), and the weighted scatter back
    (layers.py:170-177).  fp32 arithmetic.  Returns the (B, S, d) output."""
    B, S, d = x3d.shape
    r = (x3d @ w_mod.reshape(-1, 1)).squeeze(-1)
    sel = torch.topk(r, keep, dim=-1).indices.sort(dim=-1).values
    p = F.softmax(r.gather(1, sel), dim=-1)
    gidx = sel.unsqueeze(-1).expand(-1, -1, d)
    rows = torch.gather(x3d, 1, gidx).reshape(-1, d)
    w, idx, _ = router_tc(rows, w_in, w_out, k)
    T = rows.shape[0]
    flat_e = idx.reshape(-1)
    tok = torch.arange(T).unsqueeze(1).expand(-1, k).reshape(-1)
    order = torch.argsort(flat_e, stable=True)
    s_tok, s_e, s_w = tok[order], flat_e[order], w.reshape(-1)[order]
    counts = torch.bincount(flat_e, minlength=w1q.shape[0])
    starts = torch.cumsum(counts, 0) - counts
    pos = torch.arange(s_tok.numel()) - starts[s_e]
    m = int(counts.max().item())
    xq = _fake_e4m3_rows(rows)
    padded = rows.new_zeros(w1q.shape[0], m, d).index_put((s_e, pos), xq[s_tok])
    h = F.silu(torch.bmm(padded, w1q)) * torch.bmm(padded, w2q)
    # h is held in bf16 (the layer's activation dtype) before its re-quantisation
    out = torch.bmm(_fake_e4m3_rows(h.to(torch.bfloat16).to(h.dtype)), w3q)
    y = rows.new_zeros(T, d).index_add(0, s_tok, out[s_e, pos] * s_w.unsqueeze(1))
    return torch.zeros_like(x3d).scatter_add(1, gidx, p.unsqueeze(-1) * y.view(B, keep, d))
