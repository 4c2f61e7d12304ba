"""Seeded sweep of layer shapes against the oracle: the token-choice MoELayer forward
(moe.py:759-813), the fused FFN block (layers.py:142-147, 184-187) and the backward over
random (T, d, E, k, F, capacity, bias) draws (E up to 64, k up to 8), including T not a
multiple of the router's 64-token blocks, F not a multiple of 128, experts that receive
no rows and the capacity drop.

Bars (as the per-kernel tests): routing indices and per-expert counts bit-exact from the
kernel's own fp32 logits; router logits within 2e-5 abs / 1e-4 rel of fp64; the layer
output rel-L2 <= 1e-2 of the fp32 oracle on the same bf16 inputs; the aux loss within
1e-4 relative."""
import os

import numpy as np
import pytest
import torch

from kmoe import ops, synth
from kmoe.block import MoEFFNBlock
from kmoe.config import AdvancedMoEConfig
from kmoe.moe import MoELayer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

# KMOE_SWEEP_DRAWS=N runs N draws of each sweep instead of the default 16 / 6 / 6
_DRAWS = int(os.environ.get("KMOE_SWEEP_DRAWS", "0"))


def _draw(i):
    r = np.random.default_rng(1000 + i)
    E = int(r.choice([2, 3, 4, 8, 16, 33, 64]))
    k = int(r.integers(1, min(E, 8) + 1))
    d = int(64 * r.integers(1, 9))
    F = int(r.choice([8 * r.integers(1, 40), 128 * r.integers(1, 6), 352]))
    T = int(r.integers(1, 1300))
    cap = bool(r.integers(0, 2)) and T * k >= E
    bias = bool(r.integers(0, 2))
    return T, d, E, k, F, cap, bias


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _layer(dev, T, d, E, k, F, cap, bias, seed):
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F, moe_capacity_factor=1.0,
                            moe_drop_overflow=cap,
                            moe_router_bias=synth.zipf_bias(E, seed).tolist() if bias else None)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        layer.router.router[2].weight.copy_(torch.randn(E, 128, generator=g) * 0.05)
        for w in (layer.grouped_experts.w1, layer.grouped_experts.w2, layer.grouped_experts.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)
    return cfg, layer, g


@pytest.mark.parametrize("i", range(_DRAWS or 16))
def test_layer_forward_sweep(dev, i):
    T, d, E, k, F, cap, bias = _draw(i)
    print(f"sweep {i}: T={T} d={d} E={E} k={k} F={F} cap={cap} bias={bias}", flush=True)
    cfg, layer, g = _layer(dev, T, d, E, k, F, cap, bias, 500 + i)
    layer.train()
    x = torch.randn(1, T, d, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        y = layer(x)
        r = layer.router.route(x.reshape(T, d))
    torch.cuda.synchronize()
    f = lambda t: t.detach().float().cpu().numpy()
    b = None if layer.router.logit_bias is None else f(layer.router.logit_bias)
    capacity = ops.capacity_of(1.0, T, k, E) if cap else 0
    lg = f(r.logits)
    ref_lg = O.router_logits(f(x.reshape(T, d)), f(layer.router.router[0].weight), f(layer.router.router[2].weight), b)
    np.testing.assert_allclose(lg, ref_lg, atol=2e-5, rtol=1e-4)
    ge = layer.grouped_experts
    ref = O.moe_forward_tc(f(x.reshape(T, d)), f(layer.router.router[0].weight), f(layer.router.router[2].weight),
                           f(ge.w1), f(ge.w2), f(ge.w3), k, capacity=capacity, logits=lg, bias=b)
    assert np.array_equal(r.idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(layer.last_expert_counts.cpu().numpy(), ref["counts"])
    assert _rel(f(y.reshape(T, d)), ref["y"]) <= 1e-2
    aux = float(layer.aux_loss)
    assert abs(aux - ref["aux"][0]) <= 1e-4 * abs(ref["aux"][0]) + 1e-7


@pytest.mark.parametrize("i", range(_DRAWS or 8))
def test_ec_layer_forward_sweep(dev, i):
    """Expert-choice layers (moe.py:465-530, 588-673) over random shapes: B 1-3, S 8-700, d
    64-384, E 2-64, F from 8 up, capacity factors 0.5-8 (C = min(ceil(S cf / E), S), up to
    every token of a sequence).  The selection is bit-exact against the oracle on the
    kernel's logits, the output within 1e-2 rel-L2 of the oracle on a token sample, and
    tokens no expert selected give 0."""
    r = np.random.default_rng(3000 + i)
    B = int(r.integers(1, 4))
    S = int(r.integers(8, 701))
    E = int(r.choice([2, 4, 8, 16, 33, 64]))
    d = int(64 * r.integers(1, 7))
    F = int(r.choice([8 * r.integers(1, 40), 128 * r.integers(1, 5), 352]))
    cf = float(r.choice([0.5, 1.0, 1.25, 2.0, 8.0]))
    print(f"ec sweep {i}: B={B} S={S} d={d} E={E} F={F} cf={cf}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, d_ff_expert=F, moe_capacity_factor=cf, moe_routing="expert_choice")
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(4000 + i)
    ge = layer.grouped_experts_ec
    with torch.no_grad():
        layer.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        layer.router.router[2].weight.copy_(torch.randn(E, 128, generator=g) * 0.05)
        for w in (ge.w1, ge.w2, ge.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)
    layer.eval()
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        y = layer(x)
        rr, sel, C = layer.router.route(x)
    torch.cuda.synchronize()
    f = lambda t: t.detach().float().cpu().numpy()
    idx_ref, w_ref = O.ec_select(f(rr.logits), B, S, E, C)
    assert np.array_equal(sel.idx.cpu().numpy(), idx_ref)
    _, _, src_row, src_w = O.ec_tables(idx_ref, w_ref, S)
    fan = (src_row >= 0).sum(1)
    X = f(x).reshape(B * S, d).astype(np.float64)
    W1, W2, W3 = (f(w).astype(np.float64) for w in (ge.w1, ge.w2, ge.w3))
    tokens = np.arange(B * S) if B * S <= 600 else np.unique(np.concatenate(
        [r.choice(B * S, 400, replace=False), [int(np.argmax(fan)), int(np.argmin(fan))]]))
    yref = np.zeros((len(tokens), d))
    for n, t in enumerate(tokens):
        for e in np.nonzero(src_row[t] >= 0)[0]:
            gg, uu = X[t] @ W1[e], X[t] @ W2[e]
            yref[n] += src_w[t, e] * ((gg / (1.0 + np.exp(-gg)) * uu) @ W3[e])
    yk = f(y).reshape(B * S, d)[tokens]
    assert _rel(yk, yref) <= 1e-2
    assert np.all(yk[fan[tokens] == 0] == 0)


@pytest.mark.parametrize("i", range(_DRAWS or 6))
def test_ffn_block_sweep(dev, i):
    T, d, E, k, F, cap, bias = _draw(100 + i)
    print(f"block sweep {i}: T={T} d={d} E={E} k={k} F={F} cap={cap} bias={bias}", flush=True)
    cfg, layer, g = _layer(dev, T, d, E, k, F, cap, bias, 700 + i)
    blk = MoEFFNBlock(cfg, 0, ffn=layer)
    blk.ffn_norm.weight = torch.nn.Parameter((1.0 + 0.3 * torch.randn(d, generator=g)).to(dev))
    blk.eval()
    h = (torch.randn(1, T, d, generator=g) * 2).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        out = blk(h)
        w_in_g, w_out_b, _ = blk._fused_weights()
        r = ops.router(h.reshape(T, d), w_in_g, w_out_b, k, bias=layer.router.logit_bias, rms_eps=blk.ffn_norm.eps)
    torch.cuda.synchronize()
    assert blk.last_path == "fused"
    f = lambda t: t.detach().float().cpu().numpy()
    b = None if layer.router.logit_bias is None else f(layer.router.logit_bias)
    capacity = ops.capacity_of(1.0, T, k, E) if cap else 0
    hr = f(h.reshape(T, d)).astype(np.float64)
    ge = layer.grouped_experts
    ref = O.ffn_block_tc(hr, f(blk.ffn_norm.weight), blk.ffn_norm.eps, f(layer.router.router[0].weight),
                         f(layer.router.router[2].weight), f(ge.w1), f(ge.w2), f(ge.w3), k, capacity=capacity,
                         logits=f(r.logits), bias=b)
    assert np.array_equal(layer.last_expert_counts.cpu().numpy(), ref["counts"])
    # f32 output (f32 norm weight): the MoE part at the layer bar
    assert _rel(f(out.reshape(T, d)) - hr, ref["y"] - hr) <= 1e-2


@pytest.mark.parametrize("i", range(_DRAWS or 6))
def test_backward_sweep(dev, i):
    """Gradients of the training path (HIP backward) against fp64 autograd of the oracle's
    restatement of the reference forward at the kernel's routing (as test_gpu_backward.py):
    rel-L2 <= 1e-2 for dx and the expert weights, 2e-2 for the router weights."""
    from oracle import torch_port as P
    T, d, E, k, F, cap, bias = _draw(200 + i)
    print(f"backward sweep {i}: T={T} d={d} E={E} k={k} F={F} cap={cap} bias={bias}", flush=True)
    cfg, layer, g = _layer(dev, T, d, E, k, F, cap, bias, 900 + i)
    layer.train()
    x = torch.randn(1, T, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = torch.randn(1, T, d, generator=g).to(torch.bfloat16)
    loss = (layer(x).float() * dy.to(dev).float()).sum() + layer.aux_loss
    loss.backward()
    torch.cuda.synchronize()
    with torch.no_grad():
        idx = layer.router.route(x.detach().reshape(T, d)).idx.cpu()
    f64 = lambda t: t.detach().double().cpu().clone().requires_grad_(True)
    ge = layer.grouped_experts
    params = [f64(layer.router.router[0].weight), f64(layer.router.router[2].weight), f64(ge.w1), f64(ge.w2),
              f64(ge.w3)]
    xr = f64(x.reshape(T, d))
    b = None if layer.router.logit_bias is None else layer.router.logit_bias.double().cpu()
    ref = P.moe_loss_tc_routed(xr, *params, idx, dy.reshape(T, d).double(),
                               capacity=ops.capacity_of(1.0, T, k, E) if cap else 0, bias=b, training=True,
                               w_lb=layer.load_balance_loss_weight, w_z=layer.router_z_loss_weight)
    ref.backward()
    got = [x.grad.reshape(T, d), layer.router.router[0].weight.grad, layer.router.router[2].weight.grad, ge.w1.grad,
           ge.w2.grad, ge.w3.grad]
    want = [xr.grad] + [p.grad for p in params]
    bars = [1e-2, 2e-2, 2e-2, 1e-2, 1e-2, 1e-2]
    for name, a, w, bar in zip(("dx", "dW_in", "dW_out", "dW1", "dW2", "dW3"), got, want, bars):
        a64 = a.detach().double().cpu()
        if float(w.norm()) == 0.0:
            assert float(a64.norm()) == 0.0, name
            continue
        e = float((a64 - w).norm() / w.norm())
        assert e <= bar, (name, e)
