"""Non-gated experts (an activation other than swiglu: y = silu(x w1) w2 with w2 (E, F, d),
moe.py:180-191, 281-283) on the HIP kernels: the packed layouts against the host-built
layout bit for bit, the layer forward (token choice with and without the capacity drop,
expert choice) against the oracle's plain_rows / torch port at the kernel's own routing,
and the backward against fp64 autograd of the oracle's routed losses with w3 None (pinned
on the CPU by tests/test_oracle.py).

Tolerance: forward rel-L2 <= 1e-2 (bf16 operands, h rounded to bf16 once); gradients as in
test_gpu_backward.py: 1e-2 for dx and the expert weights, 2e-2 for the router weights."""
import numpy as np
import pytest
import torch

from kmoe import AdvancedMoEConfig, MoELayer, ops
from kmoe import backward as BW
from kmoe.moe import GroupedExperts
from oracle import moe_oracle as O
from oracle import torch_port as P

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = torch.as_tensor(a).double().cpu()
    b = torch.as_tensor(b).double().cpu()
    return float((a - b).norm() / max(b.norm(), 1e-30))


def f64(t):
    return t.detach().double().cpu().clone().requires_grad_(True)


def _bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy()


@pytest.mark.parametrize("E,d,F", [(3, 192, 200), (2, 64, 13), (4, 256, 512)])
def test_plain_packs_match_host_layout(dev, E, d, F):
    print(f"plain packs E={E} d={d} F={F}", flush=True)
    g = torch.Generator().manual_seed(E + d + F)
    w1, w2 = torch.randn(E, d, F, generator=g), torch.randn(E, F, d, generator=g)
    pp = ops.pack_weights_plain(w1.to(dev), w2.to(dev))
    bw = BW.pack_bwd_weights(w1.to(dev), w2.to(dev), None, None)
    torch.cuda.synchronize()
    assert bw.plain
    Fp, F256, dp = (F + 127) // 128 * 128, (F + 255) // 256 * 256, (d + 255) // 256 * 256
    b1, b2 = _bits(w1), _bits(w2)
    w1t = np.zeros((E, F256, d + 64), np.int16)
    w2t = np.zeros((E, dp, Fp + 64), np.int16)
    w2n = np.zeros((E, F256, d + 64), np.int16)
    w1n = np.zeros((E, dp, Fp + 64), np.int16)
    for e in range(E):
        w1t[e, :F, :d] = b1[e].T
        w2t[e, :d, :F] = b2[e].T
        w2n[e, :F, :d] = b2[e]
        w1n[e, :d, :F] = b1[e]
    for got, want in ((pp.w1t, w1t), (pp.w2t, w2t), (bw.w3n, w2n), (bw.w13t, w1n)):
        assert np.array_equal(got.cpu().view(torch.int16).numpy().reshape(want.shape), want)


def _layer(dev, cfg, seed):
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    return layer, g


@pytest.mark.parametrize("T,d,E,k,F,cap", [(1000, 256, 8, 2, 352, None), (700, 384, 16, 4, 200, 1.0)])
def test_plain_layer_forward(dev, T, d, E, k, F, cap):
    print(f"plain forward T={T} d={d} E={E} k={k} F={F} cap={cap}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F, ffn_activation="gelu",
                            moe_capacity_factor=cap or 1.25, moe_drop_overflow=cap is not None)
    layer, g = _layer(dev, cfg, T + d)
    layer.eval()
    x = torch.randn(1, T, d, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        y = layer(x)
        r = layer.router.route(x.reshape(T, d))
    torch.cuda.synchronize()
    ge = layer.grouped_experts
    capacity = int(np.ceil(cap * T * k / E)) if cap is not None else 0
    # routing from the kernel's logits; experts: the oracle's non-gated rows
    idx, w = O.topk_select(r.logits.cpu().numpy(), k)
    dp = O.dispatch(idx, E, capacity)
    xr = x.reshape(T, d).float().cpu().numpy().astype(np.float64)
    rows = xr[dp["row_token"][: dp["offsets"][E]]]
    yr = O.plain_rows(rows, dp["offsets"], ge.w1.detach().float().cpu().numpy(), ge.w2.detach().float().cpu().numpy(),
                      dtype=np.float64)
    want = O.combine(yr, dp["slot_row"].reshape(T, k), w)
    assert np.array_equal(layer.last_expert_counts.cpu().numpy(), dp["counts"])
    assert _rel(y.reshape(T, d).float(), want) <= 1e-2


def test_plain_expert_choice_forward(dev):
    print("plain expert-choice forward", flush=True)
    B, S, d, E, F = 2, 256, 256, 8, 320
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, d_ff_expert=F, ffn_activation="relu", moe_routing="expert_choice",
                            moe_capacity_factor=2.0)
    layer, g = _layer(dev, cfg, 77)
    layer.eval()
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        y = layer(x)
        _, sel, C = layer.router.route(x)
    torch.cuda.synchronize()
    ge = layer.grouped_experts_ec
    want = P.grouped_experts_ec_tc(x.double().cpu(), sel.w.double().cpu(), sel.idx.cpu(), ge.w1.detach().double().cpu(),
                                   ge.w2.detach().double().cpu(), None)
    assert _rel(y.float(), want) <= 1e-2


@pytest.mark.parametrize("B,S,d,E,k,F,cap", [(2, 256, 256, 8, 2, 352, None), (1, 600, 384, 16, 4, 200, 1.0)])
def test_plain_layer_backward(dev, B, S, d, E, k, F, cap):
    print(f"plain backward B={B} S={S} d={d} E={E} k={k} F={F} cap={cap}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F, ffn_activation="gelu",
                            moe_capacity_factor=cap or 1.25, moe_drop_overflow=cap is not None)
    layer, g = _layer(dev, cfg, B * S + d)
    layer.train()
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(torch.bfloat16)
    y = layer(x)
    ((y.float() * dy.to(dev).float()).sum() + layer.aux_loss).backward()
    torch.cuda.synchronize()
    T = B * S
    with torch.no_grad():
        idx = layer.router.route(x.detach().reshape(T, d)).idx.cpu()
    ge = layer.grouped_experts
    mods = [layer.router.router[0].weight, layer.router.router[2].weight, ge.w1, ge.w2]
    params = [f64(p) for p in mods]
    xr = f64(x.reshape(T, d))
    capacity = int(np.ceil(cap * T * k / E)) if cap is not None else 0
    ref = P.moe_loss_tc_routed(xr, params[0], params[1], params[2], params[3], None, idx, dy.reshape(T, d).double(),
                               capacity=capacity, training=True, w_lb=layer.load_balance_loss_weight,
                               w_z=layer.router_z_loss_weight)
    ref.backward()
    errs = {"dx": _rel(x.grad.reshape(T, d), xr.grad)}
    errs.update({n: _rel(p.grad, q.grad) for n, p, q in zip(["dw_in", "dw_out", "dw1", "dw2"], mods, params)})
    print("  rel-L2:", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (2e-2 if n in ("dw_in", "dw_out") else 1e-2), (n, e)


def test_plain_ec_backward(dev):
    print("plain expert-choice backward", flush=True)
    B, S, d, E, F = 2, 256, 256, 8, 512
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, d_ff_expert=F, ffn_activation="gelu", moe_routing="expert_choice",
                            moe_capacity_factor=2.0, moe_router_z_loss_weight=0.01)
    layer, g = _layer(dev, cfg, 91)
    layer.train()
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(torch.bfloat16)
    y = layer(x)
    ((y.float() * dy.to(dev).float()).sum() + layer.aux_loss).backward()
    torch.cuda.synchronize()
    with torch.no_grad():
        _, sel, C = layer.router.route(x.detach())
    ge = layer.grouped_experts_ec
    mods = [layer.router.router[0].weight, layer.router.router[2].weight, ge.w1, ge.w2]
    params = [f64(p) for p in mods]
    xr = f64(x)
    ref = P.moe_loss_ec_routed(xr, params[0], params[1], params[2], params[3], None, sel.idx.cpu(), dy.double(),
                               training=True, w_z=0.01)
    ref.backward()
    errs = {"dx": _rel(x.grad, xr.grad)}
    errs.update({n: _rel(p.grad, q.grad) for n, p, q in zip(["dw_in", "dw_out", "dw1", "dw2"], mods, params)})
    print("  rel-L2:", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (2e-2 if n in ("dw_in", "dw_out") else 1e-2), (n, e)


def test_plain_grouped_experts_direct(dev):
    """GroupedExperts(activation != swiglu) called on its own, trained directly."""
    print("plain direct experts backward", flush=True)
    T, d, E, k, F = 500, 256, 8, 2, 256
    ge = GroupedExperts(E, d, F, activation="silu").to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in ge.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(dev)
    w = torch.softmax(torch.randn(T, k, generator=g), -1).to(dev).requires_grad_(True)
    dy = torch.randn(T, d, generator=g).to(torch.bfloat16)
    y = ge(x, idx, w)
    (y.float() * dy.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    xr, wr, p1, p2 = f64(x), f64(w), f64(ge.w1), f64(ge.w2)
    ref = (P.grouped_experts_tc(xr, idx.cpu(), wr, p1, p2, None) * dy.double()).sum()
    ref.backward()
    errs = {"y": _rel(y.float(), P.grouped_experts_tc(xr.detach(), idx.cpu(), wr.detach(), p1.detach(), p2.detach(),
                                                         None)),
            "dx": _rel(x.grad, xr.grad), "dw": _rel(w.grad, wr.grad), "dw1": _rel(ge.w1.grad, p1.grad),
            "dw2": _rel(ge.w2.grad, p2.grad)}
    print("  rel-L2:", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (2e-2 if n == "dw" else 1e-2), (n, e)
