"""Backward of the expert-choice MoE layer and of the router / expert modules called on
their own (the reference's distillation code trains Router + GroupedExperts and the
expert-choice router directly, distill.py:289-314) on the HIP kernels, against fp64
autograd of the oracle's restatements at the kernel's own routing
(oracle/torch_port.py: moe_loss_ec_routed, grouped_experts_tc, grouped_experts_ec_tc,
router_loss_routed, ec_weights_routed; pinned on the CPU by tests/test_oracle.py), fed
the bf16 values of the inputs and parameters.

Tolerance: rel-L2 <= 1e-2 for dx and the expert weight gradients, 2e-2 for the router
and routing-weight gradients (bf16 intermediates, as in test_gpu_backward.py)."""
import pytest
import torch
import torch.nn.functional as F

from kmoe import AdvancedMoEConfig, MoELayer
from kmoe.moe import ExpertChoiceRouter, GroupedExperts, GroupedExpertsExpertChoice, Router
from oracle import torch_port as P

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / max(b.norm(), 1e-30))


def f64(t):
    return t.detach().double().cpu().clone().requires_grad_(True)


def _init(mod, g, scale=0.05):
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * scale)


def _check(errs, loose=()):
    print("rel-L2:", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (2e-2 if n in loose else 1e-2), (n, e, errs)


@pytest.mark.parametrize("B,S,d,E,F,cf,train,fp8", [(2, 256, 256, 8, 512, 2.0, True, False),
                                                    (1, 512, 384, 4, 320, 1.0, True, False),
                                                    (2, 192, 256, 16, 256, 2.0, False, False),
                                                    (2, 256, 256, 8, 512, 2.0, True, True)])
def test_ec_layer_backward(dev, B, S, d, E, F, cf, train, fp8):
    """fp8: the experts straight-through, against the fake-quantised restatement."""
    print(f"ec layer backward B={B} S={S} d={d} E={E} F={F} cf={cf} train={train} fp8={fp8}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, d_ff_expert=F, moe_routing="expert_choice",
                            moe_capacity_factor=cf, moe_router_z_loss_weight=0.01, moe_fp8=fp8)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(B * S + E)
    _init(layer, g)
    layer.train(train)
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(torch.bfloat16)
    y = layer(x)
    loss = (y.float() * dy.to(dev).float()).sum()
    if train:
        loss = loss + layer.aux_loss
    loss.backward()
    torch.cuda.synchronize()
    with torch.no_grad():
        _, sel, C = layer.router.route(x.detach())
    ti = sel.idx.cpu()
    ge = layer.grouped_experts_ec
    mods = [layer.router.router[0].weight, layer.router.router[2].weight, ge.w1, ge.w2, ge.w3]
    params = [f64(p) for p in mods]
    xr = f64(x)
    ref = P.moe_loss_ec_routed(xr, *params, ti, dy.double(), training=train, w_z=0.01, fp8=fp8)
    ref.backward()
    names = ["dx", "dw_in", "dw_out", "dw1", "dw2", "dw3"]
    got = [x.grad] + [p.grad for p in mods]
    want = [xr.grad] + [p.grad for p in params]
    _check({n: _rel(a, b) for n, a, b in zip(names, got, want)}, loose=("dw_in", "dw_out"))


@pytest.mark.parametrize("T,d,E,k,F,fp8", [(600, 256, 8, 2, 512, False), (333, 128, 16, 4, 256, False),
                                            (600, 256, 8, 2, 512, True)])
def test_grouped_experts_direct_backward(dev, T, d, E, k, F, fp8):
    """GroupedExperts.forward(x, idx, w) trained directly: gradients of x, of the routing
    weights w and of w1 / w2 / w3 (moe.py:213-294); fp8: straight-through."""
    print(f"grouped experts direct backward T={T} E={E} k={k} fp8={fp8}", flush=True)
    ge = GroupedExperts(E, d, F).to(dev, torch.bfloat16)
    ge.use_fp8 = fp8
    g = torch.Generator().manual_seed(T + E)
    _init(ge, g)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(dev)
    w = torch.softmax(torch.randn(T, k, generator=g), -1).to(dev).requires_grad_(True)
    dy = torch.randn(T, d, generator=g).to(torch.bfloat16)
    y = ge(x, idx, w)
    (y.float() * dy.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    params = [f64(ge.w1), f64(ge.w2), f64(ge.w3)]
    xr, wr = f64(x), f64(w)
    ref = (P.grouped_experts_tc(xr, idx.cpu(), wr, *params, fp8=fp8) * dy.double()).sum()
    ref.backward()
    names = ["dx", "dw", "dw1", "dw2", "dw3"]
    got = [x.grad, w.grad, ge.w1.grad, ge.w2.grad, ge.w3.grad]
    want = [xr.grad, wr.grad] + [p.grad for p in params]
    _check({n: _rel(a, b) for n, a, b in zip(names, got, want)}, loose=("dw",))


def test_grouped_experts_ec_direct_backward(dev):
    """GroupedExpertsExpertChoice.forward(x, w, idx) trained directly (moe.py:626-673)."""
    B, S, d, E, C, F = 2, 96, 128, 4, 40, 256
    ge = GroupedExpertsExpertChoice(E, d, F).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(3)
    _init(ge, g)
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    ti = torch.stack([torch.stack([torch.randperm(S, generator=g)[:C] for _ in range(E)]) for _ in range(B)]).to(dev)
    w = torch.rand(B, E, C, generator=g).to(dev).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(torch.bfloat16)
    y = ge(x, w, ti)
    (y.float() * dy.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    params = [f64(ge.w1), f64(ge.w2), f64(ge.w3)]
    xr, wr = f64(x), f64(w)
    ref = (P.grouped_experts_ec_tc(xr, wr, ti.cpu(), *params) * dy.double()).sum()
    ref.backward()
    names = ["dx", "dw", "dw1", "dw2", "dw3"]
    got = [x.grad, w.grad, ge.w1.grad, ge.w2.grad, ge.w3.grad]
    want = [xr.grad, wr.grad] + [p.grad for p in params]
    _check({n: _rel(a, b) for n, a, b in zip(names, got, want)}, loose=("dw",))


def test_router_direct_backward(dev):
    """Router.forward trained on its own: gradients through the renormalised top-k
    weights and the logits to x, w_in, w_out (moe.py:423-462)."""
    T, d, E, k = 500, 256, 8, 2
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k)
    router = Router(cfg).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    _init(router, g, 0.1)
    x = torch.randn(1, T, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    gw, gl = torch.randn(1, T, k, generator=g), torch.randn(1, T, E, generator=g)
    w, idx, logits = router(x)
    ((w.float() * gw.to(dev)).sum() + (logits.float() * gl.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    params = [f64(router.router[0].weight), f64(router.router[2].weight)]
    xr = f64(x[0])
    ref = P.router_loss_routed(xr, *params, idx[0].cpu(), gw[0].double(), gl[0].double())
    ref.backward()
    errs = {"dx": _rel(x.grad[0], xr.grad), "dw_in": _rel(router.router[0].weight.grad, params[0].grad),
            "dw_out": _rel(router.router[2].weight.grad, params[1].grad)}
    _check(errs, loose=("dx", "dw_in", "dw_out"))


def test_ec_router_direct_backward(dev):
    """ExpertChoiceRouter.forward trained on its own: gradients through the (B, E, C)
    weights (softmax over tokens, per-expert normalisation) and the logits."""
    B, S, d, E = 2, 256, 128, 8
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_routing="expert_choice", moe_capacity_factor=2.0)
    router = ExpertChoiceRouter(cfg).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(8)
    _init(router, g, 0.1)
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    w, ti, logits, C = router(x)
    gw, gl = torch.randn(w.shape, generator=g), torch.randn(logits.shape, generator=g)
    ((w.float() * gw.to(dev)).sum() + (logits.float() * gl.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    params = [f64(router.router[0].weight), f64(router.router[2].weight)]
    xr = f64(x)
    lg = F.linear(F.silu(F.linear(xr, params[0])), params[1])
    ref = (P.ec_weights_routed(lg, ti.cpu()) * gw.double()).sum() + (lg * gl.double()).sum()
    ref.backward()
    errs = {"dx": _rel(x.grad, xr.grad), "dw_in": _rel(router.router[0].weight.grad, params[0].grad),
            "dw_out": _rel(router.router[2].weight.grad, params[1].grad)}
    _check(errs, loose=("dx", "dw_in", "dw_out"))
