"""Backward pass of the token-choice MoE layer on the HIP kernels vs autograd of
the oracle's fp64 restatement of the reference forward at a fixed routing
(oracle/torch_port.moe_loss_tc_routed: moe.py:423-462 router, moe.py:213-294
experts + combine, moe.py:840-939 aux losses; pinned on the CPU by
tests/test_oracle.py), fed the kernel's own routing (the selection is pinned
bit-exactly by the forward tests) and the bf16 values of the inputs and parameters.

Tolerance: rel-L2 <= 1e-2 for dx and the expert weight gradients, 2e-2 for the
router weight gradients (bf16 intermediates: the permuted dy rows, dh, dg/du, the
saved g/u and the router's da are rounded to bf16 once each).
"""
import numpy as np
import pytest
import torch

import kmoe  # noqa: F401
from kmoe import synth
from oracle import torch_port as P
from kmoe.config import AdvancedMoEConfig
from kmoe.moe import MoELayer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / max(b.norm(), 1e-30))


def _run(dev, B, S, d, E, k, F, seed, drop_cf=None, train=True, zipf=False, empty_expert=None, dy_zero=False,
         fp8=False):
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F,
                            moe_capacity_factor=drop_cf or 1.25, moe_drop_overflow=drop_cf is not None,
                            moe_router_bias=synth.zipf_bias(E, seed).tolist() if zipf else None, moe_fp8=fp8)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        layer.router.router[2].weight.copy_(torch.randn(E, 128, generator=g) * 0.05)
        if empty_expert is not None:
            # a large negative logit bias keeps expert `empty_expert` out of every top-k
            b = torch.zeros(E)
            b[empty_expert] = -1e4
            layer.router.logit_bias = b.to(dev)
        for w in (layer.grouped_experts.w1, layer.grouped_experts.w2, layer.grouped_experts.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)
    layer.train(train)
    x = (torch.randn(B, S, d, generator=g)).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(torch.bfloat16)
    if dy_zero:
        dy.zero_()
    y = layer(x)
    loss = (y.float() * dy.to(dev).float()).sum()
    if train:
        loss = loss + layer.aux_loss
    loss.backward()
    torch.cuda.synchronize()
    # the kernel's routing (deterministic: same call as the forward's)
    with torch.no_grad():
        r = layer.router.route(x.detach().reshape(B * S, d))
    idx = r.idx.cpu()
    f64 = lambda t: t.detach().double().cpu().clone().requires_grad_(True)
    ge = layer.grouped_experts
    params = [f64(layer.router.router[0].weight), f64(layer.router.router[2].weight), f64(ge.w1), f64(ge.w2),
              f64(ge.w3)]
    xr = f64(x.reshape(B * S, d))
    cap = int(np.ceil(drop_cf * B * S * k / E)) if drop_cf is not None else 0
    bias = None if layer.router.logit_bias is None else layer.router.logit_bias.double().cpu()
    ref = P.moe_loss_tc_routed(xr, *params, idx, dy.reshape(B * S, d).double(), capacity=cap, bias=bias,
                               training=train, w_lb=layer.load_balance_loss_weight, w_z=layer.router_z_loss_weight,
                               fp8=fp8)
    ref.backward()
    got = [x.grad.reshape(B * S, d), layer.router.router[0].weight.grad, layer.router.router[2].weight.grad,
           ge.w1.grad, ge.w2.grad, ge.w3.grad]
    want = [xr.grad] + [p.grad for p in params]
    names = ["dx", "dw_in", "dw_out", "dw1", "dw2", "dw3"]
    errs = {n: _rel(a, b) for n, a, b in zip(names, got, want)}
    for t in got:
        assert torch.isfinite(t.float()).all()
    return errs, layer, idx


def _check(errs):
    print("rel-L2:", {n: f"{e:.2e}" for n, e in errs.items()})
    for n, e in errs.items():
        tol = 2e-2 if n in ("dw_in", "dw_out") else 1e-2
        assert e <= tol, (n, e, errs)


@pytest.mark.parametrize("B,S,d,E,k,F", [(2, 256, 256, 8, 2, 512), (1, 640, 384, 4, 2, 320),
                                         (2, 512, 512, 16, 2, 768)])
def test_backward_parity(dev, B, S, d, E, k, F):
    errs, _, _ = _run(dev, B, S, d, E, k, F, seed=100 + F)
    _check(errs)


@pytest.mark.parametrize("B,S,d,E,k,F,drop_cf", [(2, 256, 256, 8, 2, 512, None), (1, 640, 384, 4, 2, 320, None),
                                                 (2, 512, 256, 8, 2, 256, 1.0)])
def test_backward_fp8_straight_through(dev, B, S, d, E, k, F, drop_cf):
    """fp8 experts (config 5's e4m3 scheme) train straight-through on bf16 master
    weights: against fp64 autograd of the fake-quantised restatement
    (oracle/torch_port._expert_bmm_fp8_ste, pinned by tests/test_oracle.py), whose
    gradients pass the quantisers unchanged and multiply by the dequantised operands.
    Same bars as the bf16 backward."""
    print(f"fp8 straight-through backward B={B} S={S} d={d} E={E} F={F} cf={drop_cf}", flush=True)
    errs, _, _ = _run(dev, B, S, d, E, k, F, seed=300 + F, drop_cf=drop_cf, fp8=True)
    _check(errs)


def test_backward_capacity_drop(dev):
    """Capacity drop (cf 1.0, Zipf bias): dropped slots contribute no gradient."""
    errs, layer, idx = _run(dev, 2, 256, 256, 8, 2, 512, seed=7, drop_cf=1.0, zipf=True)
    counts = np.bincount(idx.numpy().reshape(-1), minlength=8)
    assert counts.max() > int(np.ceil(1.0 * 512 * 2 / 8)), "the test needs an overflowing expert"
    _check(errs)


def test_backward_empty_expert(dev):
    """An expert that receives no rows gets exactly zero weight gradients."""
    errs, layer, idx = _run(dev, 1, 512, 256, 8, 2, 256, seed=9, empty_expert=3)
    assert not (idx.numpy() == 3).any()
    ge = layer.grouped_experts
    for w in (ge.w1, ge.w2, ge.w3):
        assert torch.count_nonzero(w.grad[3]) == 0
    _check(errs)


def test_backward_eval_mode_no_aux(dev):
    """Eval mode: aux_loss is 0.0 and the gradients come from y alone."""
    errs, layer, _ = _run(dev, 2, 256, 256, 8, 2, 512, seed=11, train=False)
    assert layer.aux_loss == 0.0
    _check(errs)


def test_backward_aux_only(dev):
    """Loss = aux alone: the router gradients come only from the load-balance and z
    losses (softmax backward of mean_t p and of lse^2); the experts get exact zeros."""
    errs, layer, _ = _run(dev, 2, 256, 256, 8, 2, 512, seed=13, dy_zero=True)
    ge = layer.grouped_experts
    for w in (ge.w1, ge.w2, ge.w3):
        assert torch.count_nonzero(w.grad) == 0
    assert torch.count_nonzero(layer.router.router[0].weight.grad) > 0
    errs.pop("dw1"), errs.pop("dw2"), errs.pop("dw3")
    _check(errs)


def test_backward_deterministic(dev):
    """Two backward passes over the same inputs give bit-identical gradients."""
    cfg = AdvancedMoEConfig(d_model=512, n_experts=8, moe_top_k=2, d_ff_expert=512)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16).train()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 512, 512, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(2, 512, 512, generator=g).to(torch.bfloat16).to(dev)
    grads = []
    for _ in range(2):
        layer.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        y = layer(xx)
        ((y.float() * dy.float()).sum() + layer.aux_loss).backward()
        grads.append([xx.grad.clone()] + [p.grad.clone() for p in layer.parameters()])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_backward_full_size(dev):
    """Config-2 shape (T=16384, d=2048, E=16, top-2, F=2816): dx on 64 sampled tokens
    against an fp64 per-token restatement (aux terms with the global counts and T),
    dW_out against fp64 from the saved router tensors, dW3 / dW1 of the smallest expert
    on sampled columns / rows against fp64 of the saved h, g/u and the weighted dy
    rows; a second backward over the same saved forward is bit-identical."""
    from kmoe import backward as BW
    wl = synth.WORKLOADS[2]
    t = synth.make_tensors(wl, "cpu")
    layer = synth.build_layer(wl, dev, {kk: v.to(dev) for kk, v in t.items()}).train()
    T, d, E, k, F = wl.T, wl.d, wl.E, wl.k, wl.F
    x2d = t["x"].reshape(T, d).to(dev)
    g = torch.Generator().manual_seed(77)
    dy = torch.randn(T, d, generator=g).to(torch.bfloat16)
    w_out = layer.router.router[2].weight
    wlb, wz = layer.load_balance_loss_weight, layer.router_z_loss_weight
    with torch.no_grad():
        _, _, sv = layer._train_forward(x2d, T, torch.bfloat16)
        ga = torch.ones((), device=dev)
        bw = layer._bwd_weights()
        g1 = BW.moe_backward(sv, dy.to(dev), ga, w_out, bw, E, F, wlb, wz)
        g2 = BW.moe_backward(sv, dy.to(dev), ga, w_out, bw, E, F, wlb, wz)
    torch.cuda.synchronize()
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    for a in g1:
        assert torch.isfinite(a.float()).all()
    cpu = lambda z: z.detach().cpu()
    idx, counts = cpu(sv.idx), cpu(sv.disp.counts).double()
    f = counts / (T * k)
    W = {n: cpu(p).double() for n, p in (("w_in", layer.router.router[0].weight), ("w_out", w_out))}
    ge = layer.grouped_experts

    # 1) dx on a token sample: the gradient w.r.t. x_S of the loss restricted to S
    S = torch.randperm(T, generator=g)[:64]
    xs = cpu(x2d)[S].double().requires_grad_(True)
    logits = torch.nn.functional.silu(xs @ W["w_in"].T) @ W["w_out"].T
    p = torch.softmax(logits, -1)
    ids = idx[S]
    v = p.gather(1, ids)
    wsel = v / v.sum(1, keepdim=True)
    y = torch.zeros_like(xs)
    for e in torch.unique(ids).tolist():
        w1, w2, w3 = (cpu(w[e]).double() for w in (ge.w1, ge.w2, ge.w3))
        rr, jj = torch.nonzero(ids == e, as_tuple=True)
        h = torch.nn.functional.silu(xs[rr] @ w1) * (xs[rr] @ w2)
        y = y.index_add(0, rr, wsel[rr, jj, None] * (h @ w3))
    loss = (y * dy[S].double()).sum()
    loss = loss + wlb * E * (f * p.sum(0) / T).sum() + wz * (torch.logsumexp(logits, -1) ** 2).sum() / T
    loss.backward()
    e_dx = _rel(cpu(g1.dx)[S], xs.grad)

    # 2) dW_out over all tokens from the saved router tensors (fp64)
    slot_row, slot_w = cpu(sv.disp.slot_row).long(), cpu(sv.disp.slot_w).double()
    yp = cpu(sv.yperm).double()
    dyd = dy.double()
    dw = (dyd.repeat_interleave(k, 0) * yp[slot_row.clamp(min=0)]).sum(1) * (slot_row >= 0)
    dw = dw.view(T, k)
    wk = cpu(sv.w).double()
    dl = torch.zeros(T, E, dtype=torch.float64)
    dl.scatter_add_(1, idx, wk * (dw - (wk * dw).sum(1, keepdim=True)))
    lg = cpu(sv.logits).double()
    pp = torch.softmax(lg, -1)
    lse = torch.logsumexp(lg, -1, keepdim=True)
    dl += wlb * E / T * pp * (f - (pp * f).sum(1, keepdim=True)) + wz * 2.0 / T * lse * pp
    s_act = torch.nn.functional.silu(cpu(sv.hidden).double())
    e_dwout = _rel(cpu(g1.dw_out), dl.T @ s_act)

    # 3) dW3 / dW1 of the smallest expert on sampled columns / rows
    offs = cpu(sv.disp.offsets).long()
    e = int(torch.argmin(offs[1:] - offs[:-1]))
    lo, hi = int(offs[e]), int(offs[e + 1])
    wr = torch.zeros(T * k, dtype=torch.float64)
    keep = slot_row >= 0
    wr[slot_row[keep]] = slot_w[keep]
    tok = cpu(sv.disp.row_token).long()[lo:hi]
    dY = wr[lo:hi, None] * dyd[tok]                      # weighted dy rows of the expert
    Fp = (F + 127) // 128 * 128
    h = cpu(sv.h)[lo:hi, :F].double()
    cols = torch.randperm(d, generator=g)[:16]
    e_dw3 = _rel(cpu(g1.dw3[e])[:, cols], h.T @ dY[:, cols])
    gu = cpu(sv.gu)[lo:hi].double()
    fcol = torch.arange(F)
    gc = (fcol // 128) * 256 + fcol % 128
    gg, uu = gu[:, gc], gu[:, gc + 128]
    dh = dY @ cpu(ge.w3[e]).double().T
    sg = torch.sigmoid(gg)
    dg = dh * uu * sg * (1 + gg * (1 - sg))
    rows_i = torch.randperm(d, generator=g)[:16]
    xe = cpu(x2d)[tok].double()
    e_dw1 = _rel(cpu(g1.dw1[e])[rows_i], xe[:, rows_i].T @ dg)
    errs = {"dx_sample": e_dx, "dw_out": e_dwout, "dw3_e": e_dw3, "dw1_e": e_dw1}
    print("full-size rel-L2:", {n: f"{v:.2e}" for n, v in errs.items()}, "expert", e, "rows", hi - lo)
    assert e_dx <= 1e-2 and e_dw3 <= 1e-2 and e_dw1 <= 1e-2 and e_dwout <= 2e-2, errs


def test_second_backward_raises(dev):
    """A second backward through the same graph (retain_graph=True) fails with a clear
    error instead of inside the kernels."""
    print("second backward", flush=True)
    cfg = AdvancedMoEConfig(d_model=128, n_experts=4, moe_top_k=2, d_ff_expert=256)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16).train()
    x = torch.randn(1, 64, 128, device=dev, dtype=torch.bfloat16, requires_grad=True)
    y = layer(x)
    loss = y.float().square().sum() + layer.aux_loss
    loss.backward(retain_graph=True)
    with pytest.raises(RuntimeError, match="once per forward"):
        loss.backward()


def test_backward_balanced_routing(dev):
    """Balanced routing (moe.py:353-421) trains through the same kernels: the gradients at
    the balanced picks match fp64 autograd of the routed restatement."""
    print("backward balanced routing", flush=True)
    B, S, d, E, k, F = 2, 256, 256, 8, 2, 512
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F, moe_balanced_routing=True)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16).train()
    g = torch.Generator().manual_seed(17)
    with torch.no_grad():
        layer.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        w_out = torch.randn(E, 128, generator=g) * 0.05
        # experts 0 and 1 are every token's top two, each the first choice of about half
        # the tokens: both fill up in the first round, so the second round moves picks
        v = torch.randn(128, generator=g) * 0.2
        w_out[0] += 0.3 + v
        w_out[1] += 0.3 - v
        layer.router.router[2].weight.copy_(w_out)
        for w in (layer.grouped_experts.w1, layer.grouped_experts.w2, layer.grouped_experts.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(torch.bfloat16)
    y = layer(x)
    ((y.float() * dy.to(dev).float()).sum() + layer.aux_loss).backward()
    torch.cuda.synchronize()
    with torch.no_grad():
        r = layer.router.route(x.detach().reshape(B * S, d))
    idx = r.idx.cpu()
    f64 = lambda t: t.detach().double().cpu().clone().requires_grad_(True)
    ge = layer.grouped_experts
    params = [f64(layer.router.router[0].weight), f64(layer.router.router[2].weight), f64(ge.w1), f64(ge.w2),
              f64(ge.w3)]
    xr = f64(x.reshape(B * S, d))
    ref = P.moe_loss_tc_routed(xr, *params, idx, dy.reshape(B * S, d).double(), training=True,
                               w_lb=layer.load_balance_loss_weight, w_z=layer.router_z_loss_weight)
    ref.backward()
    got = [x.grad.reshape(B * S, d), layer.router.router[0].weight.grad, layer.router.router[2].weight.grad,
           ge.w1.grad, ge.w2.grad, ge.w3.grad]
    want = [xr.grad] + [p.grad for p in params]
    errs = {n: _rel(a, b) for n, a, b in zip(["dx", "dw_in", "dw_out", "dw1", "dw2", "dw3"], got, want)}
    plain = torch.topk(r.logits, k, dim=1).indices.cpu()
    assert (plain.sort(1).values != idx.sort(1).values).any(), "the capacity rule must have moved some picks"
    _check(errs)
