"""Training through the Mixture-of-Depths composition and the FFN half of
TransformerBlock on the HIP kernels (layers.py:142-187: RMSNorm, MoD selection and
weighting, the MoE, the scatter and the residual add), against fp64 autograd of the
oracle's restatement oracle/torch_port.ffn_half_loss_routed (pinned on the CPU by
tests/test_oracle.py against the numpy oracle and finite differences), fed the
kernel's own MoD selection and routing (both pinned bit-exactly by the forward tests)
and the bf16 values of the inputs and parameters.  Then the new kernels on their own:
kmoe_rmsnorm / kmoe_rmsnorm_bwd, kmoe_mod_bwd and kmoe_combine_bwd_rows against fp64.

Tolerance: rel-L2 <= 1e-2 for input and expert-weight gradients and the forward's MoE
part, 2e-2 for the router, MoD-router and norm-weight gradients (bf16 intermediates,
rounded once each)."""
import pytest
import torch
import torch.nn.functional as F

from kmoe import _lib, ops
from kmoe.block import MoEFFNBlock
from kmoe.config import AdvancedMoEConfig
from kmoe.mod import MoDMoE
from oracle import torch_port as P

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / max(b.norm(), 1e-30))


def _f64(t):
    return t.detach().double().cpu().clone().requires_grad_(True)


def _init_ffn(ffn, g, d, E):
    with torch.no_grad():
        ffn.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        ffn.router.router[2].weight.copy_(torch.randn(E, 128, generator=g) * 0.05)
        for w in (ffn.grouped_experts.w1, ffn.grouped_experts.w2, ffn.grouped_experts.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)


def _check(errs, tight=("dx", "dh", "dres", "dw1", "dw2", "dw3", "y")):
    print("  rel-L2: " + ", ".join(f"{n} {e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e <= (1e-2 if n in tight else 2e-2), (n, e)


# ------------------------------------------------------------------ MoDMoE
@pytest.mark.parametrize("B,S,d,E,k,F_,cf,with_res", [
    (2, 256, 256, 8, 2, 352, 0.75, False),
    (2, 300, 256, 8, 2, 352, 0.5, True),
    (1, 1000, 384, 16, 4, 320, 0.75, True),
])
def test_mod_moe_backward(dev, B, S, d, E, k, F_, cf, with_res):
    print(f"mod backward B={B} S={S} d={d} E={E} k={k} cf={cf} res={with_res}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F_, mod_capacity_factor=cf)
    m = MoDMoE(cfg).to(dev, BF).train()
    g = torch.Generator().manual_seed(300 + S)
    _init_ffn(m.ffn, g, d, E)
    with torch.no_grad():
        m.ffn_mod_router.router.weight.copy_(torch.randn(1, d, generator=g) * 0.08)
    x = torch.randn(B, S, d, generator=g).to(BF).to(dev).requires_grad_(True)
    res = torch.randn(B, S, d, generator=g).to(BF).to(dev).requires_grad_(True) if with_res else None
    dy = torch.randn(B, S, d, generator=g).to(BF)
    y = m(x, residual=res)
    ((y.float() * dy.to(dev).float()).sum() + m.aux_loss).backward()
    torch.cuda.synchronize()
    keep = m.ffn_mod_router.keep_count(S)
    with torch.no_grad():
        sel = ops.mod_select(x.detach(), m.ffn_mod_router.router.weight, keep)
        xs = x.detach().reshape(B * S, d)[sel.token_rows.long()]
        idx = m.ffn.router.route(xs).idx.cpu()
    ffn, ge = m.ffn, m.ffn.grouped_experts
    names = ["w_mod", "w_in", "w_out", "w1", "w2", "w3"]
    mods = [m.ffn_mod_router.router.weight, ffn.router.router[0].weight, ffn.router.router[2].weight, ge.w1, ge.w2,
            ge.w3]
    p64 = [_f64(t) for t in mods]
    x64 = _f64(x)
    r64 = _f64(res) if with_res else None
    loss, out = P.ffn_half_loss_routed(x64, *p64[1:], idx, dy.double(), w_mod=p64[0], sel_idx=sel.sel_idx.cpu(),
                                       residual=r64, w_lb=ffn.load_balance_loss_weight, w_z=ffn.router_z_loss_weight,
                                       return_out=True)
    loss.backward()
    # with a residual the bf16 output's rounding of residual + MoD-weighted MoE part
    # dominates the MoE part: the whole output is compared then
    errs = {"y": _rel(y.detach(), out.detach()), "dx": _rel(x.grad, x64.grad)}
    if with_res:
        errs["dres"] = _rel(res.grad, r64.grad)
    errs.update({"d" + n: _rel(t.grad, p.grad) for n, t, p in zip(names, mods, p64)})
    _check(errs)


@pytest.mark.parametrize("B,S,d,E,F_,cf,ec_cf,with_res,train", [
    (2, 256, 256, 8, 352, 0.75, 2.0, False, True),
    (2, 300, 256, 8, 352, 0.5, 1.0, True, True),
    (1, 400, 384, 4, 320, 0.75, 2.0, True, False),
])
def test_mod_expert_choice(dev, B, S, d, E, F_, cf, ec_cf, with_res, train):
    """MoD around an expert-choice layer: forward and gradients against fp64 autograd of
    oracle/torch_port.ffn_half_loss_ec_routed (pinned on the CPU against the numpy
    oracle's pieces) at the kernels' own MoD selection and expert-choice selection."""
    print(f"mod ec B={B} S={S} d={d} E={E} cf={cf} ec_cf={ec_cf} res={with_res} train={train}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, d_ff_expert=F_, mod_capacity_factor=cf,
                            moe_routing="expert_choice", moe_capacity_factor=ec_cf, moe_router_z_loss_weight=0.01)
    m = MoDMoE(cfg).to(dev, BF).train(train)
    g = torch.Generator().manual_seed(500 + S)
    ffn, ge = m.ffn, m.ffn.grouped_experts_ec
    with torch.no_grad():
        ffn.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        ffn.router.router[2].weight.copy_(torch.randn(E, 128, generator=g) * 0.05)
        for w in (ge.w1, ge.w2, ge.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)
        m.ffn_mod_router.router.weight.copy_(torch.randn(1, d, generator=g) * 0.08)
    x = torch.randn(B, S, d, generator=g).to(BF).to(dev).requires_grad_(True)
    res = torch.randn(B, S, d, generator=g).to(BF).to(dev).requires_grad_(True) if with_res else None
    dy = torch.randn(B, S, d, generator=g).to(BF)
    y = m(x, residual=res)
    loss = (y.float() * dy.to(dev).float()).sum()
    if train:
        loss = loss + m.aux_loss
    loss.backward()
    torch.cuda.synchronize()
    keep = m.ffn_mod_router.keep_count(S)
    with torch.no_grad():
        sel = ops.mod_select(x.detach(), m.ffn_mod_router.router.weight, keep)
        xs = x.detach().reshape(B * S, d)[sel.token_rows.long()].view(B, keep, d)
        ti = ffn.router.route(xs)[1].idx.cpu()
    names = ["w_mod", "w_in", "w_out", "w1", "w2", "w3"]
    mods = [m.ffn_mod_router.router.weight, ffn.router.router[0].weight, ffn.router.router[2].weight, ge.w1, ge.w2,
            ge.w3]
    p64 = [_f64(t) for t in mods]
    x64 = _f64(x)
    r64 = _f64(res) if with_res else None
    ref, out = P.ffn_half_loss_ec_routed(x64, *p64[1:], ti, dy.double(), w_mod=p64[0], sel_idx=sel.sel_idx.cpu().long(),
                                         residual=r64, training=train, w_z=0.01, return_out=True)
    ref.backward()
    errs = {"y": _rel(y.detach(), out.detach()), "dx": _rel(x.grad, x64.grad)}
    if with_res:
        errs["dres"] = _rel(res.grad, r64.grad)
    errs.update({"d" + n: _rel(t.grad, p.grad) for n, t, p in zip(names, mods, p64)})
    _check(errs)


@pytest.mark.parametrize("path", ["tc", "ec", "block", "block_ec"])
def test_mod_aux_router_loss(dev, path):
    """The MoD router's auxiliary BCE loss (mod.py:141-171) in training: its value and the
    auxiliary router's weight gradients against fp64 autograd of oracle/torch_port.
    mod_aux_loss (pinned on the CPU against torch's BCE on the numpy router MLP) at the
    kernel's selection, fed the bf16 values of the MoD input (the block: the kernel's
    normalised rows; the input is detached in the reference, so it takes no gradient)."""
    B, S, d, E, F_ = 2, 256, 256, 8, 352
    print(f"mod aux path={path}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, d_ff_expert=F_, mod_enabled=True, mod_capacity_factor=0.75,
                            residual_dropout=0.0, mod_load_balance_loss_weight=0.05,
                            moe_routing="expert_choice" if path.endswith("ec") else "token_choice")
    m = (MoEFFNBlock(cfg, 0) if path.startswith("block") else MoDMoE(cfg)).to(dev, BF).train()
    g = torch.Generator().manual_seed(620 + len(path))
    with torch.no_grad():
        for p_ in m.parameters():
            p_.copy_(torch.randn(p_.shape, generator=g) * 0.05 + (1.0 if p_.dim() == 1 else 0.0))
    x = torch.randn(B, S, d, generator=g).to(BF).to(dev).requires_grad_(True)
    y = m(x)
    if path.startswith("block"):
        # expert choice: the unfused composition (the block's norm module, then MoD around the layer)
        assert m.last_path == ("unfused" if path == "block_ec" else "fused_train")
    mr = m.ffn_mod_router
    aux_mod = mr.aux_loss
    (y.float().square().mean() + m.aux_loss).backward()
    torch.cuda.synchronize()
    keep = mr.keep_count(S)
    with torch.no_grad():
        if path == "block":
            xin = ops.rmsnorm(x.detach().reshape(B * S, d), m.ffn_norm.weight, m.ffn_norm.eps).n
        elif path == "block_ec":
            xin = m.ffn_norm(x.detach())
        else:
            xin = x.detach()
        xin = xin.reshape(B, S, d)
        sel = ops.mod_select(xin, mr.router.weight, keep)
    w_a, w_b = mr.aux_router[0].weight, mr.aux_router[2].weight
    a64, b64 = _f64(w_a), _f64(w_b)
    ref = P.mod_aux_loss(xin.double().cpu(), a64, b64, sel.sel_idx.cpu().long(), 0.05)
    ref.backward()
    with torch.no_grad():  # the forward-only form: the same kernels, no autograd record
        assert float(mr.aux(xin.reshape(B * S, d), sel.token_rows)) == float(aux_mod)
        # and through the module (the block's no-grad forward normalises with its norm
        # module: its bf16 rows may differ from the norm kernel's by a rounding, 3e-4 of the
        # loss measured)
        m(x)
        tol = 2e-3 if path.startswith("block") else 1e-6
        assert abs(float(mr.aux_loss) - float(aux_mod)) <= tol * abs(float(aux_mod))
    errs = {"aux": abs(float(aux_mod) - float(ref)) / abs(float(ref)), "dw_a": _rel(w_a.grad, a64.grad),
            "dw_b": _rel(w_b.grad, b64.grad)}
    _check(errs, tight=("aux",))


# ------------------------------------------------------------------ the block in training
@pytest.mark.parametrize("mod,norm_dtype,h_dtype,p_drop,fp8", [
    (False, torch.float32, BF, 0.0, False),
    (True, torch.float32, BF, 0.0, False),
    (True, BF, BF, 0.0, False),
    (True, torch.float32, torch.float32, 0.0, False),
    (False, torch.float32, BF, 0.1, False),   # the reference's default residual_dropout (config.py:87)
    (True, torch.float32, BF, 0.1, False),
    (False, torch.float32, torch.float32, 0.5, False),
    # config 5's composition, MoD + fp8 experts, trained straight-through
    (True, torch.float32, BF, 0.0, True),
    (True, torch.float32, BF, 0.1, True),
])
def test_block_training_backward(dev, mod, norm_dtype, h_dtype, p_drop, fp8):
    B, S, d, E, k, F_ = 2, 256, 256, 8, 2, 352
    print(f"block training mod={mod} norm={norm_dtype} h={h_dtype} p={p_drop} fp8={fp8}", flush=True)
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=F_, mod_enabled=mod,
                            mod_capacity_factor=0.75, residual_dropout=p_drop, moe_fp8=fp8)
    blk = MoEFFNBlock(cfg, 0).to(dev, BF).train()
    g = torch.Generator().manual_seed(410 + int(mod))
    drop_keep = None
    if p_drop > 0:
        # a fixed keep mask, drawn on the CPU: the fused path applies it in the combine
        drop_keep = torch.rand(B * S, d, generator=torch.Generator().manual_seed(77)) >= p_drop
        blk.keep_mask_fn = lambda shape, device, p: drop_keep.to(device)
    _init_ffn(blk.ffn, g, d, E)
    blk.ffn_norm.weight = torch.nn.Parameter((1.0 + 0.3 * torch.randn(d, generator=g)).to(dev, norm_dtype))
    if mod:
        with torch.no_grad():
            blk.ffn_mod_router.router.weight.copy_(torch.randn(1, d, generator=g) * 0.08)
    h = (torch.randn(B, S, d, generator=g) * 1.5).to(BF).to(dev, h_dtype).requires_grad_(True)
    dy = torch.randn(B, S, d, generator=g).to(BF)
    out = blk(h)
    assert blk.last_path == "fused_train"
    assert out.dtype == torch.promote_types(h_dtype, norm_dtype)
    ((out.float() * dy.to(dev).float()).sum() + blk.aux_loss).backward()
    torch.cuda.synchronize()
    T = B * S
    ffn, ge = blk.ffn, blk.ffn.grouped_experts
    with torch.no_grad():
        n = ops.rmsnorm(h.detach().reshape(T, d), blk.ffn_norm.weight, blk.ffn_norm.eps).n
        sel = None
        if mod:
            keep = blk.ffn_mod_router.keep_count(S)
            # the selection from n's own logits kernel: the block took it from the logits
            # its norm kernel wrote (bit-identical, test_rmsnorm_mod_logits)
            sel = ops.mod_select(n.view(B, S, d), blk.ffn_mod_router.router.weight, keep)
            idx = ffn.router.route(n[sel.token_rows.long()]).idx.cpu()
        else:
            idx = ffn.router.route(n).idx.cpu()
    names = ["w_in", "w_out", "w1", "w2", "w3", "norm"] + (["w_mod"] if mod else [])
    mods = [ffn.router.router[0].weight, ffn.router.router[2].weight, ge.w1, ge.w2, ge.w3, blk.ffn_norm.weight]
    if mod:
        mods.append(blk.ffn_mod_router.router.weight)
    p64 = [_f64(t) for t in mods]
    h64 = _f64(h)
    loss, ref = P.ffn_half_loss_routed(h64, *p64[:5], idx, dy.double(), norm_w=p64[5], eps=blk.ffn_norm.eps,
                                       w_mod=p64[6] if mod else None, sel_idx=None if sel is None else
                                       sel.sel_idx.cpu(), w_lb=ffn.load_balance_loss_weight,
                                       w_z=ffn.router_z_loss_weight, return_out=True,
                                       drop_keep=None if drop_keep is None else drop_keep.view(B, S, d),
                                       p_drop=p_drop, fp8=fp8)
    loss.backward()
    hd = h.detach().double().cpu()
    # an f32 output carries the MoE part exactly; a bf16 one rounds h + MoE part
    y_err = _rel(out.detach().double().cpu() - hd, ref.detach() - hd) if out.dtype == torch.float32 else \
        _rel(out.detach(), ref.detach())
    errs = {"y": y_err, "dh": _rel(h.grad, h64.grad)}
    errs.update({"d" + n: _rel(t.grad, p.grad) for n, t, p in zip(names, mods, p64)})
    _check(errs)


def test_block_dropout_mask_statistics(dev):
    """Active residual dropout trains on the fused path with a fresh Bernoulli(1-p) mask
    per call: the dropped elements of out - h are exactly 0, the kept fraction is 1-p,
    and two calls draw different masks."""
    print("block dropout mask", flush=True)
    cfg = AdvancedMoEConfig(d_model=256, n_experts=8, d_ff_expert=352, residual_dropout=0.25, mod_enabled=False)
    blk = MoEFFNBlock(cfg, 0).to(dev, BF).train()
    blk.ffn_norm.to(torch.float32)
    # f32 h and norm weight: out is f32, so out - h is the dropped-out MoE part exactly
    h = torch.randn(2, 512, 256, device=dev).requires_grad_(True)
    outs = []
    for _ in range(2):
        out = blk(h)
        assert blk.last_path == "fused_train"
        outs.append((out.float() - h.detach().float()) != 0)
        out.float().sum().backward()
    kept = outs[0].float().mean().item()
    assert abs(kept - 0.75) < 0.01, kept
    assert (outs[0] != outs[1]).float().mean().item() > 0.2
    assert h.grad is not None and torch.isfinite(h.grad.float()).all()
    assert blk.ffn.grouped_experts.w1.grad is not None


# ------------------------------------------------------------------ kernels
@pytest.mark.parametrize("T,d,x_dtype,w_dtype", [
    (1000, 256, BF, torch.float32), (333, 200, torch.float32, BF), (4096, 2048, BF, BF), (70, 8192, BF, torch.float32),
    (5, 8, torch.float32, torch.float32),
])
def test_rmsnorm_kernels(dev, T, d, x_dtype, w_dtype):
    print(f"rmsnorm T={T} d={d} x={x_dtype} w={w_dtype}", flush=True)
    g = torch.Generator().manual_seed(T + d)
    x = (torch.randn(T, d, generator=g) * 2.0).to(x_dtype)
    w = (1.0 + 0.3 * torch.randn(d, generator=g)).to(w_dtype)
    dn = torch.randn(T, d, generator=g).to(BF)
    dres = torch.randn(T, d, generator=g).to(x_dtype)
    eps = 1e-5
    n, rrms, _ = ops.rmsnorm(x.to(dev), w.to(dev), eps)
    dx, dw = ops.rmsnorm_bwd(dn.to(dev), x.to(dev), w.to(dev), rrms, dres=dres.to(dev))
    torch.cuda.synchronize()
    x64, w64 = x.double().requires_grad_(True), w.double().requires_grad_(True)
    r64 = 1.0 / torch.sqrt((x64.detach() ** 2).mean(-1) + eps)
    n64 = F.rms_norm(x64, (d,), w64, eps=eps)
    n64.backward(dn.double())
    assert torch.allclose(rrms.double().cpu(), r64, rtol=4e-6, atol=0)
    # n: one bf16 rounding of the f32 product
    ref = n64.detach()
    assert bool(((n.double().cpu() - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-30).all())
    dx_ref = x64.grad + dres.double()
    tol = 1e-5 if x_dtype == torch.float32 else 4e-3
    assert _rel(dx, dx_ref) <= tol
    assert _rel(dw, w64.grad) <= (1e-5 if w_dtype == torch.float32 else 4e-3)


def test_rmsnorm_bwd_no_rows(dev):
    w = torch.ones(64, device=dev)
    dx, dw = ops.rmsnorm_bwd(torch.empty(0, 64, device=dev, dtype=BF), torch.empty(0, 64, device=dev, dtype=BF), w,
                             torch.empty(0, device=dev))
    torch.cuda.synchronize()
    assert dx.shape == (0, 64) and torch.equal(dw.cpu(), torch.zeros(64))


@pytest.mark.parametrize("B,keep,d,dw_f32", [(2, 192, 256, True), (4, 1536, 2048, False), (1, 1, 64, True)])
def test_mod_bwd_kernel(dev, B, keep, d, dw_f32):
    print(f"mod_bwd B={B} keep={keep} d={d}", flush=True)
    g = torch.Generator().manual_seed(keep)
    sel_w = torch.softmax(torch.randn(B, keep, generator=g), -1)
    dsel = torch.randn(B, keep, generator=g)
    x_sel = torch.randn(B * keep, d, generator=g).to(BF)
    stride = 3
    tab = torch.full((B * keep, stride), 7.0)
    tab_d = tab.to(dev)
    dw_mod = torch.empty(d, device=dev, dtype=torch.float32 if dw_f32 else BF)
    lib = _lib.load()
    wsb = lib.kmoe_mod_bwd_workspace_bytes(B * keep, d)
    ws = torch.empty(max(wsb, 4), device=dev, dtype=torch.uint8)
    sw_d, ds_d, xs_d = sel_w.to(dev), dsel.to(dev), x_sel.to(dev)
    _lib.call("kmoe_mod_bwd", _lib.ptr(sw_d), _lib.ptr(ds_d), B, keep, _lib.ptr(xs_d), d, _lib.ptr(tab_d[:, 2:]),
              stride, _lib.ptr(dw_mod), _lib.DTYPE_F32 if dw_f32 else _lib.DTYPE_BF16, _lib.ptr(ws), wsb,
              _lib.stream_ptr(dev))
    torch.cuda.synchronize()
    p, ds = sel_w.double(), dsel.double()
    dlog = p * (ds - (p * ds).sum(-1, keepdim=True))
    got = tab_d.cpu()
    assert torch.equal(got[:, :2], tab[:, :2])  # only the strided column is written
    assert torch.allclose(got[:, 2].double(), dlog.reshape(-1), rtol=1e-5, atol=1e-7)
    want = (dlog.reshape(-1, 1) * x_sel.double()).sum(0)
    assert _rel(dw_mod, want) <= (1e-5 if dw_f32 else 4e-3)


@pytest.mark.parametrize("T,k,d,T_out", [(300, 2, 256, 500), (1000, 4, 384, 1000)])
def test_combine_bwd_rows_kernel(dev, T, k, d, T_out):
    print(f"combine_bwd_rows T={T} k={k} d={d}", flush=True)
    g = torch.Generator().manual_seed(T + k)
    A = T * k
    perm = torch.randperm(A, generator=g).to(torch.int32)
    slot_row = perm.view(T, k).clone()
    slot_row[::7, -1] = -1  # dropped slots
    slot_w = torch.rand(T, k, generator=g)
    rows = torch.randperm(T_out, generator=g)[:T].to(torch.int32)
    scale = torch.rand(T, generator=g)
    dy = torch.randn(T_out, d, generator=g).to(BF)
    yperm = torch.randn(A, d, generator=g).to(BF)
    dyperm = torch.zeros(A, d, device=dev, dtype=BF)
    dw = torch.empty(T, k, device=dev)
    dscale = torch.empty(T, device=dev)
    ins = [t.to(dev) for t in (dy, yperm, slot_row, slot_w, rows, scale)]
    _lib.call("kmoe_combine_bwd_rows", _lib.ptr(ins[0]), _lib.ptr(ins[1]), _lib.ptr(ins[2]), _lib.ptr(ins[3]), k, d,
              T, _lib.ptr(ins[4]), _lib.ptr(ins[5]), _lib.ptr(dyperm), _lib.ptr(dw), _lib.ptr(dscale),
              _lib.stream_ptr(dev))
    torch.cuda.synchronize()
    dyr = dy.double()[rows.long()]
    kept = slot_row >= 0
    yr = yperm.double()[slot_row.clamp(min=0).long()]                   # (T, k, d)
    dots = (dyr[:, None, :] * yr).sum(-1) * kept
    assert torch.allclose(dw.cpu().double(), dots * scale.double()[:, None], rtol=1e-5, atol=1e-4)
    assert torch.allclose(dscale.cpu().double(), (dots * slot_w.double()).sum(1), rtol=1e-5, atol=1e-4)
    want = torch.zeros(A, d, dtype=torch.float64)
    want[slot_row[kept].long()] = ((scale[:, None] * slot_w).double()[..., None] * dyr[:, None, :])[kept]
    got = dyperm.cpu().double()
    assert bool(((got - want).abs() <= want.abs() * 2.0 ** -8 + 1e-30).all())


@pytest.mark.parametrize("B,S,d", [(2, 300, 256), (4, 2048, 2048), (1, 7, 8200 - 8)])
def test_rmsnorm_mod_logits(dev, B, S, d):
    """The MoD logits the norm kernel writes equal, bit for bit, those kmoe_mod_select
    computes from the normalised rows, and so does the selection made from them."""
    print(f"rmsnorm mod logits B={B} S={S} d={d}", flush=True)
    g = torch.Generator().manual_seed(S + d)
    x = torch.randn(B * S, d, generator=g).to(BF).to(dev)
    w = (1.0 + 0.3 * torch.randn(d, generator=g)).to(dev)
    w_mod = (torch.randn(1, d, generator=g) * 0.05).to(BF).to(dev)
    out = ops.rmsnorm(x, w, 1e-5, w_mod=w_mod)
    keep = max(1, int(S * 0.75))
    ref = ops.mod_select(out.n.view(B, S, d), w_mod, keep)
    got = ops.mod_select(out.n.view(B, S, d), w_mod, keep, logits=out.mod_logits)
    torch.cuda.synchronize()
    assert torch.equal(out.mod_logits.view(B, S), ref.logits)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
