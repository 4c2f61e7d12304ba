"""The FFN half of TransformerBlock (layers.py:142-147, 184-187: out = h + MoE(RMSNorm(h)))
with RMSNorm folded into the router and the gate/up GEMM and the residual add folded
into the combine, against the oracle (oracle/moe_oracle.rms_norm / ffn_block_tc,
pinned on the CPU by tests/test_oracle.py).

Bars: routing indices bit-exact from the kernel's own logits; the RMSNorm scale within
1e-5 relative of fp64; router logits within 2e-5 abs / 1e-4 rel of fp64 on the folded
weights; the MoE part of the block output rel-L2 <= 1e-2 of fp64 (the norm weight is
folded into bf16 weights: one more bf16 rounding); the residual combine within one
bf16 ulp of the fp64 sum (f32 out: 1e-5 rel)."""
import numpy as np
import pytest
import torch

from kmoe import ops
from kmoe.block import MoEFFNBlock
from kmoe.config import AdvancedMoEConfig
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def relL2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def npf(t):
    return t.detach().float().cpu().numpy()


def bf(t):
    return t.to(torch.bfloat16)


# ------------------------------------------------------------------ router on RMSNorm(x)
@pytest.mark.parametrize("T,d,E,k", [(512, 256, 8, 2), (16384, 2048, 16, 2), (1000, 192, 64, 4), (33, 64, 5, 1)])
def test_router_rms_parity(dev, T, d, E, k):
    print(f"router_rms T={T} d={d} E={E} k={k}", flush=True)
    g = torch.Generator().manual_seed(200 + E)
    x = torch.randn(T, d, generator=g) * 2.5
    nw = 1.0 + 0.3 * torch.randn(d, generator=g)
    w_in = torch.randn(128, d, generator=g) * 0.02
    w_out = torch.randn(E, 128, generator=g) * 0.02
    xb = bf(x).to(dev)
    w_in_g = bf(w_in * nw[None, :]).to(dev)
    r = ops.router(xb, w_in_g, bf(w_out).to(dev), k, rms_eps=1e-5)
    torch.cuda.synchronize()
    xr = npf(xb).astype(np.float64)
    rs_ref = 1.0 / np.sqrt(np.mean(xr * xr, axis=1) + 1e-5)
    np.testing.assert_allclose(npf(r.rscale)[:T], rs_ref, rtol=1e-5)
    # the kernel's arithmetic: r * (x . w_in_g^T) on the folded weights
    lg = npf(r.logits)
    ref = O.router_logits(xr * rs_ref[:, None], npf(w_in_g), npf(bf(w_out)))
    np.testing.assert_allclose(lg, ref, atol=2e-5, rtol=1e-4)
    idx, w = O.topk_select(lg, k)
    assert np.array_equal(r.idx.cpu().numpy(), idx)
    np.testing.assert_allclose(npf(r.w), w, rtol=2e-6, atol=1e-7)
    # the reference's semantics: the router MLP on RMSNorm(x) with the unfolded weights
    ref_sem = O.router_logits(O.rms_norm(xr, npf(nw), 1e-5), npf(bf(w_in)), npf(bf(w_out)))
    assert relL2(lg, ref_sem) <= 1e-2


# ------------------------------------------------------------------ row-scaled gate/up GEMM
@pytest.mark.parametrize("with_row_index", [False, True])
def test_gate_up_scaled(dev, with_row_index):
    print(f"gate_up_scaled row_index={with_row_index}", flush=True)
    T, d, E, k, Fd = 1500, 256, 8, 2, 352
    g = torch.Generator().manual_seed(210)
    x = torch.randn(T + 37, d, generator=g)
    w1, w2 = (torch.randn(E, d, Fd, generator=g) * 0.05 for _ in range(2))
    w3 = torch.randn(E, Fd, d, generator=g) * 0.05
    rscale = torch.rand(T, generator=g) * 1.5 + 0.25
    idx = torch.randint(0, E, (T, k), generator=g)
    idx[:, 1] = (idx[:, 0] + 1 + torch.randint(0, E - 1, (T,), generator=g)) % E
    wts = torch.rand(T, k, generator=g)
    row_index = torch.randperm(T + 37, generator=g)[:T].to(torch.int32) if with_row_index else None
    xb = bf(x).to(dev)
    pw = ops.pack_weights(bf(w1).to(dev), bf(w2).to(dev), bf(w3).to(dev))
    ri = None if row_index is None else row_index.to(dev)
    disp = ops.dispatch(xb, idx.to(dev), wts.to(dev), E, row_index=ri, materialize=False)
    h = ops.gemm_gate_up_rows(xb, ri, disp.row_token, disp.offsets, pw, T * k, rscale=rscale.to(dev))
    # scale 1 everywhere: bit-identical to the unscaled kernel
    h1 = ops.gemm_gate_up_rows(xb, ri, disp.row_token, disp.offsets, pw, T * k,
                               rscale=torch.ones(T, device=dev))
    h0 = ops.gemm_gate_up_rows(xb, ri, disp.row_token, disp.offsets, pw, T * k)
    torch.cuda.synchronize()
    assert torch.equal(h1.view(torch.int16), h0.view(torch.int16))
    rt = disp.row_token.cpu().numpy()[:T * k]
    rows = rt if row_index is None else row_index.numpy()[rt]
    xs = npf(xb)[rows].astype(np.float64) * rscale.numpy()[rt, None]
    off = disp.offsets.cpu().numpy()
    ref = O.swiglu_rows(xs, off, npf(bf(w1)), npf(bf(w2)), npf(bf(w3)), dtype=np.float64)
    y = ops.gemm_down(h, None, disp.offsets, pw, T * k)
    torch.cuda.synchronize()
    assert relL2(npf(y)[:T * k], ref) <= 1e-2


# ------------------------------------------------------------------ residual combine
@pytest.mark.parametrize("out_f32", [False, True])
def test_combine_residual_parity(dev, out_f32):
    print(f"combine_residual f32={out_f32}", flush=True)
    T, fan, d, R = 1000, 3, 384, 2500
    g = torch.Generator().manual_seed(220)
    yperm = bf(torch.randn(R, d, generator=g))
    src = torch.randint(-1, R, (T, fan), generator=g).to(torch.int32)
    w = torch.rand(T, fan, generator=g)
    out_map = torch.randint(-1, T, (T + 100,), generator=g).to(torch.int32)
    scale = torch.rand(T, generator=g)
    odt = torch.float32 if out_f32 else torch.bfloat16
    res = (torch.randn(T + 100, d, generator=g) * 2.0).to(odt)
    y = ops.combine(yperm.to(dev), src.to(dev), w.to(dev), T + 100, out_map=out_map.to(dev), scale=scale.to(dev),
                    out_dtype=odt, residual=res.to(dev))
    torch.cuda.synchronize()
    comb = O.combine(npf(yperm), src.numpy(), w.numpy(), out_map=out_map.numpy(), scale=scale.numpy(), T_out=T + 100)
    ref = comb + npf(res).astype(np.float64)
    got = npf(y)
    # rows without a source set are the residual itself
    empty = out_map.numpy() < 0
    assert np.array_equal(got[empty], npf(res)[empty])
    if out_f32:
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    else:
        mag = O.combine(np.abs(npf(yperm)), src.numpy(), np.abs(w.numpy()), out_map=out_map.numpy(),
                        scale=scale.numpy(), T_out=T + 100) + np.abs(npf(res))
        assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -22)


def test_combine_residual_top2_path(dev):
    """fan 2, d 2048, bf16: the two-source kernel with a residual equals the generic
    kernel (reached with a third, always-dropped source) bit for bit."""
    print("combine_residual top2", flush=True)
    T, d, R = 3000, 2048, 6000
    g = torch.Generator().manual_seed(221)
    yperm = bf(torch.randn(R, d, generator=g)).to(dev)
    src = torch.randint(-1, R, (T, 2), generator=g).to(torch.int32)
    w = torch.rand(T, 2, generator=g)
    out_map = torch.randint(-1, T, (T + 50,), generator=g).to(torch.int32).to(dev)
    res = bf(torch.randn(T + 50, d, generator=g)).to(dev)
    src3 = torch.cat([src, torch.full((T, 1), -1, dtype=torch.int32)], 1).to(dev)
    w3 = torch.cat([w, torch.rand(T, 1, generator=g)], 1).to(dev)
    a = ops.combine(yperm, src.to(dev), w.to(dev), T + 50, out_map=out_map, residual=res)
    b = ops.combine(yperm, src3, w3, T + 50, out_map=out_map, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    ref = O.combine(npf(yperm), src.numpy(), w.numpy(), out_map=out_map.cpu().numpy(), T_out=T + 50) + npf(res)
    mag = O.combine(np.abs(npf(yperm)), src.numpy(), w.numpy(), out_map=out_map.cpu().numpy(), T_out=T + 50) \
        + np.abs(npf(res))
    assert np.all(np.abs(npf(a) - ref) <= np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -22)


@pytest.mark.parametrize("T,fan,d,out_f32", [(1000, 3, 384, False), (1000, 3, 384, True), (3000, 2, 2048, False)])
def test_combine_residual_dropout(dev, T, fan, d, out_f32):
    """kmoe_combine_residual_dropout at a fixed keep mask: residual + keep * (1/(1-p)) *
    the weighted sum, one rounding; rows without a source set are the residual; with an
    all-kept mask and keep_scale 1 it equals kmoe_combine_residual bit for bit (the
    two-source and the generic kernel)."""
    print(f"combine_residual_dropout T={T} fan={fan} d={d} f32={out_f32}", flush=True)
    g = torch.Generator().manual_seed(222 + fan)
    R = 2 * T
    yperm = bf(torch.randn(R, d, generator=g))
    src = torch.randint(-1, R, (T, fan), generator=g).to(torch.int32)
    w = torch.rand(T, fan, generator=g)
    out_map = torch.randint(-1, T, (T + 50,), generator=g).to(torch.int32)
    odt = torch.float32 if out_f32 else torch.bfloat16
    res = (torch.randn(T + 50, d, generator=g) * 2.0).to(odt)
    p = 0.3
    keep = torch.rand(T + 50, d, generator=g) >= p
    args = (yperm.to(dev), src.to(dev), w.to(dev), T + 50)
    y = ops.combine(*args, out_map=out_map.to(dev), out_dtype=odt, residual=res.to(dev), keep_mask=keep.to(dev),
                    keep_scale=1.0 / (1.0 - p))
    torch.cuda.synchronize()
    comb = O.combine(npf(yperm), src.numpy(), w.numpy(), out_map=out_map.numpy(), T_out=T + 50)
    ref = npf(res).astype(np.float64) + keep.numpy() * comb / (1.0 - p)
    got = npf(y)
    empty = out_map.numpy() < 0
    assert np.array_equal(got[empty], npf(res)[empty])
    # dropped elements are the residual exactly
    assert np.array_equal(got[~keep.numpy()], npf(res)[~keep.numpy()])
    mag = O.combine(np.abs(npf(yperm)), src.numpy(), w.numpy(), out_map=out_map.numpy(), T_out=T + 50) / (1 - p) \
        + np.abs(npf(res))
    tol = (2.0 ** -23 if out_f32 else 2.0 ** -8) * np.abs(ref) + mag * 2.0 ** -21
    assert np.all(np.abs(got - ref) <= tol)
    # all kept, scale 1: the plain residual combine's bits
    a = ops.combine(*args, out_map=out_map.to(dev), out_dtype=odt, residual=res.to(dev),
                    keep_mask=torch.ones(T + 50, d, dtype=torch.bool, device=dev), keep_scale=1.0)
    b = ops.combine(*args, out_map=out_map.to(dev), out_dtype=odt, residual=res.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16) if not out_f32 else a.view(torch.int32),
                       b.view(torch.int16) if not out_f32 else b.view(torch.int32))


# ------------------------------------------------------------------ the block
def _block(dev, d, E, k, Fd, seed, norm_dtype, cap=None):
    cfg = AdvancedMoEConfig(d_model=d, n_experts=E, moe_top_k=k, d_ff_expert=Fd,
                            moe_capacity_factor=cap or 1.25, moe_drop_overflow=cap is not None)
    blk = MoEFFNBlock(cfg, 0).to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        ffn = blk.ffn
        ffn.router.router[0].weight.copy_(torch.randn(128, d, generator=g) * 0.05)
        ffn.router.router[2].weight.copy_(torch.randn(E, 128, generator=g) * 0.05)
        for w in (ffn.grouped_experts.w1, ffn.grouped_experts.w2, ffn.grouped_experts.w3):
            w.copy_(torch.randn(w.shape, generator=g) * 0.05)
    blk.ffn_norm.weight = torch.nn.Parameter((1.0 + 0.3 * torch.randn(d, generator=g)).to(dev, norm_dtype))
    return blk, g


@pytest.mark.parametrize("B,S,d,E,k,Fd,cap,norm_dtype", [
    (2, 300, 256, 8, 2, 352, None, torch.float32),
    (1, 1000, 384, 16, 2, 320, 1.0, torch.float32),
    (2, 257, 256, 8, 2, 352, None, torch.bfloat16),
])
def test_ffn_block_fused_parity(dev, B, S, d, E, k, Fd, cap, norm_dtype):
    print(f"ffn_block B={B} S={S} d={d} E={E} cap={cap} norm={norm_dtype}", flush=True)
    blk, g = _block(dev, d, E, k, Fd, 230 + d, norm_dtype, cap)
    blk.eval()
    h = bf(torch.randn(B, S, d, generator=g) * 1.5).to(dev)
    with torch.no_grad():
        out = blk(h)
    assert blk.last_path == "fused"
    assert out.dtype == torch.promote_types(h.dtype, norm_dtype)
    T = B * S
    # the kernel's routing (the same deterministic call as the block's)
    w_in_g, w_out_b, _ = blk._fused_weights()
    r = ops.router(h.reshape(T, d), w_in_g, w_out_b, k, rms_eps=blk.ffn_norm.eps)
    torch.cuda.synchronize()
    ffn = blk.ffn
    ge = ffn.grouped_experts
    capacity = int(np.ceil(cap * T * k / E)) if cap is not None else 0
    hr = npf(h.reshape(T, d)).astype(np.float64)
    ref = O.ffn_block_tc(hr, npf(blk.ffn_norm.weight), blk.ffn_norm.eps, npf(ffn.router.router[0].weight),
                         npf(ffn.router.router[2].weight), npf(ge.w1), npf(ge.w2), npf(ge.w3), k,
                         capacity=capacity, logits=npf(r.logits))
    assert np.array_equal(ffn.last_expert_counts.cpu().numpy(), ref["counts"])
    got = npf(out.reshape(T, d)).astype(np.float64)
    moe_ref = ref["y"] - hr
    if out.dtype == torch.float32:
        # exact residual add: the MoE part alone at the MoE bar
        assert relL2(got - hr, moe_ref) <= 1e-2
    else:
        # one bf16 rounding of the sum on top of the MoE error
        assert relL2(got, ref["y"]) <= 1e-2
        assert relL2(got - hr, moe_ref) <= 2e-2


def test_ffn_block_fused_vs_unfused(dev):
    """The fused block against the unfused composition (torch RMSNorm, the kmoe layer,
    torch add) on the tokens both route identically."""
    print("ffn_block fused vs unfused", flush=True)
    blk, g = _block(dev, 256, 8, 2, 352, 240, torch.float32)
    blk.eval()
    h = bf(torch.randn(2, 512, 256, generator=g)).to(dev)
    with torch.no_grad():
        out_f = blk(h)
        xn = blk.ffn_norm(h)
        out_u = h + blk.ffn(xn)
        r_u = blk.ffn.router.route(xn.reshape(-1, 256).to(torch.bfloat16))
        w_in_g, w_out_b, _ = blk._fused_weights()
        r_f = ops.router(h.reshape(-1, 256), w_in_g, w_out_b, 2, rms_eps=blk.ffn_norm.eps)
    torch.cuda.synchronize()
    same = (torch.sort(r_u.idx, 1).values == torch.sort(r_f.idx, 1).values).all(1).cpu().numpy()
    assert same.mean() > 0.97
    hr = npf(h.reshape(-1, 256))
    a = npf(out_f.reshape(-1, 256))[same] - hr[same]
    b = npf(out_u.reshape(-1, 256))[same] - hr[same]
    assert relL2(a, b) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mod_moe_residual(dev, dtype):
    """MoDMoE(h, residual) = residual + MoDMoE(h) (layers.py:175-187) from one combine:
    unselected tokens are the residual itself, selected ones within one rounding of the sum."""
    from kmoe import MoDMoE
    print(f"mod residual {dtype}", flush=True)
    cfg = AdvancedMoEConfig(d_model=256, n_experts=8, moe_top_k=2, d_ff_expert=352, mod_capacity_factor=0.5)
    torch.manual_seed(11)
    m = MoDMoE(cfg).to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(12)
    h = torch.randn(2, 300, 256, generator=g).to(dev, dtype)
    res = torch.randn(2, 300, 256, generator=g).to(dev, dtype)
    with torch.no_grad():
        a = m(h)
        b = m(h, residual=res)
    torch.cuda.synchronize()
    sel = (a != 0).any(-1)
    assert 0.3 < sel.float().mean().item() < 0.7
    assert torch.equal(b[~sel], res[~sel])
    want = (res.double() + a.double())[sel]
    tol = 2.0 ** -22 if dtype == torch.float32 else 2.0 ** -8
    err = (b[sel].double() - want).abs()
    assert bool((err <= want.abs() * tol + a.double().abs()[sel] * tol + 1e-30).all())
