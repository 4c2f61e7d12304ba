"""GPU parity of the whole MoE layer on the five BASELINE configurations.

Routing (indices, per-expert counts, permutation, capacity drops, expert-choice
and MoD selections) is compared bit-exactly with the oracle fed the kernel's
own fp32 scores; outputs within rel-L2 1e-2 (bf16) / 3e-2 (fp8) of the oracle
computed in fp32.  Full-size configs check outputs on a token sample plus
size-independent properties (count sums, permutation bijection, determinism)."""
import numpy as np
import pytest
import torch

from kmoe import ops, synth
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def f(t):
    return t.detach().float().cpu().numpy()


def relL2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def token_outputs(x, idx, w, keep, W, tokens, fp8=False):
    """Oracle y for a subset of tokens: sum_j w[t,j] * expert_{idx[t,j]}(x[t]) over kept slots."""
    w1, w2, w3 = W
    y = np.zeros((len(tokens), x.shape[1]), dtype=np.float64)
    for e in range(w1.shape[0]):
        sel = [(i, j) for i, t in enumerate(tokens) for j in range(idx.shape[1]) if idx[t, j] == e and keep[t, j]]
        if not sel:
            continue
        ii = np.array([s[0] for s in sel])
        jj = np.array([s[1] for s in sel])
        xr = x[np.array(tokens)[ii]]
        if fp8:
            q, s = O.quant_rows(xr)
            ye = O.swiglu_rows_fp8(q, s, np.array([0, len(ii)]), w1[e:e + 1], w2[e:e + 1], w3[e:e + 1])
        else:
            ye = O.swiglu_rows(xr, np.array([0, len(ii)]), w1[e:e + 1], w2[e:e + 1], w3[e:e + 1])
        np.add.at(y, ii, w[np.array(tokens)[ii], jj][:, None] * ye)
    return y


@pytest.fixture(scope="module")
def cfg_cache():
    return {}


def setup(cfg_cache, n, dev):
    if n not in cfg_cache:
        wl = synth.WORKLOADS[n]
        t = synth.make_tensors(wl, "cpu")
        layer = synth.build_layer(wl, dev, {k: v.to(dev) for k, v in t.items()}).train()
        cfg_cache.clear()
        cfg_cache[n] = (wl, t, layer)
    return cfg_cache[n]


def test_cfg1_small_full_parity(dev, cfg_cache):
    """Config 1 (T=512, d=256, E=8, F=512) in fp32 activations: every token checked."""
    wl, t, layer = setup(cfg_cache, 1, dev)
    x = t["x"].to(dev)
    with torch.no_grad():
        y = layer(x)
        r = layer.router.route(x.reshape(wl.T, wl.d).to(torch.bfloat16))
    assert y.dtype == torch.float32 and y.shape == x.shape
    lg = f(r.logits)
    # the kernels compute in bf16: oracle on the bf16-rounded inputs, in fp32
    bf = lambda a: f(a.to(torch.bfloat16))
    ref = O.moe_forward_tc(bf(t["x"]).reshape(wl.T, wl.d), bf(t["w_in"]), bf(t["w_out"]), bf(t["w1"]),
                           bf(t["w2"]), bf(t["w3"]), wl.k, logits=lg)
    assert np.array_equal(r.idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(layer.last_expert_counts.cpu().numpy(), ref["counts"])
    assert relL2(f(y).reshape(wl.T, wl.d), ref["y"]) <= 1e-2
    # the fp32 reference on the unrounded inputs (what the reference computes on CPU)
    ref32 = O.moe_forward_tc(f(t["x"]).reshape(wl.T, wl.d), f(t["w_in"]), f(t["w_out"]), f(t["w1"]), f(t["w2"]),
                             f(t["w3"]), wl.k, logits=lg)
    assert relL2(f(y).reshape(wl.T, wl.d), ref32["y"]) <= 1e-2
    assert abs(float(layer.aux_loss) - ref["aux"][0]) <= 1e-4 * ref["aux"][0]
    # reference API contract: router(h) 3-tuple, eval mode aux 0.0
    w3_, i3_, l3_ = layer.router(x)
    assert w3_.shape == (wl.B, wl.S, wl.k) and i3_.dtype == torch.int64 and l3_.shape == (wl.B, wl.S, wl.E)
    np.testing.assert_allclose(f(w3_).sum(-1), 1.0, atol=1e-5)  # test_phase2_moe.py:84-85
    layer.eval()
    with torch.no_grad():
        y2, aux2 = layer(x, return_aux=True)
    layer.train()
    assert aux2 == 0.0 and torch.equal(y2, y)


def test_balanced_routing_layer(dev):
    """moe_balanced_routing=True (moe.py:443-451): config 1 dimensions with a logit
    skew so that capacity bites; routing bit-exact from the kernel's fp32 logits,
    output against the oracle experts."""
    wl = synth.WORKLOADS[1]
    t = synth.make_tensors(wl, "cpu")
    cfg = wl.config()
    cfg.moe_balanced_routing = True
    from kmoe.moe import MoELayer
    layer = synth.load_into(MoELayer(cfg, 0).to(device=dev, dtype=wl.dtype), {k: v.to(dev) for k, v in t.items()})
    with torch.no_grad():
        layer.router.router[2].weight[:2] += 0.05  # experts 0 and 1 preferred by most tokens
        x = t["x"].to(dev)
        y = layer(x)
        r = layer.router.route(x.reshape(wl.T, wl.d).to(torch.bfloat16))
    lg = f(r.logits)
    idx, w = O.balanced_topk(lg, wl.k)
    assert np.array_equal(r.idx.cpu().numpy(), idx)
    counts = np.bincount(idx.reshape(-1), minlength=wl.E)
    assert np.array_equal(layer.last_expert_counts.cpu().numpy(), counts)
    plain, _ = O.topk_select(lg, wl.k)
    assert not np.array_equal(plain, idx)  # the capacity rule changed some picks
    bf = lambda a: f(a.to(torch.bfloat16))
    W = (bf(t["w1"]), bf(t["w2"]), bf(t["w3"]))
    tokens = list(range(wl.T))
    ref = token_outputs(bf(t["x"]).reshape(wl.T, wl.d), idx, w, np.ones_like(idx, dtype=bool), W, tokens)
    assert relL2(f(y).reshape(wl.T, wl.d), ref) <= 1e-2


def test_cfg2_full_size(dev, cfg_cache):
    wl, t, layer = setup(cfg_cache, 2, dev)
    x = t["x"].to(dev)
    T, d = wl.T, wl.d
    with torch.no_grad():
        y = layer(x)
        y_again = layer(x)
        x2 = x.reshape(T, d)
        r = layer.router.route(x2)
        disp = ops.dispatch(x2, r.idx, r.w, wl.E)
    torch.cuda.synchronize()
    assert torch.equal(y, y_again), "forward is not bit-reproducible"
    lg = f(r.logits)
    idx_ref, w_ref = O.topk_select(lg, wl.k)
    assert np.array_equal(r.idx.cpu().numpy(), idx_ref)
    np.testing.assert_allclose(f(r.w), w_ref, rtol=2e-6, atol=1e-7)
    dref = O.dispatch(idx_ref, wl.E)
    assert np.array_equal(disp.counts.cpu().numpy(), dref["counts"])
    assert np.array_equal(disp.offsets.cpu().numpy(), dref["offsets"])
    assert np.array_equal(disp.slot_row.cpu().numpy(), dref["slot_row"])
    # permutation is a bijection onto [0, T*k)
    assert np.array_equal(np.sort(disp.slot_row.cpu().numpy()), np.arange(T * wl.k))
    # logits close to fp64
    sample = np.random.default_rng(0).choice(T, 768, replace=False)
    W = tuple(f(t[k]) for k in ("w1", "w2", "w3"))
    lref = O.router_logits(f(t["x"]).reshape(T, d)[sample], f(t["w_in"]), f(t["w_out"]))
    np.testing.assert_allclose(lg[sample], lref, atol=1e-5, rtol=1e-4)
    yref = token_outputs(f(t["x"]).reshape(T, d), idx_ref, w_ref, np.ones_like(idx_ref, bool), W, list(sample))
    assert relL2(f(y).reshape(T, d)[sample], yref) <= 1e-2
    aux_ref = O.aux_losses(lg, dref["counts"], T, wl.k, wl.E)
    assert abs(float(layer.aux_loss) - aux_ref[0]) <= 1e-4 * aux_ref[0]


def test_cfg3_zipf_capacity(dev, cfg_cache):
    wl, t, layer = setup(cfg_cache, 3, dev)
    x = t["x"].to(dev)
    T, d, E, k = wl.T, wl.d, wl.E, wl.k
    with torch.no_grad():
        y = layer(x)
        x2 = x.reshape(T, d)
        r = layer.router.route(x2)
        cap = ops.capacity_of(wl.capacity_factor, T, k, E)
        disp = ops.dispatch(x2, r.idx, r.w, E, capacity=cap)
    assert cap == 2560
    lg = f(r.logits)
    bias = synth.zipf_bias(E, wl.seed)
    lref = O.router_logits(f(t["x"]).reshape(T, d)[:512], f(t["w_in"]), f(t["w_out"]), bias)
    np.testing.assert_allclose(lg[:512], lref, atol=1e-5, rtol=1e-4)
    idx_ref, w_ref = O.topk_select(lg, k)
    assert np.array_equal(r.idx.cpu().numpy(), idx_ref)
    dref = O.dispatch(idx_ref, E, cap)
    frac = dref["counts"] / T
    assert 2 <= int((frac > 0.30).sum()) <= 3, frac
    assert np.array_equal(disp.counts.cpu().numpy(), dref["counts"])
    assert np.array_equal(disp.offsets.cpu().numpy(), dref["offsets"])
    assert np.array_equal(disp.slot_row.cpu().numpy(), dref["slot_row"])  # drop mask bit-exact
    keep = (dref["slot_row"] >= 0).reshape(T, k)
    rng = np.random.default_rng(1)
    sample = list(rng.choice(T, 512, replace=False))
    W = tuple(f(t[kk]) for kk in ("w1", "w2", "w3"))
    yref = token_outputs(f(t["x"]).reshape(T, d), idx_ref, w_ref, keep, W, sample)
    assert relL2(f(y).reshape(T, d)[sample], yref) <= 1e-2
    # fully dropped tokens produce exact zeros
    dropped = np.nonzero(~keep.any(axis=1))[0]
    if dropped.size:
        assert np.all(f(y).reshape(T, d)[dropped] == 0)


def test_cfg4_expert_choice(dev, cfg_cache):
    wl, t, layer = setup(cfg_cache, 4, dev)
    x = t["x"].to(dev)
    B, S, d, E = wl.B, wl.S, wl.d, wl.E
    with torch.no_grad():
        y = layer(x)
        r, sel, C = layer.router.route(x)
    assert C == 2048
    lg = f(r.logits)
    idx_ref, w_ref = O.ec_select(lg, B, S, E, C)
    assert np.array_equal(sel.idx.cpu().numpy(), idx_ref)
    np.testing.assert_allclose(f(sel.w), w_ref, rtol=1e-4, atol=1e-8)
    row_token, offsets, src_row, src_w = O.ec_tables(idx_ref, w_ref, S)
    assert np.array_equal(sel.src_row.cpu().numpy(), src_row)
    fan = (src_row >= 0).sum(1)
    assert fan.min() == 0 and fan.max() > 2  # variable fan-in (0..E)
    # oracle y on a token sample, including tokens with fan-in 0 and the largest fan-in
    X = f(t["x"]).reshape(B * S, d)
    W = tuple(f(t[kk]) for kk in ("w1", "w2", "w3"))
    rng = np.random.default_rng(2)
    sample = sorted(set(rng.choice(B * S, 384, replace=False).tolist()) | {int(np.argmax(fan)), int(np.argmin(fan))})
    keep = src_row >= 0
    e_idx = np.tile(np.arange(E), (B * S, 1))
    yref = token_outputs(X, e_idx, src_w, keep, W, sample)
    assert relL2(f(y).reshape(B * S, d)[sample], yref) <= 1e-2
    assert np.all(f(y).reshape(B * S, d)[fan == 0] == 0)
    if layer.training:
        _, _, z = O.aux_losses(lg, None, B * S, 1, E)
        assert abs(float(layer.aux_loss) - 0.001 * z) <= 1e-4 * 0.001 * z


def test_cfg5_fp8_mod(dev, cfg_cache):
    wl, t, layer = setup(cfg_cache, 5, dev)
    x = t["x"].to(dev)
    B, S, d, E, k = wl.B, wl.S, wl.d, wl.E, wl.k
    with torch.no_grad():
        y = layer(x)
        msel = layer.ffn_mod_router.select(x)
        keep = msel.sel_idx.shape[1]
        r = layer.ffn.router.route(x.reshape(B * S, d), row_index=msel.token_rows, T=B * keep)
    assert keep == 1536
    X = f(t["x"]).reshape(B * S, d)
    rr = f(msel.logits)
    np.testing.assert_allclose(rr, O.mod_logits(f(t["x"]), f(t["w_mod"])), atol=1e-4, rtol=1e-4)
    sel_ref, selw_ref = O.mod_select(rr, keep)
    assert np.array_equal(msel.sel_idx.cpu().numpy(), sel_ref)
    rows = (np.arange(B)[:, None] * S + sel_ref).reshape(-1)
    lg = f(r.logits)
    idx_ref, w_ref = O.topk_select(lg, k)
    assert np.array_equal(r.idx.cpu().numpy(), idx_ref)
    assert np.array_equal(layer.ffn.last_expert_counts.cpu().numpy(), np.bincount(idx_ref.reshape(-1), minlength=E))
    # y on a sample of kept tokens: mod weight * MoE, fp8-faithful and vs the fp32 reference
    W = tuple(f(t[kk]) for kk in ("w1", "w2", "w3"))
    Wq = tuple(O.quant_weight_cols(w) for w in W)
    rng = np.random.default_rng(3)
    sample = list(rng.choice(B * keep, 384, replace=False))
    Xk = X[rows]
    allk = np.ones_like(idx_ref, bool)
    y32 = token_outputs(Xk, idx_ref, w_ref, allk, W, sample) * selw_ref.reshape(-1)[sample][:, None]
    y8 = token_outputs(Xk, idx_ref, w_ref, allk, Wq, sample, fp8=True) * selw_ref.reshape(-1)[sample][:, None]
    got = f(y).reshape(B * S, d)[rows[sample]]
    # bar: the fp32 fake-quant reference; the unquantised fp32 one is informative only
    assert relL2(got, y8) <= 3e-2
    assert relL2(got, y32) <= 1e-1
    skipped = np.setdiff1d(np.arange(B * S), rows)
    assert np.all(f(y).reshape(B * S, d)[skipped] == 0)


def test_direct_experts_call_after_drop_layer_drops_nothing(dev):
    """GroupedExperts.forward (the reference's secondary boundary, moe.py:213-294) never
    drops, also right after a drop_overflow layer forward on the same module."""
    from kmoe import AdvancedMoEConfig, MoELayer
    print("direct experts after drop layer", flush=True)
    cfg = AdvancedMoEConfig(d_model=128, n_experts=4, moe_top_k=2, d_ff_expert=256, moe_capacity_factor=0.5,
                            moe_drop_overflow=True)
    torch.manual_seed(3)
    layer = MoELayer(cfg, 0).to(dev, torch.bfloat16).eval()
    x = torch.randn(1, 300, 128, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        layer(x)  # capacity ceil(0.5*300*2/4) = 75 < the routed counts: drops
        assert int(layer.last_expert_counts.max()) > 75
        T = 300
        idx = torch.stack([torch.zeros(T, dtype=torch.int64), torch.ones(T, dtype=torch.int64)], 1).to(dev)
        w = torch.full((T, 2), 0.5, device=dev)
        y = layer.grouped_experts(x.view(T, 128), idx, w)
        ge = layer.grouped_experts
        W = [f(t) for t in (ge.w1, ge.w2, ge.w3)]
        ref = token_outputs(f(x.view(T, 128)), f(idx), f(w), np.ones((T, 2), bool), W, list(range(T)))
    assert relL2(f(y), ref) <= 1e-2  # every token has both of its experts
