"""GPU parity of each HIP kernel against the CPU oracle (same seeded inputs).

Bars: integer/index outputs bit-exact; fp32 router logits within 1e-5 abs /
1e-4 rel of fp64; expert GEMMs rel-L2 <= 1e-2 (bf16) / 3e-2 (fp8) against the
fp32 oracle; the combine within one bf16 ulp of the fp64 sum."""
import numpy as np
import pytest
import torch

from kmoe import ops
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def relL2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bf16(t):
    return t.to(torch.bfloat16)


def npf(t):
    return t.detach().float().cpu().numpy()


def gen(seed, *shapes, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g) * scale for s in shapes]


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("T,d,E,k", [(512, 256, 8, 2), (16384, 2048, 16, 2), (1000, 128, 64, 4), (33, 64, 5, 1)])
def test_router_parity(dev, T, d, E, k):
    x, w_in, w_out = gen(100 + E, (T, d), (128, d), (E, 128), scale=1.0)
    w_in, w_out = w_in * 0.02, w_out * 0.02
    xb, wib, wob = bf16(x).to(dev), bf16(w_in).to(dev), bf16(w_out).to(dev)
    r = ops.router(xb, wib, wob, k)
    torch.cuda.synchronize()
    lg = npf(r.logits)
    ref = O.router_logits(npf(xb), npf(wib), npf(wob))
    np.testing.assert_allclose(lg, ref, atol=1e-5, rtol=1e-4)
    # routing from the kernel's own fp32 logits: bit-exact indices
    idx, w = O.topk_select(lg, k)
    assert np.array_equal(r.idx.cpu().numpy(), idx)
    np.testing.assert_allclose(npf(r.w), w, rtol=2e-6, atol=1e-7)
    # near-ties only: routing from fp64 logits differs on very few tokens
    idx64, _ = O.topk_select(ref, k)
    assert np.mean(np.any(idx64 != idx, axis=1)) < 0.01


@pytest.mark.parametrize("T,d,E", [(8192, 2048, 1), (8155, 512, 1), (100, 256, 8), (1000, 128, 64), (33, 64, 5)])
def test_router_logits_only_tiles(dev, T, d, E):
    """k = 0 without aux partials (the MoD auxiliary router's call): no partials buffer,
    logits and the saved pre-activation bit-identical to the call that writes partials,
    and within the fp64 bar (32-token tiles at these sizes; test_router_tiles_bit_identical
    compares the two tile sizes)."""
    x, w_in, w_out = gen(300 + E, (T, d), (128, d), (E, 128))
    xb, wib, wob = bf16(x).to(dev), bf16(w_in * 0.02).to(dev), bf16(w_out * 0.1).to(dev)
    r64 = ops.router(xb, wib, wob, 0, save_hidden=True)
    r32 = ops.router(xb, wib, wob, 0, save_hidden=True, partials=False)
    torch.cuda.synchronize()
    assert r32.partials is None
    assert torch.equal(r32.logits, r64.logits) and torch.equal(r32.hidden, r64.hidden)
    np.testing.assert_allclose(npf(r32.logits), O.router_logits(npf(xb), npf(wib), npf(wob)), atol=1e-5, rtol=1e-4)


def test_router_ties_lowest_index(dev):
    T, d, E = 256, 128, 8
    x, w_in, w_out = gen(7, (T, d), (128, d), (E, 128))
    v = w_out[0] * 0.05
    w_out = torch.zeros(E, 128)
    w_out[[2, 5, 7]] = v  # experts 2, 5, 7: bit-identical logits; the rest tie at 0
    r = ops.router(bf16(x).to(dev), bf16(w_in * 0.05).to(dev), bf16(w_out).to(dev), 2)
    lg = npf(r.logits)
    assert np.all(lg[:, 2] == lg[:, 5]) and np.all(lg[:, 2] == lg[:, 7])
    idx = r.idx.cpu().numpy()
    top_is_tie = lg[:, 2] > lg[:, 0]
    assert top_is_tie.any()
    assert np.all(idx[top_is_tie] == np.array([2, 5]))
    assert np.all(idx[~top_is_tie, 0] == 0) and np.all(idx[~top_is_tie, 1] == 1)


def test_router_bias_and_row_index(dev):
    T, d, E = 300, 256, 16
    x, w_in, w_out, b = gen(8, (T, d), (128, d), (E, 128), (E,))
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(1))[:100].to(torch.int32)
    xb, wib, wob = bf16(x).to(dev), bf16(w_in * 0.02).to(dev), bf16(w_out * 0.02).to(dev)
    r = ops.router(xb, wib, wob, 2, bias=b.to(dev), row_index=rows.to(dev))
    ref = O.router_logits(npf(xb)[rows.numpy()], npf(wib), npf(wob), b.numpy())
    np.testing.assert_allclose(npf(r.logits), ref, atol=1e-5, rtol=1e-4)
    assert np.array_equal(r.idx.cpu().numpy(), O.topk_select(npf(r.logits), 2)[0])


def test_aux_loss_parity(dev):
    T, d, E, k = 4096, 512, 16, 2
    x, w_in, w_out = gen(9, (T, d), (128, d), (E, 128))
    r = ops.router(bf16(x).to(dev), bf16(w_in * 0.05).to(dev), bf16(w_out * 0.05).to(dev), k)
    disp = ops.dispatch(bf16(x).to(dev), r.idx, r.w, E)
    out = ops.aux_loss(r.partials, T, E, disp.counts, k, 0.01, 0.001)
    lg = npf(r.logits)
    counts = np.bincount(r.idx.cpu().numpy().reshape(-1), minlength=E)
    aux, lb, z = O.aux_losses(lg, counts, T, k, E)
    np.testing.assert_allclose(npf(out), [aux, lb, z], rtol=2e-5)
    z_only = ops.aux_loss(r.partials, T, E, None, 1, 0.0, 0.001)
    np.testing.assert_allclose(npf(z_only), [0.001 * z, 0.0, z], rtol=2e-5)


# ------------------------------------------------------------------ balanced top-k
@pytest.mark.parametrize("T,E,k,mode", [(16384, 16, 2, "skew"), (3000, 8, 3, "ties"), (4096, 64, 8, "skew"),
                                        (8, 4, 3, "fallback"), (1, 5, 2, "plain"), (700, 6, 6, "ties")])
def test_balanced_topk_parity(dev, T, E, k, mode):
    g = torch.Generator().manual_seed(60 + T)
    lg = torch.randn(T, E, generator=g)
    if mode == "skew":
        lg = lg + 2.0 * torch.linspace(1, 0, E)  # popular early experts: capacity bites
    elif mode == "ties":
        lg = torch.round(lg * 2) / 2
    elif mode == "fallback":
        lg = torch.tensor([[3.0, 2.0, 1.0, 0.0]] * 6 + [[1.0, 0.0, 3.0, 2.0]] * 2)  # last round: 2 tokens all-full
    idx, w = ops.balanced_topk(lg.to(dev), k)
    ri, rw = O.balanced_topk(lg.numpy(), k)
    assert np.array_equal(idx.cpu().numpy(), ri)
    np.testing.assert_allclose(npf(w), rw, rtol=2e-6, atol=1e-7)


# ------------------------------------------------------------------ dispatch
def _routing(T, k, E, seed, skew=False):
    g = torch.Generator().manual_seed(seed)
    if skew:
        p = torch.tensor([0.5 ** (i / 2) for i in range(E)])
        first = torch.multinomial(p, T, replacement=True, generator=g)
    else:
        first = torch.randint(0, E, (T,), generator=g)
    idx = torch.empty(T, k, dtype=torch.int64)
    idx[:, 0] = first
    for j in range(1, k):
        idx[:, j] = (idx[:, j - 1] + 1 + torch.randint(0, E - 1, (T,), generator=g)) % E
    w = torch.rand(T, k, generator=g)
    return idx, w / w.sum(1, keepdim=True)


@pytest.mark.parametrize("T,k,E,cap,skew", [(16384, 2, 16, 0, False), (16384, 2, 16, 2560, True),
                                            (777, 3, 7, 50, True), (1, 1, 1, 0, False), (5000, 8, 64, 0, True)])
def test_dispatch_parity(dev, T, k, E, cap, skew):
    d = 256
    (x,) = gen(11, (T, d))
    idx, w = _routing(T, k, E, 12, skew)
    xb = bf16(x).to(dev)
    out = ops.dispatch(xb, idx.to(dev), w.to(dev), E, capacity=cap)
    torch.cuda.synchronize()
    ref = O.dispatch(idx.numpy(), E, cap)
    A_kept = int(ref["offsets"][-1])
    assert np.array_equal(out.counts.cpu().numpy(), ref["counts"])
    assert np.array_equal(out.offsets.cpu().numpy(), ref["offsets"])
    assert np.array_equal(out.slot_row.cpu().numpy()[: T * k], ref["slot_row"])
    assert np.array_equal(out.row_token.cpu().numpy()[:A_kept], ref["row_token"][:A_kept])
    assert torch.equal(out.slot_w[: T * k].cpu(), w.reshape(-1))
    assert torch.equal(out.xperm[:A_kept].cpu(), xb.cpu()[torch.from_numpy(ref["row_token"][:A_kept])])


@pytest.mark.parametrize("T,d,E,k,rows", [(16384, 2048, 16, 2, False), (1000, 128, 64, 4, False), (33, 64, 5, 1, False),
                                           (3000, 256, 16, 2, True)])
def test_router_block_counts(dev, T, d, E, k, rows):
    """kmoe_router_hist's per-block expert counts (blocks of router_block_tokens(T) tokens:
    32 when the 32-token workgroups fit the device at once) = the bincount of its own top-k
    ids per block (numpy), also with a row_index (MoD's selected rows) and a ragged last
    block; its logits and ids are those of kmoe_router."""
    x, w_in, w_out = gen(300 + E, (T + 100, d), (128, d), (E, 128))
    xb, wib, wob = bf16(x).to(dev), bf16(w_in * 0.02).to(dev), bf16(w_out * 0.02).to(dev)
    ri = None
    if rows:
        ri = torch.randperm(T + 100, generator=torch.Generator().manual_seed(4))[:T].to(torch.int32).to(dev)
    r = ops.router(xb, wib, wob, k, row_index=ri, T=T)
    r0 = ops.router(xb, wib, wob, k, row_index=ri, T=T, hist=False)
    torch.cuda.synchronize()
    assert r.block_counts is not None and r0.block_counts is None
    assert torch.equal(r.idx, r0.idx) and torch.equal(r.logits, r0.logits)
    idx = r.idx.cpu().numpy()
    hb = ops.router_block_tokens(T)
    assert hb == (32 if T <= 32 * torch.cuda.get_device_properties(dev).multi_processor_count else 64)
    nb = -(-T // hb)
    ref = np.zeros((nb, E), np.int64)
    for b in range(nb):
        ref[b] = np.bincount(idx[hb * b:hb * b + hb].reshape(-1), minlength=E)
    assert np.array_equal(r.block_counts.cpu().numpy(), ref)


@pytest.mark.parametrize("n,E,k", [(4096, 16, 2), (1000, 64, 4), (8192, 8, 8)])
def test_router_tiles_bit_identical(dev, n, E, k):
    """The first n tokens of a 16384-token call (64-token workgroups) and a call over those
    n tokens alone (32-token workgroups) give the same logits, ids and weights bit for
    bit: a token's K order depends on its 64-token block only."""
    T, d = 16384, 512
    x, w_in, w_out = gen(500 + E, (T, d), (128, d), (E, 128))
    xb, wib, wob = bf16(x).to(dev), bf16(w_in * 0.02).to(dev), bf16(w_out * 0.05).to(dev)
    assert ops.router_block_tokens(T) == 64 and ops.router_block_tokens(n) == 32
    big = ops.router(xb, wib, wob, k, save_hidden=True)
    small = ops.router(xb[:n].contiguous(), wib, wob, k, save_hidden=True)
    torch.cuda.synchronize()
    assert torch.equal(small.logits, big.logits[:n]) and torch.equal(small.hidden, big.hidden[:n])
    assert torch.equal(small.idx, big.idx[:n]) and torch.equal(small.w, big.w[:n])


@pytest.mark.parametrize("T,k,E,cap,fp8,mat", [(16384, 2, 16, 2560, False, True), (16384, 2, 16, 0, False, False),
                                               (70000, 2, 8, 0, False, True), (777, 3, 7, 50, True, True),
                                               (5000, 8, 64, 0, False, True)])
def test_dispatch_counted_matches_dispatch(dev, T, k, E, cap, fp8, mat):
    """kmoe_dispatch_counted with the router's block histograms gives kmoe_dispatch's
    results bit for bit (tables, permuted rows, fp8 codes and scales); T = 70000 takes
    the separate scan kernel."""
    d = 128
    x, w_in, w_out = gen(400 + T % 97, (T, d), (128, d), (E, 128))
    xb, wib, wob = bf16(x).to(dev), bf16(w_in * 0.05).to(dev), bf16(w_out * 0.05).to(dev)
    r = ops.router(xb, wib, wob, k)
    a = ops.dispatch(xb, r.idx, r.w, E, capacity=cap, fp8=fp8, materialize=mat)
    b = ops.dispatch(xb, r.idx, r.w, E, capacity=cap, fp8=fp8, materialize=mat, block_counts=r.block_counts)
    torch.cuda.synchronize()
    n = int(a.offsets[-1])
    for name in ("counts", "offsets", "slot_row", "slot_w"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert torch.equal(a.row_token[:n], b.row_token[:n])
    if mat:
        assert torch.equal(a.xperm[:n].view(torch.uint8), b.xperm[:n].view(torch.uint8))
    if fp8:
        assert torch.equal(a.xscale[:n], b.xscale[:n])
    ref = O.dispatch(r.idx.cpu().numpy(), E, cap)
    assert np.array_equal(b.slot_row.cpu().numpy()[: T * k], ref["slot_row"])


@pytest.mark.parametrize("T,k,E,cap,fp8,mat", [(16384, 2, 16, 0, False, False), (16384, 2, 16, 2560, False, True),
                                               (777, 3, 7, 50, True, True), (70000, 2, 8, 0, False, False),
                                               (65536, 1, 64, 0, False, False), (1, 1, 4, 0, False, False),
                                               (63, 8, 64, 3, False, True), (8192, 2, 16, 0, False, False),
                                               (8193, 2, 16, 1100, True, True)])
def test_dispatch_counted_aux(dev, T, k, E, cap, fp8, mat):
    """kmoe_dispatch_counted_aux: the tables, rows and codes of kmoe_dispatch_counted and the
    aux losses of kmoe_aux_loss, bit for bit (one more workgroup of the table launch up to
    65536 tokens, the separate launch beyond: T = 70000; router histograms and partials per
    32 tokens up to 8192 tokens, per 64 from 8193); the losses against the oracle."""
    d = 128
    x, w_in, w_out = gen(500 + T % 89, (T, d), (128, d), (E, 128))
    xb, wib, wob = bf16(x).to(dev), bf16(w_in * 0.05).to(dev), bf16(w_out * 0.05).to(dev)
    r = ops.router(xb, wib, wob, k)
    a = ops.dispatch(xb, r.idx, r.w, E, capacity=cap, fp8=fp8, materialize=mat, block_counts=r.block_counts)
    b = ops.dispatch(xb, r.idx, r.w, E, capacity=cap, fp8=fp8, materialize=mat, block_counts=r.block_counts,
                     aux=(r.partials, 0.01, 0.001))
    ref_aux = ops.aux_loss(r.partials, T, E, a.counts, k, 0.01, 0.001)
    torch.cuda.synchronize()
    assert a.aux is None and b.aux is not None
    n = int(a.offsets[-1])
    for name in ("counts", "offsets", "slot_row", "slot_w"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert torch.equal(a.row_token[:n], b.row_token[:n])
    if mat:
        assert torch.equal(a.xperm[:n].view(torch.uint8), b.xperm[:n].view(torch.uint8))
    if fp8:
        assert torch.equal(a.xscale[:n], b.xscale[:n])
    assert torch.equal(b.aux, ref_aux)
    counts = np.bincount(r.idx.cpu().numpy().reshape(-1), minlength=E)
    np.testing.assert_allclose(npf(b.aux), O.aux_losses(npf(r.logits), counts, T, k, E), rtol=2e-5)


def test_dispatch_rows_bf16_row_index_wide(dev):
    """The materialising bf16 dispatch through a row_index with the capacity drop, and a
    row wider than one register pass (d = 10240: the row copy loops)."""
    for T, d, E, k, cap in ((3000, 512, 16, 2, 300), (300, 10240, 4, 2, 0)):
        (x,) = gen(17, (T + 200, d))
        rows = torch.randperm(T + 200, generator=torch.Generator().manual_seed(3))[:T].to(torch.int32)
        idx, w = _routing(T, k, E, 18, True)
        xb = bf16(x).to(dev)
        out = ops.dispatch(xb, idx.to(dev), w.to(dev), E, capacity=cap, row_index=rows.to(dev))
        torch.cuda.synchronize()
        ref = O.dispatch(idx.numpy(), E, cap)
        n = int(ref["offsets"][-1])
        assert np.array_equal(out.row_token.cpu().numpy()[:n], ref["row_token"][:n])
        src = xb.cpu()[rows.long()][torch.from_numpy(ref["row_token"][:n])]
        assert torch.equal(out.xperm[:n].cpu(), src)


def test_dispatch_fp8_and_row_index(dev):
    T, k, E, d = 3000, 2, 16, 512
    (x,) = gen(13, (T + 500, d))
    x[7] = 0.0
    rows = torch.randperm(T + 500, generator=torch.Generator().manual_seed(2))[:T].to(torch.int32)
    rows[0] = 7  # an all-zero token row
    idx, w = _routing(T, k, E, 14, True)
    xb = bf16(x).to(dev)
    out = ops.dispatch(xb, idx.to(dev), bf16(w).to(dev), E, fp8=True, row_index=rows.to(dev))
    ref = O.dispatch(idx.numpy(), E)
    A = T * k
    src = npf(xb)[rows.numpy()][ref["row_token"]]
    q, s = O.quant_rows(src)
    assert np.array_equal(out.xperm[:A].cpu().numpy(), q)
    assert np.array_equal(npf(out.xscale[:A]), s)
    assert np.array_equal(npf(out.slot_w[:A]), npf(bf16(w)).reshape(-1))


@pytest.mark.parametrize("rows,cols,bound", [(12288, 2816, 11000), (4096, 1024, None), (300, 8192, 299),
                                             (5, 64, None), (1000, 512, 0)])
def test_quant_rows_fp8(dev, rows, cols, bound):
    """kmoe_quant_rows_fp8 (h before the fp8 down GEMM) against the oracle's per-row e4m3
    rule, codes and scales bit for bit, for every register-set width (2 to 16 vectors per
    lane) and a device-side row bound (only the rows below it are quantised); zero rows
    give scale 0 and zero codes."""
    g = torch.Generator().manual_seed(rows + cols)
    m = torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g) * 3)
    m[rows // 2] = 0.0
    mb = bf16(m).to(dev)
    nb = None if bound is None else torch.tensor([bound], dtype=torch.int32, device=dev)
    q, sc = ops.quant_rows_fp8(mb, n_rows_dev=nb)
    n = rows if bound is None else bound
    qr, sr = O.quant_rows(npf(mb[:n]))
    assert np.array_equal(q[:n].cpu().numpy(), qr)
    assert np.array_equal(npf(sc[:n]), sr)


def test_gather_rows(dev):
    (x,) = gen(15, (100, 128))
    xb = bf16(x).to(dev)
    rt = torch.tensor([5, -1, 99, 0, 5], dtype=torch.int32)
    out, _ = ops.gather_rows(xb, rt.to(dev), 5)
    exp = xb.cpu()[rt.clamp(min=0).long()]
    exp[1] = 0
    assert torch.equal(out.cpu(), exp)
    q, s = ops.gather_rows(xb, rt.to(dev), 5, fp8=True)
    qr, sr = O.quant_rows(npf(exp))
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(npf(s), sr)


# ------------------------------------------------------------------ grouped GEMMs
def _experts(E, d, F, seed, scale=0.02):
    return gen(seed, (E, d, F), (E, d, F), (E, F, d), scale=scale)


@pytest.mark.parametrize("d,F,counts", [
    (512, 768, [0, 1, 255, 256, 257, 513, 0, 1000, 31, 64, 0, 0, 300, 7, 2, 600]),
    (256, 352, [100, 0, 260, 3]),          # F not a multiple of 128, d < 256
    (2048, 2816, [300, 0, 257, 40]),       # full model width
])
def test_grouped_swiglu_bf16(dev, d, F, counts):
    E = len(counts)
    w1, w2, w3 = _experts(E, d, F, 20)
    A = sum(counts)
    (x,) = gen(21, (A, d))
    offsets = np.zeros(E + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    xb = bf16(x).to(dev)
    pw = ops.pack_weights(bf16(w1).to(dev), bf16(w2).to(dev), bf16(w3).to(dev))
    off = torch.from_numpy(offsets).to(torch.int32).to(dev)
    y = ops.grouped_ffn(xb, None, off, pw, A + 37)  # max_rows above the live rows
    torch.cuda.synchronize()
    ref = O.swiglu_rows(npf(xb), offsets, npf(bf16(w1)), npf(bf16(w2)), npf(bf16(w3)))
    err = relL2(npf(y[:A]), ref)
    assert err <= 1e-2, err
    # per-expert check (a wrong expert offset would show up here)
    for e in range(E):
        lo, hi = offsets[e], offsets[e + 1]
        if hi > lo:
            assert relL2(npf(y[lo:hi]), ref[lo:hi]) <= 1e-2


@pytest.mark.parametrize("with_row_index,cap", [(False, 0), (True, 0), (False, 300)])
def test_gate_up_gather_fused(dev, with_row_index, cap):
    """The gate/up GEMM that gathers its rows (x[row_index[row_token[r]]]) equals
    the one on the materialised permuted rows bit for bit, and the table-only
    dispatch writes the same tables as the materialising one."""
    T, k, E, d, F = 3000, 2, 8, 512, 768
    n_x = T + 321 if with_row_index else T
    (x,) = gen(30, (n_x, d))
    idx, w = _routing(T, k, E, 31, True)
    rows = (torch.randperm(n_x, generator=torch.Generator().manual_seed(3))[:T].to(torch.int32).to(dev)
            if with_row_index else None)
    xb = bf16(x).to(dev)
    w1, w2, w3 = _experts(E, d, F, 32)
    pw = ops.pack_weights(bf16(w1).to(dev), bf16(w2).to(dev), bf16(w3).to(dev))
    full = ops.dispatch(xb, idx.to(dev), w.to(dev), E, capacity=cap, row_index=rows)
    tab = ops.dispatch(xb, idx.to(dev), w.to(dev), E, capacity=cap, row_index=rows, materialize=False)
    assert tab.xperm is None
    A_kept = int(full.offsets[-1])
    for name in ("counts", "offsets", "slot_row", "slot_w"):
        assert torch.equal(getattr(full, name), getattr(tab, name)), name
    assert torch.equal(full.row_token[:A_kept], tab.row_token[:A_kept])
    h_ref = ops.gemm_gate_up(full.xperm, None, full.offsets, pw, T * k)
    h = ops.gemm_gate_up_rows(xb, rows, tab.row_token, tab.offsets, pw, T * k)
    torch.cuda.synchronize()
    assert torch.equal(h[:A_kept], h_ref[:A_kept])
    # and against the oracle on the gathered rows
    src = npf(xb)[rows.cpu().numpy()] if with_row_index else npf(xb)
    xg = src[tab.row_token[:A_kept].cpu().numpy()]
    off = tab.offsets.cpu().numpy().astype(np.int64)
    g = np.concatenate([xg[off[e]:off[e + 1]] @ npf(bf16(w1))[e] for e in range(E)])
    u = np.concatenate([xg[off[e]:off[e + 1]] @ npf(bf16(w2))[e] for e in range(E)])
    assert relL2(npf(h[:A_kept, :F]), O.silu(g) * u) <= 1e-2


def test_grouped_swiglu_f32_weights_and_kernels_api(dev):
    """fp32 parameters are packed directly; the reference's native-extension
    signature (kernels/__init__.py:105) runs on the same GEMMs."""
    from kmoe import kernels
    E, d, F = 4, 256, 512
    w1, w2, w3 = (t.to(dev) for t in _experts(E, d, F, 22))
    counts = torch.tensor([10, 0, 300, 50])
    ends = torch.cumsum(counts, 0)
    starts = ends - counts
    (x,) = gen(23, (int(ends[-1]), d))
    y = kernels.grouped_swiglu_forward(bf16(x).to(dev), w1, w2, w3, None, starts.to(dev), ends.to(dev))
    ref = O.swiglu_rows(npf(bf16(x)), np.concatenate([[0], ends.numpy()]), npf(w1), npf(w2), npf(w3))
    assert relL2(npf(y), ref) <= 1e-2


def test_grouped_swiglu_fp8(dev):
    E, d, F = 8, 1024, 1408
    counts = [500, 0, 260, 1, 700, 256, 33, 129]
    A = sum(counts)
    w1, w2, w3 = _experts(E, d, F, 24)
    (x,) = gen(25, (A, d))
    offsets = np.zeros(E + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    xb = bf16(x).to(dev)
    pw = ops.pack_weights(bf16(w1).to(dev), bf16(w2).to(dev), bf16(w3).to(dev), fp8=True)
    off = torch.from_numpy(offsets).to(torch.int32).to(dev)
    rt = torch.arange(A, dtype=torch.int32, device=dev)
    xq, xs = ops.gather_rows(xb, rt, A, fp8=True)
    y = ops.grouped_ffn(xq, xs, off, pw, A)
    torch.cuda.synchronize()
    W1, W2, W3 = npf(bf16(w1)), npf(bf16(w2)), npf(bf16(w3))
    # fp8-faithful oracle (same quantisation) and the unquantised fp32 reference
    qx, sx = O.quant_rows(npf(xb))
    faithful = O.swiglu_rows_fp8(qx, sx, offsets, O.quant_weight_cols(W1), O.quant_weight_cols(W2),
                                 O.quant_weight_cols(W3))
    # bar: the fp32 fake-quant reference (e4m3 casts, per-token / per-row scales)
    assert relL2(npf(y[:A]), faithful) <= 3e-2
    assert relL2(npf(y[:A]), faithful) <= 1e-2  # measured well inside the bar
    # e4m3 (3 mantissa bits) on Gaussian data costs ~6-7% against unquantised fp32
    ref = O.swiglu_rows(npf(xb), offsets, W1, W2, W3)
    assert relL2(npf(y[:A]), ref) <= 1e-1


@pytest.mark.parametrize("path", ["bf16", "gather", "save_gu", "rscale", "fp8", "fp8_gu"])
@pytest.mark.parametrize("rest", [4, 84, 144])
def test_split_tail_tiles_bit_identical(dev, path, rest):
    """The last partial round of tiles runs as narrow tiles (a quarter of the columns when
    at most n_cu/4 tiles are left, a half when at most n_cu/2, whole tiles otherwise).
    They compute every output element with the same MFMAs as a full tile: the experts
    of a launch whose tail they fill (`rest` tiles past the last full round: split 4,
    2, 1) give the same bits as in a launch with an extra expert appended, which has no
    partial round at all, for the gate/up (plain, gathered, g/u-saving, RMS-scaled,
    fp8, fp8 g/u-saving) and the down GEMMs."""
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    d, F = 512, 256  # 2 column tiles per slot in both GEMMs
    assert rest % 2 == 0 and rest < n_cu
    slots_a = (n_cu + rest) // 2  # tiles: n_cu + rest
    slots_b = n_cu                # tiles: 2 n_cu (two full rounds)
    rng = np.random.default_rng(rest)
    # slots per expert (7 experts), rows 256 (s - 1) + r with r in [1, 256]
    sl = np.full(7, slots_a // 7)
    sl[: slots_a - sl.sum()] += 1
    counts = [int(256 * (s - 1) + r) for s, r in zip(sl, rng.integers(1, 257, 7))]
    counts[1] = 256 * (int(sl[1]) - 1) + 256  # a slot of exactly 256 rows
    counts[2] = 256 * (int(sl[2]) - 1) + 1    # and one of a single row
    counts_b = counts + [256 * (slots_b - slots_a)]
    A, Ab = sum(counts), sum(counts_b)
    w1, w2, w3 = _experts(8, d, F, 40)
    (x,) = gen(41, (Ab, d))
    xb = bf16(x).to(dev)
    fp8 = path.startswith("fp8")
    pws = [ops.pack_weights(bf16(w1[:E]).to(dev), bf16(w2[:E]).to(dev), bf16(w3[:E]).to(dev), fp8=fp8)
           for E in (7, 8)]
    rs = (torch.rand(Ab, generator=torch.Generator().manual_seed(42)) + 0.5).to(dev)
    outs = []
    for cnt, pw in zip((counts, counts_b), pws):
        n = sum(cnt)
        off = torch.tensor(np.concatenate([[0], np.cumsum(cnt)]), dtype=torch.int32, device=dev)
        rt = torch.arange(n, dtype=torch.int32, device=dev)
        xs = xb[:n]
        gu = None
        if path == "bf16":
            h = ops.gemm_gate_up(xs, None, off, pw, n)
        elif path == "gather":
            h = ops.gemm_gate_up_rows(xs, None, rt, off, pw, n)
        elif path == "save_gu":
            h, gu = ops.gemm_gate_up_rows(xs, None, rt, off, pw, n, save_gu=True)
        elif path == "rscale":
            h = ops.gemm_gate_up_rows(xs, None, rt, off, pw, n, rscale=rs[:n].contiguous())
        if fp8:
            xq, xsc = ops.gather_rows(xb, rt, n, fp8=True)
            if path == "fp8_gu":
                h, gu = ops.gemm_gate_up(xq, xsc, off, pw, n, save_gu=True)
            else:
                h = ops.gemm_gate_up(xq, xsc, off, pw, n)
            y = ops.grouped_ffn(xq, xsc, off, pw, n)
        else:
            y = ops.gemm_down(h, None, off, pw, n)
        outs.append((h, gu, y))
    torch.cuda.synchronize()
    (ha, gua, ya), (hb, gub, yb) = outs
    assert torch.equal(ha[:A].view(torch.int16), hb[:A].view(torch.int16))
    assert torch.equal(ya[:A].view(torch.int16), yb[:A].view(torch.int16))
    if gua is not None:
        assert torch.equal(gua[:A].view(torch.int16), gub[:A].view(torch.int16))
    if path == "bf16":
        off = np.concatenate([[0], np.cumsum(counts)])
        ref = O.swiglu_rows(npf(xb[:A]), off, npf(bf16(w1[:7])), npf(bf16(w2[:7])), npf(bf16(w3[:7])))
        assert relL2(npf(ya[:A]), ref) <= 1e-2


# ------------------------------------------------------------------ fp8 straight-through operands
def test_gate_up_fp8_gu(dev):
    """kmoe_gemm_gate_up_fp8_gu: h bit-identical to kmoe_gemm_gate_up's, and the saved
    descaled gate / up values (packed order: per 128 columns of f, 128 gate then 128 up)
    against the fp32 products of the oracle's dequantised operands (e4m3 rows times
    their scales, per-column fake-quantised weights); bf16 rounding of the stored value
    is the only difference (rel-L2 ~1e-3, bar 4e-3)."""
    E, d, F = 4, 256, 320
    counts = [300, 0, 17, 256]
    A = sum(counts)
    Fp = 384
    w1, w2, w3 = _experts(E, d, F, 51)
    (x,) = gen(52, (A, d))
    xb = bf16(x).to(dev)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    off = torch.tensor(offsets, dtype=torch.int32, device=dev)
    pw = ops.pack_weights(bf16(w1).to(dev), bf16(w2).to(dev), bf16(w3).to(dev), fp8=True)
    xq, xs = ops.gather_rows(xb, torch.arange(A, dtype=torch.int32, device=dev), A, fp8=True)
    h_plain = ops.gemm_gate_up(xq, xs, off, pw, A)
    h, gu = ops.gemm_gate_up(xq, xs, off, pw, A, save_gu=True)
    torch.cuda.synchronize()
    assert torch.equal(h[:A].view(torch.int16), h_plain[:A].view(torch.int16))
    g4 = npf(gu[:A]).reshape(A, Fp // 128, 2, 128)
    g_got, u_got = g4[:, :, 0].reshape(A, Fp)[:, :F], g4[:, :, 1].reshape(A, Fp)[:, :F]
    qx, sx = O.quant_rows(npf(xb))
    xd = O.dequant_rows(qx, sx).astype(np.float64)
    W1q, W2q = O.quant_weight_cols(npf(bf16(w1))), O.quant_weight_cols(npf(bf16(w2)))
    g_ref = np.zeros((A, F))
    u_ref = np.zeros((A, F))
    for e in range(E):
        r = slice(offsets[e], offsets[e + 1])
        g_ref[r] = xd[r] @ W1q[e]
        u_ref[r] = xd[r] @ W2q[e]
    assert relL2(g_got, g_ref) <= 4e-3 and relL2(u_got, u_ref) <= 4e-3


@pytest.mark.parametrize("rows,cols,bound", [(700, 384, None), (700, 384, 513), (64, 2816, 0), (5, 8, None)])
def test_dequant_rows_fp8(dev, rows, cols, bound):
    """kmoe_dequant_rows_fp8 against the oracle's dequantisation rounded to bf16, bit for
    bit, on codes and scales from kmoe_quant_rows_fp8; rows at or past the device-side
    bound are left as they were."""
    from kmoe import _lib
    from kmoe._lib import ptr
    g = torch.Generator().manual_seed(rows + cols)
    m = torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g) * 2)
    q, sc = ops.quant_rows_fp8(bf16(m).to(dev))
    nb = None if bound is None else torch.tensor([bound], dtype=torch.int32, device=dev)
    out = torch.full((rows, cols), 7.0, device=dev, dtype=torch.bfloat16)
    _lib.call("kmoe_dequant_rows_fp8", ptr(q), ptr(sc), rows, ptr(nb), cols, ptr(out), None)
    torch.cuda.synchronize()
    n = rows if bound is None else bound
    want = torch.from_numpy(O.dequant_rows(q[:n].cpu().numpy(), npf(sc[:n]))).to(torch.bfloat16)
    assert torch.equal(out[:n].cpu().view(torch.int16), want.view(torch.int16))
    assert bool((out[n:] == 7.0).all())
    assert torch.equal(ops.dequant_rows_fp8(q, sc, nb)[:n].view(torch.int16), out[:n].view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fake_quant_cols_e4m3(dev, dtype):
    """kmoe_fake_quant_e4m3_cols against the oracle's per-output-column weight
    quantisation (the fp8 packing's), dequantised and rounded to bf16, bit for bit,
    including a zero column and columns past the last full 64-column block."""
    E, K, N = 3, 200, 130
    (w,) = gen(53, (E, K, N), scale=0.05)
    w[1, :, 7] = 0.0
    wd = w.to(dtype)
    got = ops.fake_quant_cols_e4m3(wd.to(dev))
    torch.cuda.synchronize()
    want = torch.from_numpy(O.quant_weight_cols(wd.float().numpy())).to(torch.bfloat16)
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
    assert bool((got[1, :, 7] == 0).all())


# ------------------------------------------------------------------ combine
def test_combine_parity(dev):
    T, fan, d, R = 1000, 3, 384, 2500
    g = torch.Generator().manual_seed(30)
    yperm = bf16(torch.randn(R, d, generator=g))
    src = torch.randint(-1, R, (T, fan), generator=g).to(torch.int32)
    w = torch.rand(T, fan, generator=g)
    out_map = torch.randint(-1, T, (T + 100,), generator=g).to(torch.int32)
    scale = torch.rand(T, generator=g)
    y = ops.combine(yperm.to(dev), src.to(dev), w.to(dev), T + 100, out_map=out_map.to(dev), scale=scale.to(dev))
    ref = O.combine(npf(yperm), src.numpy(), w.numpy(), out_map=out_map.numpy(), scale=scale.numpy(), T_out=T + 100)
    got = npf(y)
    # one bf16 rounding of the result plus fp32 accumulation error of the terms
    mag = O.combine(np.abs(npf(yperm)), src.numpy(), np.abs(w.numpy()), out_map=out_map.numpy(),
                    scale=scale.numpy(), T_out=T + 100)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -22)
    yf = ops.combine(yperm.to(dev), src.to(dev), w.to(dev), T + 100, out_map=out_map.to(dev), scale=scale.to(dev),
                     out_dtype=torch.float32)
    np.testing.assert_allclose(npf(yf), ref, rtol=1e-5, atol=1e-6)


def test_combine_top2_path_matches_generic(dev):
    """fan 2, d 2048, bf16 out runs a two-source kernel; it must equal the generic
    kernel bit for bit (the generic one is reached with a third, always-dropped source),
    and the oracle to the combine bar.  Dropped sources, out_map and scale included."""
    T, d, R = 3000, 2048, 6000
    g = torch.Generator().manual_seed(32)
    yperm = bf16(torch.randn(R, d, generator=g))
    src = torch.randint(-1, R, (T, 2), generator=g).to(torch.int32)
    w = torch.rand(T, 2, generator=g)
    out_map = torch.randint(-1, T, (T + 50,), generator=g).to(torch.int32)
    scale = torch.rand(T, generator=g)
    src3 = torch.cat([src, torch.full((T, 1), -1, dtype=torch.int32)], 1)
    w3 = torch.cat([w, torch.rand(T, 1, generator=g)], 1)
    for om, sc in ((None, None), (out_map, scale)):
        a = ops.combine(yperm.to(dev), src.to(dev), w.to(dev), T if om is None else T + 50,
                        out_map=None if om is None else om.to(dev), scale=None if sc is None else sc.to(dev))
        b = ops.combine(yperm.to(dev), src3.to(dev), w3.to(dev), T if om is None else T + 50,
                        out_map=None if om is None else om.to(dev), scale=None if sc is None else sc.to(dev))
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        ref = O.combine(npf(yperm), src.numpy(), w.numpy(), out_map=None if om is None else om.numpy(),
                        scale=None if sc is None else sc.numpy(), T_out=T if om is None else T + 50)
        mag = O.combine(np.abs(npf(yperm)), src.numpy(), w.numpy(), out_map=None if om is None else om.numpy(),
                        scale=None if sc is None else sc.numpy(), T_out=T if om is None else T + 50)
        assert np.all(np.abs(npf(a) - ref) <= np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -22)


def test_combine_is_deterministic(dev):
    T, fan, d, R = 4096, 16, 512, 20000
    g = torch.Generator().manual_seed(31)
    yperm = bf16(torch.randn(R, d, generator=g)).to(dev)
    src = torch.randint(-1, R, (T, fan), generator=g).to(torch.int32).to(dev)
    w = torch.rand(T, fan, generator=g).to(dev)
    a = ops.combine(yperm, src, w, T)
    b = ops.combine(yperm, src, w, T)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ expert choice / MoD selection
@pytest.mark.parametrize("B,S,E,C,ties", [(1, 16384, 16, 2048, False), (2, 300, 4, 75, True), (3, 64, 8, 64, False),
                                         (1, 12000, 4, 5000, True)])
def test_ec_select_parity(dev, B, S, E, C, ties):
    g = torch.Generator().manual_seed(40)
    lg = torch.randn(B * S, E, generator=g) * 0.2
    if ties:
        lg = torch.round(lg * 8) / 8  # many exactly equal logits
    out = ops.ec_select(lg.to(dev), B, S, E, C)
    idx, w = O.ec_select(lg.numpy(), B, S, E, C)
    assert np.array_equal(out.idx.cpu().numpy(), idx)
    np.testing.assert_allclose(npf(out.w), w, rtol=1e-4, atol=1e-7)
    row_token, offsets, src_row, _ = O.ec_tables(idx, w, S)
    assert np.array_equal(out.row_token.cpu().numpy(), row_token)
    assert np.array_equal(out.offsets.cpu().numpy(), offsets)
    assert np.array_equal(out.src_row.cpu().numpy(), src_row)


@pytest.mark.parametrize("B,S,E,C,ties", [(1, 16384, 16, 2048, False), (2, 300, 4, 75, True), (1, 12000, 4, 5000, True)])
def test_ec_select_token_order(dev, B, S, E, C, ties):
    """order 0 (the layer forward's): the descending selection with each expert's
    slots in ascending token order; weights bit-identical per (token, expert)."""
    g = torch.Generator().manual_seed(42)
    lg = torch.randn(B * S, E, generator=g) * 0.2
    if ties:
        lg = torch.round(lg * 8) / 8
    desc = ops.ec_select(lg.to(dev), B, S, E, C)
    asc = ops.ec_select(lg.to(dev), B, S, E, C, descending=False)
    di, dw = desc.idx.cpu().numpy(), desc.w.cpu().numpy()
    ai, aw = asc.idx.cpu().numpy(), asc.w.cpu().numpy()
    order = np.argsort(di, axis=-1, kind="stable")
    assert np.array_equal(ai, np.take_along_axis(di, order, axis=-1))
    assert np.array_equal(aw, np.take_along_axis(dw, order, axis=-1))  # bit-identical
    row_token, offsets, src_row, src_w = O.ec_tables(ai, aw, S)
    assert np.array_equal(asc.row_token.cpu().numpy(), row_token)
    assert np.array_equal(asc.offsets.cpu().numpy(), offsets)
    assert np.array_equal(asc.src_row.cpu().numpy(), src_row)
    sel = src_row >= 0
    assert np.array_equal(asc.src_w.cpu().numpy()[sel], desc.src_w.cpu().numpy()[sel])
    assert np.array_equal(asc.src_w.cpu().numpy()[sel], src_w[sel].astype(np.float32))


@pytest.mark.parametrize(
    "B,S,keep,ties",
    [(4, 2048, 1536, None), (2, 100, 75, "some"), (1, 7, 1, None), (1, 4096, 3000, "some"), (2, 333, 333, None),
     (2, 1000, 250, "all"), (1, 5000, 1234, "some")],  # S > 4096: the one-workgroup-per-sequence kernel
)
def test_mod_select_parity(dev, B, S, keep, ties):
    d = 256
    g = torch.Generator().manual_seed(41)
    x = torch.randn(B, S, d, generator=g)
    wm = torch.randn(1, d, generator=g) * 0.05
    if ties == "some":
        x[:, ::3] = x[:, :1]  # repeated rows -> equal router logits
    elif ties == "all":
        x[:] = x[:, :1]  # every logit of a sequence equal: the lowest indices are kept
    xb, wb = bf16(x).to(dev), bf16(wm).to(dev)
    out = ops.mod_select(xb, wb, keep)
    r = npf(out.logits)
    np.testing.assert_allclose(r, O.mod_logits(npf(xb), npf(wb)), atol=1e-4, rtol=1e-4)
    sel, w = O.mod_select(r, keep)
    assert np.array_equal(out.sel_idx.cpu().numpy(), sel)
    np.testing.assert_allclose(npf(out.sel_w), w, rtol=1e-5, atol=1e-8)
    exp_rows = (np.arange(B)[:, None] * S + sel).reshape(-1)
    assert np.array_equal(out.token_rows.cpu().numpy(), exp_rows)
    om = np.full(B * S, -1)
    om[exp_rows] = np.arange(B * keep)
    assert np.array_equal(out.out_map.cpu().numpy(), om)
