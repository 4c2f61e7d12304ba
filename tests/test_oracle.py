"""Pins the CPU oracle (oracle/moe_oracle.py) against independent checks:
brute force, library routines (numpy/torch), closed forms and the golden
fixtures.  CPU only."""
import itertools
import math
import os

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import moe_oracle as O
from oracle import torch_port as P

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ router logits
def test_router_logits_bruteforce():
    r = rng(0)
    T, d, E = 5, 16, 4
    x = r.standard_normal((T, d))
    w_in = r.standard_normal((128, d)) * 0.1
    w_out = r.standard_normal((E, 128)) * 0.1
    lg = O.router_logits(x, w_in, w_out)
    for t in range(T):
        for e in range(E):
            acc = 0.0
            for j in range(128):
                h = sum(x[t, i] * w_in[j, i] for i in range(d))
                acc += (h / (1.0 + math.exp(-h))) * w_out[e, j]
            assert abs(acc - lg[t, e]) < 1e-12


def test_router_logits_match_torch_modules():
    """Same math as the reference's nn.Sequential(Linear, SiLU, Linear) (moe.py:347-351)."""
    r = rng(1)
    T, d, E = 64, 32, 8
    x = r.standard_normal((T, d))
    seq = nn.Sequential(nn.Linear(d, 128, bias=False), nn.SiLU(), nn.Linear(128, E, bias=False)).double()
    ref = seq(torch.from_numpy(x)).detach().numpy()
    lg = O.router_logits(x, seq[0].weight.detach().numpy(), seq[2].weight.detach().numpy())
    np.testing.assert_allclose(lg, ref, rtol=1e-12, atol=1e-12)
    bias = r.standard_normal(E)
    np.testing.assert_allclose(O.router_logits(x, seq[0].weight.detach().numpy(), seq[2].weight.detach().numpy(),
                                               bias), ref + bias, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ top-k
def test_topk_bruteforce_with_ties():
    r = rng(2)
    lg = r.integers(0, 3, size=(200, 6)).astype(np.float64)  # many ties
    idx, w = O.topk_select(lg, 3)
    for t in range(lg.shape[0]):
        order = sorted(range(6), key=lambda e: (-lg[t, e], e))[:3]
        assert list(idx[t]) == order
        ex = np.exp(lg[t, order] - lg[t].max())
        np.testing.assert_allclose(w[t], ex / ex.sum(), rtol=1e-12)


def test_topk_matches_torch_on_tie_free():
    r = rng(3)
    lg = r.standard_normal((500, 16))
    idx, w = O.topk_select(lg, 2)
    p = torch.softmax(torch.from_numpy(lg), -1)
    tv, ti = torch.topk(p, 2, dim=-1)
    assert np.array_equal(idx, ti.numpy())
    np.testing.assert_allclose(w, (tv / tv.sum(-1, keepdim=True)).numpy(), rtol=1e-12)
    np.testing.assert_allclose(w.sum(1), 1.0, atol=1e-12)  # test_phase2_moe.py:84-85 invariant
    assert np.all(w[:, 0] >= w[:, 1])


# ------------------------------------------------------------------ balanced top-k
@pytest.mark.parametrize("T,E,k,skew", [(500, 16, 2, 0.0), (300, 8, 3, 2.0), (64, 4, 4, 3.0), (37, 5, 2, 1.0)])
def test_balanced_matches_torch_port(T, E, k, skew):
    """Logit-ranked restatement vs the reference's probability-masked op sequence
    (tie-free data): same experts, same weights."""
    r = rng(50 + T)
    lg = r.standard_normal((T, E)) + skew * np.linspace(1, 0, E)[None, :]  # skew: early experts popular
    idx, w = O.balanced_topk(lg, k)
    wt, it = P.balanced_topk_tc(torch.softmax(torch.from_numpy(lg), -1), k)
    assert np.array_equal(idx, it.numpy())
    np.testing.assert_allclose(w, wt.numpy(), rtol=1e-12)
    assert np.all(np.sort(idx, axis=1)[:, 1:] != np.sort(idx, axis=1)[:, :-1])  # distinct per token


def test_balanced_capacity_closed_form():
    """All tokens rank the experts 0 > 1 > 2 > 3.  Round 0: everyone takes expert
    0 (capacity is only checked between rounds), so its count (T) exceeds
    cap = T*k/E and it is masked afterwards; round 1: everyone takes expert 1;
    round 2 (k=3): experts 0 and 1 are full (T > cap = 3T/4), so everyone takes 2."""
    T, E = 40, 4
    lg = np.tile(np.array([3.0, 2.0, 1.0, 0.0]), (T, 1))
    idx, w = O.balanced_topk(lg, 3)
    assert np.all(idx == np.array([0, 1, 2]))
    p = np.exp(lg[0] - 3.0) / np.exp(lg[0] - 3.0).sum()
    np.testing.assert_allclose(w[0], p[:3] / (p[:3].sum() + 1e-9), rtol=1e-12)
    # capacity bites: 30 of the 40 tokens prefer expert 3 first; cap = T*2/4 = 20
    lg2 = lg.copy()
    lg2[:30, 3] = 5.0  # 30 tokens take expert 3 in round 0 -> 3 is full for round 1
    idx2, _ = O.balanced_topk(lg2, 2)
    assert np.all(idx2[:30, 0] == 3) and np.all(idx2[30:, 0] == 0)
    assert np.all(idx2[:30, 1] == 0) and np.all(idx2[30:, 1] == 1)  # expert 0 (10 picks) is not full


def test_balanced_fallback_when_all_full():
    """A token whose remaining experts are all full takes its best expert not
    picked yet, ignoring capacity (moe.py:402-407)."""
    # T=8, E=4, k=3, cap=6.  Tokens 2-7 rank 0 > 1 > 2 > 3, tokens 0-1 rank 2 > 3 > 0 > 1.
    # Round 0: six take expert 0 (full), two take 2.  Round 1: six take 1 (0 is full:
    # full too), two take 3.  Round 2: tokens 0-1 have only 0 and 1 left, both full:
    # they fall back to the better of the two (0); the others take 2.
    lg = np.tile(np.array([3.0, 2.0, 1.0, 0.0]), (8, 1))
    lg[:2] = [1.0, 0.0, 3.0, 2.0]
    idx, w = O.balanced_topk(lg, 3)
    assert np.all(idx[:2] == np.array([2, 3, 0])) and np.all(idx[2:] == np.array([0, 1, 2]))
    wt, it = P.balanced_topk_tc(torch.softmax(torch.from_numpy(lg), -1), 3)
    assert np.array_equal(idx, it.numpy())
    np.testing.assert_allclose(w, wt.numpy(), rtol=1e-12)
    lg3 = np.tile(np.array([2.0, 1.0, 0.0]), (12, 1))  # E=3, k=3, cap=12: round 2 has expert 2 free
    idx3, w3 = O.balanced_topk(lg3, 3)
    assert np.all(idx3 == np.array([0, 1, 2]))
    lg4 = np.tile(np.array([2.0, 1.0, 0.0]), (12, 1))
    lg4[:, 2] = [3.0] * 12  # everyone takes 2 first (count 12 = cap: full), then 0 (full), then 1 (fallback-free)
    idx4, _ = O.balanced_topk(lg4, 3)
    assert np.all(idx4 == np.array([2, 0, 1]))
    wt, it = P.balanced_topk_tc(torch.softmax(torch.from_numpy(lg4), -1), 3)
    assert np.array_equal(idx4, it.numpy())


def test_balanced_bruteforce_with_ties():
    """Integer logits (many ties): a per-token, per-round loop with the
    lowest-index rule."""
    r = rng(9)
    T, E, k = 120, 6, 3
    lg = r.integers(0, 3, size=(T, E)).astype(np.float64)
    idx, _ = O.balanced_topk(lg, k)
    cap = max(T * k // E, 1)
    counts = [0] * E
    chosen = [[] for _ in range(T)]
    for rr in range(k):
        full = [counts[e] >= cap for e in range(E)]
        picks = []
        for t in range(T):
            cand = [e for e in range(E) if e not in chosen[t] and not full[e]]
            if not cand:
                cand = [e for e in range(E) if e not in chosen[t]]
            best = min(cand, key=lambda e: (-lg[t, e], e))
            picks.append(best)
        for t, b in enumerate(picks):
            chosen[t].append(b)
            counts[b] += 1
    assert np.array_equal(idx, np.array(chosen))


# ------------------------------------------------------------------ aux
def test_aux_closed_forms():
    E, T, k = 8, 64, 2
    lg = np.zeros((T, E))
    counts = np.full(E, T * k // E)
    aux, lb, z = O.aux_losses(lg, counts, T, k, E)
    assert abs(z - math.log(E) ** 2) < 1e-12
    assert abs(lb - 1.0) < 1e-12
    assert abs(aux - (0.01 * lb + 0.001 * z)) < 1e-15
    # all routed to expert 0 with all probability on it -> LB = E
    lg2 = np.full((T, E), -1e4)
    lg2[:, 0] = 0.0
    _, lb2, _ = O.aux_losses(lg2, np.array([T * k] + [0] * (E - 1)), T, k, E)
    assert abs(lb2 - E) < 1e-9


def test_aux_matches_bruteforce_and_torch():
    r = rng(4)
    T, E, k = 50, 6, 2
    lg = r.standard_normal((T, E))
    idx, _ = O.topk_select(lg, k)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    aux, lb, z = O.aux_losses(lg, counts, T, k, E)
    p = np.array([[math.exp(v) / sum(math.exp(u) for u in row) for v in row] for row in lg])
    lb_bf = E * sum((counts[e] / (T * k)) * p[:, e].mean() for e in range(E))
    z_bf = np.mean([math.log(sum(math.exp(v) for v in row)) ** 2 for row in lg])
    assert abs(lb - lb_bf) < 1e-12 and abs(z - z_bf) < 1e-12
    ref = P.aux_tc(torch.from_numpy(lg).view(1, T, E), torch.from_numpy(idx).view(1, T, k), E)
    assert abs(float(ref) - aux) < 1e-7 * abs(aux)  # the port builds f in float32 (one_hot().float())


# ------------------------------------------------------------------ dispatch
@pytest.mark.parametrize("cap", [0, 3, 40])
def test_dispatch_matches_stable_argsort(cap):
    r = rng(5)
    T, k, E = 97, 2, 7
    idx = r.integers(0, E, size=(T, k))
    idx[:, 1] = (idx[:, 0] + 1 + r.integers(0, E - 1, size=T)) % E
    dp = O.dispatch(idx, E, cap)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    torder = torch.argsort(torch.from_numpy(flat), stable=True).numpy()
    assert np.array_equal(order, torder)
    assert np.array_equal(dp["counts"], np.bincount(flat, minlength=E))
    # without capacity the permutation is exactly argsort(stable)
    if cap == 0:
        assert np.array_equal(dp["row_token"], order // k)
        inv = np.empty_like(order)
        inv[order] = np.arange(order.size)
        assert np.array_equal(dp["slot_row"], inv)
    # brute force of the capacity rule
    seen = [0] * E
    row = 0
    rows = {}
    for e in range(E):
        for a in range(T * k):
            if flat[a] == e:
                if cap <= 0 or seen[e] < cap:
                    rows[a] = row
                    row += 1
                seen[e] += 1
    for a in range(T * k):
        assert dp["slot_row"][a] == rows.get(a, -1)
    assert dp["offsets"][-1] == row


# ------------------------------------------------------------------ experts / combine
def test_swiglu_rows_bruteforce():
    r = rng(6)
    E, d, F_ = 3, 8, 5
    w1, w2, w3 = (r.standard_normal(s) for s in [(E, d, F_), (E, d, F_), (E, F_, d)])
    offsets = np.array([0, 2, 2, 5])
    x = r.standard_normal((5, d))
    y = O.swiglu_rows(x, offsets, w1, w2, w3, dtype=np.float64)
    for e in range(E):
        for row in range(offsets[e], offsets[e + 1]):
            g = [sum(x[row, i] * w1[e, i, f] for i in range(d)) for f in range(F_)]
            u = [sum(x[row, i] * w2[e, i, f] for i in range(d)) for f in range(F_)]
            h = [g[f] / (1 + math.exp(-g[f])) * u[f] for f in range(F_)]
            ref = [sum(h[f] * w3[e, f, n] for f in range(F_)) for n in range(d)]
            np.testing.assert_allclose(y[row], ref, rtol=1e-12, atol=1e-12)


def test_combine_bruteforce():
    r = rng(7)
    yrows = r.standard_normal((6, 4))
    src = np.array([[0, 3], [-1, 5], [2, -1]])
    w = r.standard_normal((3, 2))
    out = O.combine(yrows, src, w, out_map=np.array([2, -1, 0, 1]), scale=np.array([2.0, 3.0, 4.0]), T_out=4)
    exp = np.zeros((4, 4))
    exp[0] = 4.0 * (w[2, 0] * yrows[2])
    exp[2] = 2.0 * (w[0, 0] * yrows[0] + w[0, 1] * yrows[3])
    exp[3] = 3.0 * (w[1, 1] * yrows[5])
    np.testing.assert_allclose(out, exp, rtol=1e-12)


def test_oracle_layer_matches_torch_port():
    """Two independent restatements agree: numpy oracle vs the op-for-op torch port."""
    r = rng(8)
    B, S, d, E, k, F_ = 2, 24, 32, 4, 2, 48
    x = r.standard_normal((B, S, d))
    w_in = r.standard_normal((128, d)) * 0.2
    w_out = r.standard_normal((E, 128)) * 0.2
    w1, w2 = r.standard_normal((E, d, F_)) * 0.2, r.standard_normal((E, d, F_)) * 0.2
    w3 = r.standard_normal((E, F_, d)) * 0.2
    res = O.moe_forward_tc(x.reshape(-1, d), w_in, w_out, w1, w2, w3, k, dtype=np.float64)
    tt = [torch.from_numpy(a) for a in (x, w_in, w_out, w1, w2, w3)]
    y, aux = P.moe_layer_tc(*tt, k)
    np.testing.assert_allclose(res["y"].reshape(B, S, d), y.numpy(), rtol=1e-9, atol=1e-9)
    assert abs(res["aux"][0] - float(aux)) < 1e-7 * abs(float(aux))  # f built in float32 by the port


# ------------------------------------------------------------------ expert choice
def test_ec_select_bruteforce_and_torch():
    r = rng(9)
    B, S, E, C = 2, 40, 4, 10
    lg = r.integers(0, 5, size=(B * S, E)).astype(np.float64)  # ties
    idx, w = O.ec_select(lg, B, S, E, C)
    L = lg.reshape(B, S, E)
    for b in range(B):
        for e in range(E):
            order = sorted(range(S), key=lambda s: (-L[b, s, e], s))[:C]
            assert list(idx[b, e]) == order
            p = np.exp(L[b, :, e] - L[b, :, e].max())
            p /= p.sum()
            np.testing.assert_allclose(w[b, e], p[order] / (p[order].sum() + 1e-9), rtol=1e-12)
    lg2 = r.standard_normal((B * S, E))
    idx2, w2 = O.ec_select(lg2, B, S, E, C)
    pr = torch.softmax(torch.from_numpy(lg2).view(B, S, E).transpose(1, 2), -1)
    tv, ti = torch.topk(pr, C, dim=-1)
    assert np.array_equal(idx2, ti.numpy())
    np.testing.assert_allclose(w2, (tv / (tv.sum(-1, keepdim=True) + 1e-9)).numpy(), rtol=1e-12)


def test_ec_layer_matches_torch_port():
    r = rng(10)
    B, S, d, E, F_, cf = 2, 32, 16, 4, 24, 2.0
    x = r.standard_normal((B, S, d))
    w_in, w_out = r.standard_normal((128, d)) * 0.3, r.standard_normal((E, 128)) * 0.3
    w1, w2, w3 = r.standard_normal((E, d, F_)) * 0.3, r.standard_normal((E, d, F_)) * 0.3, r.standard_normal((E, F_, d)) * 0.3
    C = math.ceil(S * cf / E)
    lg = O.router_logits(x.reshape(-1, d), w_in, w_out)
    idx, w = O.ec_select(lg, B, S, E, C)
    row_token, offsets, src_row, src_w = O.ec_tables(idx, w, S)
    yrows = O.swiglu_rows(x.reshape(-1, d)[row_token], offsets, w1, w2, w3, dtype=np.float64)
    y = O.combine(yrows, src_row, src_w)
    ref = P.moe_layer_ec(*[torch.from_numpy(a) for a in (x, w_in, w_out, w1, w2, w3)], cf)
    np.testing.assert_allclose(y.reshape(B, S, d), ref.numpy(), rtol=1e-9, atol=1e-9)


# ------------------------------------------------------------------ MoD
def test_mod_select_bruteforce_and_torch():
    r = rng(11)
    B, S, keep = 3, 30, 22
    rr = r.integers(0, 4, size=(B, S)).astype(np.float64)
    sel, w = O.mod_select(rr, keep)
    for b in range(B):
        order = sorted(sorted(range(S), key=lambda s: (-rr[b, s], s))[:keep])
        assert list(sel[b]) == order
        ex = np.exp(rr[b, order] - rr[b, order].max())
        np.testing.assert_allclose(w[b], ex / ex.sum(), rtol=1e-12)
    rr2 = r.standard_normal((B, S))
    sel2, w2 = O.mod_select(rr2, keep)
    tv, ti = torch.topk(torch.from_numpy(rr2), keep, dim=-1)
    si, so = torch.sort(ti, dim=-1)
    assert np.array_equal(sel2, si.numpy())
    np.testing.assert_allclose(w2, torch.softmax(torch.gather(tv, -1, so), -1).numpy(), rtol=1e-12)


# ------------------------------------------------------------------ fp8
def _torch_e4m3(v):
    t = torch.from_numpy(np.asarray(v, dtype=np.float32)).clamp(-448, 448)
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_exhaustive_against_torch():
    codes = np.arange(256, dtype=np.uint32)
    codes = codes[(codes & 0x7F) != 0x7F]
    vals = O.e4m3_to_f32(codes)
    # every code decodes/encodes to itself (except -0 -> 0x80 handled by sign)
    assert np.array_equal(O.f32_to_e4m3(vals), codes.astype(np.uint8))
    assert np.array_equal(_torch_e4m3(vals), codes.astype(np.uint8))
    # every rounding midpoint and its neighbours, plus out-of-range values
    pos = np.sort(np.unique(np.abs(vals)))
    mids = (pos[:-1].astype(np.float64) + pos[1:]) / 2
    probe = np.concatenate([mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                            np.nextafter(mids.astype(np.float32), np.float32(1e9)), [449.0, 464.0, 500.0, 1e6, 1e-12]])
    probe = np.concatenate([probe, -probe]).astype(np.float32)
    assert np.array_equal(O.f32_to_e4m3(probe), _torch_e4m3(probe))
    r = rng(12)
    rnd = (r.standard_normal(200000) * np.exp(r.uniform(-12, 7, 200000))).astype(np.float32)
    assert np.array_equal(O.f32_to_e4m3(rnd), _torch_e4m3(rnd))


def test_quant_rows_roundtrip():
    r = rng(13)
    m = r.standard_normal((8, 64)).astype(np.float32)
    m[3] = 0.0
    q, s = O.quant_rows(m)
    assert s[3] == 0 and np.all(q[3] == 0)
    dq = O.dequant_rows(q, s)
    rel = np.abs(dq - m).max(axis=1) / np.maximum(np.abs(m).max(axis=1), 1e-30)
    assert np.all(rel[[0, 1, 2, 4, 5, 6, 7]] <= 2 ** -4)  # e4m3 has 3 mantissa bits
    # amax element maps exactly to +-448
    for i in [0, 1, 2]:
        j = np.argmax(np.abs(m[i]))
        assert O.e4m3_to_f32(q[i, j:j + 1])[0] == np.sign(m[i, j]) * 448.0


def test_bf16_round_matches_torch():
    """bf16_round = torch's fp32 -> bfloat16 cast (round to nearest even) and back."""
    r = rng(14)
    v = (r.standard_normal(100000) * np.exp(r.uniform(-80, 80, 100000))).astype(np.float32)
    # exact ties (low half 0x8000, both parities of the kept bit), their neighbours,
    # the largest finite values (round to inf), subnormals, +-0, +-inf
    hi = r.integers(0, 1 << 16, 4000, dtype=np.uint64).astype(np.uint32) << 16
    ties = hi | np.uint32(0x8000)
    special = np.array([0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x00008000, 0x00018000, 0x00000001, 0x80000000,
                        0x00000000, 0x7F800000, 0xFF800000], dtype=np.uint32)
    bits = np.concatenate([v.view(np.uint32), ties, ties - 1, ties + 1, special])
    vals = bits.view(np.float32)
    vals = vals[~np.isnan(vals)]
    ref = torch.from_numpy(vals.copy()).to(torch.bfloat16).float().numpy()
    got = O.bf16_round(vals)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # NaN stays NaN (also payloads that only have low mantissa bits), sign kept
    nans = np.array([0x7FC00000, 0x7F800001, 0xFF800001, 0x7FFFFFFF], dtype=np.uint32).view(np.float32)
    out = O.bf16_round(nans)
    assert np.all(np.isnan(out))
    assert np.array_equal(np.signbit(out), np.signbit(nans))


def _torch_quant_cols(w):
    """Per-expert, per-output-column e4m3 fake-quant of w (E, K, N) in torch: scale =
    amax over K of column n / 448, q = e4m3(clamp(w * (448 / amax))), dequantised."""
    t = torch.from_numpy(np.asarray(w, dtype=np.float32))
    amax = t.abs().amax(dim=1, keepdim=True)                       # (E, 1, N)
    inv = torch.where(amax > 0, torch.tensor(448.0) / amax, torch.zeros_like(amax))
    q = (t * inv).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    return (q * (amax / 448.0)).numpy()


def test_quant_weight_cols_matches_torch_and_axis():
    """quant_weight_cols: one scale per (expert, output column n) = amax over the K
    (input) axis / 448 (cfg 5: per-expert per-output-row scales of w^T)."""
    r = rng(15)
    E, K, N = 3, 40, 24
    w = r.standard_normal((E, K, N)).astype(np.float32) * 0.02
    # columns of very different magnitudes and an all-zero column: a scale taken over
    # the wrong axis (per input row, per expert) would crush the small columns
    w[:, :, 3] *= 1e3
    w[:, :, 7] *= 1e-3
    w[1, :, 5] = 0.0
    got = O.quant_weight_cols(w)
    ref = _torch_quant_cols(w)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.all(got[1, :, 5] == 0.0)
    # brute force, element by element: every column's largest |w| maps to exactly
    # +-amax, and every element is within half an e4m3 step of the scaled value
    for e in range(E):
        for n in range(N):
            col = w[e, :, n].astype(np.float64)
            amax = np.abs(col).max()
            if amax == 0:
                continue
            j = int(np.argmax(np.abs(col)))
            assert got[e, j, n] == np.float32(np.sign(col[j]) * np.float32(amax / np.float32(448.0)) * 448.0)
            err = np.abs(got[e, :, n] - col) / amax
            assert err.max() <= 2.0 ** -4 * 1.0001  # 3 mantissa bits, relative to the column amax
    # per-column precision: a small column keeps its own relative precision
    rel7 = np.abs(got[:, :, 7] - w[:, :, 7]).max() / np.abs(w[:, :, 7]).max()
    assert rel7 <= 2.0 ** -4


def _torch_swiglu_fp8(xq, xs, offsets, w1q, w2q, w3q):
    """fp32 fake-quant restatement in torch of the cfg 5 expert path: x dequantised from
    its per-token scales, h = silu(x w1) * (x w2) rounded to bf16 by torch's cast,
    re-quantised per row with torch's e4m3 cast, y = h' w3."""
    x = torch.from_numpy(O.e4m3_to_f32(xq)) * torch.from_numpy(np.asarray(xs, np.float32))[:, None]
    y = torch.zeros(x.shape[0], w3q.shape[2])
    for e in range(w1q.shape[0]):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        xe = x[lo:hi]
        g = xe @ torch.from_numpy(w1q[e])
        u = xe @ torch.from_numpy(w2q[e])
        h = (g / (1.0 + torch.exp(-g)) * u).to(torch.bfloat16).float()
        amax = h.abs().amax(dim=1, keepdim=True)
        inv = torch.where(amax > 0, torch.tensor(448.0) / amax, torch.zeros_like(amax))
        hq = (h * inv).clamp(-448, 448).to(torch.float8_e4m3fn).float() * (amax / 448.0)
        y[lo:hi] = hq @ torch.from_numpy(w3q[e])
    return y.numpy()


def _fp8_case(seed, E=4, d=32, F_=24, T=37):
    r = rng(seed)
    x = r.standard_normal((T, d)).astype(np.float32)
    w1, w2, w3 = (r.standard_normal(s).astype(np.float32) * 0.1 for s in [(E, d, F_), (E, d, F_), (E, F_, d)])
    cuts = np.sort(r.integers(0, T + 1, E - 1))
    offsets = np.concatenate([[0], cuts, [T]]).astype(np.int64)
    offsets[2] = offsets[1]  # an empty expert
    xq, xs = O.quant_rows(O.bf16_round(x))
    return x, xq, xs, offsets, O.quant_weight_cols(w1), O.quant_weight_cols(w2), O.quant_weight_cols(w3)


def test_swiglu_rows_fp8_matches_torch_restatement():
    """swiglu_rows_fp8 = the torch fake-quant restatement (library casts for bf16 and
    e4m3).  The two differ only in fp32 summation order, which flips an e4m3 code of h
    about once in a million; dropping the bf16 rounding of h moves rel-L2 to ~6e-3,
    taking h's scales per column instead of per row to ~2e-2."""
    for seed in (16, 17):
        _, xq, xs, offsets, w1q, w2q, w3q = _fp8_case(seed)
        got = O.swiglu_rows_fp8(xq, xs, offsets, w1q, w2q, w3q)
        ref = _torch_swiglu_fp8(xq, xs, offsets, w1q, w2q, w3q)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 1e-4, rel
        close = np.abs(got - ref) <= 1e-5 * np.abs(ref).max()
        assert close.mean() >= 0.999


def test_swiglu_rows_fp8_bruteforce_fp64():
    """Per-token fp64 brute force of the fp8 expert path (tiny shape): dequantised x and
    weights, h in fp64 -> bf16 -> per-row e4m3 (torch casts), y summed in fp64."""
    E, d, F_, T = 3, 8, 6, 11
    x, xq, xs, offsets, w1q, w2q, w3q = _fp8_case(18, E=E, d=d, F_=F_, T=T)
    got = O.swiglu_rows_fp8(xq, xs, offsets, w1q, w2q, w3q)
    xd = O.e4m3_to_f32(xq).astype(np.float64) * xs.astype(np.float64)[:, None]
    for e in range(E):
        for t in range(int(offsets[e]), int(offsets[e + 1])):
            h = []
            for f in range(F_):
                g = sum(xd[t, i] * float(w1q[e, i, f]) for i in range(d))
                u = sum(xd[t, i] * float(w2q[e, i, f]) for i in range(d))
                h.append(g / (1.0 + math.exp(-g)) * u)
            hb = torch.tensor(h, dtype=torch.float64).float().to(torch.bfloat16).float()
            amax = float(hb.abs().max())
            sc = np.float32(amax) / np.float32(448.0)
            inv = np.float32(448.0) / np.float32(amax)
            hq = (hb * float(inv)).clamp(-448, 448).to(torch.float8_e4m3fn).float().double() * float(sc)
            for n in range(d):
                ref = sum(float(hq[f]) * float(w3q[e, f, n]) for f in range(F_))
                assert abs(got[t, n] - ref) <= 1e-5 * max(1.0, abs(ref)), (e, t, n, got[t, n], ref)


def test_mod_logits_matches_linear():
    """mod_logits = nn.Linear(d, 1, bias=False) of the MoD router (mod.py:93), fp64."""
    r = rng(19)
    B, S, d = 2, 9, 24
    x = r.standard_normal((B, S, d))
    lin = nn.Linear(d, 1, bias=False).double()
    ref = lin(torch.from_numpy(x)).squeeze(-1).detach().numpy()
    got = O.mod_logits(x, lin.weight.detach().numpy())
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-13)
    # brute force on one token
    assert abs(got[1, 4] - sum(x[1, 4, i] * float(lin.weight.detach()[0, i]) for i in range(d))) < 1e-12


# ------------------------------------------------------------------ golden fixtures
def test_golden_fixture_cfg1():
    path = os.path.join(GOLDEN, "cfg1_small.npz")
    g = np.load(path)
    res = O.moe_forward_tc(g["x"], g["w_in"], g["w_out"], g["w1"], g["w2"], g["w3"], int(g["k"]))
    assert np.array_equal(res["idx"], g["idx"])
    assert np.array_equal(res["counts"], g["counts"])
    np.testing.assert_allclose(res["y"], g["y"], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(res["aux"][0], float(g["aux"]), rtol=1e-5)


def test_golden_fixture_e4m3():
    g = np.load(os.path.join(GOLDEN, "e4m3_kat.npz"))
    assert np.array_equal(O.f32_to_e4m3(g["inputs"]), g["codes"])


# ---------------------------------------------------------------- backward oracle
def _tiny_layer(seed, T=6, d=4, E=3, k=2, F_=5, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: (torch.randn(*s, generator=g, dtype=torch.float64) * scale).requires_grad_(True)
    return (mk(T, d), mk(128, d), mk(E, 128), mk(E, d, F_), mk(E, d, F_), mk(E, F_, d),
            torch.randn(T, d, generator=g, dtype=torch.float64))


def test_routed_loss_matches_port_forward():
    """At the port's own top-k routing, the routed loss equals sum(y * dy) + aux of
    torch_port.moe_layer_tc (two restatements of moe.py:213-294, 423-462, 840-939)."""
    x, w_in, w_out, w1, w2, w3, dy = _tiny_layer(1, T=40, d=16, E=5, k=2, F_=12)
    with torch.no_grad():
        y, aux = P.moe_layer_tc(x[None], w_in, w_out, w1, w2, w3, 2, training=True)
        _, idx, _ = P.router_tc(x[None], w_in, w_out, 2)
        got_y = P.moe_loss_tc_routed(x, w_in, w_out, w1, w2, w3, idx[0], dy, training=False)
        got = P.moe_loss_tc_routed(x, w_in, w_out, w1, w2, w3, idx[0], dy)
    assert got_y == (y[0] * dy).sum()  # same ops, same order
    # the port forms its one-hot counts in float32 (as the reference's .float() does)
    assert abs(float(got - ((y[0] * dy).sum() + aux))) <= 1e-9


@pytest.mark.parametrize("cap,training,bias", [(0, True, False), (3, True, True), (0, False, False)])
def test_routed_loss_gradcheck(cap, training, bias):
    """At a fixed routing the layer is smooth: autograd of the routed loss equals
    central finite differences (fp64) for x and every parameter, with the capacity
    drop, a logit bias and without the aux losses."""
    x, w_in, w_out, w1, w2, w3, dy = _tiny_layer(2)
    with torch.no_grad():
        logits = F.linear(F.silu(F.linear(x, w_in)), w_out)
        idx = torch.topk(logits, 2, dim=-1).indices
    b = torch.tensor([0.3, -0.2, 0.1], dtype=torch.float64) if bias else None
    fn = lambda *a: P.moe_loss_tc_routed(*a, idx, dy, capacity=cap, bias=b, training=training)
    assert torch.autograd.gradcheck(fn, (x, w_in, w_out, w1, w2, w3), eps=1e-6, atol=1e-7, rtol=1e-5)


# ------------------------------------------------------------------ block boundary (RMSNorm + residual)
def test_rms_norm_pins():
    g = torch.Generator().manual_seed(60)
    x = torch.randn(37, 96, generator=g, dtype=torch.float64) * 3.0
    w = 1.0 + 0.3 * torch.randn(96, generator=g, dtype=torch.float64)
    got = O.rms_norm(x.numpy(), w.numpy(), 1e-5)
    # library routine
    ref = F.rms_norm(x, (96,), w, eps=1e-5).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)
    # weight 1, eps 0: every row has mean square 1; scaling x changes nothing
    u = O.rms_norm(x.numpy(), np.ones(96), 0.0)
    np.testing.assert_allclose(np.mean(u * u, axis=1), 1.0, rtol=1e-12)
    np.testing.assert_allclose(O.rms_norm(7.5 * x.numpy(), np.ones(96), 0.0), u, rtol=1e-12, atol=1e-14)
    # per-element brute force on a tiny input
    xs, ws = x[:3, :5].numpy(), w[:5].numpy()
    bf = np.zeros_like(xs)
    for i in range(3):
        ms = sum(float(v) * float(v) for v in xs[i]) / 5
        for j in range(5):
            bf[i, j] = ws[j] * xs[i, j] / math.sqrt(ms + 1e-5)
    np.testing.assert_allclose(O.rms_norm(xs, ws, 1e-5), bf, rtol=1e-13)


def test_ffn_block_matches_torch_port():
    T, d, E, k, Fd = 48, 64, 4, 2, 40
    g = torch.Generator().manual_seed(61)
    h = torch.randn(1, T, d, generator=g, dtype=torch.float64)
    nw = 1.0 + 0.3 * torch.randn(d, generator=g, dtype=torch.float64)
    w_in = torch.randn(128, d, generator=g, dtype=torch.float64) * 0.1
    w_out = torch.randn(E, 128, generator=g, dtype=torch.float64) * 0.1
    w1, w2 = (torch.randn(E, d, Fd, generator=g, dtype=torch.float64) * 0.1 for _ in range(2))
    w3 = torch.randn(E, Fd, d, generator=g, dtype=torch.float64) * 0.1
    r = O.ffn_block_tc(h[0].numpy(), nw.numpy(), 1e-5, w_in.numpy(), w_out.numpy(), w1.numpy(), w2.numpy(),
                       w3.numpy(), k)
    y, _ = P.moe_layer_tc(F.rms_norm(h, (d,), nw, eps=1e-5), w_in, w_out, w1, w2, w3, k, training=False)
    np.testing.assert_allclose(r["y"], (h + y)[0].numpy(), rtol=1e-9, atol=1e-12)


# ---------------------------------------------------------------- expert-choice backward oracle
def _tiny_ec(seed, B=2, S=10, d=6, E=3, F_=5, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: (torch.randn(*s, generator=g, dtype=torch.float64) * scale).requires_grad_(True)
    return (mk(B, S, d), mk(128, d), mk(E, 128), mk(E, d, F_), mk(E, d, F_), mk(E, F_, d),
            torch.randn(B, S, d, generator=g, dtype=torch.float64))


def test_ec_routed_loss_matches_layer_forward():
    """At its own top-C selection, moe_loss_ec_routed's output term equals moe_layer_ec's
    y (two restatements of moe.py:494-530, 626-673), and its z term the closed form."""
    x, w_in, w_out, w1, w2, w3, dy = _tiny_ec(5, B=2, S=16, d=8, E=4, F_=6)
    with torch.no_grad():
        y = P.moe_layer_ec(x, w_in, w_out, w1, w2, w3, 2.0)
        logits = torch.nn.functional.linear(torch.nn.functional.silu(torch.nn.functional.linear(x, w_in)), w_out)
        C = int(math.ceil(16 * 2.0 / 4))
        ti = torch.topk(torch.softmax(logits.transpose(1, 2), -1), C, dim=-1).indices
        l0 = P.moe_loss_ec_routed(x, w_in, w_out, w1, w2, w3, ti, dy, training=False)
        l1 = P.moe_loss_ec_routed(x, w_in, w_out, w1, w2, w3, ti, dy, training=True, w_z=0.5)
        z = (torch.logsumexp(logits, -1) ** 2).mean()
    assert abs(float(l0) - float((y * dy).sum())) < 1e-10
    assert abs(float(l1) - float(l0) - 0.5 * float(z)) < 1e-10


def test_ec_routed_loss_gradcheck():
    x, w_in, w_out, w1, w2, w3, dy = _tiny_ec(6)
    with torch.no_grad():
        logits = torch.nn.functional.linear(torch.nn.functional.silu(torch.nn.functional.linear(x, w_in)), w_out)
        ti = torch.topk(torch.softmax(logits.transpose(1, 2), -1), 4, dim=-1).indices
    f = lambda *a: P.moe_loss_ec_routed(*a, ti, dy, training=True, w_z=0.3)
    assert torch.autograd.gradcheck(f, (x, w_in, w_out, w1, w2, w3), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_router_loss_routed_gradcheck_and_forward():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(9, 6, generator=g, dtype=torch.float64, requires_grad=True)
    w_in = (torch.randn(128, 6, generator=g, dtype=torch.float64) * 0.3).requires_grad_(True)
    w_out = (torch.randn(4, 128, generator=g, dtype=torch.float64) * 0.3).requires_grad_(True)
    w, idx, logits = P.router_tc(x[None], w_in, w_out, 2)
    gw, gl = torch.randn(9, 2, generator=g, dtype=torch.float64), torch.randn(9, 4, generator=g, dtype=torch.float64)
    with torch.no_grad():
        ref = float((w[0] * gw).sum() + (logits[0] * gl).sum())
        got = float(P.router_loss_routed(x, w_in, w_out, idx[0], gw, gl))
    assert abs(ref - got) < 1e-12  # at its own routing: Router.forward's (w, logits)
    f = lambda *a: P.router_loss_routed(*a, idx[0], gw, gl)
    assert torch.autograd.gradcheck(f, (x, w_in, w_out), eps=1e-6, atol=1e-6, rtol=1e-5)


def _tiny_ffn_half(seed=21):
    g = torch.Generator().manual_seed(seed)
    B, S, d, E, k, F_ = 2, 10, 8, 4, 2, 6
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g, dtype=torch.float64) * sc)
    return dict(h=r(B, S, d), w_in=r(128, d, sc=0.3), w_out=r(E, 128, sc=0.3), w1=r(E, d, F_, sc=0.4),
                w2=r(E, d, F_, sc=0.4), w3=r(E, F_, d, sc=0.4), nw=1.0 + 0.2 * r(d), w_mod=r(1, d, sc=0.5),
                dy=r(B, S, d), k=k, keep=7)


@pytest.mark.parametrize("with_norm", [False, True])
def test_ffn_half_loss_matches_numpy_composition(with_norm):
    """ffn_half_loss_routed (the torch restatement of layers.py:142-187 with MoD) against
    the numpy oracle's own pieces: rms_norm, mod_logits / mod_select (argsort-based),
    moe_forward_tc (routing from its own logits) and an explicit scatter of the weighted
    rows; the loss is sum(out * dy) + the MoE aux on the kept tokens."""
    c = _tiny_ffn_half()
    B, S, d = c["h"].shape
    k, keep = c["k"], c["keep"]
    h = c["h"].numpy()
    x = O.rms_norm(h, c["nw"].numpy(), 1e-5) if with_norm else h
    r = O.mod_logits(x, c["w_mod"].numpy())
    sel, sw = O.mod_select(r, keep)
    rows = np.concatenate([x[b, sel[b]] for b in range(B)])
    ref = O.moe_forward_tc(rows, c["w_in"].numpy(), c["w_out"].numpy(), c["w1"].numpy(), c["w2"].numpy(),
                           c["w3"].numpy(), k, dtype=np.float64)
    out = np.zeros_like(x)
    for b in range(B):
        out[b, sel[b]] = sw[b][:, None] * ref["y"][b * keep:(b + 1) * keep]
    base = h if with_norm else 0.0
    want = float(((base + out) * c["dy"].numpy()).sum() + ref["aux"][0])
    got = float(P.ffn_half_loss_routed(c["h"], c["w_in"], c["w_out"], c["w1"], c["w2"], c["w3"],
                                       torch.from_numpy(ref["idx"]), c["dy"], norm_w=c["nw"] if with_norm else None,
                                       w_mod=c["w_mod"], sel_idx=torch.from_numpy(sel)))
    assert abs(got - want) <= 1e-10 * max(1.0, abs(want))
    # without MoD: h + MoE(RMSNorm(h)) of ffn_block_tc
    if with_norm:
        blk = O.ffn_block_tc(h.reshape(-1, d), c["nw"].numpy(), 1e-5, c["w_in"].numpy(), c["w_out"].numpy(),
                             c["w1"].numpy(), c["w2"].numpy(), c["w3"].numpy(), k)
        want2 = float((blk["y"] * c["dy"].numpy().reshape(-1, d)).sum() + blk["aux"][0])
        got2 = float(P.ffn_half_loss_routed(c["h"], c["w_in"], c["w_out"], c["w1"], c["w2"], c["w3"],
                                            torch.from_numpy(blk["idx"]), c["dy"], norm_w=c["nw"]))
        assert abs(got2 - want2) <= 1e-10 * max(1.0, abs(want2))


def test_ffn_half_loss_ec_matches_numpy_composition():
    """ffn_half_loss_ec_routed (MoD around the expert-choice layer, layers.py:148-187)
    against the numpy oracle's pieces: mod_logits / mod_select, then on the kept rows
    router_logits, ec_select (capacity from the kept length), ec_tables, swiglu_rows and
    combine, an explicit scatter of the weighted rows and the z-loss of the kept rows'
    logits; plus the same with w_z = 0 and no residual."""
    c = _tiny_ffn_half(23)
    B, S, d = c["h"].shape
    keep, E, cf, w_z = c["keep"], c["w_out"].shape[0], 2.0, 0.3
    h = c["h"].numpy()
    res = 0.5 * c["dy"].numpy()[:, ::-1].copy()
    sel, sw = O.mod_select(O.mod_logits(h, c["w_mod"].numpy()), keep)
    xs = np.concatenate([h[b, sel[b]] for b in range(B)])
    C = math.ceil(keep * cf / E)
    lg = O.router_logits(xs, c["w_in"].numpy(), c["w_out"].numpy())
    idx, w = O.ec_select(lg, B, keep, E, C)
    row_token, offsets, src_row, src_w = O.ec_tables(idx, w, keep)
    yrows = O.swiglu_rows(xs[row_token], offsets, c["w1"].numpy(), c["w2"].numpy(), c["w3"].numpy(),
                          dtype=np.float64)
    y = O.combine(yrows, src_row, src_w).reshape(B, keep, d)
    out = np.zeros_like(h)
    for b in range(B):
        out[b, sel[b]] = sw[b][:, None] * y[b]
    m = lg.max(axis=-1)
    z = np.mean((m + np.log(np.exp(lg - m[:, None]).sum(axis=-1))) ** 2)
    dy = c["dy"].numpy()
    args = [c[n] for n in ("h", "w_in", "w_out", "w1", "w2", "w3")] + [torch.from_numpy(idx), c["dy"]]
    kw = dict(w_mod=c["w_mod"], sel_idx=torch.from_numpy(sel))
    want = float(((res + out) * dy).sum() + w_z * z)
    got = float(P.ffn_half_loss_ec_routed(*args, residual=torch.from_numpy(res), w_z=w_z, **kw))
    assert abs(got - want) <= 1e-10 * max(1.0, abs(want))
    want0 = float((out * dy).sum())
    got0 = float(P.ffn_half_loss_ec_routed(*args, training=False, **kw))
    assert abs(got0 - want0) <= 1e-10 * max(1.0, abs(want0))


def test_mod_aux_loss_matches_library_bce():
    """mod_aux_loss against torch's binary_cross_entropy_with_logits on the numpy
    oracle's router MLP (router_logits with one output) and mod_select's kept set."""
    c = _tiny_ffn_half(24)
    B, S, d = c["h"].shape
    g = torch.Generator().manual_seed(7)
    w_a = torch.randn(128, d, generator=g, dtype=torch.float64) * 0.3
    w_b = torch.randn(1, 128, generator=g, dtype=torch.float64) * 0.3
    h = c["h"].numpy()
    sel, _ = O.mod_select(O.mod_logits(h, c["w_mod"].numpy()), c["keep"])
    lg = torch.from_numpy(O.router_logits(h.reshape(-1, d), w_a.numpy(), w_b.numpy())).view(B, S)
    t = torch.zeros(B, S, dtype=torch.float64)
    for b in range(B):
        t[b, torch.from_numpy(sel[b])] = 1.0
    want = 0.25 * float(F.binary_cross_entropy_with_logits(lg, t))
    got = float(P.mod_aux_loss(c["h"], w_a, w_b, torch.from_numpy(sel), 0.25))
    assert abs(got - want) <= 1e-12 * max(1.0, abs(want))


def test_ffn_half_loss_gradcheck():
    """Finite differences of the MoD + norm composition at a fixed selection and routing
    (the gradients the GPU backward is compared with)."""
    c = _tiny_ffn_half(22)
    B, S, d = c["h"].shape
    x = O.rms_norm(c["h"].numpy(), c["nw"].numpy(), 1e-5)
    sel, _ = O.mod_select(O.mod_logits(x, c["w_mod"].numpy()), c["keep"])
    rows = np.concatenate([x[b, sel[b]] for b in range(B)])
    idx = O.moe_forward_tc(rows, c["w_in"].numpy(), c["w_out"].numpy(), c["w1"].numpy(), c["w2"].numpy(),
                           c["w3"].numpy(), c["k"], dtype=np.float64)["idx"]
    ins = [c[n].clone().requires_grad_(True) for n in ("h", "nw", "w_mod", "w_in", "w_out", "w1", "w2", "w3")]

    def f(h, nw, w_mod, w_in, w_out, w1, w2, w3):
        return P.ffn_half_loss_routed(h, w_in, w_out, w1, w2, w3, torch.from_numpy(idx), c["dy"], norm_w=nw,
                                      w_mod=w_mod, sel_idx=torch.from_numpy(sel))
    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-5, rtol=1e-4)


# ------------------------------------------------------------------ non-gated experts
def test_plain_rows_bruteforce():
    """plain_rows (silu(x W1[e]) W2[e], moe.py:281-283) against a per-token, per-unit fp64
    loop; and the torch port's padded-bmm experts with w3 None against dispatch +
    plain_rows + combine of the numpy oracle (two restatements)."""
    rng = np.random.default_rng(41)
    T, d, E, k, F_ = 13, 6, 3, 2, 5
    x = rng.standard_normal((T, d))
    w1 = rng.standard_normal((E, d, F_)) * 0.4
    w2 = rng.standard_normal((E, F_, d)) * 0.4
    idx, w = O.topk_select(rng.standard_normal((T, E)), k)
    dp = O.dispatch(idx, E)
    rows = x[dp["row_token"][: dp["offsets"][E]]]
    got = O.plain_rows(rows, dp["offsets"], w1, w2, dtype=np.float64)
    want = np.zeros_like(got)
    for e in range(E):
        for r in range(int(dp["offsets"][e]), int(dp["offsets"][e + 1])):
            for f in range(F_):
                a = sum(rows[r, i] * w1[e, i, f] for i in range(d))
                want[r] += a / (1.0 + math.exp(-a)) * w2[e, f]
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    assert np.array_equal(O.swiglu_rows(rows, dp["offsets"], w1, w2, None, dtype=np.float64), got)
    y_np = O.combine(got, dp["slot_row"].reshape(T, k), w)
    y_t = P.grouped_experts_tc(torch.from_numpy(x), torch.from_numpy(idx), torch.from_numpy(w), torch.from_numpy(w1),
                               torch.from_numpy(w2), None)
    assert np.allclose(y_t.numpy(), y_np, rtol=1e-12, atol=1e-12)


def test_plain_routed_losses_gradcheck():
    """The backward references with non-gated experts: token choice at its own routing
    equals moe_layer_tc's forward, and both routed losses pass finite differences."""
    g = torch.Generator().manual_seed(43)
    mk = lambda *s: (torch.randn(*s, generator=g, dtype=torch.float64) * 0.5).requires_grad_(True)
    x, w_in, w_out, w1, w2 = mk(9, 6), mk(128, 6), mk(4, 128), mk(4, 6, 5), mk(4, 5, 6)
    dy = torch.randn(9, 6, generator=g, dtype=torch.float64)
    with torch.no_grad():
        y, aux = P.moe_layer_tc(x[None], w_in, w_out, w1, w2, None, 2, training=True)
        _, idx, _ = P.router_tc(x[None], w_in, w_out, 2)
        got = P.moe_loss_tc_routed(x, w_in, w_out, w1, w2, None, idx[0], dy, training=True)
    # (aux_tc counts in float32: 1e-8 relative)
    assert abs(float(got) - float((y[0] * dy).sum() + aux)) < 1e-8 * max(1.0, abs(float(got)))
    f = lambda *a: P.moe_loss_tc_routed(*a, None, idx[0], dy, training=True)
    assert torch.autograd.gradcheck(f, (x, w_in, w_out, w1, w2), eps=1e-6, atol=1e-6, rtol=1e-5)
    xe, wi, wo, e1, e2, _, dye = _tiny_ec(44)
    e2 = (torch.randn(3, 5, 6, generator=g, dtype=torch.float64) * 0.5).requires_grad_(True)
    with torch.no_grad():
        logits = torch.nn.functional.linear(torch.nn.functional.silu(torch.nn.functional.linear(xe, wi)), wo)
        ti = torch.topk(torch.softmax(logits.transpose(1, 2), -1), 4, dim=-1).indices
    fe = lambda *a: P.moe_loss_ec_routed(*a, None, ti, dye, training=True, w_z=0.3)
    assert torch.autograd.gradcheck(fe, (xe, wi, wo, e1, e2), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_fp8_mod_port_matches_numpy_oracle():
    """oracle/torch_port.py moe_layer_fp8_mod (config 5's CPU baseline) against the numpy
    oracle's pieces: mod_select, then the fp8 token-choice layer (moe_forward_tc fp8=True)
    on the gathered rows, weighted and scattered back.  Same selection and routing; the
    products' fp32 summation order differs, which moves an occasional value across an e4m3
    rounding boundary (one code = 1/8 relative): 0.4% rel-L2 on this draw, where a missing
    or misplaced step of the composition costs O(1)."""
    g = torch.Generator().manual_seed(21)
    B, S, d, E, k, F_, keep = 2, 40, 64, 6, 2, 96, 30
    # bf16-representable activations, as the layer's input always is (the oracle rounds
    # the rows to bf16 before their per-token scale)
    x = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(torch.float32)
    w_mod = torch.randn(1, d, generator=g) * 0.05
    w_in, w_out = torch.randn(128, d, generator=g) * 0.05, torch.randn(E, 128, generator=g) * 0.05
    w1, w2, w3 = (torch.randn(E, d, F_, generator=g) * 0.05, torch.randn(E, d, F_, generator=g) * 0.05,
                  torch.randn(E, F_, d, generator=g) * 0.05)
    w1q, w2q, w3q = P.fake_quant_expert_weights(w1, w2, w3)
    # the weight fake quantisation is the oracle's per-output-column scheme
    np.testing.assert_array_equal(w1q.numpy(), O.quant_weight_cols(w1.numpy()))
    got = P.moe_layer_fp8_mod(x, w_mod, w_in, w_out, w1q, w2q, w3q, k, keep).numpy()
    xn = x.numpy()
    sel, pw = O.mod_select(O.mod_logits(xn, w_mod.numpy(), dtype=np.float32), keep)
    ref = np.zeros_like(xn)
    for b in range(B):
        rows = xn[b, sel[b]]
        r = O.moe_forward_tc(rows, w_in.numpy(), w_out.numpy(), w1.numpy(), w2.numpy(), w3.numpy(), k, fp8=True)
        ref[b, sel[b]] = pw[b][:, None].astype(np.float32) * r["y"]
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err < 1e-2, err
    # the skipped tokens stay zero, the kept ones do not
    mask = np.zeros((B, S), dtype=bool)
    for b in range(B):
        mask[b, sel[b]] = True
    assert np.all(got[~mask] == 0) and np.all(np.abs(got[mask]).sum(-1) > 0)


def test_fp8_ste_forward_matches_fp8_port():
    """The straight-through fp8 restatement (ffn_half_loss_routed fp8=True, the GPU
    training tests' reference) computes the same forward as the pinned config 5 port
    moe_layer_fp8_mod at the same MoD selection and routing."""
    g = torch.Generator().manual_seed(22)
    B, S, d, E, k, F_, keep = 2, 24, 64, 5, 2, 80, 16
    x = torch.randn(B, S, d, generator=g, dtype=torch.float64).to(torch.bfloat16).to(torch.float64)
    w_mod = torch.randn(1, d, generator=g, dtype=torch.float64) * 0.05
    w_in = torch.randn(128, d, generator=g, dtype=torch.float64) * 0.05
    w_out = torch.randn(E, 128, generator=g, dtype=torch.float64) * 0.05
    w1, w2 = (torch.randn(E, d, F_, generator=g, dtype=torch.float64) * 0.05 for _ in range(2))
    w3 = torch.randn(E, F_, d, generator=g, dtype=torch.float64) * 0.05
    want = P.moe_layer_fp8_mod(x, w_mod, w_in, w_out, *P.fake_quant_expert_weights(w1, w2, w3), k, keep)
    r = (x @ w_mod.reshape(-1, 1)).squeeze(-1)
    sel = torch.topk(r, keep, dim=-1).indices.sort(dim=-1).values
    rows = torch.gather(x, 1, sel.unsqueeze(-1).expand(-1, -1, d)).reshape(-1, d)
    idx = P.router_tc(rows, w_in, w_out, k)[1]
    _, got = P.ffn_half_loss_routed(x, w_in, w_out, w1, w2, w3, idx, torch.zeros_like(x), w_mod=w_mod,
                                    sel_idx=sel, training=False, return_out=True, fp8=True)
    assert torch.allclose(got, want, rtol=0, atol=1e-12 * float(want.abs().max()))
    # and it differs from the unquantised layer by the quantisation (a few per cent)
    _, plain = P.ffn_half_loss_routed(x, w_in, w_out, w1, w2, w3, idx, torch.zeros_like(x), w_mod=w_mod,
                                      sel_idx=sel, training=False, return_out=True)
    assert 1e-3 < float((plain - got).norm() / got.norm()) < 0.2


def test_fp8_ste_gradients_use_dequantised_operands():
    """Straight-through gradients of _expert_bmm_fp8_ste: the quantisers pass the gradient
    unchanged (ste's own gradient is the identity), and with h unquantised the gradients
    of x, w1, w2, w3 equal those of the plain SwiGLU product evaluated at the
    fake-quantised operands as leaves (a backward multiplying by the master weights or
    rows instead would differ by the quantisation, a few per cent).  With h quantised,
    dw3 is the closed form hq^T dout of each expert with hq = e4m3(bf16(h))."""
    g = torch.Generator().manual_seed(23)
    E, m, d, F_ = 3, 7, 32, 48
    x = torch.randn(E, m, d, generator=g, dtype=torch.float64)
    ws = [torch.randn(E, d, F_, generator=g, dtype=torch.float64) * 0.1 for _ in range(2)]
    ws.append(torch.randn(E, F_, d, generator=g, dtype=torch.float64) * 0.1)
    dout = torch.randn(E, m, d, generator=g, dtype=torch.float64)
    # ste: value fq(t), gradient of t
    t = torch.randn(5, 9, generator=g, dtype=torch.float64, requires_grad=True)
    c = torch.randn(5, 9, generator=g, dtype=torch.float64)
    q = P.ste(P._fake_e4m3_rows, t)
    assert torch.equal(q.detach(), P._fake_e4m3_rows(t.detach()))
    (q * c).sum().backward()
    assert torch.equal(t.grad, c)

    def grads(fn, leaves):
        leaves = [v.clone().requires_grad_(True) for v in leaves]
        (fn(*leaves) * dout).sum().backward()
        return [v.grad for v in leaves]

    fqw = lambda w: P._fake_e4m3_rows(w.transpose(1, 2)).transpose(1, 2)
    ste_g = grads(lambda a, b, c_, e: P._expert_bmm_fp8_ste(a, b, c_, e, quant_h=False), [x] + ws)
    at_q = grads(P._expert_bmm, [P._fake_e4m3_rows(x)] + [fqw(w) for w in ws])
    master = grads(P._expert_bmm, [x] + ws)
    for a, b, c_ in zip(ste_g, at_q, master):
        assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)
        assert float((c_ - b).norm() / b.norm()) > 1e-3
    # quantised h: dw3 = hq^T dout per expert
    xq = P._fake_e4m3_rows(x)
    h = F.silu(torch.bmm(xq, fqw(ws[0]))) * torch.bmm(xq, fqw(ws[1]))
    hq = P._fake_e4m3_rows(h.to(torch.bfloat16).to(torch.float64))
    dw3 = grads(P._expert_bmm_fp8_ste, [x] + ws)[3]
    for e in range(E):
        assert torch.allclose(dw3[e], hq[e].T @ dout[e], rtol=1e-12, atol=1e-12)


def test_dropout_keep_convention_matches_torch():
    """ffn_half_loss_routed's residual dropout (ffn_out * keep * (1 / (1 - p)), layers.py:190)
    against nn.functional.dropout itself: the mask read off torch's output reproduces it
    exactly; the block's output is residual + that."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 33, 16, generator=g, dtype=torch.float64) + 3.0  # no exact zeros
    for p in (0.1, 0.5):
        torch.manual_seed(123)
        out = F.dropout(x, p=p, training=True)
        keep = out != 0
        assert 0 < keep.double().mean().item() < 1
        assert torch.equal(x * keep.to(x.dtype) * (1.0 / (1.0 - p)), out)
        # (dividing by 1 - p instead differs in the last bit: the reciprocal is the convention)
