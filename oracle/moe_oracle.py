"""numpy restatement of the reference MoE forward (TEST INFRASTRUCTURE ONLY).

Each function cites the reference code it follows (paths into
JBedichek/Kolmogorov-MoE-Architecture).  Where the reference leaves a choice
open (tie order of torch.topk, the capacity-drop rule, fp8 scaling), the rule
this build specifies is stated in the docstring; the HIP kernels implement the
same rule.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


# ----------------------------------------------------------------------------- router
def silu(x):
    """SiLU(x) = x * sigmoid(x) (nn.SiLU in moe.py:349)."""
    return x / (1.0 + np.exp(-x))


def router_logits(x, w_in, w_out, bias=None, dtype=np.float64):
    """Router MLP: SiLU(x . w_in^T) . w_out^T (+ bias)  (moe.py:345-351, 438).

    x: (T, d); w_in: (128, d) (nn.Linear [out, in]); w_out: (E, 128).
    The optional per-expert bias is added to the logits before the softmax
    (the DeepSeek-style bias of Experiments/sparse_distillation/distill.py:337-338)."""
    h = silu(x.astype(dtype) @ w_in.astype(dtype).T)
    lg = h @ w_out.astype(dtype).T
    if bias is not None:
        lg = lg + np.asarray(bias, dtype=dtype)
    return lg


def softmax(lg, axis=-1):
    """F.softmax (moe.py:441)."""
    m = np.max(lg, axis=axis, keepdims=True)
    e = np.exp(lg - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def topk_select(logits, k):
    """Top-k experts per token and renormalised weights (moe.py:455-460).

    Rule: rank by logit descending; equal logits -> lowest expert index first
    (torch.topk leaves the tie order unspecified).  Softmax is monotone in the
    logit, so this is the same set as top-k of the probabilities.  Weights are
    p_j / sum_sel p = exp(l_j - m) / sum_sel exp(l - m)."""
    lg = np.asarray(logits, dtype=np.float64)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :k]
    sel = np.take_along_axis(lg, order, axis=1)
    m = lg.max(axis=1, keepdims=True)
    ex = np.exp(sel - m)
    return order.astype(np.int64), ex / ex.sum(axis=1, keepdims=True)


def balanced_topk(logits, k):
    """Capacity-balanced greedy assignment (Router._balanced_topk_assignment,
    moe.py:353-421), in k rounds over all tokens at once.

    cap = max(T*k // E, 1).  Round r: experts whose count after rounds < r has
    reached cap are masked for every token, as are the token's own earlier picks;
    each token takes its best remaining expert (fp32 logit descending, equal logits
    -> lowest expert index, the rule of topk_select; softmax is monotone, so this
    is the argmax of the probabilities); a token with every remaining expert
    masked takes its best expert not picked yet, ignoring capacity (moe.py:402-407).
    Counts then add the round's picks (moe.py:414).  Weights: the picks'
    probabilities / (their sum + 1e-9) (moe.py:411,420)."""
    lg = np.asarray(logits, dtype=np.float64)
    T, E = lg.shape
    cap = max((T * k) // E, 1)
    p = softmax(lg)
    counts = np.zeros(E, dtype=np.int64)
    taken = np.zeros((T, E), dtype=bool)
    idx = np.zeros((T, k), dtype=np.int64)
    wraw = np.zeros((T, k), dtype=np.float64)
    for r in range(k):
        masked = np.where(taken | (counts >= cap)[None, :], -np.inf, lg)
        best = np.argmax(masked, axis=1)  # first maximum: lowest index
        none = np.isneginf(masked.max(axis=1))
        if none.any():
            best[none] = np.argmax(np.where(taken[none], -np.inf, lg[none]), axis=1)
        idx[:, r] = best
        wraw[:, r] = p[np.arange(T), best]
        counts += np.bincount(best, minlength=E)
        taken[np.arange(T), best] = True
    return idx, wraw / (wraw.sum(axis=1, keepdims=True) + 1e-9)


def aux_losses(logits, counts, T, k, E, w_lb=0.01, w_z=0.001):
    """Load-balance and z losses (moe.py:840-939).

    LB = E * sum_e f_e * P_e, f_e = counts_e / (T*k), P_e = mean_t softmax_e;
    z = mean_t logsumexp_t^2; aux = w_lb*LB + w_z*z.  counts=None -> LB = 0
    (expert-choice uses w_z*z only, moe.py:833-836)."""
    lg = np.asarray(logits, dtype=np.float64)
    P = softmax(lg).mean(axis=0)
    m = lg.max(axis=1)
    lse = m + np.log(np.exp(lg - m[:, None]).sum(axis=1))
    z = float(np.mean(lse ** 2))
    lb = 0.0
    if counts is not None:
        f = np.asarray(counts, dtype=np.float64) / (T * k)
        lb = float(E * np.sum(f * P))
    return w_lb * lb + w_z * z, lb, z


# ----------------------------------------------------------------------------- dispatch
def dispatch(idx, E, capacity=0):
    """Stable counting sort of assignments a = t*k + j by expert
    (= argsort(flat, stable=True), bincount, cumsum; moe.py:238-253).

    Capacity rule (config 3, this build's): keep the first `capacity`
    assignments of each expert in assignment (= token) order; dropped
    assignments get slot_row = -1.  capacity <= 0 keeps all."""
    idx = np.asarray(idx, dtype=np.int64)
    T, k = idx.shape
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=E)[:E].astype(np.int64)
    kept = np.minimum(counts, capacity) if capacity > 0 else counts.copy()
    offsets = np.zeros(E + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(kept)
    slot_row = np.full(T * k, -1, dtype=np.int64)
    row_token = np.full(T * k, -1, dtype=np.int64)
    for e in range(E):
        a = np.nonzero(flat == e)[0][: kept[e]]  # ascending assignment order
        rows = offsets[e] + np.arange(a.size)
        slot_row[a] = rows
        row_token[rows] = a // k
    return dict(counts=counts, offsets=offsets, slot_row=slot_row, row_token=row_token)


# ----------------------------------------------------------------------------- experts
def swiglu_rows(xrows, offsets, w1, w2, w3, dtype=np.float32):
    """Per-expert SwiGLU on expert-contiguous rows:
    y = (silu(x W1[e]) * (x W2[e])) W3[e]  (moe.py:275-279, ffn.py:17-64,
    kernels/__init__.py:59-102).  w3 None: the non-gated experts of an activation other
    than swiglu, y = silu(x W1[e]) W2[e] with W2 (E, F, d) (moe.py:180-191, 281-283)."""
    if w3 is None:
        return plain_rows(xrows, offsets, w1, w2, dtype=dtype)
    E = w1.shape[0]
    y = np.zeros((xrows.shape[0], w3.shape[2]), dtype=dtype)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        xe = xrows[lo:hi].astype(dtype)
        h = silu(xe @ w1[e].astype(dtype)) * (xe @ w2[e].astype(dtype))
        y[lo:hi] = h @ w3[e].astype(dtype)
    return y


def plain_rows(xrows, offsets, w1, w2, dtype=np.float32):
    """Non-gated experts on expert-contiguous rows: y = silu(x W1[e]) W2[e] (moe.py:281-283)."""
    E = w1.shape[0]
    y = np.zeros((xrows.shape[0], w2.shape[2]), dtype=dtype)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        y[lo:hi] = silu(xrows[lo:hi].astype(dtype) @ w1[e].astype(dtype)) @ w2[e].astype(dtype)
    return y


def combine(yrows, src_row, src_w, out_map=None, scale=None, T_out=None):
    """y[o] = scale[s] * sum_j w[s,j] * yrows[src[s,j]], s = out_map[o]
    (moe.py:285-292 index_add_; moe.py:132-158 scatter_add_; layers.py:175-185)."""
    src_row = np.asarray(src_row)
    src_w = np.asarray(src_w, dtype=np.float64)
    n_src = src_row.shape[0]
    T_out = n_src if T_out is None else T_out
    acc = np.zeros((n_src, yrows.shape[1]), dtype=np.float64)
    for j in range(src_row.shape[1]):
        valid = src_row[:, j] >= 0
        acc[valid] += src_w[valid, j, None] * yrows[src_row[valid, j]].astype(np.float64)
    if scale is not None:
        acc *= np.asarray(scale, dtype=np.float64)[:, None]
    if out_map is None:
        return acc
    out = np.zeros((T_out, yrows.shape[1]), dtype=np.float64)
    om = np.asarray(out_map)
    v = om >= 0
    out[v] = acc[om[v]]
    return out


# ----------------------------------------------------------------------------- expert choice
def ec_select(logits, B, S, E, C):
    """Expert-choice selection (moe.py:494-530): per sequence b and expert e the
    C tokens of largest softmax-over-tokens probability, in descending order.

    Rule: rank by logit (monotone in that probability), equal logits -> lowest
    token index first; w = p / (sum_sel p + 1e-9)."""
    lg = np.asarray(logits, dtype=np.float64).reshape(B, S, E)
    idx = np.zeros((B, E, C), dtype=np.int64)
    w = np.zeros((B, E, C), dtype=np.float64)
    for b in range(B):
        p = softmax(lg[b], axis=0)  # (S, E), softmax over tokens
        for e in range(E):
            order = np.argsort(-lg[b, :, e], kind="stable")[:C]
            idx[b, e] = order
            ps = p[order, e]
            w[b, e] = ps / (ps.sum() + 1e-9)
    return idx, w


def ec_tables(idx, w, S):
    """Expert-major permuted rows (row = e*B*C + b*C + c) and per-token (B*S, E)
    source tables for the combine (moe.py:649-671)."""
    B, E, C = idx.shape
    row_token = np.zeros(E * B * C, dtype=np.int64)
    src_row = np.full((B * S, E), -1, dtype=np.int64)
    src_w = np.zeros((B * S, E), dtype=np.float64)
    for b in range(B):
        for e in range(E):
            rows = e * B * C + b * C + np.arange(C)
            toks = b * S + idx[b, e]
            row_token[rows] = toks
            src_row[toks, e] = rows
            src_w[toks, e] = w[b, e]
    offsets = np.arange(E + 1, dtype=np.int64) * (B * C)
    return row_token, offsets, src_row, src_w


# ----------------------------------------------------------------------------- MoD
def mod_logits(x3d, w_mod, dtype=np.float64):
    """r = x . w  (mod.py:93; nn.Linear(d, 1, bias=False))."""
    return x3d.astype(dtype) @ np.asarray(w_mod, dtype=dtype).reshape(-1)


def mod_select(r, keep):
    """Top-`keep` tokens per sequence, sorted ascending, softmax over the kept
    logits (mod.py:97-112).  Rule: equal logits -> lowest token index first."""
    r = np.asarray(r, dtype=np.float64)
    B, S = r.shape
    sel = np.zeros((B, keep), dtype=np.int64)
    w = np.zeros((B, keep), dtype=np.float64)
    for b in range(B):
        order = np.argsort(-r[b], kind="stable")[:keep]
        s = np.sort(order)
        sel[b] = s
        w[b] = softmax(r[b, s])
    return sel, w


# ----------------------------------------------------------------------------- fp8 e4m3
def f32_to_e4m3(v):
    """fp32 -> OCP e4m3fn codes: saturate to +-448, round to nearest even
    (config 5's scheme; cast mechanics as fp8_moe.py:112-125: clamp, then
    .to(float8_e4m3fn)).  Returns uint8 codes."""
    v = np.asarray(v, dtype=np.float32)
    u = v.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    nan = np.isnan(v)
    a = np.minimum(np.abs(v), np.float32(E4M3_MAX)).astype(np.float32)
    ua = a.view(np.uint32)
    exp = (ua >> 23).astype(np.int64) - 127
    # subnormal: rint(a * 2^9) (RNE)
    sub = np.rint(a.astype(np.float64) * 512.0).astype(np.uint32)
    mant = ua & 0x7FFFFF
    m3 = mant >> 20
    rest = mant & 0xFFFFF
    e = np.clip(exp + 7, 0, 15).astype(np.uint32)
    code = (e << 3) | m3
    up = (rest > 0x80000) | ((rest == 0x80000) & ((m3 & 1) == 1))
    code = code + up.astype(np.uint32)
    code = np.minimum(code, 0x7E)
    code = np.where(exp < -6, sub, code)
    code = np.where(nan, 0x7F, code)
    return (sign | code).astype(np.uint8)


def e4m3_to_f32(c):
    """Decode e4m3fn codes (0x7f/0xff are NaN)."""
    c = np.asarray(c, dtype=np.uint32)
    s = (c >> 7) & 1
    e = (c >> 3) & 15
    m = c & 7
    v = np.where(e == 0, m.astype(np.float64) / 512.0, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    v = np.where((c & 0x7F) == 0x7F, np.nan, v)
    return np.where(s == 1, -v, v).astype(np.float32)


def quant_rows(m):
    """Per-row e4m3 quantisation: scale = amax/448, q = e4m3(x * (448/amax)), all
    fp32 arithmetic (amax = 0 -> scale 0, q = 0).  Returns (codes, scale)."""
    m = np.asarray(m, dtype=np.float32)
    amax = np.max(np.abs(m), axis=1).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(448.0) / amax, np.float32(0.0)).astype(np.float32)
    q = f32_to_e4m3((m * inv[:, None]).astype(np.float32))
    return q, (amax / np.float32(448.0)).astype(np.float32)


def dequant_rows(q, scale):
    return e4m3_to_f32(q) * np.asarray(scale, dtype=np.float32)[:, None]


def quant_weight_cols(w):
    """Per-expert per-output-column quantisation of w (E, K, N) (columns are the
    output rows of x @ w): returns dequantised weights (E, K, N) in fp32."""
    E, K, N = w.shape
    out = np.zeros((E, K, N), dtype=np.float32)
    for e in range(E):
        q, s = quant_rows(np.ascontiguousarray(w[e].T))
        out[e] = dequant_rows(q, s).T
    return out


def swiglu_rows_fp8(xq, xs, offsets, w1q, w2q, w3q):
    """fp8 expert path: x rows dequantised from per-token scales, weights from
    per-output-row scales (already dequantised), h re-quantised per row before
    the down GEMM; fp32 accumulation."""
    x = dequant_rows(xq, xs)
    E = w1q.shape[0]
    y = np.zeros((x.shape[0], w3q.shape[2]), dtype=np.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        xe = x[lo:hi]
        h = (silu(xe @ w1q[e]) * (xe @ w2q[e])).astype(np.float32)
        # the kernel stores h in bf16 before re-quantising it
        h = bf16_round(h)
        hq, hs = quant_rows(h)
        y[lo:hi] = dequant_rows(hq, hs) @ w3q[e]
    return y


def bf16_round(v):
    """Round fp32 to bf16 (RNE) and back to fp32; NaN stays a (quiet) NaN with its
    sign (the kernels' f32_to_bf16 rule)."""
    v = np.asarray(v, dtype=np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(np.isnan(v), ((u >> 16) | 0x40) << 16, r)
    return r.astype(np.uint32).view(np.float32)


# ----------------------------------------------------------------------------- full layer
def moe_forward_tc(x, w_in, w_out, w1, w2, w3, k, capacity=0, logits=None, bias=None, w_lb=0.01, w_z=0.001,
                   fp8=False, dtype=np.float32):
    """Token-choice MoELayer forward (moe.py:782-813) in fp32 arithmetic.

    If `logits` is given (the kernel's fp32 logits), routing is derived from
    them, so indices/counts/permutation can be compared bit-exactly."""
    x = np.asarray(x, dtype=dtype)
    T = x.shape[0]
    E = w_out.shape[0]
    if logits is None:
        logits = router_logits(x, w_in, w_out, bias)
    idx, w = topk_select(logits, k)
    dp = dispatch(idx, E, capacity)
    xrows = x[dp["row_token"][: dp["offsets"][E]]]
    if fp8:
        xq, xs = quant_rows(bf16_round(xrows))
        w1q, w2q, w3q = quant_weight_cols(w1), quant_weight_cols(w2), quant_weight_cols(w3)
        yrows = swiglu_rows_fp8(xq, xs, dp["offsets"], w1q, w2q, w3q)
    else:
        yrows = swiglu_rows(xrows, dp["offsets"], w1, w2, w3, dtype=dtype)
    y = combine(yrows, dp["slot_row"].reshape(T, k), w)
    aux = aux_losses(logits, dp["counts"], T, k, E, w_lb, w_z)
    return dict(y=y, logits=np.asarray(logits), idx=idx, w=w, aux=aux, **dp)


# ----------------------------------------------------------------------------- block boundary
def rms_norm(x, weight, eps=1e-5, dtype=np.float64):
    """RMSNorm.forward (embeddings.py:182-195): weight * x / sqrt(mean(x^2, -1) + eps)."""
    x = np.asarray(x, dtype=dtype)
    rms = np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return np.asarray(weight, dtype=dtype) * (x / rms)


def ffn_block_tc(h, norm_w, eps, w_in, w_out, w1, w2, w3, k, capacity=0, logits=None, bias=None,
                 dtype=np.float64):
    """The FFN half of TransformerBlock.forward (layers.py:142-147, 184-187) without MoD
    and without residual dropout: out = h + MoELayer(RMSNorm(h)).  `logits` as in
    moe_forward_tc (routing from the kernel's own fp32 logits)."""
    xn = rms_norm(h, norm_w, eps, dtype=dtype)
    r = moe_forward_tc(xn, w_in, w_out, w1, w2, w3, k, capacity=capacity, logits=logits, bias=bias, dtype=dtype)
    r["y"] = np.asarray(h, dtype=dtype) + r["y"]
    r["xn"] = xn
    return r
