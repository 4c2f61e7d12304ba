"""Packed-weight cache on disk (kmoe/checkpoint.py save_packed / load_packed): the packed
buffers read back are bit-identical to a fresh pack, a layer using them gives a
bit-identical forward, and a file made from other parameters is not installed.  The fp8
pack itself (codes and per-row scales) is checked bit for bit against the oracle."""
import numpy as np
import pytest
import torch

from kmoe import AdvancedMoEConfig, MoELayer, checkpoint as C

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fp8", [False, True])
def test_packed_roundtrip(dev, tmp_path, fp8):
    print(f"packed roundtrip fp8={fp8}", flush=True)
    cfg = AdvancedMoEConfig(d_model=256, n_experts=8, d_ff_expert=352, moe_fp8=fp8)
    torch.manual_seed(5)
    a = MoELayer(cfg, 0).to(dev, torch.bfloat16).eval()
    x = torch.randn(2, 200, 256, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        ya = a(x)
    path = str(tmp_path / "packed.safetensors")
    C.save_packed(a.grouped_experts, path)
    meta = C.describe_packed(path)
    assert (meta["E"], meta["d"], meta["F"], meta["fp8"]) == ("8", "256", "352", str(int(fp8)))
    b = MoELayer(cfg, 0).to(dev, torch.bfloat16).eval()
    b.load_state_dict(a.state_dict())
    assert C.load_packed(b.grouped_experts, path)
    pa, pb = a.grouped_experts.packed(), b.grouped_experts.packed()
    assert pb.w13.data_ptr() != pa.w13.data_ptr()  # read back, not shared
    for u, v in ((pa.w13, pb.w13), (pa.w3, pb.w3), (pa.s13, pb.s13), (pa.s3, pb.s3)):
        if u is not None:
            assert torch.equal(u, v)
    key_before = b.grouped_experts._packed[0]
    with torch.no_grad():
        yb = b(x)
    torch.cuda.synchronize()
    assert b.grouped_experts._packed[0] == key_before  # no re-pack
    assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
    # different parameters: the file is not installed
    c = MoELayer(cfg, 0).to(dev, torch.bfloat16)
    with torch.no_grad():
        c.load_state_dict(a.state_dict())
        c.grouped_experts.w3[0, 0, 0] += 1.0
    assert not C.load_packed(c.grouped_experts, path)


def _unpack_fp8(pw):
    """Host view of the fp8 packed layout: w13 rows (E, 2*F_pad, d + 128 pad bytes),
    gate row of f at (f//128)*256 + f%128 and up row at +128; w3 rows (E, d_pad,
    F_pad + 128) with row n = column n of w3[e]; s13 (E, 2*F_pad), s3 (E, d_pad)."""
    E, d, F = pw.E, pw.d, pw.F
    Fp = (F + 127) // 128 * 128
    dp = (d + 255) // 256 * 256
    w13 = pw.w13.cpu().numpy().reshape(E, 2 * Fp, d + 128)
    w3 = pw.w3.cpu().numpy().reshape(E, dp, Fp + 128)
    s13 = pw.s13.cpu().numpy().reshape(E, 2 * Fp)
    s3 = pw.s3.cpu().numpy().reshape(E, dp)
    f = np.arange(F)
    gate_rows = (f // 128) * 256 + f % 128
    return (w13[:, gate_rows, :d], s13[:, gate_rows], w13[:, gate_rows + 128, :d], s13[:, gate_rows + 128],
            w3[:, :d, :F], s3[:, :d], w13, w3)


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_packed_fp8_codes_match_oracle(dev, wdtype):
    """kmoe_pack_weights' fp8 codes and per-row scales equal the oracle's per-output-column
    quantisation (quant_rows of w[e]^T: scale amax/448, RNE e4m3) bit for bit, and the
    padding is zero."""
    from oracle import moe_oracle as O
    from kmoe import ops

    E, d, F = 3, 192, 200  # F_pad 256: a partial f block; d_pad 256: 64 zero rows in w3
    g = torch.Generator().manual_seed(11)
    w1, w2, w3 = (torch.randn(*s, generator=g) * 0.02 for s in [(E, d, F), (E, d, F), (E, F, d)])
    w1[1, :, 7] *= 300.0  # one column far larger than the rest
    w2[2, :, 9] = 0.0     # an all-zero column: scale 0, codes 0
    w1, w2, w3 = (w.to(wdtype) for w in (w1, w2, w3))
    print(f"packed fp8 codes wdtype={wdtype}", flush=True)
    pw = ops.pack_weights(w1.to(dev), w2.to(dev), w3.to(dev), fp8=True)
    torch.cuda.synchronize()
    c1, s1, c2, s2, c3, s3, w13, w3p = _unpack_fp8(pw)
    for e in range(E):
        for codes, scales, w in ((c1, s1, w1), (c2, s2, w2), (c3, s3, w3)):
            q, s = O.quant_rows(np.ascontiguousarray(w[e].float().numpy().T))
            assert np.array_equal(codes[e], q), e
            assert np.array_equal(scales[e].view(np.uint32), s.view(np.uint32)), e
    assert np.all(s2[2, 9] == 0) and np.all(c2[2, 9] == 0)
    # padding: the 128 bytes after each row, the f rows past F and the d rows past d
    assert not w13[:, :, d:].any() and not w3p[:, :, F:].any() and not w3p[:, d:, :].any()
    Fp = (F + 127) // 128 * 128
    pad_f = [(f // 128) * 256 + h * 128 + f % 128 for f in range(F, Fp) for h in (0, 1)]
    assert not w13[:, pad_f, :].any()
    assert not pw.s13.cpu().numpy().reshape(E, 2 * Fp)[:, pad_f].any()
    assert not pw.s3.cpu().numpy().reshape(E, -1)[:, d:].any()


def _bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy()


@pytest.mark.parametrize("E,d,F,wdtype", [(3, 192, 200, torch.bfloat16), (2, 128, 13, torch.float32),
                                          (2, 256, 384, torch.float32), (1, 64, 136, torch.bfloat16)])
def test_bf16_packs_match_host_layout(dev, E, d, F, wdtype):
    """kmoe_pack_weights (bf16) and kmoe_pack_weights_bwd against the packed layouts built on
    the host from w1/w2/w3: every element, the zero pads after each row and the zero
    padding rows (F and d not multiples of the tile sizes; f32 inputs rounded to bf16)."""
    from kmoe import backward as BW, ops

    g = torch.Generator().manual_seed(21)
    w1, w2, w3 = (torch.randn(*s, generator=g).to(wdtype) for s in [(E, d, F), (E, d, F), (E, F, d)])
    print(f"bf16 packs E={E} d={d} F={F} {wdtype}", flush=True)
    pw = ops.pack_weights(w1.to(dev), w2.to(dev), w3.to(dev))
    bw = BW.pack_bwd_weights(w1.to(dev), w2.to(dev), w3.to(dev), torch.zeros(128, d, dtype=wdtype, device=dev))
    torch.cuda.synchronize()
    Fp = (F + 127) // 128 * 128
    dp = (d + 255) // 256 * 256
    b1, b2, b3 = _bf16_bits(w1), _bf16_bits(w2), _bf16_bits(w3)
    w13 = np.zeros((E, 2 * Fp, d + 64), np.int16)
    w3p = np.zeros((E, dp, Fp + 64), np.int16)
    f = np.arange(F)
    rows = (f // 128) * 256 + f % 128
    for e in range(E):
        w13[e, rows, :d] = b1[e].T
        w13[e, rows + 128, :d] = b2[e].T
        w3p[e, :d, :F] = b3[e].T
    assert np.array_equal(pw.w13.cpu().view(torch.int16).numpy().reshape(w13.shape), w13)
    assert np.array_equal(pw.w3.cpu().view(torch.int16).numpy().reshape(w3p.shape), w3p)
    F256 = (F + 255) // 256 * 256
    w3n = np.zeros((E, F256, d + 64), np.int16)
    w13t = np.zeros((E, dp, 2 * Fp + 64), np.int16)
    c = np.arange(2 * Fp)
    src_f = (c >> 8) * 128 + (c & 127)
    half = (c >> 7) & 1
    ok = src_f < F
    for e in range(E):
        w3n[e, :F, :d] = b3[e]
        for i in range(d):
            w13t[e, i, c[ok & (half == 0)]] = b1[e, i, src_f[ok & (half == 0)]]
            w13t[e, i, c[ok & (half == 1)]] = b2[e, i, src_f[ok & (half == 1)]]
    assert np.array_equal(bw.w3n.cpu().view(torch.int16).numpy().reshape(w3n.shape), w3n)
    assert np.array_equal(bw.w13t.cpu().view(torch.int16).numpy().reshape(w13t.shape), w13t)
