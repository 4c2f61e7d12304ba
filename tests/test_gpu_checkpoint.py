"""Packed-weight cache on disk (kmoe/checkpoint.py save_packed / load_packed): the packed
buffers read back are bit-identical to a fresh pack, a layer using them gives a
bit-identical forward, and a file made from other parameters is not installed."""
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
