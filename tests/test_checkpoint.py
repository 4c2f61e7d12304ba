"""CPU tests of the checkpoint helpers (kmoe/checkpoint.py): the reference checkpoint
layout (trainer.py:340-362, layers.py:70-74), the safe loader, and the expert copy of
tools/reallocate_experts.py with the real state-dict keys."""
import pickle

import pytest
import torch

import kmoe
from kmoe import AdvancedMoEConfig, MoELayer, checkpoint as C


class _Opaque:  # stands for the config object a reference trainer checkpoint pickles
    pass


def _model_sd(cfg, n_layers=3):
    sd = {"embed.weight": torch.randn(10, cfg.d_model)}
    for i in range(n_layers):
        blk = kmoe.MoEFFNBlock(cfg, i)
        for k, v in blk.state_dict().items():
            sd[f"layers.{i}.{k}"] = v.clone()
        sd[f"layers.{i}.seq_norm.weight"] = torch.ones(cfg.d_model)
        sd[f"layers.{i}.seq_layer.q_proj.weight"] = torch.randn(4, cfg.d_model)
    return sd


def test_layer_state_dict_loads_strict():
    cfg = AdvancedMoEConfig(d_model=64, n_experts=4, d_ff_expert=96)
    sd = _model_sd(cfg)
    m = MoELayer(cfg, 1)
    m.load_state_dict(C.layer_state_dict(sd, 1), strict=True)
    assert torch.equal(m.grouped_experts.w2, sd["layers.1.ffn.grouped_experts.w2"])
    b = kmoe.MoEFFNBlock(cfg, 2)
    b.load_state_dict(C.layer_state_dict(sd, 2, part="block"), strict=True)
    assert torch.equal(b.ffn_norm.weight, sd["layers.2.ffn_norm.weight"])
    assert torch.equal(b.ffn.router.router[0].weight, sd["layers.2.ffn.router.router.0.weight"])
    assert torch.equal(b.ffn_mod_router.router.weight, sd["layers.2.ffn_mod_router.router.weight"])
    # a block without MoD takes the FFN half alone
    nomod = AdvancedMoEConfig(d_model=64, n_experts=4, d_ff_expert=96, mod_enabled=False)
    sd2 = {k: v for k, v in sd.items() if ".ffn_mod_router." not in k}
    kmoe.MoEFFNBlock(nomod, 2).load_state_dict(C.layer_state_dict(sd2, 2, part="block"), strict=True)
    with pytest.raises(KeyError):
        C.layer_state_dict(sd, 7)


def test_safe_loader(tmp_path):
    cfg = AdvancedMoEConfig(d_model=64, n_experts=4, d_ff_expert=96)
    sd = _model_sd(cfg, 1)
    p = tmp_path / "ckpt.pt"
    torch.save({"model_state_dict": sd, "step": 12, "epoch": 0}, p)
    got = C.load_model_state_dict(str(p))
    assert set(got) == set(sd) and all(torch.equal(got[k], sd[k]) for k in sd)
    bare = tmp_path / "bare.pt"
    torch.save(sd, bare)
    assert set(C.load_model_state_dict(str(bare))) == set(sd)
    # a checkpoint whose pickle holds an arbitrary object is refused, not executed
    bad = tmp_path / "bad.pt"
    torch.save({"model_state_dict": sd, "config": _Opaque()}, bad, pickle_module=pickle)
    with pytest.raises(ValueError, match="weights_only"):
        C.load_model_state_dict(str(bad))


def test_copy_experts_uses_real_keys():
    cfg = AdvancedMoEConfig(d_model=64, n_experts=4, d_ff_expert=96)
    sd = _model_sd(cfg)
    before = {k: v.clone() for k, v in sd.items()}
    out = C.copy_experts(sd, [(0, 3, 2, 1), (1, 0, 2, 2)])
    for w in ("w1", "w2", "w3"):
        dst = out[f"layers.2.ffn.grouped_experts.{w}"]
        assert torch.equal(dst[1], sd[f"layers.0.ffn.grouped_experts.{w}"][3])
        assert torch.equal(dst[2], sd[f"layers.1.ffn.grouped_experts.{w}"][0])
        assert torch.equal(dst[0], before[f"layers.2.ffn.grouped_experts.{w}"][0])
        assert torch.equal(dst[3], before[f"layers.2.ffn.grouped_experts.{w}"][3])
    # the input dict is not modified; untouched entries are shared
    assert all(torch.equal(sd[k], before[k]) for k in sd)
    assert out["layers.0.ffn.router.router.0.weight"] is sd["layers.0.ffn.router.router.0.weight"]
    with pytest.raises(KeyError):
        C.copy_experts(sd, [(0, 0, 5, 0)])


def _packed_file(tmp_path, ge, name, meta_over=None, drop=(), shape_over=None):
    """A packed-weight file for `ge` as save_packed writes it (zero buffers of the sizes the
    library packs), with metadata entries replaced / removed and tensor sizes changed."""
    from safetensors.torch import save_file

    E, d, F, fp8 = ge.n_experts, ge.d_model, ge.d_ff, ge.use_fp8
    meta = {"kmoe_packed": "1", "E": str(E), "d": str(d), "F": str(F), "fp8": str(int(fp8)),
            "fingerprint": C._fingerprint(ge), **C._layout_meta(E, d, F, fp8)}
    meta.update(meta_over or {})
    for k in drop:
        meta.pop(k)
    sizes = {"w13": int(meta.get("w13_bytes", 0) or C._layout_meta(E, d, F, fp8)["w13_bytes"]),
             "w3": int(C._layout_meta(E, d, F, fp8)["w3_bytes"])}
    Fp, dp = (F + 127) // 128 * 128, (d + 255) // 256 * 256
    if fp8:
        sizes.update({"s13": E * 2 * Fp, "s3": E * dp})
    sizes.update(shape_over or {})
    t = {k: torch.zeros(n, dtype=torch.uint8 if k in ("w13", "w3") else torch.float32) for k, n in sizes.items()}
    path = str(tmp_path / name)
    save_file(t, path, metadata=meta)
    return path


@pytest.mark.parametrize("fp8", [False, True])
def test_packed_file_layout_checks(tmp_path, fp8):
    """A packed-weight file is accepted only with this library's packed-layout and ABI
    versions and the buffer sizes it packs; anything else is refused (re-pack)."""
    cfg = AdvancedMoEConfig(d_model=128, n_experts=4, d_ff_expert=200, moe_fp8=fp8)
    ge = MoELayer(cfg, 0).grouped_experts
    assert C.packed_file_matches(ge, _packed_file(tmp_path, ge, "ok.st"))
    lay = C._layout_meta(4, 128, 200, fp8)
    bad = [
        dict(meta_over={"layout": str(int(lay["layout"]) + 1)}),
        dict(meta_over={"layout": "1"}),  # the layout before the packed-row padding
        dict(meta_over={"abi": "0"}),
        dict(drop=("layout",)),
        dict(meta_over={"w13_bytes": str(int(lay["w13_bytes"]) - 128)}),
        dict(shape_over={"w3": int(lay["w3_bytes"]) - 4096}),
        dict(meta_over={"F": "192"}),
        dict(meta_over={"fingerprint": "0" * 16}),
    ]
    if fp8:
        bad.append(dict(shape_over={"s13": 4 * 2 * 256 - 1}))
    for i, kw in enumerate(bad):
        assert not C.packed_file_matches(ge, _packed_file(tmp_path, ge, f"bad{i}.st", **kw)), kw
        assert not C.load_packed(ge, str(tmp_path / f"bad{i}.st"))
