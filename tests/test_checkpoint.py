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
        sd[f"layers.{i}.ffn_mod_router.router.0.weight"] = torch.randn(4, cfg.d_model)
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
