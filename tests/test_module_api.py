"""CPU tests of the drop-in Python API: constructor config, attributes,
parameter names/shapes (the reference's state-dict keys), and that the
product path refuses to run without a GPU (no silent CPU fallback)."""
import pytest
import torch

import kmoe
from kmoe import AdvancedMoEConfig, MoELayer, get_test_config


def test_config_defaults_match_reference():
    c = AdvancedMoEConfig()  # moe_arch/model/config.py:17-56
    assert (c.d_model, c.d_ff_expert, c.n_experts, c.moe_top_k) == (2048, 2816, 16, 2)
    assert c.moe_capacity_factor == 1.25
    assert (c.moe_load_balance_loss_weight, c.moe_router_z_loss_weight) == (0.01, 0.001)
    assert (c.moe_implementation, c.moe_routing, c.moe_balanced_routing) == ("batched", "token_choice", False)
    assert (c.mod_capacity_factor, c.ffn_activation) == (0.75, "swiglu")
    t = get_test_config()
    assert (t.d_model, t.d_ff_expert, t.n_experts) == (256, 352, 4)


def test_token_choice_state_dict_keys():
    cfg = AdvancedMoEConfig(d_model=256, n_experts=8, d_ff_expert=512)
    m = MoELayer(cfg, layer_idx=3)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert shapes == {
        "router.router.0.weight": (128, 256),
        "router.router.2.weight": (8, 128),
        "grouped_experts.w1": (8, 256, 512),
        "grouped_experts.w2": (8, 256, 512),
        "grouped_experts.w3": (8, 512, 256),
    }
    for attr in ("config", "layer_idx", "n_experts", "top_k", "capacity_factor", "routing_type", "implementation",
                 "router", "grouped_experts", "grouped_experts_ec", "experts", "load_balance_loss_weight",
                 "router_z_loss_weight", "aux_loss"):
        assert hasattr(m, attr), attr
    assert m.layer_idx == 3 and m.experts is None and m.grouped_experts_ec is None and m.aux_loss == 0.0
    # reference init bound 1/sqrt(fan_in) per expert (moe.py:194-211)
    assert m.grouped_experts.w1.abs().max() <= 1 / 256 ** 0.5 + 1e-7
    assert m.grouped_experts.w3.abs().max() <= 1 / 512 ** 0.5 + 1e-7


def test_expert_choice_state_dict_keys():
    cfg = AdvancedMoEConfig(d_model=128, n_experts=4, d_ff_expert=256, moe_routing="expert_choice")
    m = MoELayer(cfg, 0)
    assert sorted(m.state_dict()) == ["grouped_experts_ec.w1", "grouped_experts_ec.w2", "grouped_experts_ec.w3",
                                      "router.router.0.weight", "router.router.2.weight"]
    assert m.grouped_experts is None
    assert m.router.capacity(2048) == 640  # ceil(2048*1.25/4), moe.py:511


def test_mod_module_keys():
    cfg = AdvancedMoEConfig(d_model=128, n_experts=4, d_ff_expert=256)
    m = kmoe.MoDMoE(cfg)
    keys = set(m.state_dict())
    assert "ffn_mod_router.router.weight" in keys and "ffn_mod_router.aux_router.0.weight" in keys
    assert m.ffn_mod_router.keep_count(2048) == 1536 and m.ffn_mod_router.keep_count(1) == 1


def test_unsupported_modes_fail_loudly():
    with pytest.raises(NotImplementedError):
        MoELayer(AdvancedMoEConfig(d_model=128, moe_implementation="expert_parallel"), 0)
    with pytest.raises(NotImplementedError):
        MoELayer(AdvancedMoEConfig(d_model=128, ffn_activation="gelu", moe_fp8=True), 0)


@pytest.mark.parametrize("kw, what", [
    (dict(n_experts=164), "n_experts=164"),            # configs/1b_150m_active.yaml:26
    (dict(d_model=1512, d_ff=4096, d_ff_expert=512), "d_model=1512"),  # configs/1b_150m_active.yaml:15
    (dict(n_experts=8, moe_top_k=9), "moe_top_k=9"),
    (dict(n_experts=4, moe_top_k=5), "moe_top_k=5"),
    (dict(n_experts=65, moe_routing="expert_choice"), "n_experts=65"),
])
def test_out_of_range_configs_fail_at_construction(kw, what):
    """Shapes the HIP kernels do not take are refused by MoELayer.__init__ with the
    offending field named, not at the first forward inside the C ABI."""
    with pytest.raises(ValueError, match=what):
        MoELayer(AdvancedMoEConfig(**kw), 0)
    # the limits themselves are accepted
    MoELayer(AdvancedMoEConfig(d_model=128, d_ff_expert=256, n_experts=64, moe_top_k=8), 0)


@pytest.mark.parametrize("routing", ["token_choice", "expert_choice"])
def test_non_gated_expert_keys(routing):
    """An activation other than swiglu gives the reference's two-matrix experts
    (moe.py:180-191): w1 (E, d, F), w2 (E, F, d), no w3; silu(x w1) w2 whatever the name."""
    cfg = AdvancedMoEConfig(d_model=128, n_experts=4, d_ff_expert=96, ffn_activation="gelu", moe_routing=routing)
    m = MoELayer(cfg, 0)
    ge = m.grouped_experts if routing == "token_choice" else m.grouped_experts_ec
    pre = "grouped_experts." if routing == "token_choice" else "grouped_experts_ec."
    sd = m.state_dict()
    assert {k for k in sd if k.startswith(pre)} == {pre + "w1", pre + "w2"}
    assert ge.w1.shape == (4, 128, 96) and ge.w2.shape == (4, 96, 128) and ge.w3 is None and not ge.gated
    bound = 1.0 / 128 ** 0.5  # per-expert kaiming-uniform bound of w1 (fan_in d), moe.py:194-211
    assert float(ge.w1.detach().abs().max()) <= bound and float(ge.w2.detach().abs().max()) <= 1.0 / 96 ** 0.5


def test_cpu_input_is_rejected():
    m = MoELayer(AdvancedMoEConfig(d_model=128, n_experts=4, d_ff_expert=256), 0)
    with pytest.raises(ValueError, match="GPU"):
        m(torch.randn(1, 8, 128))


def test_ffn_block_keys_and_norm():
    """MoEFFNBlock: a TransformerBlock's FFN-half keys (layers.py:70-74), the config's norm
    (embeddings.py:196-212), and the RMSNorm module's formula (embeddings.py:190-195)."""
    cfg = AdvancedMoEConfig(d_model=256, n_experts=8, d_ff_expert=512)
    assert (cfg.norm_type, cfg.norm_eps, cfg.residual_dropout) == ("rmsnorm", 1e-5, 0.1)
    blk = kmoe.MoEFFNBlock(cfg, 0)
    keys = set(blk.state_dict())
    ffn_keys = {"ffn_norm.weight", "ffn.router.router.0.weight", "ffn.router.router.2.weight",
                "ffn.grouped_experts.w1", "ffn.grouped_experts.w2", "ffn.grouped_experts.w3"}
    # mod_enabled (the reference's default) adds the FFN's MoD router (layers.py:84-88)
    assert ffn_keys | {"ffn_mod_router.router.weight", "ffn_mod_router.aux_router.0.weight",
                       "ffn_mod_router.aux_router.2.weight"} == keys
    nomod = kmoe.MoEFFNBlock(AdvancedMoEConfig(d_model=256, n_experts=8, d_ff_expert=512, mod_enabled=False), 0)
    assert set(nomod.state_dict()) == ffn_keys and nomod.ffn_mod_router is None
    x = torch.randn(3, 5, 256, dtype=torch.float64)
    blk.ffn_norm.weight.data = torch.rand(256) + 0.5
    ref = torch.nn.functional.rms_norm(x, (256,), blk.ffn_norm.weight.double(), eps=1e-5)
    torch.testing.assert_close(blk.ffn_norm(x), ref, rtol=1e-6, atol=1e-7)
    ln = kmoe.MoEFFNBlock(AdvancedMoEConfig(d_model=256, n_experts=8, d_ff_expert=512, norm_type="layernorm"), 0)
    assert isinstance(ln.ffn_norm, torch.nn.LayerNorm)
    # wrapping an existing layer shares its parameters
    m = MoELayer(cfg, 0)
    assert kmoe.MoEFFNBlock(cfg, 0, ffn=m).ffn is m
    with pytest.raises(ValueError):
        blk.eval()(x.float())  # the fused path refuses CPU tensors
