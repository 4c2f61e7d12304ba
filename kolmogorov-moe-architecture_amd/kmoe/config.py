"""Constructor config of the MoE layer.

Mirrors the MoE/MoD/FFN fields of ``AdvancedMoEConfig``
(moe_arch/model/config.py:12-56, defaults identical).  ``MoELayer`` reads its
settings with ``getattr`` so the reference's own config object works as well;
the build-only fields below default to the reference's behaviour.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence


@dataclass
class AdvancedMoEConfig:
    # model size (config.py:17-20)
    vocab_size: int = 50000
    d_model: int = 2048
    n_layers: int = 32
    max_seq_len: int = 2048
    # FFN (config.py:28-30)
    d_ff: int = 5632
    d_ff_expert: int = 2816
    ffn_activation: str = "swiglu"
    # MoE (config.py:33-50)
    n_experts: int = 16
    moe_top_k: int = 2
    moe_capacity_factor: float = 1.25
    moe_load_balance_loss_weight: float = 0.01
    moe_router_z_loss_weight: float = 0.001
    moe_implementation: str = "batched"
    moe_routing: str = "token_choice"
    moe_balanced_routing: bool = False
    # MoD (config.py:58-62)
    mod_enabled: bool = True
    mod_capacity_factor: float = 0.75
    mod_load_balance_loss_weight: float = 0.001
    mod_router_hidden_dim: int = 128
    # regularisation / normalisation / dtype (config.py:83-108)
    dropout: float = 0.1
    residual_dropout: float = 0.1
    norm_type: str = "rmsnorm"
    norm_eps: float = 1e-5
    dtype: str = "bfloat16"
    device: str = "cuda"
    # ---- build-only fields (ignored by the reference) ----
    # Token-choice capacity drop: keep the first ceil(moe_capacity_factor*T*k/E)
    # assignments of every expert in token order, drop the rest.
    moe_drop_overflow: bool = False
    # Expert GEMMs on fp8 e4m3 with per-token activation scales and
    # per-expert per-output-row weight scales.
    moe_fp8: bool = False
    # Optional per-expert logit bias added before the softmax (E floats).
    moe_router_bias: Optional[Sequence[float]] = None


def get_5b_config() -> AdvancedMoEConfig:
    """The reference's default 5B configuration (config.py:277-279)."""
    return AdvancedMoEConfig()


def get_test_config() -> AdvancedMoEConfig:
    """MoE fields of the reference's small test config (config.py:336-353)."""
    return AdvancedMoEConfig(vocab_size=1000, d_model=256, n_layers=4, max_seq_len=128, d_ff=704,
                             d_ff_expert=352, n_experts=4)
