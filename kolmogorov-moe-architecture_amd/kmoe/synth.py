"""Seeded synthetic inputs for the five benchmark configurations.

All tensors are drawn on the CPU with torch's seeded generator (identical on
every machine for a given torch version), as N(0,1) activations and
N(0, 0.02^2) weights, then cast and moved.  The expert weights overwrite the
reference's uniform init (moe.py:194-211) and the router weights overwrite
nn.Linear's default init.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from .config import AdvancedMoEConfig

ZIPF_S = 1.2
ZIPF_TAU = 0.1  # bias scale: 3 experts receive > 30% of tokens at config 3


@dataclass
class Workload:
    name: str
    B: int
    S: int
    d: int
    E: int
    k: int
    F: int
    dtype: torch.dtype
    seed: int
    routing: str = "token_choice"
    capacity_factor: float = 1.25
    drop_overflow: bool = False
    zipf_bias: bool = False
    fp8: bool = False
    mod: bool = False
    mod_cf: float = 0.75
    extra: dict = field(default_factory=dict)

    @property
    def T(self) -> int:
        return self.B * self.S

    def config(self) -> AdvancedMoEConfig:
        bias = zipf_bias(self.E, self.seed).tolist() if self.zipf_bias else None
        return AdvancedMoEConfig(d_model=self.d, n_experts=self.E, moe_top_k=self.k, d_ff_expert=self.F,
                                 moe_capacity_factor=self.capacity_factor, moe_routing=self.routing,
                                 moe_drop_overflow=self.drop_overflow, moe_fp8=self.fp8, moe_router_bias=bias,
                                 mod_capacity_factor=self.mod_cf)


WORKLOADS = {
    1: Workload("cfg1_cpu_small_fp32", B=2, S=256, d=256, E=8, k=2, F=512, dtype=torch.float32, seed=1),
    2: Workload("cfg2_d2048_e16_top2_bf16", B=8, S=2048, d=2048, E=16, k=2, F=2816, dtype=torch.bfloat16, seed=2),
    3: Workload("cfg3_zipf_capacity1.25", B=8, S=2048, d=2048, E=16, k=2, F=2816, dtype=torch.bfloat16, seed=3,
                drop_overflow=True, zipf_bias=True),
    4: Workload("cfg4_expert_choice_C2048", B=1, S=16384, d=2048, E=16, k=2, F=2816, dtype=torch.bfloat16, seed=4,
                routing="expert_choice", capacity_factor=2.0),
    5: Workload("cfg5_fp8_mod0.75", B=4, S=2048, d=2048, E=16, k=2, F=2816, dtype=torch.bfloat16, seed=5, fp8=True,
                mod=True),
}


def zipf_bias(E: int, seed: int) -> np.ndarray:
    """b_e = tau * ln(z_e), z_e = rank_e^-s over a seeded expert permutation."""
    perm = torch.randperm(E, generator=torch.Generator().manual_seed(seed * 11)).numpy()
    rank = np.empty(E)
    rank[perm] = np.arange(1, E + 1)
    return (ZIPF_TAU * np.log(rank ** -ZIPF_S)).astype(np.float32)


def make_tensors(wl: Workload, device="cpu", tokens: Optional[int] = None):
    """x (B,S,d) and the layer's parameters, as a dict of tensors on `device`.

    `tokens` (optional) overrides B*S with B=1 (for bounded CPU samples)."""
    g = torch.Generator().manual_seed(wl.seed)
    B, S = (wl.B, wl.S) if tokens is None else (1, tokens)
    x = torch.randn(B, S, wl.d, generator=g)
    t = dict(x=x)
    t["w_in"] = torch.randn(128, wl.d, generator=g) * 0.02
    t["w_out"] = torch.randn(wl.E, 128, generator=g) * 0.02
    t["w1"] = torch.randn(wl.E, wl.d, wl.F, generator=g) * 0.02
    t["w2"] = torch.randn(wl.E, wl.d, wl.F, generator=g) * 0.02
    t["w3"] = torch.randn(wl.E, wl.F, wl.d, generator=g) * 0.02
    if wl.mod:
        t["w_mod"] = torch.randn(1, wl.d, generator=g) * 0.02
    return {k: v.to(wl.dtype).to(device) for k, v in t.items()}


def load_into(module, t: dict):
    """Copies generated weights into a MoELayer / MoDMoE's parameters."""
    from .mod import MoDMoE
    moe = module.ffn if isinstance(module, MoDMoE) else module
    with torch.no_grad():
        moe.router.router[0].weight.copy_(t["w_in"])
        moe.router.router[2].weight.copy_(t["w_out"])
        ge = moe.grouped_experts if moe.grouped_experts is not None else moe.grouped_experts_ec
        ge.w1.copy_(t["w1"])
        ge.w2.copy_(t["w2"])
        ge.w3.copy_(t["w3"])
        if isinstance(module, MoDMoE):
            module.ffn_mod_router.router.weight.copy_(t["w_mod"])
    return module


def build_layer(wl: Workload, device, t: dict):
    """A MoELayer (or MoDMoE for config 5) of the workload, weights from `t`."""
    from .moe import MoELayer
    from .mod import MoDMoE
    cfg = wl.config()
    m = MoDMoE(cfg) if wl.mod else MoELayer(cfg, 0)
    m = m.to(device=device, dtype=wl.dtype)
    return load_into(m, t)
