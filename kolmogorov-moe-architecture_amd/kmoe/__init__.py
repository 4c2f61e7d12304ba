"""kmoe — MI355X-native MoE feed-forward layer (router, dispatch, grouped SwiGLU
GEMMs, combine) behind the Python API of moe_arch/model/moe.py."""
from ._lib import KmoeError, load as load_library
from .config import AdvancedMoEConfig, get_5b_config, get_test_config
from .moe import (ExpertChoiceRouter, GroupedExperts, GroupedExpertsExpertChoice, MoELayer, Router)
from .mod import MoDMoE, MoDRouter
from .block import MoEFFNBlock, RMSNorm
from . import ops, kernels, checkpoint

__all__ = [
    "AdvancedMoEConfig", "get_5b_config", "get_test_config", "MoELayer", "Router", "ExpertChoiceRouter",
    "GroupedExperts", "GroupedExpertsExpertChoice", "MoDRouter", "MoDMoE", "ops", "kernels", "KmoeError",
    "load_library", "MoEFFNBlock", "RMSNorm", "checkpoint",
]
