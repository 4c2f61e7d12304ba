"""Drop-in for moe_arch/kernels (the reference's native extension package).

``grouped_swiglu_forward`` keeps the signature of the reference dispatcher
(moe_arch/kernels/__init__.py:105-137) and of the pybind entry point
``moe_kernels.grouped_swiglu_forward`` (grouped_gemm.cu:186-194), but runs the
MFMA grouped GEMMs: device-resident segment bounds, one launch per GEMM, no
host sync and no stream creation.  There is no PyTorch fallback.
"""
from __future__ import annotations

import torch

from . import _lib, ops


def is_kernel_available() -> bool:
    """kernels/__init__.py:24-26."""
    try:
        _lib.load()
        return True
    except ImportError:
        return False


_PACK_CACHE = {}


def _packed(W1, W2, W3):
    key = tuple((w.data_ptr(), w._version) for w in (W1, W2, W3))
    pw = _PACK_CACHE.get(key)
    if pw is None:
        _PACK_CACHE.clear()
        pw = ops.pack_weights(W1, W2, W3)
        _PACK_CACHE[key] = pw
    return pw


def grouped_swiglu_forward(sorted_inputs, W1, W2, W3, sorted_expert_ids, seg_starts, seg_ends,
                           use_cuda_kernel: bool = True) -> torch.Tensor:
    """For each expert e: out[s_e:e_e] = (silu(x W1[e]) * (x W2[e])) W3[e].

    Segments must be contiguous and ordered (seg_starts[e+1] == seg_ends[e], as
    produced by the reference's sort, sparse_moe.py:343-359)."""
    del sorted_expert_ids, use_cuda_kernel
    E = W1.shape[0]
    A = sorted_inputs.shape[0]
    offsets = torch.empty(E + 1, device=sorted_inputs.device, dtype=torch.int32)
    offsets[:E] = seg_starts.to(torch.int32)
    offsets[E:] = seg_ends[-1:].to(torch.int32)
    pw = _packed(W1, W2, W3)
    x = sorted_inputs.to(torch.bfloat16).contiguous()
    y = ops.grouped_ffn(x, None, offsets, pw, A)
    return y[:A].to(sorted_inputs.dtype)
