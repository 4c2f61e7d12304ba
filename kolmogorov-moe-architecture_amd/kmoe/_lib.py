"""ctypes binding of libkmoe.so, the C ABI declared in include/kmoe.h.

The library is built in-tree (``make`` in the package directory, or
``__graft_entry__.build()``).  Loading it is mandatory: there is no CPU
fallback, so a missing library raises immediately.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkmoe.so")
HEADER_PATH = os.path.abspath(os.path.join(_HERE, "..", "..", "include", "kmoe.h"))

KMOE_OK = 0
DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_FP8_E4M3 = 2
MAX_EXPERTS = 64
ROUTER_HIDDEN = 128

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/kmoe.h
_SIGNATURES = {
    "kmoe_last_error": (ctypes.c_char_p, []),
    "kmoe_abi_version": (_i32, []),
    "kmoe_pack_layout_version": (_i32, []),
    "kmoe_router_partials_len": (_i64, [_i64, _i32]),
    "kmoe_router_block_tokens": (_i32, [_i64]),
    "kmoe_router": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_aux_loss": (_i32, [_vp, _i64, _i32, _vp, _i32, _f32, _f32, _vp, _vp]),
    "kmoe_mod_aux_bce": (_i32, [_vp, _i64, _vp, _i64, _f32, _vp, _vp]),
    "kmoe_dispatch_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "kmoe_dispatch": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp,
                             _vp, _i32, _vp, _vp, _sz, _vp]),
    "kmoe_dispatch_counted": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _i32, _vp, _vp, _sz, _vp]),
    "kmoe_dispatch_counted_aux": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _vp, _i32, _vp, _vp, _sz, _vp, _f32, _f32, _vp, _vp]),
    "kmoe_dispatch_noalloc": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _i32, _vp, _vp]),
    "kmoe_gather_rows": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _vp]),
    "kmoe_padded_ff": (_i32, [_i32]),
    "kmoe_packed_w13_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "kmoe_packed_w3_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "kmoe_pack_weights": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_gemm_gate_up": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp]),
    "kmoe_gemm_gate_up_rows": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp]),
    "kmoe_gemm_down": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp]),
    "kmoe_quant_rows_fp8": (_i32, [_vp, _i64, _vp, _i32, _vp, _vp, _vp]),
    "kmoe_grouped_swiglu": (_i32, [_vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_combine": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _i32, _vp]),
    "kmoe_balanced_workspace_bytes": (_sz, [_i32, _i32]),
    "kmoe_balanced_topk": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "kmoe_ec_workspace_bytes": (_sz, [_i32, _i64, _i32]),
    "kmoe_ec_select": (_i32, [_vp, _i32, _i64, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "kmoe_mod_workspace_bytes": (_sz, [_i32, _i64]),
    "kmoe_mod_select": (_i32, [_vp, _i32, _i64, _i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    # backward pass
    "kmoe_router_hist": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_router_train": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_gemm_gate_up_rows_gu": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp]),
    "kmoe_gemm_gate_up_fp8_gu": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_dequant_rows_fp8": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp, _vp]),
    "kmoe_fake_quant_e4m3_cols": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "kmoe_router_rms": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _f32, _vp, _vp]),
    "kmoe_gemm_gate_up_rows_scaled": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp]),
    "kmoe_combine_residual": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _vp, _i32, _vp]),
    "kmoe_combine_residual_dropout": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _f32, _i64, _vp, _i32,
                                             _vp]),
    "kmoe_combine_bwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i64, _vp, _vp, _vp]),
    "kmoe_combine_bwd_rows": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_mod_bwd_workspace_bytes": (_sz, [_i64, _i32]),
    "kmoe_mod_bwd": (_i32, [_vp, _vp, _i32, _i64, _vp, _i32, _vp, _i64, _vp, _i32, _vp, _sz, _vp]),
    "kmoe_rmsnorm": (_i32, [_vp, _i32, _vp, _i32, _f32, _i64, _i32, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_rmsnorm_bwd_workspace_bytes": (_sz, [_i64, _i32]),
    "kmoe_rmsnorm_bwd": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _sz, _vp]),
    "kmoe_packed_w3n_bytes": (_sz, [_i32, _i32, _i32]),
    "kmoe_packed_w13t_bytes": (_sz, [_i32, _i32, _i32]),
    "kmoe_pack_weights_bwd": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "kmoe_packed_w1t_bytes": (_sz, [_i32, _i32, _i32]),
    "kmoe_packed_w1n_bytes": (_sz, [_i32, _i32, _i32]),
    "kmoe_pack_weights_plain": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "kmoe_pack_weights_plain_bwd": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "kmoe_silu_rows": (_i32, [_vp, _i64, _vp, _i32, _vp, _vp]),
    "kmoe_silu_bwd": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp, _vp]),
    "kmoe_gemm_grouped": (_i32, [_vp, _vp, _i32, _i32, _i64, _vp, _i64, _i32, _vp, _i64, _i32, _vp]),
    "kmoe_swiglu_bwd": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp, _vp]),
    "kmoe_reduce_f32": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp]),
    "kmoe_gemm_wgrad_rows": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _vp, _vp, _i32, _i64, _i32,
                                    _vp]),
    "kmoe_router_dlogits": (_i32, [_vp, _i64, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _f32, _vp, _vp]),
    "kmoe_ec_dlogits": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "kmoe_router_bwd_workspace_bytes": (_sz, [_i64, _i32]),
    "kmoe_router_mlp_bwd": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
    "kmoe_packed_w_in_t_bytes": (_sz, [_i32]),
    "kmoe_pack_w_in_t": (_i32, [_vp, _i32, _i32, _vp, _vp]),
}


class KmoeError(RuntimeError):
    """A kmoe C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


_LIB = None


def header_functions(path: str = HEADER_PATH) -> list:
    """Names of every function declared in include/kmoe.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kmoe_[a-z0-9_]+)\s*\(", text)))


def load():
    """Loads libkmoe.so (once) and binds every signature.  Raises if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"kmoe: HIP library {LIB_PATH} is not built; run `make` in "
            f"{os.path.dirname(_HERE)} or __graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def call(name: str, *args):
    """Calls a status-returning entry point and raises KmoeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != KMOE_OK:
        raise KmoeError(name, rc, lib.kmoe_last_error().decode())
    return rc


def ptr(t):
    """Device pointer of a tensor (None for None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_ptr(device=None):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
