"""Checkpoints around the MoE layer: the reference's state-dict format in, the derived
packed-weight cache on disk, and the expert copy of tools/reallocate_experts.py with the
state-dict keys the model actually has.

* The reference saves ``{"model_state_dict": model.state_dict(), ...}`` with torch.save
  (trainer.py:340-362, train.py:186-208).  An MoE block ``i`` of MoETransformer holds its
  layer under ``layers.{i}.ffn.`` and its pre-FFN norm under ``layers.{i}.ffn_norm.``
  (layers.py:70-74); the kmoe modules use the same key suffixes, so the sub-dict loads
  with ``load_state_dict`` unchanged.  Files are read with ``weights_only=True``: a file
  whose pickle holds other objects (the reference stores its config object) is refused
  by torch's safe loader, and the error says so; nothing in a checkpoint is executed.
* The packed expert weights (and, for fp8, the per-row quantisation scales) are a
  derived cache of w1/w2/w3.  ``save_packed`` writes them with a fingerprint of the
  source parameters and the library's packed-layout version, ABI version and buffer
  sizes (safetensors); ``load_packed`` installs them only when all of these match the
  layer's current parameters and the loaded library, so a large layer (or an fp8 one,
  quantised once) skips the pack at load time and a file from a build with another
  packed layout is re-packed instead of being read with the wrong strides.
* ``copy_experts`` is the expert copy of tools/reallocate_experts.py:254-266 with the
  keys ``...grouped_experts.w1/w2/w3`` (the reference tool looks for ``gate_proj`` /
  ``up_proj`` / ``down_proj``, which no MoELayer has, so it copies nothing).
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional, Tuple

import torch
import xxhash
from safetensors.torch import load_file, save_file

from . import ops

_EXPERT_KEYS = ("w1", "w2", "w3")


def load_model_state_dict(path: str, map_location="cpu") -> Dict[str, torch.Tensor]:
    """The ``model_state_dict`` of a reference checkpoint (or a bare state dict), loaded
    with torch's safe loader only."""
    try:
        obj = torch.load(path, map_location=map_location, weights_only=True)
    except Exception as e:  # the safe unpickler refuses non-tensor objects
        raise ValueError(f"kmoe: {path} cannot be read with torch.load(weights_only=True) ({e}); "
                         "re-save its model_state_dict alone (torch.save(ckpt['model_state_dict'], ...))") from e
    if isinstance(obj, dict) and "model_state_dict" in obj:
        obj = obj["model_state_dict"]
    if not isinstance(obj, dict):
        raise ValueError(f"kmoe: {path} does not hold a state dict")
    return obj


def layer_state_dict(model_sd: Dict[str, torch.Tensor], layer_idx: int, part: str = "ffn",
                     prefix: str = "layers.") -> Dict[str, torch.Tensor]:
    """Entries of block `layer_idx` for a kmoe module: part="ffn" gives the MoELayer's
    keys (``router.router.0.weight``, ``grouped_experts.w1``, ...), part="block" the
    MoEFFNBlock's (``ffn_norm.weight``, ``ffn.*`` and, with MoD, ``ffn_mod_router.*``)."""
    base = f"{prefix}{layer_idx}."
    if part == "ffn":
        head = base + "ffn."
        out = {k[len(head):]: v for k, v in model_sd.items() if k.startswith(head)}
    elif part == "block":
        out = {k[len(base):]: v for k, v in model_sd.items()
               if k.startswith((base + "ffn.", base + "ffn_norm.", base + "ffn_mod_router."))}
    else:
        raise ValueError(f"kmoe.layer_state_dict: part must be 'ffn' or 'block', not {part!r}")
    if not out:
        raise KeyError(f"kmoe: no '{base}{'ffn' if part == 'ffn' else 'ffn*'}' entries in the state dict")
    return out


def copy_experts(model_sd: Dict[str, torch.Tensor], moves: Iterable[Tuple[int, int, int, int]],
                 prefix: str = "layers.") -> Dict[str, torch.Tensor]:
    """New state dict with expert weights copied: each (src_layer, src_expert, dst_layer,
    dst_expert) copies w1/w2/w3[src_expert] of block src_layer over [dst_expert] of
    dst_layer (the reallocation step of tools/reallocate_experts.py:254-266).  Sources
    are read from the input dict, so moves do not see each other's writes."""
    out = {k: v for k, v in model_sd.items()}
    copied = set()
    for sl, se, dl, de in moves:
        for w in _EXPERT_KEYS:
            sk = f"{prefix}{sl}.ffn.grouped_experts.{w}"
            dk = f"{prefix}{dl}.ffn.grouped_experts.{w}"
            if w == "w3" and sk not in model_sd and dk not in model_sd:
                continue  # non-gated experts have w1 and w2 only
            if sk not in model_sd or dk not in model_sd:
                raise KeyError(f"kmoe.copy_experts: missing {sk if sk not in model_sd else dk}")
            src, dst = model_sd[sk], model_sd[dk]
            if src.shape[1:] != dst.shape[1:]:
                raise ValueError(f"kmoe.copy_experts: {sk} {tuple(src.shape)} vs {dk} {tuple(dst.shape)}")
            if dk not in copied:
                out[dk] = dst.clone()
                copied.add(dk)
            out[dk][de] = src[se]
    return out


# ---------------------------------------------------------------- packed-weight cache
def _fingerprint(experts) -> str:
    """xxh64 over the bytes of w1, w2, w3 (with their shapes and dtypes) and the fp8 flag."""
    h = xxhash.xxh64()
    for name in _EXPERT_KEYS:
        w = getattr(experts, name).detach()
        h.update(f"{name}:{tuple(w.shape)}:{w.dtype};".encode())
        h.update(w.contiguous().view(torch.uint8).cpu().numpy().tobytes())
    h.update(b"fp8" if experts.use_fp8 else b"bf16")
    return h.hexdigest()


def _layout_meta(E: int, d: int, F: int, fp8: bool) -> Dict[str, str]:
    """What a packed buffer's layout depends on besides E/d/F/fp8: the library's packed
    layout version and ABI version, and the byte sizes of the packed buffers."""
    from . import _lib

    lib = _lib.load()
    pdt = _lib.DTYPE_FP8_E4M3 if fp8 else _lib.DTYPE_BF16
    return {"layout": str(lib.kmoe_pack_layout_version()), "abi": str(lib.kmoe_abi_version()),
            "w13_bytes": str(lib.kmoe_packed_w13_bytes(E, d, F, pdt)),
            "w3_bytes": str(lib.kmoe_packed_w3_bytes(E, d, F, pdt))}


def save_packed(experts, path: str) -> None:
    """Write the experts' packed weights (GroupedExperts / GroupedExpertsExpertChoice,
    bf16 or fp8 with scales), the source fingerprint and the packed layout's version
    and sizes to a safetensors file.  Gated (swiglu) experts only."""
    if not getattr(experts, "gated", True):
        raise ValueError("kmoe: packed-weight files hold gated (swiglu) experts only")
    pw = experts.packed()
    tensors = {"w13": pw.w13, "w3": pw.w3}
    if pw.fp8:
        tensors["s13"], tensors["s3"] = pw.s13, pw.s3
    meta = {"kmoe_packed": "1", "E": str(pw.E), "d": str(pw.d), "F": str(pw.F), "fp8": str(int(pw.fp8)),
            "fingerprint": _fingerprint(experts), **_layout_meta(pw.E, pw.d, pw.F, pw.fp8)}
    save_file({k: v.detach().contiguous().cpu() for k, v in tensors.items()}, path, metadata=meta)


def packed_file_matches(experts, path: str) -> bool:
    """Whether the packed-weight file at `path` was made from exactly the experts' current
    parameters (fingerprint, shapes, fp8 mode) by a library with this build's packed layout
    (layout and ABI versions, buffer sizes).  Reads the metadata and tensor shapes only."""
    from safetensors import safe_open

    if not getattr(experts, "gated", True):
        return False  # packed-weight files hold gated (swiglu) experts only
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("kmoe_packed") != "1":
            raise ValueError(f"kmoe.load_packed: {path} is not a kmoe packed-weight file")
        shapes = {k: tuple(f.get_slice(k).get_shape()) for k in f.keys()}
    E, d, F, fp8 = experts.n_experts, experts.d_model, experts.d_ff, experts.use_fp8
    try:
        if (int(meta["E"]), int(meta["d"]), int(meta["F"]), bool(int(meta["fp8"]))) != (E, d, F, fp8):
            return False
    except (KeyError, ValueError):
        return False
    want = _layout_meta(E, d, F, fp8)
    if any(meta.get(k) != v for k, v in want.items()):
        return False
    # the tensors themselves: byte buffers of the sizes the library packs, and one fp32
    # scale per packed row for fp8
    Fp = (F + 127) // 128 * 128
    dp = (d + 255) // 256 * 256
    exp_shapes = {"w13": (int(want["w13_bytes"]),), "w3": (int(want["w3_bytes"]),)}
    if fp8:
        exp_shapes.update({"s13": (E * 2 * Fp,), "s3": (E * dp,)})
    if shapes != exp_shapes:
        return False
    return meta.get("fingerprint") == _fingerprint(experts)


def load_packed(experts, path: str, device: Optional[torch.device] = None) -> bool:
    """Install packed weights saved by save_packed if they were made from exactly the
    experts' current parameters by a build with the same packed layout
    (packed_file_matches); returns whether they were installed (False: the next forward
    packs as usual)."""
    if not packed_file_matches(experts, path):
        return False
    dev = device if device is not None else experts.w1.device
    t = load_file(path, device=str(dev))
    if t["w13"].dtype != torch.uint8 or t["w3"].dtype != torch.uint8:
        return False
    pw = ops.PackedWeights(t["w13"], t["w3"], t.get("s13"), t.get("s3"), experts.n_experts, experts.d_model,
                           experts.d_ff, experts.use_fp8)
    experts.install_packed(pw)
    return True


def describe_packed(path: str) -> dict:
    """Metadata of a packed-weight file (shapes, mode, fingerprint)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        return dict(f.metadata() or {})
