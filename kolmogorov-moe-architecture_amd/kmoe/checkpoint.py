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
  source parameters (safetensors); ``load_packed`` installs them after checking the
  fingerprint against the layer's current parameters, so a large layer (or an fp8 one,
  quantised once) skips the pack at load time.
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
    MoEFFNBlock's (``ffn_norm.weight`` and ``ffn.*``)."""
    base = f"{prefix}{layer_idx}."
    if part == "ffn":
        head = base + "ffn."
        out = {k[len(head):]: v for k, v in model_sd.items() if k.startswith(head)}
    elif part == "block":
        out = {k[len(base):]: v for k, v in model_sd.items()
               if k.startswith(base + "ffn.") or k.startswith(base + "ffn_norm.")}
        # the block's MoD router (ffn_mod_router.*) is not part of the FFN half
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


def save_packed(experts, path: str) -> None:
    """Write the experts' packed weights (GroupedExperts / GroupedExpertsExpertChoice,
    bf16 or fp8 with scales) and the source fingerprint to a safetensors file."""
    pw = experts.packed()
    tensors = {"w13": pw.w13, "w3": pw.w3}
    if pw.fp8:
        tensors["s13"], tensors["s3"] = pw.s13, pw.s3
    meta = {"kmoe_packed": "1", "E": str(pw.E), "d": str(pw.d), "F": str(pw.F), "fp8": str(int(pw.fp8)),
            "fingerprint": _fingerprint(experts)}
    save_file({k: v.detach().contiguous().cpu() for k, v in tensors.items()}, path, metadata=meta)


def load_packed(experts, path: str, device: Optional[torch.device] = None) -> bool:
    """Install packed weights saved by save_packed if they were made from exactly the
    experts' current parameters (same fingerprint, shapes and fp8 mode); returns whether
    they were installed (False: the next forward packs as usual)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    if meta.get("kmoe_packed") != "1":
        raise ValueError(f"kmoe.load_packed: {path} is not a kmoe packed-weight file")
    E, d, F = experts.n_experts, experts.d_model, experts.d_ff
    if (int(meta["E"]), int(meta["d"]), int(meta["F"]), bool(int(meta["fp8"]))) != (E, d, F, experts.use_fp8):
        return False
    if meta.get("fingerprint") != _fingerprint(experts):
        return False
    dev = device if device is not None else experts.w1.device
    t = load_file(path, device=str(dev))
    pw = ops.PackedWeights(t["w13"], t["w3"], t.get("s13"), t.get("s3"), E, d, F, experts.use_fp8)
    experts.install_packed(pw)
    return True


def describe_packed(path: str) -> dict:
    """Metadata of a packed-weight file (shapes, mode, fingerprint)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        return dict(f.metadata() or {})
