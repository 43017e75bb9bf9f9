"""Checkpoint and state-dict loading for the fused modules.

The reference saves a FastWAM model as a payload dict (FB/fastwam.py:1113-1123): "mot" holds
`MoT.state_dict()`, whose keys are `mixtures.{video,action}.<expert key>` (FB/mot.py:22-31;
inside a full `FastWAM.state_dict()` they carry one more `mot.` prefix), plus "step",
"torch_dtype" and optionally "proprio_encoder"; a legacy payload holds the video expert alone
under "dit" (FB/fastwam.py:1125-1131).  The GEAK trees run on a fused attention layout
(FB/fused_qkv.py:141-199): `self_attn.{q,k,v}` concatenated along the output dimension into
`self_attn.qkv`, and `cross_attn.{k,v}` into `cross_attn.kv`.

`FusedActionDiT`, `FusedVideoDiTBlock` and `FusedVideoPrefill` take an expert's own keys
(`blocks.{i}.self_attn.q.weight`, ...; FB/action_dit.py:47-103, FB/wan_video_dit.py:93-131).
`expert_state_dicts` turns either layout, with or without the prefixes, into those.

Files are read only with loaders that execute nothing from the file: `torch.load(...,
weights_only=True)` for the reference's `torch.save` payloads, safetensors otherwise.
"""
from __future__ import annotations

import os
from typing import Dict, Mapping

import torch

EXPERTS = ("video", "action")


def load_checkpoint(path: str) -> Dict[str, object]:
    """The payload of a checkpoint file: a dict with "mot" (or "dit") for the reference's
    `FastWAM.save_checkpoint` files, or {"mot": tensors} for a .safetensors file of a MoT state
    dict.  Raises ValueError for anything else."""
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        return {"mot": load_file(path, device="cpu")}
    if not os.path.exists(path):
        raise FileNotFoundError(path)
    payload = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(payload, dict) or not ("mot" in payload or "dit" in payload):
        raise ValueError(f"checkpoint {path!r} holds neither a `mot` nor a `dit` state dict")
    return payload


def unfuse_attention(sd: Mapping[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """Inverse of the reference's fused attention layout (FB/fused_qkv.py:141-199): every
    `<p>.qkv.{weight,bias}` of a self-attention becomes `<p>.{q,k,v}.*` (three equal row
    blocks, in that order) and every `<p>.kv.{weight,bias}` of a cross-attention `<p>.{k,v}.*`.
    Other keys pass through; a state dict already in the split layout comes back unchanged."""
    out: Dict[str, torch.Tensor] = {}
    for key, val in sd.items():
        for fused, names in ((".qkv.", "qkv"), (".kv.", "kv")):
            i = key.rfind(fused)
            if i < 0 or not key.endswith(("weight", "bias")):
                continue
            prefix, leaf = key[:i], key[i + len(fused):]
            if leaf not in ("weight", "bias"):
                continue
            # as the reference fuses them: q|k|v of self-attention, k|v of cross-attention
            if "self_attn" not in prefix if names == "qkv" else "cross_attn" not in prefix:
                continue
            n = len(names)
            if val.shape[0] % n != 0:
                raise ValueError(f"{key}: {val.shape[0]} rows do not split into {n} equal blocks")
            for name, part in zip(names, val.chunk(n, dim=0)):
                out[f"{prefix}.{name}.{leaf}"] = part.contiguous()
            break
        else:
            out[key] = val
    return out


def expert_state_dicts(payload: Mapping[str, object]) -> Dict[str, Dict[str, torch.Tensor]]:
    """{"video": ..., "action": ...} expert state dicts (split q/k/v layout, expert-relative
    keys) from a checkpoint payload, a MoT state dict or a full FastWAM state dict.  A legacy
    "dit" payload yields the video expert only."""
    if "mot" in payload:
        sd = payload["mot"]
    elif "dit" in payload:
        return {"video": unfuse_attention(payload["dit"])}
    else:
        sd = payload
    out: Dict[str, Dict[str, torch.Tensor]] = {}
    for name in EXPERTS:
        for prefix in (f"mixtures.{name}.", f"mot.mixtures.{name}."):
            sub = {k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}
            if sub:
                out[name] = unfuse_attention(sub)
                break
    if not out:
        raise ValueError("no `mixtures.video.*` or `mixtures.action.*` keys in the state dict")
    return out
