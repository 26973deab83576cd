"""LoRA adapter files for a stack of blocks: save and load the trained
factors in safetensors.

Two key layouts:
- "diffusers" (the file the klein trainer writes, `pytorch_lora_weights.
  safetensors`, docs/RESEARCH.md:87-97 and its section 3.1):
  `transformer.transformer_blocks.{i}.attn.to_q.lora_A.weight` /
  `.lora_B.weight` for the double blocks (image stream to_q, to_k, to_v,
  to_out.0; the text stream's projections under the diffusers names of the
  added context projections, add_q_proj, add_k_proj, add_v_proj,
  to_add_out), `transformer.single_transformer_blocks.{i}.attn.
  to_qkv_mlp_proj` and `.attn.to_out` for the single blocks.  A is [rank,
  in], B is [out, rank], bf16.  Alpha is not a tensor: `__metadata__` holds
  `format: "pt"` and `lora_adapter_metadata`, the PEFT config as JSON with
  `transformer.`-prefixed fields (r, lora_alpha, target_modules,
  init_lora_weights "gaussian", use_rslora, use_dora).
- "foundry" (the reference harness's weight keys, throughput.rs:1078-1093):
  `weights/double.{i}.{img|txt}.{to_q|to_k|to_v|to_out}.lora_{a|b}` and
  `weights/single.{i}.{to_in|to_out}.lora_{a|b}`, with the rank and alpha as
  metadata strings.

Loading copies into the blocks' factor tensors in place (the double block's
stacked q/k/v factors stay views) and then calls refresh_adapters(), and it
adopts the file's alpha / rank as the blocks' LoRA scale when the metadata
gives them.  Files are read with safetensors' tensor loader only (nothing in
a file is executed).
"""
import json
from collections import OrderedDict
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .block import LORA_TARGETS, SINGLE_LORA_TARGETS

DIFFUSERS_DOUBLE = {
    ("img", "q"): "attn.to_q", ("img", "k"): "attn.to_k", ("img", "v"): "attn.to_v",
    ("img", "out"): "attn.to_out.0",
    ("txt", "q"): "attn.add_q_proj", ("txt", "k"): "attn.add_k_proj", ("txt", "v"): "attn.add_v_proj",
    ("txt", "out"): "attn.to_add_out",
}
DIFFUSERS_SINGLE = {"to_in": "attn.to_qkv_mlp_proj", "to_out": "attn.to_out"}
FOUNDRY_DOUBLE = {"q": "to_q", "k": "to_k", "v": "to_v", "out": "to_out"}
LAYOUTS = ("diffusers", "foundry")


def _key(layout: str, kind: str, i: int, stream: Optional[str], target: str, part: str) -> str:
    """part: "a" (the [rank, in] factor) or "b" (the [out, rank] factor)."""
    if layout == "diffusers":
        if kind == "double":
            mod = f"transformer.transformer_blocks.{i}.{DIFFUSERS_DOUBLE[(stream, target)]}"
        else:
            mod = f"transformer.single_transformer_blocks.{i}.{DIFFUSERS_SINGLE[target]}"
        return f"{mod}.lora_{part.upper()}.weight"
    if layout == "foundry":
        if kind == "double":
            return f"weights/double.{i}.{stream}.{FOUNDRY_DOUBLE[target]}.lora_{part}"
        return f"weights/single.{i}.{target}.lora_{part}"
    raise ValueError(f"unknown layout {layout!r}; expected one of {LAYOUTS}")


def _slots(doubles: Sequence, singles: Sequence, layout: str, streams: Sequence[str]):
    """(key, block, owner of the factor dicts, target, part) for every factor."""
    out = []
    for i, blk in enumerate(doubles):
        for stream in streams:
            w = blk.w[stream]
            for t in LORA_TARGETS:
                if t not in w.lora_a:
                    continue
                for part in ("a", "b"):
                    out.append((_key(layout, "double", i, stream, t, part), blk, w, t, part))
    for i, blk in enumerate(singles):
        for t in SINGLE_LORA_TARGETS:
            if t not in blk.w.lora_a:
                continue
            for part in ("a", "b"):
                out.append((_key(layout, "single", i, None, t, part), blk, blk.w, t, part))
    return out


def _rank_alpha(doubles: Sequence, singles: Sequence) -> Tuple[int, float]:
    ranks, scales = set(), set()
    for blk in list(doubles) + list(singles):
        w = blk.w["img"] if isinstance(blk.w, dict) else blk.w
        for a in w.lora_a.values():
            ranks.add(int(a.shape[0]))
        scales.add(float(blk.lora_scale))
    if len(ranks) != 1 or len(scales) != 1:
        raise ValueError(f"blocks disagree on LoRA rank {sorted(ranks)} or scale {sorted(scales)}")
    r = ranks.pop()
    return r, scales.pop() * r


def lora_state_dict(doubles: Sequence = (), singles: Sequence = (), layout: str = "diffusers",
                    streams: Sequence[str] = ("img", "txt")) -> "OrderedDict[str, torch.Tensor]":
    """The stack's LoRA factors under `layout`'s keys, as contiguous bf16 CPU
    tensors.  streams: the double blocks' streams to include (the klein
    trainer adapts the image stream only: streams=("img",))."""
    sd = OrderedDict()
    for key, _, w, t, part in _slots(doubles, singles, layout, streams):
        src = w.lora_a[t] if part == "a" else w.lora_b[t]
        sd[key] = src.detach().to(device="cpu", dtype=torch.bfloat16).contiguous()
    return sd


def save_lora(path: str, doubles: Sequence = (), singles: Sequence = (), layout: str = "diffusers",
              streams: Sequence[str] = ("img", "txt")) -> Dict[str, str]:
    """Write the stack's LoRA factors to `path` (safetensors).  Rank and alpha
    (= the blocks' LoRA scale x rank) go into the metadata; returns it."""
    from safetensors.torch import save_file
    r, alpha = _rank_alpha(doubles, singles)
    sd = lora_state_dict(doubles, singles, layout, streams)
    if layout == "diffusers":
        targets = sorted({k.split(".lora_")[0].split(".", 3)[-1] for k in sd})
        peft = {"transformer.r": r, "transformer.lora_alpha": alpha, "transformer.target_modules": targets,
                "transformer.init_lora_weights": "gaussian", "transformer.use_rslora": False,
                "transformer.use_dora": False, "transformer.lora_dropout": 0.0, "transformer.bias": "none"}
        meta = {"format": "pt", "lora_adapter_metadata": json.dumps(peft)}
    else:
        meta = {"format": "pt", "lora_rank": str(r), "lora_alpha": repr(alpha)}
    save_file(sd, path, metadata=meta)
    return meta


def read_metadata(path: str) -> Tuple[Optional[int], Optional[float]]:
    """(rank, alpha) from a LoRA file's metadata, None where absent."""
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    if "lora_adapter_metadata" in meta:
        cfg = json.loads(meta["lora_adapter_metadata"])
        r, a = cfg.get("transformer.r"), cfg.get("transformer.lora_alpha")
        return (int(r) if r is not None else None), (float(a) if a is not None else None)
    r, a = meta.get("lora_rank"), meta.get("lora_alpha")
    return (int(r) if r is not None else None), (float(a) if a is not None else None)


def load_lora(path: str, doubles: Sequence = (), singles: Sequence = (), layout: str = "diffusers",
              streams: Sequence[str] = ("img", "txt"), strict: bool = False) -> Dict[str, object]:
    """Copy the LoRA factors in `path` into the blocks.

    A factor the file lacks keeps its value (the klein trainer's files adapt
    only the image stream of the double blocks); strict=True makes that an
    error.  A key the blocks have no slot for, or a shape that differs, is
    always an error.  Returns {"loaded", "missing", "rank", "alpha",
    "scale"}; with both rank and alpha in the metadata the blocks' LoRA scale
    becomes alpha / rank."""
    from safetensors.torch import load_file
    tensors = load_file(path)
    slots = _slots(doubles, singles, layout, streams)
    known = {s[0] for s in slots}
    unexpected = sorted(k for k in tensors if k not in known)
    if unexpected:
        raise ValueError(f"{path}: keys with no LoRA slot in these blocks ({layout} layout): {unexpected[:8]}")
    loaded: List[str] = []
    missing: List[str] = []
    for key, blk, w, t, part in slots:
        if key not in tensors:
            missing.append(key)
            continue
        dst = w.lora_a[t] if part == "a" else w.lora_b[t]
        src = tensors[key]
        if tuple(src.shape) != tuple(dst.shape):
            raise ValueError(f"{key}: file shape {tuple(src.shape)} != block shape {tuple(dst.shape)}")
        dst.copy_(src.to(device=dst.device, dtype=dst.dtype))
        loaded.append(key)
    if strict and missing:
        raise ValueError(f"{path}: missing LoRA factors: {missing[:8]}")
    r, alpha = read_metadata(path)
    scale = None
    if r and alpha is not None:
        scale = alpha / r
        for blk in list(doubles) + list(singles):
            blk.lora_scale = scale
    for blk in list(doubles) + list(singles):
        blk.refresh_adapters()
    return {"loaded": loaded, "missing": missing, "rank": r, "alpha": alpha, "scale": scale}
