"""Pre-quantized FP8 weight checkpoints for FP8Linear modules (safetensors).

Converting a transformer from bf16 weights quantizes every eligible linear at load
(``FP8Linear.from_linear``, reference kernels/fp8_linear.py:65-85, reached from
runtime/model_manager.py:113).  A checkpoint written by ``save_fp8_checkpoint`` stores
what that conversion produces -- per converted module the e4m3 codes ``w8 [N, K]``, the
per-output-channel scales ``w_scale [N]`` (fp32) and the bf16 bias ``[N]`` -- so
``load_fp8_checkpoint`` rebuilds the same modules without quantizing, bit for bit, and a
model evicted to host memory can be restored from FP8 bytes (half the size of bf16).

File layout (one safetensors file):
  tensors   "<module path>.w8" (F8_E4M3 [N, K]), "<module path>.w_scale" (F32 [N]),
            "<module path>.bias" (BF16 [N], only for modules with a bias)
  metadata  "format" = "mxf8-fp8linear", "version" = "1",
            "modules" = JSON list of {"name", "in_features", "out_features", "bias", "act"}
Module paths are those of ``transformer.named_modules()``.
"""
from __future__ import annotations

import json

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

from .fp8_linear import ACT_GELU_TANH, ACT_NONE, FP8Linear

FORMAT = "mxf8-fp8linear"
VERSION = "1"


def save_fp8_checkpoint(transformer: nn.Module, path: str) -> int:
    """Write the buffers of every FP8Linear in ``transformer`` to ``path``; returns the count."""
    tensors: dict[str, torch.Tensor] = {}
    entries = []
    for name, mod in transformer.named_modules():
        if not isinstance(mod, FP8Linear):
            continue
        if not name:
            raise ValueError("save_fp8_checkpoint: the transformer itself is an FP8Linear")
        tensors[f"{name}.w8"] = mod.w8.detach().cpu().contiguous()
        tensors[f"{name}.w_scale"] = mod.w_scale.detach().reshape(-1).float().cpu().contiguous()
        if mod.bias is not None:
            tensors[f"{name}.bias"] = mod.bias.detach().to(torch.bfloat16).cpu().contiguous()
        entries.append({"name": name, "in_features": mod.in_features, "out_features": mod.out_features,
                        "bias": mod.bias is not None, "act": int(mod.act)})
    if not entries:
        raise ValueError("save_fp8_checkpoint: no FP8Linear modules in the transformer")
    save_file(tensors, path, metadata={"format": FORMAT, "version": VERSION, "modules": json.dumps(entries)})
    return len(entries)


def _set_submodule(root: nn.Module, name: str, mod: nn.Module) -> None:
    parent_name, _, attr = name.rpartition(".")
    parent = root.get_submodule(parent_name) if parent_name else root
    setattr(parent, attr, mod)


@torch.no_grad()
def load_fp8_checkpoint(transformer: nn.Module, path: str, device: torch.device | str | None = None,
                        strict: bool = True, fuse_gelu: bool = False) -> int:
    """Install the FP8Linear modules stored in ``path`` into ``transformer``; returns the count.

    A module path that names an ``nn.Linear`` is replaced by an FP8Linear built from the
    stored buffers (its LoRA ``adapters`` list carries over and its bf16 weight is freed,
    as in ``FP8Linear.from_linear``); one that names an FP8Linear has its buffers
    replaced in place.  ``device`` defaults to the linear's own device when that is a GPU, else
    ``cuda``.  With ``strict``, a stored module that the transformer lacks raises
    KeyError; shape mismatches always raise ValueError.  Modules saved with the GELU-tanh
    epilogue (``convert_transformer_to_fp8(..., fuse_gelu=True)``) need ``fuse_gelu=True``,
    which folds their tanh-GELU activation modules again (and only theirs).
    """
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or meta.get("version") != VERSION:
            raise ValueError(f"{path}: not an {FORMAT} v{VERSION} checkpoint (metadata {meta})")
        entries = json.loads(meta["modules"])
        # validate every entry before changing the transformer
        targets = []
        for e in entries:
            name = e["name"]
            try:
                target = transformer.get_submodule(name)
            except AttributeError:
                if strict:
                    raise KeyError(f"{path}: module {name!r} is not in the transformer") from None
                continue
            shape = tuple(f.get_slice(f"{name}.w8").get_shape())
            if shape != (e["out_features"], e["in_features"]):
                raise ValueError(f"{path}: {name}.w8 has shape {shape}")
            if not isinstance(target, (FP8Linear, nn.Linear)):
                raise ValueError(f"{name}: expected nn.Linear or FP8Linear, found {type(target).__name__}")
            if (target.in_features, target.out_features) != (e["in_features"], e["out_features"]):
                raise ValueError(f"{name}: {type(target).__name__} {target.in_features}->{target.out_features} does "
                                 f"not match the stored {e['in_features']}->{e['out_features']}")
            if isinstance(target, FP8Linear):
                if int(target.act) != e["act"]:
                    raise ValueError(f"{name}: the module's epilogue activation {int(target.act)} differs from the "
                                     f"stored {e['act']}")
            elif e["act"] == ACT_GELU_TANH and not fuse_gelu:
                raise ValueError(f"{path}: {name} was saved with the fused GELU-tanh epilogue; load with "
                                 f"fuse_gelu=True")
            targets.append((e, target))
        count = 0
        gelu_mods: dict[int, str] = {}
        for e, target in targets:
            name = e["name"]
            w8 = f.get_tensor(f"{name}.w8")
            w_scale = f.get_tensor(f"{name}.w_scale")
            bias = f.get_tensor(f"{name}.bias") if e["bias"] else None
            if isinstance(target, FP8Linear):
                # buffers replaced in place (a fused activation module keeps calling this module)
                dev = torch.device(device) if device is not None else target.w8.device
                src = FP8Linear.from_quantized(w8, w_scale, bias, dev)
                target.w8, target.w_scale, target.bias = src.w8, src.w_scale, src.bias
                count += 1
                continue
            if device is not None:
                dev = torch.device(device)
            else:
                w = target.weight
                dev = w.device if (w is not None and w.is_cuda) else torch.device("cuda")
            new = FP8Linear.from_quantized(w8, w_scale, bias, dev)
            if isinstance(getattr(target, "adapters", None), list):
                new.adapters = list(target.adapters)
            target.weight = None
            target.bias = None
            _set_submodule(transformer, name, new)
            if e["act"] == ACT_GELU_TANH:
                gelu_mods[id(new)] = name
            count += 1
    if gelu_mods:
        # fold the tanh-GELU module around each module saved with the fused epilogue (and
        # only those: the others keep their activation module, as when they were saved)
        for _, act_mod in transformer.named_modules():
            proj = getattr(act_mod, "proj", None)
            if id(proj) in gelu_mods and getattr(act_mod, "approximate", None) == "tanh":
                proj.act = ACT_GELU_TANH
                act_mod.forward = proj.forward
                gelu_mods.pop(id(proj))
        if gelu_mods:
            names = sorted(gelu_mods.values())
            raise ValueError(f"{path}: saved with a fused GELU-tanh, but no tanh-GELU module wraps {names}")
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return count
