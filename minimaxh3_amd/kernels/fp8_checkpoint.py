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
            "modules" = JSON list of {"name", "in_features", "out_features", "bias", "act"},
            "fingerprint" = the caller's description of how the weights were made (optional)
Module paths are those of ``transformer.named_modules()``.

The codes depend on everything that shaped the bf16 weights before the conversion (the base
weights, LoRAs fused into them, runtime/model_manager.py:109-110) and on the conversion's own
settings (exclude patterns, kept edge blocks).  ``conversion_fingerprint`` condenses those into
one string; a checkpoint saved with it is refused by a load that expects another one, so a
cache keyed by the fingerprint never hands back stale codes.
"""
from __future__ import annotations

import hashlib
import json

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

from .fp8_linear import ACT_GELU_TANH, ACT_NONE, FP8Linear

FORMAT = "mxf8-fp8linear"
VERSION = "1"


def conversion_fingerprint(exclude_patterns: str | list[str], keep_edge_blocks: int, fused_loras=(),
                           source: str = "", fuse_gelu: bool = False) -> str:
    """A digest of what decides the FP8 codes: the conversion settings
    (``convert_transformer_to_fp8``'s exclude patterns and kept edge blocks, the GELU fold),
    the LoRAs fused into the bf16 weights beforehand (any JSON-serialisable description,
    e.g. the (path, scale) specs) and a revision or hash of the base weights (``source``)."""
    if isinstance(exclude_patterns, str):
        exclude_patterns = exclude_patterns.split(",")
    desc = {
        "exclude": sorted(p.strip().lower() for p in exclude_patterns if p.strip()),
        "keep_edge_blocks": int(keep_edge_blocks),
        "fused_loras": json.loads(json.dumps(list(fused_loras), default=str)),
        "source": str(source),
        "fuse_gelu": bool(fuse_gelu),
    }
    return hashlib.sha256(json.dumps(desc, sort_keys=True).encode()).hexdigest()


def save_fp8_checkpoint(transformer: nn.Module, path: str, fingerprint: str | None = None) -> int:
    """Write the buffers of every FP8Linear in ``transformer`` to ``path``; returns the count.
    ``fingerprint`` (e.g. from ``conversion_fingerprint``) is stored with them."""
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
    meta = {"format": FORMAT, "version": VERSION, "modules": json.dumps(entries)}
    if fingerprint is not None:
        meta["fingerprint"] = str(fingerprint)
    save_file(tensors, path, metadata=meta)
    return len(entries)


def _set_submodule(root: nn.Module, name: str, mod: nn.Module) -> None:
    parent_name, _, attr = name.rpartition(".")
    parent = root.get_submodule(parent_name) if parent_name else root
    setattr(parent, attr, mod)


@torch.no_grad()
def load_fp8_checkpoint(transformer: nn.Module, path: str, device: torch.device | str | None = None,
                        strict: bool = True, fuse_gelu: bool = False, fingerprint: str | None = None) -> int:
    """Install the FP8Linear modules stored in ``path`` into ``transformer``; returns the count.

    A module path that names an ``nn.Linear`` is replaced by an FP8Linear built from the
    stored buffers (its LoRA ``adapters`` list carries over and its bf16 weight is freed,
    as in ``FP8Linear.from_linear``); one that names an FP8Linear has its buffers
    replaced in place.  ``device`` defaults to the linear's own device when that is a GPU, else
    ``cuda``.  With ``strict``, a stored module that the transformer lacks raises
    KeyError; any other mismatch (shapes, dtypes, a bias the target has or lacks, a missing
    tensor) raises ValueError.  Modules saved with the GELU-tanh epilogue
    (``convert_transformer_to_fp8(..., fuse_gelu=True)``) need ``fuse_gelu=True``, which folds
    their tanh-GELU activation modules again (and only theirs).  With ``fingerprint``, a file
    saved with another fingerprint (or none) raises ValueError.  Every check runs before the
    transformer is changed, so a refused file leaves it untouched.
    """
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or meta.get("version") != VERSION:
            raise ValueError(f"{path}: not an {FORMAT} v{VERSION} checkpoint (metadata {meta})")
        if fingerprint is not None and meta.get("fingerprint") != str(fingerprint):
            raise ValueError(f"{path}: saved for fingerprint {meta.get('fingerprint')!r}, expected {fingerprint!r} "
                             f"(the weights or the conversion settings changed)")
        entries = json.loads(meta["modules"])
        stored = set(f.keys())

        def tensor_info(key: str, what: str):
            if key not in stored:
                raise ValueError(f"{path}: {what} tensor {key!r} is missing")
            sl = f.get_slice(key)
            return str(sl.get_dtype()), tuple(sl.get_shape())

        # every check, before the transformer changes
        targets = []
        for e in entries:
            name = e["name"]
            try:
                target = transformer.get_submodule(name)
            except AttributeError:
                if strict:
                    raise KeyError(f"{path}: module {name!r} is not in the transformer") from None
                continue
            n, k = e["out_features"], e["in_features"]
            if tensor_info(f"{name}.w8", "code") != ("F8_E4M3", (n, k)):
                raise ValueError(f"{path}: {name}.w8 must be F8_E4M3 {(n, k)}, found {tensor_info(f'{name}.w8', '')}")
            if tensor_info(f"{name}.w_scale", "scale") != ("F32", (n,)):
                raise ValueError(f"{path}: {name}.w_scale must be F32 ({n},)")
            if e["bias"] and tensor_info(f"{name}.bias", "bias") != ("BF16", (n,)):
                raise ValueError(f"{path}: {name}.bias must be BF16 ({n},)")
            if not isinstance(target, (FP8Linear, nn.Linear)):
                raise ValueError(f"{name}: expected nn.Linear or FP8Linear, found {type(target).__name__}")
            if (target.in_features, target.out_features) != (k, n):
                raise ValueError(f"{name}: {type(target).__name__} {target.in_features}->{target.out_features} does "
                                 f"not match the stored {k}->{n}")
            if (target.bias is not None) != bool(e["bias"]):
                raise ValueError(f"{name}: the module {'has' if target.bias is not None else 'lacks'} a bias, the "
                                 f"stored one {'has' if e['bias'] else 'lacks'} one")
            if isinstance(target, FP8Linear):
                if int(target.act) != e["act"]:
                    raise ValueError(f"{name}: the module's epilogue activation {int(target.act)} differs from the "
                                     f"stored {e['act']}")
            elif e["act"] == ACT_GELU_TANH:
                if not fuse_gelu:
                    raise ValueError(f"{path}: {name} was saved with the fused GELU-tanh epilogue; load with "
                                     f"fuse_gelu=True")
                parent_name, _, attr = name.rpartition(".")
                parent = transformer.get_submodule(parent_name) if parent_name else transformer
                if attr != "proj" or getattr(parent, "approximate", None) != "tanh":
                    raise ValueError(f"{path}: saved with a fused GELU-tanh, but no tanh-GELU module wraps {name}")
            targets.append((e, target))

        count = 0
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
                # fold the tanh-GELU module around it (checked above), as when it was saved
                parent_name = name.rpartition(".")[0]
                act_mod = transformer.get_submodule(parent_name) if parent_name else transformer
                new.act = ACT_GELU_TANH
                act_mod.forward = new.forward
            count += 1
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return count
