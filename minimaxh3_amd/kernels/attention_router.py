"""Drop-in SDPA router (mirrors kernels/attention_router.py of the reference).

``install()`` replaces ``torch.nn.functional.scaled_dot_product_attention`` with
``routed_sdpa``, which sends a call to the FP8 kernel when it runs inside a denoiser
scope, the path is enabled, the call is non-causal without dropout or GQA, the inputs
are supported, Sq >= min_seq and the mask reduces to one value per key; every other call
goes to the original SDPA unchanged.  The router itself never raises.
"""
from __future__ import annotations

import functools
import threading
from contextlib import contextmanager

import torch
import torch.nn.functional as F

from .fp8_attention import fp8_attention, is_supported

enabled: bool = True
repair_tau: float = -1.0
min_seq: int = 4096

_tls = threading.local()
_lock = threading.Lock()
_orig_sdpa = F.scaled_dot_product_attention
_installed: bool = False


def _get_depth() -> int:
    return getattr(_tls, "depth", 0)


def configure(enabled: bool, repair_tau: float, min_seq: int) -> None:
    """Set the module-wide routing knobs (attention_router.py:25-28)."""
    globals()["enabled"] = bool(enabled)
    globals()["repair_tau"] = float(repair_tau)
    globals()["min_seq"] = int(min_seq)


def _extract_per_key_mask(attn_mask, B: int, Sk: int, device):
    """Reduce an SDPA mask to per-key form (attention_router.py:31-53).

    Returns (ok, key_mask [B, Sk] bool | None, key_bias [B, Sk] fp32 | None).  Accepted:
    None, or a 2-4 D tensor on `device` that broadcasts as [B or 1, 1, 1, Sk]; bool masks
    become key_mask, floating masks key_bias; anything else is not per-key (ok=False).
    """
    if attn_mask is None:
        return True, None, None
    if not isinstance(attn_mask, torch.Tensor) or attn_mask.device != device:
        return False, None, None
    if not 2 <= attn_mask.ndim <= 4:
        return False, None, None
    if attn_mask.shape[-2] != 1 or attn_mask.shape[-1] != Sk:
        return False, None, None
    shape4 = (1,) * (4 - attn_mask.ndim) + tuple(attn_mask.shape)
    if shape4[0] not in (1, B) or shape4[1] != 1:
        return False, None, None
    per_key = attn_mask.reshape(shape4).expand(B, 1, 1, Sk)[:, 0, 0, :]
    if per_key.dtype == torch.bool:
        return True, per_key.contiguous(), None
    if per_key.is_floating_point():
        return True, None, per_key.to(torch.float32).contiguous()
    return False, None, None


def routed_sdpa(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attn_mask: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    scale: float | None = None,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """SDPA-compatible entry point (attention_router.py:56-102)."""
    if (
        _get_depth() > 0
        and enabled
        and dropout_p == 0.0
        and not is_causal
        and not enable_gqa
        and isinstance(query, torch.Tensor)
        and isinstance(key, torch.Tensor)
        and isinstance(value, torch.Tensor)
        and query.shape[-1] == key.shape[-1] == value.shape[-1]
        and is_supported(query, key, value)
        and query.shape[2] >= min_seq
    ):
        ok, key_mask, key_bias = _extract_per_key_mask(attn_mask, query.shape[0], key.shape[2], query.device)
        if ok:
            return fp8_attention(query, key, value, scale=scale, key_mask=key_mask, key_bias=key_bias,
                                 repair_tau=repair_tau)
    return _orig_sdpa(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal,
                      scale=scale, enable_gqa=enable_gqa)


def install() -> None:
    """Patch F.scaled_dot_product_attention (and torch._C._nn's) once (attention_router.py:105-115)."""
    global _installed
    with _lock:
        if _installed:
            return
        F.scaled_dot_product_attention = routed_sdpa
        if hasattr(torch._C, "_nn") and hasattr(torch._C._nn, "scaled_dot_product_attention"):
            torch._C._nn.scaled_dot_product_attention = routed_sdpa
        _installed = True


def instrument_transformer(transformer):
    """Run transformer.forward inside a denoiser scope (attention_router.py:118-130)."""
    if getattr(transformer, "_denoiser_scope_instrumented", False):
        return transformer
    inner = transformer.forward

    @functools.wraps(inner)
    def _scoped_forward(*args, **kwargs):
        with denoiser_scope(transformer):
            return inner(*args, **kwargs)

    transformer.forward = _scoped_forward
    transformer._denoiser_scope_instrumented = True
    return transformer


@contextmanager
def denoiser_scope(transformer=None):
    """Thread-local nesting counter that enables routing (attention_router.py:133-139)."""
    _tls.depth = _get_depth() + 1
    try:
        yield transformer
    finally:
        _tls.depth = max(0, _get_depth() - 1)
