"""Drop-in FP8 attention path (mirrors kernels/fp8_attention.py of the reference).

Same public surface: ``LOG2E``, ``is_supported(q, k, v)`` and
``fp8_attention(q, k, v, scale=None, key_mask=None, key_bias=None, repair_tau=-1.0)``.
The Q / K / V quantizers and the flash-attention forward are gfx950 HIP kernels; there
is no fallback (unsupported inputs raise ValueError, like the reference).

One deliberate difference: the output is written through the strides of
``torch.empty_like(q)``, so a permuted (non-contiguous) query gives correct values in
its own layout (the reference stores contiguous [B,H,Sq,D] offsets into a buffer with
q's strides, fp8_attention.py:296 and 379, which is only right for contiguous q).
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from .. import ops
from .._native import require_gfx950

LOG2E = 1.4426950408889634


def _is_gfx950(device: torch.device) -> bool:
    try:
        require_gfx950(device)
        return True
    except RuntimeError:
        return False


def is_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Inputs the FP8 kernel accepts (fp8_attention.py:12-36).

    4-D GPU tensors on one device, all bf16 or all fp16, D in {64, 128}, equal [B, H]
    (no GQA), Sk == Sv > 0, Sq > 0, and a gfx950 device (in place of the reference's
    compute-capability >= (8, 9) test).
    """
    if not (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor)):
        return False
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if q.device != k.device or q.device != v.device:
        return False
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        return False
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    d = q.shape[-1]
    if d not in (64, 128) or k.shape[-1] != d or v.shape[-1] != d:
        return False
    if q.shape[:2] != k.shape[:2] or q.shape[:2] != v.shape[:2]:
        return False
    if k.shape[2] != v.shape[2] or q.shape[2] == 0 or k.shape[2] == 0:
        return False
    return _is_gfx950(q.device)


# Quantize Q inside the attention launch when q's layout allows it (ops.attn_fwd_q);
# False keeps the separate Q quantizer launch.  Both give the same output bit for bit.
fuse_q_quant = True


class KVStats(NamedTuple):
    """Column statistics of k and v from the QKV projection that produced them
    (``FP8Linear.forward_qkv``): ``part`` [2, ceil(B S / 128), H D] fp32 (key sums, value
    |max|), ``key`` False when only the value statistics are present."""

    part: torch.Tensor
    key: bool = True


def fp8_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float | None = None,
    key_mask: torch.Tensor | None = None,
    key_bias: torch.Tensor | None = None,
    repair_tau: float = -1.0,
    kv_stats: KVStats | None = None,
) -> torch.Tensor:
    """Non-causal FP8 attention over [B, H, S, D] tensors (fp8_attention.py:300-403).

    key_mask: bool [B, Sk] (True = attend) or None; key_bias: float [B, Sk] additive
    (natural log) bias or None, entries <= -1e8 mask the key; repair_tau < 0 disables the
    exact repair of large probabilities.  Returns [B, H, Sq, D] in q's dtype.
    kv_stats (an extension): the statistics ``FP8Linear.forward_qkv`` returned with the
    projection that k and v are views of; the K/V quantizers then read k and v once.
    """
    if not is_supported(q, k, v):
        raise ValueError("Unsupported inputs for fp8_attention")
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    c = ops.softmax_c(scale, D)
    if kv_stats is None:
        k8, sk, v8t, sv, _ = ops.attn_quant_kv(k, v)
    else:
        mean = None if kv_stats.key else ops.attn_kmean(k)
        k8, sk, v8t, sv, _ = ops.attn_quant_kv_gemm_stats(k, v, kv_stats.part, mean)
    if fuse_q_quant and ops.attn_fwd_q_supported(q):
        # the attention kernel quantizes Q itself (same codes and scales as attn_quant_q)
        return ops.attn_fwd_q(q, c, k8, v8t, sk, sv, key_mask, key_bias, float(repair_tau), Sk)
    q8, sq = ops.attn_quant_q(q, c)
    return ops.attn_fwd(q8, k8, v8t, sq, sk, sv, key_mask, key_bias, float(repair_tau), q, Sk)
