"""CPU baseline of the FP8 hot path (test infrastructure only: timed by bench.py's
cpu_baseline leg, never part of the product).

These are the torch CPU fallbacks the reference runs when the FP8 kernels do not apply:

* ``dequant_linear``  -- the fp32 dequant-matmul stand-in for ``torch._scaled_mm``
  (kernels/fp8_linear.py:95-102): ``(x8 * sa) @ (w8 * sw)^T + bias`` -> bf16.
* ``sdpa_fallback``   -- the original ``F.scaled_dot_product_attention`` that
  ``routed_sdpa`` calls for unsupported inputs (kernels/attention_router.py:93-102),
  here on fp32 dequantized Q/K/V.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def quantize_rows_torch(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row e4m3 quantization in torch CPU arithmetic (kernels/fp8_linear.py:20-22)."""
    s = x.float().abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / 448.0
    return (x.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), s


def dequant_linear(x8: torch.Tensor, sa: torch.Tensor, w8: torch.Tensor, sw: torch.Tensor,
                   bias: torch.Tensor | None) -> torch.Tensor:
    """bf16((x8 * sa) @ (w8 * sw)^T + bias) in fp32 on the CPU.

    x8 [M, K] / w8 [N, K] float8_e4m3fn, sa [M, 1] / sw [1, N] fp32, bias [N] or None.
    """
    a = x8.to(torch.float32) * sa.reshape(-1, 1)
    w = w8.to(torch.float32) * sw.reshape(-1, 1)
    out = a @ w.t()
    if bias is not None:
        out = out + bias.to(torch.float32)
    return out.to(torch.bfloat16)


def sdpa_fallback(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None) -> torch.Tensor:
    """Exact non-causal attention on the CPU in fp32 ([B, H, S, D] inputs)."""
    return F.scaled_dot_product_attention(q, k, v, scale=scale)
