"""Oracle for the FP8 linear path (test infrastructure only).

Restates kernels/fp8_linear.py of the reference:
* ``quantize_rows``      <- _quantize_rows_kernel / quantize_rows  (fp8_linear.py:8-24, 27-42)
* ``scaled_mm``          <- the torch._scaled_mm call             (fp8_linear.py:95-102)
* ``lora_branch_add``    <- apply_lora_adapters                    (fp8_linear.py:45-55)
* ``gelu_tanh``          <- the tanh-GELU that follows the MLP-up linear in the DiT FFN
* ``fp8_linear_forward`` <- FP8Linear.forward                      (fp8_linear.py:87-108)
* ``adaln_modulate``     <- the DiT block's adaLN input to its QKV / MLP-up linears:
  LayerNorm without affine, then x * (1 + scale) + shift (diffusers' AdaLayerNorm, a
  dependency the reference does not vendor, model_manager.py:79-103); the values feed
  FP8Linear.forward's quantize_rows (fp8_linear.py:94).  Pinned against torch's own
  layer_norm and bf16 ops in tests/test_oracle_linear.py.
"""
from __future__ import annotations

import numpy as np

from .mfma import mfma_f8_dot
from .numerics import E4M3_MAX, absmax_maxnum, bf16_round, clamp448_maxnum, e4m3_decode, e4m3_encode

F32 = np.float32


def quantize_rows(x):
    """Per-row dynamic e4m3 quantization (fp8_linear.py:16-24).

    x: [M, K] values (fp32 view of the bf16/fp16/fp32 input).
    Returns (codes uint8 [M, K], scale fp32 [M, 1]):
      scale = max(max_k |x|, 1e-12) / 448            (fp32, IEEE division, line 21)
      code  = e4m3(clamp(x / scale, -448, 448))      (fp32 IEEE division, line 22)
    """
    x = np.asarray(x, dtype=F32)
    if x.ndim != 2:
        raise ValueError("quantize_rows expects a 2D array")
    M, K = x.shape
    if K == 0:
        return np.zeros((M, 0), np.uint8), np.full((M, 1), F32(1e-12) / F32(E4M3_MAX), F32)
    amax = absmax_maxnum(x, axis=1)
    scale = (np.fmax(amax, F32(1e-12)) / F32(E4M3_MAX)).astype(F32)
    with np.errstate(invalid="ignore"):  # inf / inf -> NaN, clamped below
        q = (x / scale[:, None]).astype(F32)
    return e4m3_encode(clamp448_maxnum(q)), scale.reshape(M, 1)


def scaled_mm(x8, w8, sa, sw, bias=None, dot="exact"):
    """Row-wise scaled FP8 GEMM, fp32-exact accumulate (fp8_linear.py:95-102).

    out[m, n] = (sum_k dec(x8[m,k]) * dec(w8[n,k])) * sa[m] * sw[n] + bias[n]
    x8 [M,K] codes, w8 [N,K] codes, sa [M] or [M,1], sw [N] or [1,N], bias [N] or None.
    Returns fp32 [M, N] before the bf16 cast (products of e4m3 values are exact in
    fp32; the sum is done in float64, the epilogue order of torch._scaled_mm is not
    fixed by the reference).  ``dot="mfma"`` forms the sum as the gfx950 fp8 matrix
    instruction accumulates it (oracle.mfma) instead; the epilogue is the same.
    """
    if dot not in ("exact", "mfma"):
        raise ValueError(f"scaled_mm: dot must be 'exact' or 'mfma', got {dot!r}")
    a = e4m3_decode(x8).astype(np.float64)
    b = e4m3_decode(w8).astype(np.float64)
    acc = a @ b.T if dot == "exact" else mfma_f8_dot(a, b).astype(np.float64)
    out = acc * np.asarray(sa, np.float64).reshape(-1, 1) * np.asarray(sw, np.float64).reshape(1, -1)
    if bias is not None:
        out = out + np.asarray(bias, np.float64).reshape(1, -1)
    return out.astype(F32)


def gelu_tanh(z):
    """0.5 z (1 + tanh(sqrt(2/pi) (z + 0.044715 z^3))), evaluated in float64."""
    z = np.asarray(z, np.float64)
    return (0.5 * z * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (z + 0.044715 * z ** 3)))).astype(F32)


def _round_to(dtype):
    """Rounding to the stored dtype of an output: "bf16" or "fp16" (values kept as fp32)."""
    if dtype == "bf16":
        return bf16_round
    if dtype == "fp16":
        return lambda a: np.asarray(a, F32).astype(np.float16).astype(F32)
    raise ValueError(dtype)


def lora_branch_add(x, out, adapters, out_dtype="bf16"):
    """apply_lora_adapters (fp8_linear.py:45-55) with torch's bf16 matmul rounding.

    For each (A [r,K], B [N,r], scale): branch = bf16(bf16(bf16(x@A^T) @ B^T) * scale) (x is
    converted to A's dtype, bf16, line 53), converted to out's dtype and added in it (line 54):
    out = r(out + r(branch)) with r the rounding to ``out_dtype`` (bf16 or fp16; the linear
    output reaches that dtype through ``.to(x.dtype)``, line 107).  x, A, B are fp32 arrays;
    matmuls accumulate in float64 then round to bf16.
    """
    rnd = _round_to(out_dtype)
    out = rnd(out)
    x = bf16_round(x).astype(np.float64)
    for A, B, scale in adapters:
        t = bf16_round((x @ np.asarray(A, np.float64).T).astype(F32))
        branch = bf16_round((t.astype(np.float64) @ np.asarray(B, np.float64).T).astype(F32))
        branch = bf16_round((branch * F32(scale)).astype(F32))
        out = rnd((out + rnd(branch)).astype(F32))
    return out


def fp8_linear_forward(x, w8, w_scale, bias=None, adapters=(), gelu=False, in_dtype="bf16"):
    """FP8Linear.forward (fp8_linear.py:87-108) on [M, K] inputs of ``in_dtype`` (bf16 or fp16
    values), the result as fp32 holding values of that dtype.

    Padding M to a multiple of 16 (lines 91-93) only adds zero rows whose outputs are
    sliced away (line 106), so it does not change any kept value and is not modelled.  The
    bf16 linear output is converted to the input's dtype (line 107) before the LoRA adds.
    ``gelu`` applies the tanh-GELU of the following FFN activation after the LoRA add, rounded
    to that dtype.
    """
    rnd = _round_to(in_dtype)
    x = rnd(np.asarray(x, F32))
    x8, sa = quantize_rows(x)
    out = rnd(bf16_round(scaled_mm(x8, w8, sa, w_scale, bias)))
    out = lora_branch_add(x, out, adapters, in_dtype) if adapters else out
    if gelu:
        out = rnd(gelu_tanh(out))
    return out


def adaln_modulate(x, shift, scale, S, eps=1e-6, eager=False):
    """y = LayerNorm(x) * (1 + scale_b) + shift_b for x [M, C], rows of batch item b = m // S.

    LayerNorm has no affine: n = (x - mean) / sqrt(var + eps), biased variance, in float64.
    shift, scale: [B, C] bf16 values.  ``eager=False``: y rounded to bf16 once (the fused
    pointwise code of a compiled block).  ``eager=True``: torch's eager bf16 op sequence,
    n -> bf16, (1 + scale) -> bf16, product -> bf16, sum -> bf16 (each op computed in fp32
    and rounded, which float64 products / sums of bf16 values cast to fp32 reproduce).
    Returns y as fp32 holding bf16 values.
    """
    x = np.asarray(x, np.float64)
    M, C = x.shape
    b = np.arange(M) // S
    sh = np.asarray(shift, np.float64)[b]
    sc = np.asarray(scale, np.float64)[b]
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    n = (x - mean) / np.sqrt(var + eps)
    if not eager:
        return bf16_round((n * (1.0 + sc) + sh).astype(F32))
    nb = bf16_round(n.astype(F32)).astype(np.float64)
    op = bf16_round((1.0 + sc).astype(F32)).astype(np.float64)
    prod = bf16_round((nb * op).astype(F32)).astype(np.float64)
    return bf16_round((prod + sh).astype(F32))
