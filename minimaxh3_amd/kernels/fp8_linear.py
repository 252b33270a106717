"""Drop-in FP8 linear path (mirrors kernels/fp8_linear.py of the reference).

Same public surface: ``quantize_rows``, ``apply_lora_adapters``, ``FP8Linear`` (buffers
``w8``, ``w_scale``, ``bias``; attributes ``in_features``, ``out_features``, ``adapters``),
``find_primary_block_list`` and ``convert_transformer_to_fp8``.  The compute runs in the
gfx950 HIP kernels of ``minimaxh3_amd`` (per-row e4m3 quantizer, row-wise scaled FP8 GEMM
with the bias / LoRA / GELU-tanh epilogue fused); there is no fallback path.

Differences from the reference that do not change results: no padding of M to a
multiple of 16 (fp8_linear.py:91-93; the GEMM handles any M), and for bf16 inputs (the
DiT's dtype) one LoRA adapter runs inside the GEMM epilogue with the reference's three bf16
roundings instead of as separate bf16 matmuls + add.  Inputs of other dtypes apply their
adapters after the GEMM exactly as the reference does, since its final add happens in the
input's dtype; several adapters on bf16 inputs are concatenated along the rank, which
rounds their summed branch once instead of once per adapter.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import ops

ACT_NONE = 0
ACT_GELU_TANH = 1


def quantize_rows(x2d: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row dynamic e4m3 quantization (fp8_linear.py:27-42).

    Returns (x8 [M, K] float8_e4m3fn, x_scale [M, 1] fp32) with
    x_scale = max(max|row|, 1e-12) / 448 and x8 = e4m3(clamp(x / x_scale, +-448)).
    """
    if x2d.ndim != 2 or not x2d.is_cuda:
        raise ValueError("quantize_rows expects a 2D CUDA tensor")
    return ops.quant_rows(x2d)


def adaln_quantize_rows(
    x: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    eps: float = 1e-6,
    eager_rounding: bool = False,
    return_modulated: bool = False,
):
    """adaLN modulation fused with quantize_rows (an extension; no counterpart in the reference).

    For a DiT block's pre-linear input ``y = LayerNorm(x) * (1 + scale) + shift`` (LayerNorm
    without affine, ``x`` [B, S, C] bf16, adaLN ``shift`` / ``scale`` [B, C] bf16) this
    returns ``quantize_rows(y)`` -- (x8 [B*S, C] e4m3, x_scale [B*S, 1] fp32) -- reading x
    once, plus y [B*S, C] bf16 when ``return_modulated`` (needed by LoRA adapters).  y is
    rounded to bf16 once, as the fused pointwise code of a compiled block computes it, or
    after each op like torch's eager bf16 ops with ``eager_rounding``.  Feed the result to
    ``FP8Linear.forward_quantized``.
    """
    if x.ndim != 3 or not x.is_cuda:
        raise ValueError("adaln_quantize_rows expects a [B, S, C] CUDA tensor")
    x8, sa, y = ops.adaln_quant_rows(x, shift, scale, float(eps), bool(eager_rounding), bool(return_modulated))
    return (x8, sa, y) if return_modulated else (x8, sa)


def apply_lora_adapters(
    x: torch.Tensor,
    out: torch.Tensor,
    adapters: list[tuple[torch.Tensor, torch.Tensor, float]],
) -> torch.Tensor:
    """out + bf16(bf16(bf16(x A^T) B^T) * scale) for each adapter (fp8_linear.py:45-55).

    This generic form serves the bf16 ``nn.Linear`` modules that the LoRA registry wraps
    (runtime/lora.py:206-226); ``FP8Linear`` fuses the same branch into its GEMM.
    """
    if not adapters:
        return out
    for A, B, scale in adapters:
        branch = (x.to(A.dtype) @ A.t()) @ B.t()
        out = out + (branch * scale).to(out.dtype)
    return out


class FP8Linear(nn.Module):
    """nn.Linear replacement with e4m3 weights and per-output-channel scales (fp8_linear.py:58-108)."""

    def __init__(self, in_features: int, out_features: int) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.adapters: list[tuple[torch.Tensor, torch.Tensor, float]] = []
        self.act = ACT_NONE
        self._lora_cache_key = None
        self._lora_cache = None

    @classmethod
    @torch.no_grad()
    def from_linear(cls, linear: nn.Linear) -> "FP8Linear":
        """Quantize ``linear``'s weight per output channel and free it (fp8_linear.py:65-85)."""
        mod = cls(linear.in_features, linear.out_features)
        weight = linear.weight.detach()
        if not weight.is_cuda:
            weight = weight.cuda()
        w8, w_scale_col = quantize_rows(weight)
        mod.register_buffer("w8", w8)
        mod.register_buffer("w_scale", w_scale_col.view(1, -1).contiguous())
        bias = None
        if linear.bias is not None:
            bias = linear.bias.detach().to(device=w8.device, dtype=torch.bfloat16).contiguous()
        mod.register_buffer("bias", bias)
        if isinstance(getattr(linear, "adapters", None), list):
            mod.adapters = list(linear.adapters)
        linear.weight = None
        linear.bias = None
        return mod

    @classmethod
    @torch.no_grad()
    def from_quantized(cls, w8: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None,
                       device: torch.device | str | None = None) -> "FP8Linear":
        """FP8Linear from stored buffers: e4m3 codes ``w8 [N, K]``, per-output-channel fp32
        scales ``w_scale`` ([N] or [1, N]) and an optional bias [N] (stored as bf16).  These
        are the buffers ``from_linear`` computes; no quantization runs."""
        if w8.dtype != torch.float8_e4m3fn or w8.ndim != 2:
            raise ValueError("from_quantized: w8 must be a 2D float8_e4m3fn tensor")
        N, K = w8.shape
        if w_scale.dtype != torch.float32 or w_scale.numel() != N:
            raise ValueError(f"from_quantized: w_scale must hold {N} fp32 scales")
        if bias is not None and bias.numel() != N:
            raise ValueError(f"from_quantized: bias must hold {N} values")
        dev = torch.device(device) if device is not None else w8.device
        mod = cls(K, N)
        mod.register_buffer("w8", w8.to(dev).contiguous())
        mod.register_buffer("w_scale", w_scale.to(dev).reshape(1, N).contiguous())
        mod.register_buffer("bias", None if bias is None else bias.to(dev, torch.bfloat16).reshape(N).contiguous())
        return mod

    def _lora_ab(self):
        """(A, B, scale) of the fused epilogue, or None without adapters.

        One adapter is applied with exactly the reference's roundings.  Several adapters
        are concatenated along the rank with each scale folded into its B (bf16), which
        rounds the branch sum once instead of once per adapter.  Ranks are zero-padded to
        a multiple of 16 (the bf16 MFMA K step); the zero columns add nothing.
        """
        adapters = self.adapters
        if not adapters:
            return None
        if torch.compiler.is_compiling():
            # Traced (the reference compiles each block before LoRAs are appended,
            # runtime/model_manager.py:127-141 and runtime/lora.py:263-302): the operands are
            # built in the graph, which for one rank-aligned bf16 adapter is A and B as they
            # stand; the compiler's guards on the adapter list replace the cache below.
            return self._combine(adapters)
        # the key holds the adapter tensors themselves (an id() of a freed tensor can be
        # reused) and their in-place version counters
        key = [(A, B, float(s), A._version, B._version) for A, B, s in adapters]
        old = self._lora_cache_key
        hit = old is not None and len(old) == len(key) and all(
            o[0] is k[0] and o[1] is k[1] and o[2:] == k[2:] for o, k in zip(old, key))
        if not hit:
            self._lora_cache = self._combine(adapters)
            self._lora_cache_key = key
        return self._lora_cache

    def _lora_operands(self, x2d: torch.Tensor):
        """(t = bf16(x A^T), B, scale) for the fused epilogue, or (None, None, 0.0)."""
        ab = self._lora_ab()
        if ab is None:
            return None, None, 0.0
        a, b, scale = ab
        xb = x2d if x2d.dtype == torch.bfloat16 else x2d.to(torch.bfloat16)
        return ops.lora_down(xb, a), b, scale

    @classmethod
    def _combine(cls, adapters):
        """(A, B, scale) of the fused epilogue: one adapter as it is, several concatenated
        along the rank with each scale folded into its B; ranks zero-padded to 16."""
        if len(adapters) == 1:
            A, B, scale = adapters[0]
            a, b = cls._pad_rank(A.to(torch.bfloat16), B.to(torch.bfloat16))
        else:
            a = torch.cat([A.to(torch.bfloat16) for A, _, _ in adapters], 0)
            b = torch.cat([(B.float() * float(s)).to(torch.bfloat16) for _, B, s in adapters], 1)
            a, b = cls._pad_rank(a, b)
            scale = 1.0
        return a.contiguous(), b.contiguous(), float(scale)

    @staticmethod
    def _pad_rank(A: torch.Tensor, B: torch.Tensor):
        r = A.shape[0]
        rp = -(-r // 16) * 16
        if rp != r:
            A = torch.cat([A, A.new_zeros((rp - r, A.shape[1]))], 0)
            B = torch.cat([B, B.new_zeros((B.shape[0], rp - r))], 1)
        return A, B

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x2d = x.reshape(-1, self.in_features)
        if x.dtype != torch.bfloat16 and (self.adapters or self.act == ACT_GELU_TANH):
            # The reference converts the bf16 linear output to x's dtype and adds each LoRA
            # branch in that dtype (fp8_linear.py:105-108), and the FFN's tanh-GELU module
            # then acts in that dtype; the fused epilogue adds and rounds in bf16, so other
            # dtypes take the reference's sequence.
            x8, x_scale = quantize_rows(x2d)
            out = ops.gemm_rowwise(x8, self.w8, x_scale, self.w_scale, self.bias, ACT_NONE, None, None, 0.0)
            out = apply_lora_adapters(x2d, out.to(x.dtype), self.adapters)
            if self.act == ACT_GELU_TANH:
                out = torch.nn.functional.gelu(out, approximate="tanh")
            return out.reshape(*orig_shape[:-1], self.out_features)
        x8, x_scale = quantize_rows(x2d)
        lora_t, lora_b, lora_scale = self._lora_operands(x2d)
        out = ops.gemm_rowwise(x8, self.w8, x_scale, self.w_scale, self.bias, int(self.act), lora_t, lora_b,
                               lora_scale)
        return out.reshape(*orig_shape[:-1], self.out_features).to(x.dtype)

    def forward_qkv(self, x: torch.Tensor, heads: int, head_dim: int, key_stats: bool = True):
        """``forward`` of a fused QKV projection -- x [B, S, in] -> [B, S, 3 heads head_dim] with
        the q, k and v parts in that order, each head-major -- that also returns the column
        statistics its attention's K/V quantizers need (an extension with no counterpart in the
        reference; they replace the key mean and the V-scale pass of kernels/fp8_attention.py:
        338 and 140-155).  Returns (out, stats): pass stats as ``fp8_attention(..., kv_stats=)``
        with k and v the [B, H, S, D] views of out's k and v parts, and K and V are read once.
        With ``key_stats=False`` only the V statistics are taken (keys that are transformed
        after the projection, e.g. by a per-head norm or RoPE, need their own mean).

        The output equals ``forward(x)`` bit for bit.  Where the statistics epilogue does not
        apply (LoRA adapters or an activation on this module, a non-bf16 input, S < 128, or
        heads x head_dim not a multiple of 256) stats is None, which ``fp8_attention`` takes
        as "compute the statistics from k and v"."""
        if x.ndim != 3 or x.shape[2] != self.in_features:
            raise ValueError(f"forward_qkv: expected x [B, S, {self.in_features}]")
        B, S, _ = x.shape
        C = int(heads) * int(head_dim)
        if self.out_features != 3 * C:
            raise ValueError(f"forward_qkv: out_features {self.out_features} != 3 x {heads} x {head_dim}")
        if self.adapters or self.act != ACT_NONE or x.dtype != torch.bfloat16 or S < 128 or C % 256:
            return self.forward(x), None
        x8, x_scale = quantize_rows(x.reshape(-1, self.in_features))
        out, part = ops.gemm_rowwise_kv_stats(x8, self.w8, x_scale, self.w_scale, self.bias, S,
                                              C if key_stats else -1, 2 * C, C)
        from .fp8_attention import KVStats

        return out.reshape(B, S, self.out_features), KVStats(part, bool(key_stats))

    def forward_adaln(self, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6,
                      eager_rounding: bool = False) -> torch.Tensor:
        """``forward`` of the adaLN modulation y = LayerNorm(x) * (1 + scale) + shift of a DiT
        block's hidden state x [B, S, C] bf16 (shift / scale [B, C] bf16; an extension with
        no counterpart in the reference, see ``adaln_quantize_rows``) -> [B, S, N] bf16.  The
        modulation runs inside the activation quantizer; y reaches memory only when LoRA
        adapters need it for their down-projection.  Equals ``forward(y)`` bit for bit."""
        if x.ndim != 3 or x.shape[2] != self.in_features:
            raise ValueError(f"forward_adaln: expected x [B, S, {self.in_features}]")
        B, S, _ = x.shape
        lora = bool(self.adapters)
        x8, sa, y = ops.adaln_quant_rows(x, shift, scale, float(eps), bool(eager_rounding), lora)
        out = self.forward_quantized(x8, sa, y if lora else None)
        return out.reshape(B, S, self.out_features)

    def forward_quantized(self, x8: torch.Tensor, x_scale: torch.Tensor,
                          x_modulated: torch.Tensor | None = None) -> torch.Tensor:
        """``forward`` on an input quantized already (``adaln_quantize_rows``): x8 [M, K] e4m3,
        x_scale [M, 1] fp32 -> bf16 [M, N].  LoRA adapters read the bf16 input
        ``x_modulated`` [M, K] (``return_modulated=True``), as in ``forward``."""
        if x8.ndim != 2 or x8.shape[1] != self.in_features or x8.dtype != torch.float8_e4m3fn:
            raise ValueError(f"forward_quantized: expected e4m3 x8 [M, {self.in_features}]")
        if not x8.is_contiguous():
            raise ValueError("forward_quantized: x8 must be contiguous")
        M = x8.shape[0]
        if (x_scale.dtype != torch.float32 or x_scale.numel() != M or x_scale.device != x8.device
                or not x_scale.is_contiguous()):
            raise ValueError(f"forward_quantized: x_scale must hold {M} contiguous fp32 scales on {x8.device}")
        lora_t = lora_b = None
        lora_scale = 0.0
        if self.adapters:
            if x_modulated is None:
                raise ValueError("forward_quantized: LoRA adapters need the bf16 input (x_modulated)")
            lora_t, lora_b, lora_scale = self._lora_operands(x_modulated.reshape(-1, self.in_features))
        return ops.gemm_rowwise(x8, self.w8, x_scale, self.w_scale, self.bias, int(self.act), lora_t, lora_b,
                                lora_scale)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, act={self.act}"


def find_primary_block_list(transformer: nn.Module) -> tuple[str, nn.ModuleList]:
    """The longest non-empty ModuleList, preferring lists of one module type (fp8_linear.py:111-122)."""
    lists = [(n, m) for n, m in transformer.named_modules() if isinstance(m, nn.ModuleList) and len(m) > 0]
    if not lists:
        raise ValueError("No non-empty nn.ModuleList found in transformer")
    uniform = [(n, m) for n, m in lists if len({type(c) for c in m}) == 1]
    pool = uniform or lists
    return max(pool, key=lambda nm: len(nm[1]))


def _fuse_gelu_modules(block: nn.Module) -> None:
    """Fold a tanh-GELU activation module into its FP8 projection (GEMM epilogue).

    Matches the activation modules of diffusers-style FFNs: a module with a ``proj``
    sub-module and ``approximate == "tanh"`` whose forward is gelu_tanh(proj(x)).
    """
    for name, mod in list(block.named_modules()):
        proj = getattr(mod, "proj", None)
        if isinstance(proj, FP8Linear) and getattr(mod, "approximate", None) == "tanh" and proj.act == ACT_NONE:
            proj.act = ACT_GELU_TANH
            mod.forward = proj.forward  # the module's own forward would apply GELU a second time


def convert_transformer_to_fp8(
    transformer: nn.Module,
    exclude_patterns: str | list[str],
    keep_edge_blocks: int,
    fuse_gelu: bool = False,
) -> int:
    """Swap eligible nn.Linear modules of the primary blocks for FP8Linear (fp8_linear.py:125-162).

    Blocks [keep, n - keep) are converted; a Linear qualifies when in/out features are
    multiples of 16 and its lower-cased path contains none of the exclude patterns.
    Returns the number of converted modules.  ``fuse_gelu`` additionally folds tanh-GELU
    activations into the preceding FP8 GEMM (an extension; off by default).
    """
    if isinstance(exclude_patterns, str):
        exclude_patterns = exclude_patterns.split(",")
    patterns = [p.strip().lower() for p in exclude_patterns if p.strip()]
    list_name, blocks = find_primary_block_list(transformer)
    lo = max(0, int(keep_edge_blocks))
    hi = max(lo, len(blocks) - int(keep_edge_blocks))
    converted = 0
    for idx in range(lo, hi):
        block = blocks[idx]
        for sub_name, sub in list(block.named_modules()):
            if not isinstance(sub, nn.Linear):
                continue
            if sub.in_features % 16 or sub.out_features % 16:
                continue
            path = (f"{list_name}.{idx}.{sub_name}" if sub_name else f"{list_name}.{idx}").lower()
            if any(p in path for p in patterns):
                continue
            new = FP8Linear.from_linear(sub)
            if not sub_name:
                blocks[idx] = new
            else:
                parent_name, _, attr = sub_name.rpartition(".")
                parent = block.get_submodule(parent_name) if parent_name else block
                setattr(parent, attr, new)
            converted += 1
        if fuse_gelu:
            _fuse_gelu_modules(blocks[idx])
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return converted
