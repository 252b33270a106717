"""torch custom ops over libmxf8 (one per C-ABI entry point), with fake (meta) kernels.

Registering the launches as ``torch.library.custom_op`` keeps the FP8 path opaque to
torch.compile: the DiT blocks are compiled with ``fullgraph=False``
(runtime/model_manager.py:127-141) and these ops trace as single nodes without graph
breaks.  Outputs come from torch's caching allocator; launches go to the current stream.
"""
from __future__ import annotations

import math

import torch

from . import _native as N

E4M3 = torch.float8_e4m3fn


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _prep(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what}: expected a GPU tensor")
    N.require_gfx950(t.device)


def _on(t: torch.Tensor | None, device: torch.device, what: str) -> None:
    if t is not None and t.device != device:
        raise ValueError(f"{what} must be on {device}, got {t.device}")


def _check_kv_codes(k8: torch.Tensor, v8t: torch.Tensor, sk: torch.Tensor, sv: torch.Tensor, B: int, H: int,
                    Sk: int, D: int, device: torch.device, what: str) -> None:
    """The kernels address K8 / V8T / sK through Sk alone (ceil(Sk/128)*128 padded keys per
    head), so the codes must have exactly the layout attn_quant_k / attn_quant_v give for Sk
    keys: a larger Sk would read past them, a smaller one would misplace every head."""
    Skp = _cdiv(Sk, 128) * 128
    want = ((k8, (B, H, Skp, D), E4M3, "k8"), (v8t, (B, H, D, Skp), E4M3, "v8t"),
            (sk, (B, H, Skp // 128), torch.float32, "sk"), (sv, (B, H, D), torch.float32, "sv"))
    for t, shape, dtype, name in want:
        if tuple(t.shape) != shape or t.dtype != dtype or not t.is_contiguous():
            raise ValueError(f"{what}: {name} must be a contiguous {dtype} tensor of shape {shape} for Sk={Sk}, "
                             f"got {t.dtype} {tuple(t.shape)}")
        _on(t, device, f"{what}: {name}")


def key_operands(key_mask: torch.Tensor | None, key_bias: torch.Tensor | None, B: int, Sk: int,
                 device: torch.device) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """The kernel's per-key operands: a mask as uint8 [B, Sk] (nonzero = keep, the truth value
    of the reference's ``key_mask.to(torch.bool)``, fp8_attention.py:374) and a bias as fp32
    [B, Sk] (375).  Either may hold B*Sk values or Sk values shared by every batch item; it
    must be on the attention's device (ValueError otherwise)."""
    out = []
    for t, dt, name in ((key_mask, torch.bool, "key_mask"), (key_bias, torch.float32, "key_bias")):
        if t is None:
            out.append(None)
            continue
        _on(t, device, name)
        t = t.to(dt)
        if t.numel() == B * Sk:
            t = t.reshape(B, Sk)
        elif t.numel() == Sk:
            t = t.reshape(1, Sk).expand(B, Sk)
        else:
            raise ValueError(f"{name} must hold B*Sk = {B * Sk} (or Sk = {Sk}) values, got shape {tuple(t.shape)}")
        t = t.contiguous()
        out.append(t.view(torch.uint8) if dt == torch.bool else t)
    return out[0], out[1]


# ---------------------------------------------------------------------------------------
# FP8 linear
# ---------------------------------------------------------------------------------------

@torch.library.custom_op("mxf8::quant_rows", mutates_args=())
def quant_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[M, K] bf16/fp16/fp32 -> (e4m3 [M, K], fp32 scale [M, 1]) (kernels/fp8_linear.py:27-42)."""
    _prep(x, "quant_rows")
    if x.stride(1) != 1 or x.stride(0) < x.shape[1]:
        x = x.contiguous()
    M, K = x.shape
    x8 = torch.empty((M, K), dtype=E4M3, device=x.device)
    scale = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    if M > 0:
        with torch.cuda.device(x.device):
            N.check(N.load().mxf8_quant_rows(x.data_ptr(), N.dtype_code(x.dtype), M, K, max(x.stride(0), K),
                                             x8.data_ptr(), scale.data_ptr(), N.stream_of(x)), "quant_rows")
    return x8, scale


@quant_rows.register_fake
def _(x):
    M, K = x.shape
    return x.new_empty((M, K), dtype=E4M3), x.new_empty((M, 1), dtype=torch.float32)


@torch.library.custom_op("mxf8::adaln_quant_rows", mutates_args=())
def adaln_quant_rows(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float, eager: bool,
                     want_y: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """adaLN modulation + per-row e4m3 quantization in one pass.

    x [B, S, C] bf16, shift / scale [B, C] bf16 -> (x8 [B*S, C] e4m3, sa [B*S, 1] fp32,
    y [B*S, C] bf16 or an empty tensor) with y = LN(x) * (1 + scale) + shift rounded to bf16
    once (``eager=False``) or after every op like torch's eager bf16 ops (``eager=True``),
    and (x8, sa) = quant_rows(y).
    """
    _prep(x, "adaln_quant_rows")
    if x.ndim != 3 or shift.shape != (x.shape[0], x.shape[2]) or scale.shape != shift.shape:
        raise ValueError("adaln_quant_rows: expected x [B, S, C] and shift, scale [B, C]")
    if x.dtype != torch.bfloat16 or shift.dtype != torch.bfloat16 or scale.dtype != torch.bfloat16:
        raise ValueError("adaln_quant_rows: bf16 tensors expected")
    B, S, C = x.shape
    x2 = x.reshape(B * S, C)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    # one row stride for both (expanded / strided operands are copied)
    if shift.stride(1) != 1 or shift.stride(0) < C or shift.stride(0) % 8:
        shift = shift.contiguous()
    if scale.stride(1) != 1 or scale.stride(0) != shift.stride(0):
        scale = scale.contiguous()
        if scale.stride(0) != shift.stride(0):
            shift = shift.contiguous()
    M = B * S
    x8 = torch.empty((M, C), dtype=E4M3, device=x.device)
    sa = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    y = torch.empty((M, C) if want_y else (0,), dtype=torch.bfloat16, device=x.device)
    if M > 0:
        with torch.cuda.device(x.device):
            N.check(N.load().mxf8_adaln_quant_rows(
                x2.data_ptr(), M, C, x2.stride(0), S, shift.data_ptr(), scale.data_ptr(), shift.stride(0),
                float(eps), int(bool(eager)), x8.data_ptr(), sa.data_ptr(), y.data_ptr() if want_y else None,
                N.stream_of(x)), "adaln_quant_rows")
    return x8, sa, y


@adaln_quant_rows.register_fake
def _(x, shift, scale, eps, eager, want_y):
    B, S, C = x.shape
    return (x.new_empty((B * S, C), dtype=E4M3), x.new_empty((B * S, 1), dtype=torch.float32),
            x.new_empty((B * S, C) if want_y else (0,), dtype=torch.bfloat16))


@torch.library.custom_op("mxf8::gemm_rowwise", mutates_args=())
def gemm_rowwise(a8: torch.Tensor, w8: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor,
                 bias: torch.Tensor | None, act: int, lora_t: torch.Tensor | None,
                 lora_b: torch.Tensor | None, lora_scale: float) -> torch.Tensor:
    """bf16(a8 w8^T * sa * sw + bias) (+ LoRA) (+ GELU-tanh), bf16 [M, N]."""
    _prep(a8, "gemm_rowwise")
    M, K = a8.shape
    Nn = w8.shape[0]
    dev = a8.device
    if a8.dtype != E4M3 or w8.dtype != E4M3 or w8.dim() != 2 or w8.shape[1] != K:
        raise ValueError(f"gemm_rowwise: e4m3 a8 [M, K] and w8 [N, K] expected, got {a8.dtype} {tuple(a8.shape)} "
                         f"and {w8.dtype} {tuple(w8.shape)}")
    if not (a8.is_contiguous() and w8.is_contiguous()):
        raise ValueError("gemm_rowwise: a8 and w8 must be contiguous")
    if sa.dtype != torch.float32 or sa.numel() != M or sw.dtype != torch.float32 or sw.numel() != Nn:
        raise ValueError(f"gemm_rowwise: fp32 scales of {M} rows and {Nn} channels expected")
    if not (sa.is_contiguous() and sw.is_contiguous()):
        raise ValueError("gemm_rowwise: scales must be contiguous")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != Nn or not bias.is_contiguous()):
        raise ValueError(f"gemm_rowwise: bias must be {Nn} contiguous bf16 values")
    if lora_t is not None and (lora_b is None or lora_t.shape[0] != M or lora_b.shape != (Nn, lora_t.shape[1])
                               or not lora_t.is_contiguous() or not lora_b.is_contiguous()):
        raise ValueError("gemm_rowwise: LoRA operands t [M, r] and B [N, r] (contiguous bf16) expected")
    for t, name in ((w8, "w8"), (sa, "sa"), (sw, "sw"), (bias, "bias"), (lora_t, "lora_t"), (lora_b, "lora_b")):
        _on(t, dev, f"gemm_rowwise: {name}")
    out = torch.empty((M, Nn), dtype=torch.bfloat16, device=a8.device)
    if M == 0 or Nn == 0:
        return out
    r = 0 if lora_t is None else lora_t.shape[1]
    with torch.cuda.device(a8.device):
        N.check(N.load().mxf8_gemm_rowwise(
            a8.data_ptr(), w8.data_ptr(), sa.data_ptr(), sw.data_ptr(), N.ptr(bias), int(act),
            N.ptr(lora_t), N.ptr(lora_b), r, float(lora_scale), out.data_ptr(), M, Nn, K, Nn,
            N.stream_of(a8)), "gemm_rowwise")
    return out


@gemm_rowwise.register_fake
def _(a8, w8, sa, sw, bias, act, lora_t, lora_b, lora_scale):
    return a8.new_empty((a8.shape[0], w8.shape[0]), dtype=torch.bfloat16)


def kv_stats_shape(M: int, C: int) -> tuple[int, int, int]:
    """Shape of the K/V column statistics of gemm_rowwise_kv_stats: [2, ceil(M/128), C]
    (key sums, value |max|; 128-row block; column)."""
    return (2, _cdiv(M, 128), C)


@torch.library.custom_op("mxf8::gemm_rowwise_kv_stats", mutates_args=())
def gemm_rowwise_kv_stats(a8: torch.Tensor, w8: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor,
                          bias: torch.Tensor | None, seq_len: int, k_col0: int, v_col0: int,
                          cols: int) -> tuple[torch.Tensor, torch.Tensor]:
    """gemm_rowwise (no LoRA, no activation) of a fused QKV projection, plus the column
    statistics its attention's K/V quantizers need: per-channel sums of the key columns
    [k_col0, k_col0 + cols) and |max| of the value columns [v_col0, v_col0 + cols) (-1: none)
    over each batch item's seq_len rows (kernels/fp8_attention.py:338, 140-155).  Returns
    (out [M, N] bf16, equal to gemm_rowwise's bit for bit, stats [2, ceil(M/128), cols]: the
    statistic of every 128-row block inside one batch item; the other blocks' entries are
    not written)."""
    _prep(a8, "gemm_rowwise_kv_stats")
    M, K = a8.shape
    Nn = w8.shape[0]
    if a8.dtype != E4M3 or w8.dtype != E4M3 or w8.dim() != 2 or w8.shape[1] != K:
        raise ValueError("gemm_rowwise_kv_stats: e4m3 a8 [M, K] and w8 [N, K] expected")
    if not (a8.is_contiguous() and w8.is_contiguous() and sa.is_contiguous() and sw.is_contiguous()):
        raise ValueError("gemm_rowwise_kv_stats: operands must be contiguous")
    if sa.dtype != torch.float32 or sa.numel() != M or sw.dtype != torch.float32 or sw.numel() != Nn:
        raise ValueError(f"gemm_rowwise_kv_stats: fp32 scales of {M} rows and {Nn} channels expected")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != Nn or not bias.is_contiguous()):
        raise ValueError(f"gemm_rowwise_kv_stats: bias must be {Nn} contiguous bf16 values")
    for t, name in ((w8, "w8"), (sa, "sa"), (sw, "sw"), (bias, "bias")):
        _on(t, a8.device, f"gemm_rowwise_kv_stats: {name}")
    out = torch.empty((M, Nn), dtype=torch.bfloat16, device=a8.device)
    stats = torch.empty(kv_stats_shape(M, cols), dtype=torch.float32, device=a8.device)
    with torch.cuda.device(a8.device):
        N.check(N.load().mxf8_gemm_rowwise_kv_stats(
            a8.data_ptr(), w8.data_ptr(), sa.data_ptr(), sw.data_ptr(), N.ptr(bias), out.data_ptr(), M, Nn, K, Nn,
            int(seq_len), int(k_col0), int(v_col0), int(cols), stats.data_ptr(), N.stream_of(a8)),
            "gemm_rowwise_kv_stats")
    return out, stats


@gemm_rowwise_kv_stats.register_fake
def _(a8, w8, sa, sw, bias, seq_len, k_col0, v_col0, cols):
    return (a8.new_empty((a8.shape[0], w8.shape[0]), dtype=torch.bfloat16),
            a8.new_empty(kv_stats_shape(a8.shape[0], cols), dtype=torch.float32))


@torch.library.custom_op("mxf8::lora_down", mutates_args=())
def lora_down(x: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
    """t = bf16(x A^T): x [M, K] bf16, A [r, K] bf16 -> [M, r] bf16 (kernels/fp8_linear.py:53)."""
    _prep(x, "lora_down")
    if x.stride(1) != 1:
        x = x.contiguous()
    a = a.contiguous()
    M, K = x.shape
    r = a.shape[0]
    t = torch.empty((M, r), dtype=torch.bfloat16, device=x.device)
    if M > 0:
        with torch.cuda.device(x.device):
            N.check(N.load().mxf8_lora_down(x.data_ptr(), x.stride(0), a.data_ptr(), t.data_ptr(), M, K, r,
                                            N.stream_of(x)), "lora_down")
    return t


@lora_down.register_fake
def _(x, a):
    return x.new_empty((x.shape[0], a.shape[0]), dtype=torch.bfloat16)


# ---------------------------------------------------------------------------------------
# FP8 attention
# ---------------------------------------------------------------------------------------

def _workspace(B: int, H: int, Sq: int, Sk: int, D: int, device) -> torch.Tensor:
    n = int(N.load().mxf8_attn_workspace_bytes(B, H, Sq, Sk, D))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


@torch.library.custom_op("mxf8::attn_quant_q", mutates_args=())
def attn_quant_q(q: torch.Tensor, c: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(q * c) -> Q8 [B,H,ceil(Sq/128)*128,D] e4m3 + sq [B,H,ceil(Sq/128)] (fp8_attention.py:39-77)."""
    _prep(q, "attn_quant_q")
    B, H, S, D = q.shape
    nq = _cdiv(S, 128)
    q8 = torch.empty((B, H, nq * 128, D), dtype=E4M3, device=q.device)
    sq = torch.empty((B, H, nq), dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        N.check(N.load().mxf8_attn_quant_q(q.data_ptr(), N.dtype_code(q.dtype), N.strides4(q), B, H, S, D,
                                           float(c), q8.data_ptr(), sq.data_ptr(), N.stream_of(q)), "attn_quant_q")
    return q8, sq


@attn_quant_q.register_fake
def _(q, c):
    B, H, S, D = q.shape
    nq = _cdiv(S, 128)
    return q.new_empty((B, H, nq * 128, D), dtype=E4M3), q.new_empty((B, H, nq), dtype=torch.float32)


@torch.library.custom_op("mxf8::attn_kmean", mutates_args=())
def attn_kmean(k: torch.Tensor) -> torch.Tensor:
    """Mean of fp32(k) over the key axis, [B, H, D] fp32 (fp8_attention.py:338)."""
    _prep(k, "attn_kmean")
    B, H, S, D = k.shape
    mean = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    ws = _workspace(B, H, S, S, D, k.device)
    with torch.cuda.device(k.device):
        N.check(N.load().mxf8_attn_kmean(k.data_ptr(), N.dtype_code(k.dtype), N.strides4(k), B, H, S, D,
                                         mean.data_ptr(), ws.data_ptr(), N.stream_of(k)), "attn_kmean")
    return mean


@attn_kmean.register_fake
def _(k):
    B, H, S, D = k.shape
    return k.new_empty((B, H, D), dtype=torch.float32)


@torch.library.custom_op("mxf8::attn_quant_k", mutates_args=())
def attn_quant_k(k: torch.Tensor, mean: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(k - mean) -> K8 [B,H,ceil(Sk/128)*128,D] e4m3 + sk [B,H,ceil(Sk/128)] (fp8_attention.py:80-119)."""
    _prep(k, "attn_quant_k")
    B, H, S, D = k.shape
    nk = _cdiv(S, 128)
    mean = mean.to(torch.float32).contiguous()
    k8 = torch.empty((B, H, nk * 128, D), dtype=E4M3, device=k.device)
    sk = torch.empty((B, H, nk), dtype=torch.float32, device=k.device)
    with torch.cuda.device(k.device):
        N.check(N.load().mxf8_attn_quant_k(k.data_ptr(), N.dtype_code(k.dtype), N.strides4(k), mean.data_ptr(),
                                           B, H, S, D, k8.data_ptr(), sk.data_ptr(), N.stream_of(k)), "attn_quant_k")
    return k8, sk


@attn_quant_k.register_fake
def _(k, mean):
    B, H, S, D = k.shape
    nk = _cdiv(S, 128)
    return k.new_empty((B, H, nk * 128, D), dtype=E4M3), k.new_empty((B, H, nk), dtype=torch.float32)


@torch.library.custom_op("mxf8::attn_quant_v", mutates_args=())
def attn_quant_v(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """v -> V8T [B,H,D,ceil(Sk/128)*128] e4m3 (transposed) + sv [B,H,D] (fp8_attention.py:122-170)."""
    _prep(v, "attn_quant_v")
    B, H, S, D = v.shape
    nk = _cdiv(S, 128)
    v8t = torch.empty((B, H, D, nk * 128), dtype=E4M3, device=v.device)
    sv = torch.empty((B, H, D), dtype=torch.float32, device=v.device)
    ws = _workspace(B, H, S, S, D, v.device)
    with torch.cuda.device(v.device):
        N.check(N.load().mxf8_attn_quant_v(v.data_ptr(), N.dtype_code(v.dtype), N.strides4(v), B, H, S, D,
                                           v8t.data_ptr(), sv.data_ptr(), ws.data_ptr(), N.stream_of(v)),
                "attn_quant_v")
    return v8t, sv


@attn_quant_v.register_fake
def _(v):
    B, H, S, D = v.shape
    nk = _cdiv(S, 128)
    return v.new_empty((B, H, D, nk * 128), dtype=E4M3), v.new_empty((B, H, D), dtype=torch.float32)


@torch.library.custom_op("mxf8::attn_quant_kv", mutates_args=())
def attn_quant_kv(k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                                            torch.Tensor]:
    """K and V quantized together (fp8_attention.py:338-369): (K8 [B,H,Skp,D], sk [B,H,nk],
    V8T [B,H,D,Skp], sv [B,H,D], key mean [B,H,D] fp32) -- the outputs of attn_kmean +
    attn_quant_k + attn_quant_v in three launches."""
    _prep(k, "attn_quant_kv")
    if k.shape != v.shape or k.dtype != v.dtype or k.device != v.device:
        raise ValueError("attn_quant_kv: k and v must have one shape, dtype and device")
    B, H, S, D = k.shape
    nk = _cdiv(S, 128)
    k8 = torch.empty((B, H, nk * 128, D), dtype=E4M3, device=k.device)
    sk = torch.empty((B, H, nk), dtype=torch.float32, device=k.device)
    v8t = torch.empty((B, H, D, nk * 128), dtype=E4M3, device=k.device)
    sv = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    mean = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    ws = torch.empty(max(int(N.load().mxf8_attn_kv_workspace_bytes(B, H, S, D)), 16), dtype=torch.uint8,
                     device=k.device)
    with torch.cuda.device(k.device):
        N.check(N.load().mxf8_attn_quant_kv(
            k.data_ptr(), N.strides4(k), v.data_ptr(), N.strides4(v), N.dtype_code(k.dtype), B, H, S, D,
            k8.data_ptr(), sk.data_ptr(), v8t.data_ptr(), sv.data_ptr(), mean.data_ptr(), ws.data_ptr(),
            N.stream_of(k)), "attn_quant_kv")
    return k8, sk, v8t, sv, mean


@attn_quant_kv.register_fake
def _(k, v):
    B, H, S, D = k.shape
    nk = _cdiv(S, 128)
    f32 = torch.float32
    return (k.new_empty((B, H, nk * 128, D), dtype=E4M3), k.new_empty((B, H, nk), dtype=f32),
            k.new_empty((B, H, D, nk * 128), dtype=E4M3), k.new_empty((B, H, D), dtype=f32),
            k.new_empty((B, H, D), dtype=f32))


@torch.library.custom_op("mxf8::attn_quant_kv_gemm_stats", mutates_args=())
def attn_quant_kv_gemm_stats(k: torch.Tensor, v: torch.Tensor, stats: torch.Tensor,
                             key_mean: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                     torch.Tensor, torch.Tensor]:
    """attn_quant_kv for k, v [B, H, S, D] that are views of a gemm_rowwise_kv_stats output,
    from its statistics: one fold launch and one quantizing pass (K and V read once).  With
    ``key_mean`` [B, H, D] fp32 given, the key mean is that (e.g. of keys transformed after
    the projection) and only the V statistics come from ``stats``.  Same outputs as
    attn_quant_kv: (K8, sk, V8T, sv, key mean)."""
    _prep(k, "attn_quant_kv_gemm_stats")
    if k.shape != v.shape or k.dtype != v.dtype or k.device != v.device:
        raise ValueError("attn_quant_kv_gemm_stats: k and v must have one shape, dtype and device")
    B, H, S, D = k.shape
    _on(stats, k.device, "attn_quant_kv_gemm_stats: stats")
    if stats.dtype != torch.float32 or tuple(stats.shape) != kv_stats_shape(B * S, H * D) or not stats.is_contiguous():
        raise ValueError(f"attn_quant_kv_gemm_stats: stats must be contiguous fp32 {kv_stats_shape(B * S, H * D)}, "
                         f"got {stats.dtype} {tuple(stats.shape)}")
    nk = _cdiv(S, 128)
    k8 = torch.empty((B, H, nk * 128, D), dtype=E4M3, device=k.device)
    sk = torch.empty((B, H, nk), dtype=torch.float32, device=k.device)
    v8t = torch.empty((B, H, D, nk * 128), dtype=E4M3, device=k.device)
    sv = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    if key_mean is None:
        mean = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    else:
        _on(key_mean, k.device, "attn_quant_kv_gemm_stats: key_mean")
        if key_mean.numel() != B * H * D:
            raise ValueError(f"attn_quant_kv_gemm_stats: key_mean must hold B*H*D = {B * H * D} values")
        mean = key_mean.to(torch.float32).reshape(B, H, D).clone()
    with torch.cuda.device(k.device):
        N.check(N.load().mxf8_attn_quant_kv_gemm_stats(
            k.data_ptr(), N.strides4(k), v.data_ptr(), N.strides4(v), N.dtype_code(k.dtype), B, H, S, D,
            stats.data_ptr(), int(key_mean is None), k8.data_ptr(), sk.data_ptr(), v8t.data_ptr(), sv.data_ptr(),
            mean.data_ptr(), N.stream_of(k)), "attn_quant_kv_gemm_stats")
    return k8, sk, v8t, sv, mean


@attn_quant_kv_gemm_stats.register_fake
def _(k, v, stats, key_mean):
    B, H, S, D = k.shape
    nk = _cdiv(S, 128)
    f32 = torch.float32
    return (k.new_empty((B, H, nk * 128, D), dtype=E4M3), k.new_empty((B, H, nk), dtype=f32),
            k.new_empty((B, H, D, nk * 128), dtype=E4M3), k.new_empty((B, H, D), dtype=f32),
            k.new_empty((B, H, D), dtype=f32))


@torch.library.custom_op("mxf8::attn_fwd", mutates_args=())
def attn_fwd(q8: torch.Tensor, k8: torch.Tensor, v8t: torch.Tensor, sq: torch.Tensor, sk: torch.Tensor,
             sv: torch.Tensor, key_mask: torch.Tensor | None, key_bias: torch.Tensor | None, repair_tau: float,
             like: torch.Tensor, Sk: int, kv_mode: int = 0) -> torch.Tensor:
    """FP8 flash-attention forward (fp8_attention.py:185-297).

    ``like`` is the original query: the output has its shape, dtype and strides (the
    kernel writes through the strides, so permuted query layouts stay correct).  kv_mode
    0 holds a head's K/V in LDS when they fit (Sk <= 512 at D = 128, no repair), 1 always
    streams K/V tiles; both give the same bits.
    """
    _prep(q8, "attn_fwd")
    B, H, Sq, D = like.shape
    nq = _cdiv(Sq, 128)
    if (tuple(q8.shape) != (B, H, nq * 128, D) or q8.dtype != E4M3 or not q8.is_contiguous()
            or tuple(sq.shape) != (B, H, nq) or sq.dtype != torch.float32 or not sq.is_contiguous()):
        raise ValueError(f"attn_fwd: q8 [B,H,{nq * 128},D] e4m3 and sq [B,H,{nq}] fp32 (contiguous) expected for "
                         f"a query of shape {tuple(like.shape)}, got {tuple(q8.shape)} and {tuple(sq.shape)}")
    _on(sq, q8.device, "attn_fwd: sq")
    _on(like, q8.device, "attn_fwd: like")
    _check_kv_codes(k8, v8t, sk, sv, B, H, Sk, D, q8.device, "attn_fwd")
    out = torch.empty_like(like)
    km, kb = key_operands(key_mask, key_bias, B, Sk, q8.device)
    with torch.cuda.device(q8.device):
        N.check(N.load().mxf8_attn_fwd(
            q8.data_ptr(), k8.data_ptr(), v8t.data_ptr(), sq.data_ptr(), sk.data_ptr(), sv.data_ptr(),
            N.ptr(km), N.ptr(kb), float(repair_tau), out.data_ptr(), N.dtype_code(out.dtype), N.strides4(out),
            B, H, Sq, Sk, D, int(kv_mode), N.stream_of(q8)), "attn_fwd")
    return out


@attn_fwd.register_fake
def _(q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, like, Sk, kv_mode=0):
    return torch.empty_like(like)


def attn_fwd_q_supported(q: torch.Tensor) -> bool:
    """Whether attn_fwd_q takes q's layout: 16-bit, unit channel stride, the other strides
    multiples of 8 elements (other layouts use attn_quant_q + attn_fwd).  Reads only dtype,
    shape and strides, which a traced graph knows for every tensor, so it causes no graph
    break; attn_fwd_q checks the pointer's alignment when it runs."""
    return (q.dtype in (torch.bfloat16, torch.float16) and q.dim() == 4 and q.stride(3) == 1
            and all(s % 8 == 0 for s in q.stride()[:3]))


@torch.library.custom_op("mxf8::attn_fwd_q", mutates_args=())
def attn_fwd_q(q: torch.Tensor, c: float, k8: torch.Tensor, v8t: torch.Tensor, sk: torch.Tensor, sv: torch.Tensor,
               key_mask: torch.Tensor | None, key_bias: torch.Tensor | None, repair_tau: float,
               Sk: int, kv_mode: int = 0) -> torch.Tensor:
    """attn_quant_q + attn_fwd in one launch (fp8_attention.py:321-336 and 380-402): each
    128-row Q block is quantized inside the launch; same output bit for bit.  kv_mode as
    attn_fwd."""
    _prep(q, "attn_fwd_q")
    if not attn_fwd_q_supported(q):
        raise ValueError("attn_fwd_q: q must be bf16/fp16 with unit channel stride, other strides multiples of 8 "
                         "and 16-byte alignment")
    if q.data_ptr() % 16:
        # a view that starts off a 16-byte boundary: the two launches give the same bits
        q8, sq = attn_quant_q(q, c)
        return attn_fwd(q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, q, Sk, kv_mode)
    B, H, Sq, D = q.shape
    _check_kv_codes(k8, v8t, sk, sv, B, H, Sk, D, q.device, "attn_fwd_q")
    out = torch.empty_like(q)
    km, kb = key_operands(key_mask, key_bias, B, Sk, q.device)
    with torch.cuda.device(q.device):
        N.check(N.load().mxf8_attn_fwd_q(
            q.data_ptr(), N.strides4(q), float(c), k8.data_ptr(), v8t.data_ptr(), sk.data_ptr(), sv.data_ptr(),
            N.ptr(km), N.ptr(kb), float(repair_tau), None, out.data_ptr(), N.dtype_code(out.dtype), N.strides4(out),
            B, H, Sq, Sk, D, int(kv_mode), N.stream_of(q)), "attn_fwd_q")
    return out


@attn_fwd_q.register_fake
def _(q, c, k8, v8t, sk, sv, key_mask, key_bias, repair_tau, Sk, kv_mode=0):
    return torch.empty_like(q)


def softmax_c(scale: float | None, D: int) -> float:
    """c = (scale or 1/sqrt(D)) * log2(e) (kernels/fp8_attention.py:315)."""
    return (scale if scale is not None else 1.0 / math.sqrt(D)) * 1.4426950408889634
