"""Pins the FP8 linear oracle: closed forms, brute force and torch CPU routines."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle.linear import gelu_tanh, lora_branch_add, quantize_rows, scaled_mm
from oracle.numerics import bf16_round, e4m3_decode


def _bf16_randn(rng, shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def test_quantize_rows_matches_torch_restatement():
    # An independent torch CPU statement of fp8_linear.py:20-22.
    rng = np.random.default_rng(0)
    x = _bf16_randn(rng, (37, 3072))
    x[:, rng.choice(3072, 30, replace=False)] *= 20.0
    codes, scale = quantize_rows(x)
    xt = torch.from_numpy(x)
    s = xt.abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / 448.0
    ref = (xt / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(scale, s.numpy())
    np.testing.assert_array_equal(codes, ref)


def test_quantize_rows_closed_forms():
    x = np.zeros((4, 64), np.float32)
    x[1, 5] = -3.0          # the amax element maps to -448 exactly
    x[1, 6] = 1.5
    x[2] = np.linspace(-1, 1, 64, dtype=np.float32)
    x[3, 0] = 1e-30         # tiny row: the 1e-12 floor
    codes, scale = quantize_rows(x)
    assert np.all(codes[0] == 0)
    assert scale[0, 0] == np.float32(1e-12) / np.float32(448)
    assert scale[1, 0] == np.float32(3.0) / np.float32(448)
    assert codes[1, 5] == 0xFE and codes[1, 6] == 0x76  # 224 = 1.75 * 2**7
    assert codes[2, 0] == 0xFE and codes[2, 63] == 0x7E
    assert codes[3, 0] == 0x00  # 1e-30 / (1e-12/448) ~ 4.5e-16 underflows to 0
    # dequantization error is bounded by half an e4m3 step (relative 1/16 for normals)
    deq = e4m3_decode(codes) * scale
    big = np.abs(x) > 2 ** -6 * scale
    assert np.all(np.abs(deq - x)[big] <= np.abs(x[big]) / 16 + 1e-12)


def test_scaled_mm_brute_force_nonsquare():
    rng = np.random.default_rng(2)
    M, N, K = 5, 7, 33
    x8 = rng.integers(0, 256, (M, K)).astype(np.uint8)
    w8 = rng.integers(0, 256, (N, K)).astype(np.uint8)
    x8[(x8 & 0x7F) == 0x7F] = 0
    w8[(w8 & 0x7F) == 0x7F] = 0
    sa = rng.uniform(0.5, 2, M).astype(np.float32)
    sw = rng.uniform(0.5, 2, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    out = scaled_mm(x8, w8, sa, sw, bias)
    a = e4m3_decode(x8)
    b = e4m3_decode(w8)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += float(a[m, k]) * float(b[n, k])
            ref = acc * float(sa[m]) * float(sw[n]) + float(bias[n])
            assert abs(out[m, n] - ref) <= 1e-5 * max(1.0, abs(ref))


def test_gelu_tanh_matches_torch():
    z = np.linspace(-8, 8, 10001, dtype=np.float32)
    ref = F.gelu(torch.from_numpy(z).double(), approximate="tanh").float().numpy()
    np.testing.assert_allclose(gelu_tanh(z), ref, rtol=1e-6, atol=1e-7)


def test_lora_branch_matches_torch_bf16():
    rng = np.random.default_rng(3)
    M, K, N, r = 24, 64, 48, 8
    x = _bf16_randn(rng, (M, K))
    out = _bf16_randn(rng, (M, N))
    A = _bf16_randn(rng, (r, K), 0.05)
    B = _bf16_randn(rng, (N, r), 0.05)
    got = lora_branch_add(x, out, [(A, B, 0.75)])
    xt, ot = torch.from_numpy(x).bfloat16(), torch.from_numpy(out).bfloat16()
    At, Bt = torch.from_numpy(A).bfloat16(), torch.from_numpy(B).bfloat16()
    branch = (xt @ At.t()) @ Bt.t()
    ref = (ot + (branch * 0.75).to(torch.bfloat16)).float().numpy()
    # torch's CPU bf16 matmul may accumulate in a different order: allow one bf16 ulp
    np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=1e-6)


def test_lora_branch_fp16_output_matches_torch():
    """fp16 inputs: the reference converts the bf16 linear output to fp16 and adds each bf16
    branch after converting it to fp16 (fp8_linear.py:54, 107)."""
    rng = np.random.default_rng(4)
    M, K, N, r = 24, 64, 48, 8
    x = (rng.standard_normal((M, K))).astype(np.float16).astype(np.float32)
    out = _bf16_randn(rng, (M, N))
    A = _bf16_randn(rng, (r, K), 0.05)
    B = _bf16_randn(rng, (N, r), 0.05)
    got = lora_branch_add(x, out, [(A, B, 0.75)], out_dtype="fp16")
    assert np.array_equal(got, got.astype(np.float16).astype(np.float32))
    xt, ot = torch.from_numpy(x).half(), torch.from_numpy(out).bfloat16().to(torch.float16)
    At, Bt = torch.from_numpy(A).bfloat16(), torch.from_numpy(B).bfloat16()
    branch = (xt.to(torch.bfloat16) @ At.t()) @ Bt.t()
    ref = (ot + (branch * 0.75).to(torch.float16)).float().numpy()
    # torch's CPU bf16 matmul may accumulate in a different order: one bf16 ulp of the branch
    np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=1e-6)
    # and the sum is taken in fp16: it differs from the bf16 statement of the same branch
    assert not np.array_equal(got, lora_branch_add(x, out, [(A, B, 0.75)]))


# ------------------------------------------------------------------ adaLN modulation

def _bf16_ulp_diff(a, b):
    """|a - b| in units of the bf16 ulp of max(|a|, |b|) (bf16-valued fp32 inputs)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    mag = np.maximum(np.abs(a), np.abs(b))
    ulp = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7), 2.0 ** -133)
    return np.abs(a - b) / ulp


def test_adaln_modulate_closed_form():
    """Rows of +-a (a a power of two, even count, eps = 0): mean 0, var a^2, LN output exactly
    +-1, so y = bf16(+-(1 + scale) + shift) (one rounding) or
    bf16(bf16(+-bf16(1 + scale)) + shift) (eager)."""
    from oracle.linear import adaln_modulate
    rng = np.random.default_rng(0)
    B, S, C = 2, 3, 64
    sign = np.where(rng.random((B * S, C)) < 0.5, 1.0, -1.0)
    sign[:, : C // 2] = 1.0
    sign[:, C // 2:] = -1.0
    for r in range(B * S):
        rng.shuffle(sign[r])
    a = np.array([0.25, 4.0, 1.0, 0.5, 8.0, 2.0])[:, None]
    x = (sign * a).astype(np.float32)
    shift = bf16_round(rng.standard_normal((B, C)).astype(np.float32) * 0.1)
    scale = bf16_round(rng.standard_normal((B, C)).astype(np.float32) * 0.1)
    b = np.arange(B * S) // S
    fused = adaln_modulate(x, shift, scale, S, eps=0.0)
    np.testing.assert_array_equal(fused, bf16_round((sign * (1.0 + scale[b].astype(np.float64))
                                                     + shift[b]).astype(np.float32)))
    eager = adaln_modulate(x, shift, scale, S, eps=0.0, eager=True)
    op = bf16_round((1.0 + scale[b].astype(np.float64)).astype(np.float32)).astype(np.float64)
    np.testing.assert_array_equal(eager, bf16_round((sign * op + shift[b]).astype(np.float32)))


def test_adaln_modulate_matches_torch_ops():
    """Against torch's own CPU layer_norm and bf16 ops: eager (bf16 tensors, one rounding per
    op) and fused (fp32 ops, one rounding).  LayerNorm statistics in fp32 (torch) and float64
    (oracle) may round a value to the neighbouring bf16: at most 1 ulp, rarely."""
    from oracle.linear import adaln_modulate
    rng = np.random.default_rng(1)
    B, S, C, eps = 2, 37, 3072, 1e-6
    x = bf16_round((rng.standard_normal((B, S, C)) * 1.5 + 0.3).astype(np.float32))
    x[..., rng.choice(C, 30, replace=False)] *= 20.0
    x = bf16_round(x)
    shift = bf16_round((rng.standard_normal((B, C)) * 0.1).astype(np.float32))
    scale = bf16_round((rng.standard_normal((B, C)) * 0.1).astype(np.float32))
    xt, sht, sct = (torch.from_numpy(v).to(torch.bfloat16) for v in (x, shift, scale))
    with torch.no_grad():
        eager_t = F.layer_norm(xt, (C,), eps=eps) * (1 + sct[:, None]) + sht[:, None]
        fused_t = (F.layer_norm(xt.float(), (C,), eps=eps) * (1 + sct.float()[:, None]) + sht.float()[:, None])
        fused_t = fused_t.to(torch.bfloat16)
    for eager, ref in ((True, eager_t), (False, fused_t)):
        y = adaln_modulate(x.reshape(B * S, C), shift, scale, S, eps=eps, eager=eager)
        r = ref.float().numpy().reshape(B * S, C)
        d = _bf16_ulp_diff(y, r)
        err = np.abs(y.astype(np.float64) - r)
        # within 1 ulp, or 2^-17 absolute where n (1 + scale) and shift cancel
        assert ((d <= 1.0) | (err <= 2.0 ** -17)).all() and (d > 0).mean() < 5e-3, (eager, d.max())
    # the two modes differ (the eager roundings matter)
    ye = adaln_modulate(x.reshape(B * S, C), shift, scale, S, eps=eps, eager=True)
    yf = adaln_modulate(x.reshape(B * S, C), shift, scale, S, eps=eps, eager=False)
    assert (ye != yf).mean() > 0.01


def test_quantize_rows_non_finite_follow_the_reference_clamp():
    """Closed forms for non-finite rows under the reference's Triton semantics
    (kernels/fp8_linear.py:20-22: tl.max / tl.maximum / tl.minimum skip NaN): a NaN does
    not enter the row maximum and its quotient clamps to -448 (0xFE); a row maximum of inf
    gives the scale inf, finite elements x / inf = +-0 (0x00 / 0x80), +-inf -> NaN -> -448."""
    inf, nan = np.inf, np.nan
    x = np.array([[inf, 1.0, -2.0, 0.0],
                  [nan, 448.0, -224.0, 1.0],
                  [nan, nan, nan, nan],
                  [-inf, 5.0, -0.0, nan]], np.float32)
    codes, scale = quantize_rows(x)
    assert scale[0, 0] == inf and scale[3, 0] == inf
    assert scale[1, 0] == np.float32(1.0)
    assert scale[2, 0] == np.float32(np.float32(1e-12) / np.float32(448.0))
    np.testing.assert_array_equal(codes, np.array([[0xFE, 0x00, 0x80, 0x00],
                                                   [0xFE, 0x7E, 0xF6, 0x38],
                                                   [0xFE, 0xFE, 0xFE, 0xFE],
                                                   [0xFE, 0x00, 0x80, 0xFE]], np.uint8))
