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
