"""K/V statistics from the QKV projection's epilogue (FP8Linear.forward_qkv ->
fp8_attention(kv_stats=...)): the key mean (kernels/fp8_attention.py:338) and the per-channel
V scale (122-155) come from the GEMM that writes K and V, so the quantizers read K and V once.

Checks, on shapes that take both GEMM tile sizes, a K tail, D = 64, batch items whose
boundaries fall inside 128-row blocks and token tails:

* the projection's output equals FP8Linear.forward's bit for bit;
* the raw statistics equal per-block sums (fp32 bar) and maxima (exact) of the output;
* V codes and scales equal the oracle's bit for bit; K codes equal the oracle's given the
  kernel's key mean, which is within 1e-6 of max|k| of the oracle's mean;
* the chained 480p block (QKV projection -> attention, S = 20280) and the joint
  two-item self-attention shape (S = 21304) at full size, attention outputs against the
  oracle on sampled Q tiles.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle.numerics import bf16_round
from tests.helpers import assert_attn_close, codes

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _qkv_linear(g, k, heads, d):
    from minimaxh3_amd.kernels import fp8_linear as fl
    n = 3 * heads * d
    lin = torch.nn.Linear(k, n, bias=True, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn((n, k), device="cuda", generator=g) * 0.02)
        lin.bias.copy_(torch.randn((n,), device="cuda", generator=g) * 0.01)
    return fl.FP8Linear.from_linear(lin)


def _activations(g, m, k, outliers=True):
    """bf16 ~N(0,1) (with floor(1% of k) channels scaled x20 when `outliers`) plus 0.5, so that
    every output channel has a mean of its own and the key mean is far from zero."""
    x = torch.randn((m, k), device="cuda", generator=g)
    if outliers:
        idx = torch.randperm(k, device="cuda", generator=g)[: max(1, k // 100)]
        x[:, idx] *= 20.0
    return (x + 0.5).to(torch.bfloat16)


def _views(out, B, S, H, D):
    qkv = out.reshape(B, S, 3, H, D)
    return tuple(qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))


def _check_raw_stats(out2d, stats, S, H, D, key_stats):
    """stats[0/1][p][c] against numpy per-block sums / maxima of the GPU's own output, for the
    128-row blocks inside one batch item (the kernel leaves the others out)."""
    M = out2d.shape[0]
    C = H * D
    o = out2d.float().cpu().numpy()
    ks, vs = o[:, C:2 * C].astype(np.float64), np.abs(o[:, 2 * C:3 * C])
    st = stats.cpu().numpy()
    nb = -(-M // 128)
    assert st.shape == (2, nb, C)
    checked = 0
    for p in range(nb):
        a, b = 128 * p, 128 * p + 128
        if b > min((a // S + 1) * S, M):
            continue  # an item boundary or M inside the block
        checked += 1
        if key_stats:
            ref = ks[a:b].sum(0)
            tol = 2e-6 * np.abs(ks[a:b]).sum(0) + 1e-30  # fp32: <= 18 roundings of partial sums
            assert (np.abs(st[0, p] - ref) <= tol).all(), p
        np.testing.assert_array_equal(st[1, p], vs[a:b].max(0).astype(np.float32), err_msg=str(p))
    assert checked >= nb - 2 * (M // S)


def _check_quantizers(k, v, k8, sk, v8t, sv, mean, heads=None):
    """V codes / scales bit-exact; K codes / scales bit-exact given the kernel's mean; the mean
    within 1e-6 of max|k| of the oracle's (float64 sum)."""
    B, H, S, D = k.shape
    hs = range(H) if heads is None else heads
    for b in range(B):
        for h in hs:
            kn = k[b:b + 1, h:h + 1].float().cpu().numpy()
            vn = v[b:b + 1, h:h + 1].float().cpu().numpy()
            mu = mean[b:b + 1, h:h + 1].cpu().numpy().reshape(1, 1, 1, D)
            ref_mu = oa.key_mean(kn)
            assert np.abs(mu - ref_mu).max() <= 1e-6 * np.abs(kn).max(), (b, h)
            rk8, rsk = oa.quantize_k(kn, mu)
            np.testing.assert_array_equal(codes(k8[b:b + 1, h:h + 1, :S]), rk8)
            np.testing.assert_array_equal(sk[b:b + 1, h:h + 1].cpu().numpy(), rsk)
            rv8t, rsv = oa.quantize_v(vn)
            np.testing.assert_array_equal(codes(v8t[b:b + 1, h:h + 1, :, :S]), rv8t)
            np.testing.assert_array_equal(sv[b:b + 1, h:h + 1].cpu().numpy(), rsv)


@pytest.mark.parametrize("B,S,H,D,K,key_stats", [
    (2, 300, 2, 128, 256, True),    # 128 x 128 tiles, item boundary inside a block, token tail
    (2, 300, 4, 64, 272, True),     # D = 64, K tail (272 % 128 = 16)
    (3, 200, 2, 128, 256, True),    # three items, S < 256
    (1, 1000, 2, 128, 512, False),  # value statistics only; key mean from attn_kmean
    (1, 2176, 8, 128, 256, True),   # S a multiple of 128: no block crosses an item boundary
])
def test_kv_stats_small_shapes(B, S, H, D, K, key_stats):
    _say(f"kv stats B={B} S={S} H={H} D={D} K={K} key_stats={key_stats}")
    from minimaxh3_amd import ops
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention
    g = torch.Generator(device="cuda").manual_seed(11)
    mod = _qkv_linear(g, K, H, D)
    x = _activations(g, B * S, K, outliers=False).reshape(B, S, K)
    plain = mod.forward(x)
    out, stats = mod.forward_qkv(x, H, D, key_stats=key_stats)
    torch.cuda.synchronize()
    assert stats is not None and stats.key == key_stats
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16)), "projection output differs from forward"
    _check_raw_stats(out.reshape(B * S, -1), stats.part, S, H, D, key_stats)
    q, k, v = _views(out, B, S, H, D)
    mean_in = None if key_stats else ops.attn_kmean(k)
    k8, sk, v8t, sv, mean = ops.attn_quant_kv_gemm_stats(k, v, stats.part, mean_in)
    torch.cuda.synchronize()
    _check_quantizers(k, v, k8, sk, v8t, sv, mean)
    # padded key rows / columns of the FP8 layouts are zero, as in attn_quant_kv
    Sp = k8.shape[2]
    assert not codes(k8[:, :, S:]).any() and not codes(v8t[:, :, :, S:]).any() and Sp % 128 == 0
    # the attention on these statistics: against the oracle (full shape) given the kernel's key
    # mean (a one-ulp difference in the mean may move a K code by one step)
    o = fp8_attention(q, k, v, kv_stats=stats)
    torch.cuda.synchronize()
    for h in sorted({0, H - 1}):
        qn, kn, vn = (t[:, h:h + 1].float().cpu().numpy() for t in (q, k, v))
        ref, _ = oa.fp8_attention(qn, kn, vn, mu=mean[:, h:h + 1].cpu().numpy()[:, :, None, :])
        assert_attn_close(o[:, h:h + 1].float().cpu().numpy(), ref)


def test_kv_stats_bigger_tiles_and_tail():
    """256 x 256 tiles (M = 12 x 1100 = 13200 rows, N = 3 x 12 x 128 = 4608: 52 x 18 = 936 >= 512
    tiles): item boundaries inside 128-row blocks and a token tail in the last tile row."""
    B, S, H, D, K = 12, 1100, 12, 128, 384
    _say(f"kv stats 256x256 tiles B={B} S={S} H={H}")
    from minimaxh3_amd import ops
    g = torch.Generator(device="cuda").manual_seed(12)
    mod = _qkv_linear(g, K, H, D)
    x = _activations(g, B * S, K).reshape(B, S, K)
    plain = mod.forward(x)
    out, stats = mod.forward_qkv(x, H, D)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    _check_raw_stats(out.reshape(B * S, -1), stats.part, S, H, D, True)
    q, k, v = _views(out, B, S, H, D)
    k8, sk, v8t, sv, mean = ops.attn_quant_kv_gemm_stats(k, v, stats.part, None)
    torch.cuda.synchronize()
    _check_quantizers(k, v, k8, sk, v8t, sv, mean, heads=(0, 5, H - 1))


@pytest.mark.parametrize("B,S,outliers", [(1, 20280, True), (1, 20280, False), (2, 21304, False)])
def test_kv_stats_full_size_chained(B, S, outliers):
    """The 480p block's QKV projection (M = 20280, 3072 -> 9216) feeding the attention, and the
    joint two-item shape (S = 21304): statistics from the epilogue and quantizers against the
    oracle on several heads (bit-exact given the kernel's key mean).  The attention output is
    held to the attention bar (cosine >= 0.999, max-abs <= 2e-2, stated for N(0,1)-scale
    inputs) on sampled Q tiles where the activations have no x20 outlier channels: with them V
    reaches |v| ~ 12, where one bf16 ulp of the output (0.0625-0.125) is above 2e-2."""
    H, D, K = 24, 128, 3072
    _say(f"kv stats chained full size B={B} S={S} outliers={outliers}")
    from minimaxh3_amd import ops
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention
    g = torch.Generator(device="cuda").manual_seed(13)
    mod = _qkv_linear(g, K, H, D)
    x = _activations(g, B * S, K, outliers).reshape(B, S, K)
    plain = mod.forward(x)
    out, stats = mod.forward_qkv(x, H, D)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    q, k, v = _views(out, B, S, H, D)
    k8, sk, v8t, sv, mean = ops.attn_quant_kv_gemm_stats(k, v, stats.part, None)
    _, _, v8t_r, sv_r, mean_r = ops.attn_quant_kv(k, v)
    torch.cuda.synchronize()
    # V is the two-pass quantizer's bit for bit; the two key means agree to fp32 rounding
    assert torch.equal(v8t.view(torch.uint8), v8t_r.view(torch.uint8)) and torch.equal(sv, sv_r)
    kmax = float(k.float().abs().max())
    assert float((mean - mean_r).abs().max()) <= 1e-6 * kmax
    _check_quantizers(k, v, k8, sk, v8t, sv, mean, heads=(0, 11, H - 1))
    if outliers:
        _check_raw_stats(out.reshape(B * S, -1), stats.part, S, H, D, True)
        return
    o = fp8_attention(q, k, v, kv_stats=stats)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    nq = -(-S // 128)
    tiles = [0, nq // 2, nq - 1]
    c = ops.softmax_c(None, D)
    for b in range(B):
        for h in (0, H - 1):
            qn, kn, vn = (t[b:b + 1, h:h + 1].float().cpu().numpy() for t in (q, k, v))
            q8, sq = oa.quantize_q(qn, c)
            # the kernel's key mean (checked against the oracle's above)
            k8r, skr = oa.quantize_k(kn, mean[b:b + 1, h:h + 1].cpu().numpy()[:, :, None, :])
            v8r, svr = oa.quantize_v(vn)
            ref = bf16_round(oa.attn_fwd(q8, k8r, v8r, sq, skr, svr, q_tiles=tiles))
            for t in tiles:
                r0, r1 = t * 128, min(S, t * 128 + 128)
                assert_attn_close(o[b, h, r0:r1].float().cpu().numpy(), ref[0, 0, r0:r1])


def test_forward_qkv_falls_back_where_the_epilogue_does_not_apply():
    """LoRA adapters, a fused activation, a non-bf16 input or heads x head_dim not a multiple
    of 256 give (forward(x), None), and fp8_attention(kv_stats=None) takes the standard path."""
    g = torch.Generator(device="cuda").manual_seed(14)
    mod = _qkv_linear(g, 256, 1, 128)  # C = 128
    x = _activations(g, 300, 256).reshape(1, 300, 256)
    out, stats = mod.forward_qkv(x, 1, 128)
    assert stats is None and torch.equal(out.view(torch.int16), mod.forward(x).view(torch.int16))
    mod2 = _qkv_linear(g, 256, 2, 128)
    A = (torch.randn((16, 256), device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    Bm = (torch.randn((768, 16), device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    mod2.adapters.append((A, Bm, 1.0))
    out, stats = mod2.forward_qkv(x, 2, 128)
    assert stats is None and torch.equal(out.view(torch.int16), mod2.forward(x).view(torch.int16))
    with pytest.raises(ValueError):
        mod2.forward_qkv(x, 3, 128)
