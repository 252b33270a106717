"""GPU parity of the FP8 attention path against the oracle.

Quantizers: codes and scales bit-exact (K given the oracle's key mean; the mean itself
to 1e-6 of the key scale).  Forward: cosine >= 0.999 and max-abs <= 2e-2 against the
oracle's algorithm on the same codes and scales.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle.numerics import bf16_round
from tests.helpers import assert_attn_close, assert_attn_model, bf16_randn, codes, cos, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _layout(x_np, permuted, dtype=torch.bfloat16):
    """[B,H,S,D] numpy -> GPU tensor, optionally as a permuted view of [B,S,H,D] storage."""
    if permuted:
        return to_gpu(np.ascontiguousarray(x_np.transpose(0, 2, 1, 3)), dtype).permute(0, 2, 1, 3)
    return to_gpu(x_np, dtype)


@pytest.mark.parametrize("B,H,S,D,permuted,dtype", [
    (2, 2, 300, 128, False, torch.bfloat16), (1, 3, 700, 128, True, torch.bfloat16),
    (2, 1, 130, 64, False, torch.float16), (1, 2, 128, 64, True, torch.bfloat16),
    (1, 1, 5, 128, False, torch.bfloat16),
])
def test_attention_quantizers_bit_exact(B, H, S, D, permuted, dtype):
    _say(f"attn quantizers B={B} H={H} S={S} D={D} perm={permuted} {dtype}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(S + D)
    q, k, v = (bf16_randn(rng, (B, H, S, D)) for _ in range(3))
    k = bf16_round(k + bf16_randn(rng, (1, 1, 1, D), 2.0))  # a non-zero key mean
    if dtype == torch.float16:
        q, k, v = (t.astype(np.float16).astype(np.float32) for t in (q, k, v))
    qg, kg, vg = (_layout(t, permuted, dtype) for t in (q, k, v))
    c = np.float32(oa.LOG2E / math.sqrt(D))
    q8, sq = ops.attn_quant_q(qg, float(c))
    rq8, rsq = oa.quantize_q(q, c)
    nq = -(-S // 128)
    assert q8.shape == (B, H, nq * 128, D)
    np.testing.assert_array_equal(sq.cpu().numpy(), rsq)
    np.testing.assert_array_equal(codes(q8)[:, :, :S], rq8)
    assert not codes(q8)[:, :, S:].any()
    mu = ops.attn_kmean(kg)
    rmu = oa.key_mean(k)[:, :, 0, :]
    assert np.abs(mu.cpu().numpy() - rmu).max() <= 1e-6 * np.abs(k).max()
    k8, sk = ops.attn_quant_k(kg, to_gpu(rmu, torch.float32))
    rk8, rsk = oa.quantize_k(k, rmu[:, :, None, :])
    np.testing.assert_array_equal(sk.cpu().numpy(), rsk)
    np.testing.assert_array_equal(codes(k8)[:, :, :S], rk8)
    assert not codes(k8)[:, :, S:].any()
    v8t, sv = ops.attn_quant_v(vg)
    rv8t, rsv = oa.quantize_v(v)
    np.testing.assert_array_equal(sv.cpu().numpy(), rsv)
    np.testing.assert_array_equal(codes(v8t)[..., :S], rv8t)
    assert not codes(v8t)[..., S:].any()


@pytest.mark.parametrize("B,H,S,D,layout,dtype", [
    (2, 3, 333, 128, "packed", torch.bfloat16), (1, 2, 700, 128, "contig", torch.bfloat16),
    (2, 2, 130, 64, "packed", torch.float16), (1, 3, 5, 128, "permuted", torch.bfloat16),
    (1, 2, 256, 64, "strided", torch.bfloat16), (2, 24, 2600, 128, "packed", torch.bfloat16),
])
def test_attention_quant_kv_matches_separate_and_oracle(B, H, S, D, layout, dtype):
    """attn_quant_kv (one pass for both statistics, one fold, one pass quantizing K and V)
    equals attn_kmean + attn_quant_k + attn_quant_v bit for bit, and the oracle: V codes
    and scales bit-exact, K codes and scales bit-exact given the kernel's own key mean, the
    mean within 1e-6 of max|k|.  Layouts: K and V halves of one [B, S, 2, H, D] projection
    (packed), contiguous, permuted [B, S, H, D] views, and a channel stride of 2 (strided)."""
    _say(f"attn quant_kv B={B} H={H} S={S} D={D} {layout} {dtype}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(S * 3 + D + B)
    k, v = bf16_randn(rng, (B, H, S, D)), bf16_randn(rng, (B, H, S, D), 2.0)
    k = bf16_round(k + bf16_randn(rng, (1, H, 1, D), 2.0))  # a non-zero key mean per head
    if dtype == torch.float16:
        k, v = (t.astype(np.float16).astype(np.float32) for t in (k, v))
    if layout == "packed":
        kv = np.ascontiguousarray(np.stack([k, v], 2).transpose(0, 3, 2, 1, 4))  # [B, S, 2, H, D]
        g = to_gpu(kv, dtype)
        kg, vg = g[:, :, 0].permute(0, 2, 1, 3), g[:, :, 1].permute(0, 2, 1, 3)
    elif layout == "strided":
        kg = to_gpu(np.repeat(k, 2, axis=-1), dtype)[..., ::2]
        vg = to_gpu(np.repeat(v, 2, axis=-1), dtype)[..., ::2]
        assert kg.stride(-1) == 2
    else:
        kg, vg = _layout(k, layout == "permuted", dtype), _layout(v, layout == "permuted", dtype)
    k8, sk, v8t, sv, mu = ops.attn_quant_kv(kg, vg)
    mu_s = ops.attn_kmean(kg)
    k8s, sks = ops.attn_quant_k(kg, mu_s)
    v8ts, svs = ops.attn_quant_v(vg)
    assert torch.equal(mu, mu_s) and torch.equal(sk, sks) and torch.equal(sv, svs)
    assert torch.equal(k8.view(torch.uint8), k8s.view(torch.uint8))
    assert torch.equal(v8t.view(torch.uint8), v8ts.view(torch.uint8))
    rmu = oa.key_mean(k)[:, :, 0, :]
    assert np.abs(mu.cpu().numpy() - rmu).max() <= 1e-6 * np.abs(k).max()
    rk8, rsk = oa.quantize_k(k, mu.cpu().numpy()[:, :, None, :])
    np.testing.assert_array_equal(sk.cpu().numpy(), rsk)
    np.testing.assert_array_equal(codes(k8)[:, :, :S], rk8)
    assert not codes(k8)[:, :, S:].any()
    rv8t, rsv = oa.quantize_v(v)
    np.testing.assert_array_equal(sv.cpu().numpy(), rsv)
    np.testing.assert_array_equal(codes(v8t)[..., :S], rv8t)
    assert not codes(v8t)[..., S:].any()


def _fwd_case(rng, B, H, Sq, Sk, D, mask=None, bias=None, tau=-1.0, permuted=False, dtype=torch.bfloat16,
              dot="exact"):
    """Runs the GPU forward on the oracle's own codes/scales; returns it with the oracle's
    output (its fp8 products formed as ``dot`` says, see oracle.attention.attn_fwd)."""
    from minimaxh3_amd import ops
    q, = (bf16_randn(rng, (B, H, Sq, D)),)
    k, v = bf16_randn(rng, (B, H, Sk, D)), bf16_randn(rng, (B, H, Sk, D))
    ref, inter = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=bias, repair_tau=tau,
                                  out_dtype="bf16" if dtype == torch.bfloat16 else "fp16", dot=dot)
    nq, nk = -(-Sq // 128), -(-Sk // 128)

    def pad(a, axis, n):
        w = [(0, 0)] * a.ndim
        w[axis] = (0, n - a.shape[axis])
        return np.pad(a, w)

    q8 = to_gpu(pad(inter["q8"], 2, nq * 128), torch.uint8).view(torch.float8_e4m3fn)
    k8 = to_gpu(pad(inter["k8"], 2, nk * 128), torch.uint8).view(torch.float8_e4m3fn)
    v8t = to_gpu(pad(inter["v8t"], 3, nk * 128), torch.uint8).view(torch.float8_e4m3fn)
    like = _layout(q, permuted, dtype)
    out = ops.attn_fwd(q8, k8, v8t, to_gpu(inter["sq"], torch.float32), to_gpu(inter["sk"], torch.float32),
                       to_gpu(inter["sv"], torch.float32),
                       None if mask is None else to_gpu(mask.astype(np.uint8), torch.bool),
                       None if bias is None else to_gpu(bias, torch.float32), float(tau), like, Sk)
    assert out.shape == (B, H, Sq, D) and out.dtype == dtype and out.stride() == like.stride()
    return out.float().cpu().numpy(), ref


@pytest.mark.parametrize("tau", [-1.0, 0.5, 0.0])
def test_attn_fwd_matches_oracle(tau):
    _say(f"attn fwd tau={tau}")
    rng = np.random.default_rng(11)
    out, ref = _fwd_case(rng, 2, 2, 300, 700, 128, tau=tau)
    assert_attn_close(out, ref)
    assert cos(out, ref) > 0.9999
    # with the fp8 instruction's arithmetic the oracle gives the kernel's bits (the repair within 2 ulps)
    out_m, ref_m = _fwd_case(np.random.default_rng(11), 2, 2, 300, 700, 128, tau=tau, dot="mfma")
    np.testing.assert_array_equal(out_m, out)
    assert_attn_model(out_m, ref_m, "bf16", tau)


@pytest.mark.parametrize("tau", [500.0, 1e30])
def test_attn_fwd_repair_above_every_code_is_plain(tau):
    """A repair threshold above the largest e4m3 value (448) corrects no P code: the repair
    kernel clears every hi / lo byte, its extra products add exact zeros, and its output equals
    the kernel without the repair bit for bit (mask and bias included)."""
    _say(f"attn fwd repair tau={tau} against no repair")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(21)
    B, H, Sq, Sk, D = 2, 3, 400, 900, 128
    q = to_gpu(bf16_randn(rng, (B, H, Sq, D)), torch.bfloat16)
    k = to_gpu(bf16_randn(rng, (B, H, Sk, D)), torch.bfloat16)
    v = to_gpu(bf16_randn(rng, (B, H, Sk, D)), torch.bfloat16)
    mask = np.ones((B, Sk), bool)
    mask[1, 700:] = False
    bias = (rng.standard_normal((B, Sk)) * 0.5).astype(np.float32)
    km, kb = to_gpu(mask.astype(np.uint8), torch.bool), to_gpu(bias, torch.float32)
    c = ops.softmax_c(None, D)
    k8, sk, v8t, sv, _ = ops.attn_quant_kv(k, v)
    for m, b in ((None, None), (km, kb)):
        plain = ops.attn_fwd_q(q, c, k8, v8t, sk, sv, m, b, -1.0, Sk, 1)
        rep = ops.attn_fwd_q(q, c, k8, v8t, sk, sv, m, b, float(tau), Sk, 1)
        torch.cuda.synchronize()
        assert torch.equal(plain.view(torch.int16), rep.view(torch.int16))


def test_attn_fwd_mask_bias_permuted():
    _say("attn fwd mask+bias permuted")
    rng = np.random.default_rng(12)
    B, Sk = 2, 700
    mask = np.ones((B, Sk), bool)
    mask[1, 520:] = False
    mask[0, rng.choice(Sk, 50, replace=False)] = False
    bias = (rng.standard_normal((B, Sk)) * 0.5).astype(np.float32)
    bias[0, :20] = -1e9
    for m, b in ((mask, None), (None, bias), (mask, bias)):
        out, ref = _fwd_case(rng, B, 2, 300, Sk, 128, mask=m, bias=b, permuted=True)
        assert_attn_close(out, ref)


@pytest.mark.parametrize("Sq,Sk,D,dtype", [
    (130, 200, 64, torch.bfloat16), (64, 100, 128, torch.float16), (257, 512, 128, torch.bfloat16),
    (128, 1, 128, torch.bfloat16), (1, 300, 64, torch.bfloat16),
])
def test_attn_fwd_shapes(Sq, Sk, D, dtype):
    _say(f"attn fwd Sq={Sq} Sk={Sk} D={D} {dtype}")
    rng = np.random.default_rng(Sq * 7 + Sk)
    out, ref = _fwd_case(rng, 1, 2, Sq, Sk, D, dtype=dtype)
    assert_attn_close(out, ref)


def test_attn_fwd_fully_masked_rows_are_zero():
    _say("attn fwd fully masked")
    rng = np.random.default_rng(13)
    mask = np.ones((2, 300), bool)
    mask[1] = False
    out, ref = _fwd_case(rng, 2, 1, 200, 300, 128, mask=mask)
    assert np.all(out[1] == 0) and np.all(ref[1] == 0)
    assert_attn_close(out[0], ref[0])


def test_fp8_attention_end_to_end():
    _say("fp8_attention end to end")
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention, is_supported
    rng = np.random.default_rng(14)
    B, H, S, D = 2, 3, 333, 128
    q, k, v = (bf16_randn(rng, (B, H, S, D)) for _ in range(3))
    mask = np.ones((B, S), bool)
    mask[1, 300:] = False
    qg, kg, vg = (_layout(t, True) for t in (q, k, v))
    assert is_supported(qg, kg, vg)
    out = fp8_attention(qg, kg, vg, key_mask=to_gpu(mask, torch.bool), repair_tau=0.5)
    ref, inter = oa.fp8_attention(q, k, v, key_mask=mask, repair_tau=0.5)
    from minimaxh3_amd import ops
    q8, sq = ops.attn_quant_q(qg, float(inter["c"]))
    np.testing.assert_array_equal(codes(q8)[:, :, :S], inter["q8"])
    v8t, sv = ops.attn_quant_v(vg)
    np.testing.assert_array_equal(codes(v8t)[..., :S], inter["v8t"])
    mu = ops.attn_kmean(kg).cpu().numpy()
    assert np.abs(mu - inter["mu"][:, :, 0]).max() <= 1e-6 * np.abs(k).max()
    assert_attn_close(out.float().cpu().numpy(), ref)
    with pytest.raises(ValueError):
        fp8_attention(qg[..., :32], kg[..., :32], vg[..., :32])


def test_router_routes_to_fp8_on_gpu():
    _say("router on gpu")
    from minimaxh3_amd.kernels import attention_router as ar
    rng = np.random.default_rng(15)
    q, k, v = (to_gpu(bf16_randn(rng, (1, 2, 256, 128))) for _ in range(3))
    ar.configure(enabled=True, repair_tau=-1.0, min_seq=128)
    try:
        with ar.denoiser_scope():
            out = ar.routed_sdpa(q, k, v)
        ref, _ = oa.fp8_attention(*(t.float().cpu().numpy() for t in (q, k, v)))
        assert_attn_close(out.float().cpu().numpy(), ref)
        out2 = ar.routed_sdpa(q, k, v)  # outside the scope: plain SDPA
        exact = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
        assert cos(out2.float().cpu().numpy(), exact.cpu().numpy()) > 0.99999
    finally:
        ar.configure(enabled=True, repair_tau=-1.0, min_seq=4096)


@pytest.mark.parametrize("B,Sq,Sk,H,mask_tail", [
    (1, 20280, 20280, 24, 0),      # 480p video self-attention
    (2, 21304, 21304, 24, 384),    # joint video + audio self-attention, item 1 key-masked
    (2, 21304, 512, 24, 0),        # text cross-attention
    (1, 77648, 77648, 24, 0),      # 720p video + audio self-attention
])
def test_full_size_sampled_tiles(B, Sq, Sk, H, mask_tail):
    """Full-size GPU runs of the DiT attention shapes; the oracle on sampled Q tiles of
    sampled heads (Q tiles are independent), and on one tile per item with the fp8
    instruction's arithmetic, bit for bit but for rare 1-ulp cases."""
    _say(f"full size B={B} Sq={Sq} Sk={Sk} H={H} mask_tail={mask_tail}")
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention
    from minimaxh3_amd import ops
    D = 128
    g = torch.Generator(device="cuda").manual_seed(0)
    mk = lambda S: torch.randn((B, S, H, D), device="cuda", generator=g).to(torch.bfloat16).permute(0, 2, 1, 3)
    q, k, v = mk(Sq), mk(Sk), mk(Sk)
    mask = None
    if mask_tail:
        mask = torch.ones((B, Sk), dtype=torch.bool, device="cuda")
        mask[1, Sk - mask_tail:] = False
    out = fp8_attention(q, k, v, key_mask=mask)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    heads = [0, H - 1]
    tiles = [0, (Sq // 128) // 2, -(-Sq // 128) - 1]
    for b in range(B):
        for h in heads:
            qn, kn, vn = (t[b:b + 1, h:h + 1].float().cpu().numpy() for t in (q, k, v))
            c = ops.softmax_c(None, D)
            q8, sq = oa.quantize_q(qn, c)
            mu = oa.key_mean(kn)
            k8, sk = oa.quantize_k(kn, mu)
            v8t, sv = oa.quantize_v(vn)
            km = None if mask is None else mask[b:b + 1].cpu().numpy()
            ref = bf16_round(oa.attn_fwd(q8, k8, v8t, sq, sk, sv, key_mask=km, q_tiles=tiles))
            for t in tiles:
                r0, r1 = t * 128, min(Sq, t * 128 + 128)
                assert_attn_close(out[b, h, r0:r1].float().cpu().numpy(), ref[0, 0, r0:r1])
    # head 0 of every item, middle Q tile: the oracle with the fp8 instruction's arithmetic and
    # the key mean the GPU path used gives the kernel's bits
    _, _, _, _, mean = ops.attn_quant_kv(k, v)
    t = (Sq // 128) // 2
    r0, r1 = t * 128, min(Sq, t * 128 + 128)
    for b in range(B):
        qn, kn, vn = (x[b:b + 1, :1].float().cpu().numpy() for x in (q, k, v))
        q8, sq = oa.quantize_q(qn, ops.softmax_c(None, D))
        k8, sk = oa.quantize_k(kn, mean[b:b + 1, :1].cpu().numpy().reshape(1, 1, 1, D))
        v8t, sv = oa.quantize_v(vn)
        km = None if mask is None else mask[b:b + 1].cpu().numpy()
        ref = bf16_round(oa.attn_fwd(q8, k8, v8t, sq, sk, sv, key_mask=km, q_tiles=[t], dot="mfma"))
        _say(f"  item {b}: tile {t} against the instruction-model oracle")
        assert_attn_model(out[b, 0, r0:r1].float().cpu().numpy(), ref[0, 0, r0:r1], "bf16", -1.0)


def test_full_size_repair_matches_the_instruction_model():
    """The reference's quality profile (repair tau = 0.5) at the 480p shape, B=1 H=24 S=20280
    D=128: one Q tile of heads 0 and 23 against the oracle with the fp8 instructions'
    arithmetic and the key mean the GPU path used (within 2 ulps, mostly bit-identical)."""
    _say("full size repair tau=0.5 S=20280")
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention
    from minimaxh3_amd import ops
    B, S, H, D, tau = 1, 20280, 24, 128, 0.5
    g = torch.Generator(device="cuda").manual_seed(3)
    mk = lambda: torch.randn((B, S, H, D), device="cuda", generator=g).to(torch.bfloat16).permute(0, 2, 1, 3)
    q, k, v = mk(), mk(), mk()
    out = fp8_attention(q, k, v, repair_tau=tau)
    _, _, _, _, mean = ops.attn_quant_kv(k, v)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    t = 40
    r0, r1 = t * 128, t * 128 + 128
    for h in (0, H - 1):
        qn, kn, vn = (x[:, h:h + 1].float().cpu().numpy() for x in (q, k, v))
        q8, sq = oa.quantize_q(qn, ops.softmax_c(None, D))
        k8, sk = oa.quantize_k(kn, mean[:, h:h + 1].cpu().numpy().reshape(1, 1, 1, D))
        v8t, sv = oa.quantize_v(vn)
        ref = bf16_round(oa.attn_fwd(q8, k8, v8t, sq, sk, sv, repair_tau=tau, q_tiles=[t], dot="mfma"))
        assert_attn_model(out[0, h, r0:r1].float().cpu().numpy(), ref[0, 0, r0:r1], "bf16", tau)


@pytest.mark.parametrize("use_mask,use_bias,tau", [
    (True, False, 0.5), (True, False, -1.0), (False, False, 0.5), (True, False, 0.0), (False, True, -1.0),
    (True, True, 0.5),
])
def test_attn_fwd_tail_tile_mask_bias(use_mask, use_bias, tau):
    """Mask / bias whose last KV tile is partial (S = 333; the tail keys carry real values)
    combined with the exact repair (B=2, H=3, permuted output)."""
    _say(f"attn fwd tail mask={use_mask} bias={use_bias} tau={tau}")
    rng = np.random.default_rng(14)
    B, S = 2, 333
    mask = bias = None
    if use_mask:
        mask = np.ones((B, S), bool)
        mask[1, 300:] = False
    if use_bias:
        bias = np.zeros((B, S), np.float32)
        bias[:, 320:] = 3.0                      # the tail keys dominate when their bias is read
        bias[1, :10] = -1e9
    out, ref = _fwd_case(rng, B, 3, S, S, 128, mask=mask, bias=bias, tau=tau, permuted=True)
    assert_attn_close(out, ref)


def test_attention_rejects_codes_of_another_length():
    """K8 / V8T / sK are addressed through Sk alone: codes quantized for another number of
    keys (or of another dtype or layout) raise ValueError before anything is launched."""
    _say("attn operand checks")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(15)
    B, H, S, D = 1, 2, 300, 128
    q, k, v = (to_gpu(bf16_randn(rng, (B, H, S, D))) for _ in range(3))
    k8, sk = ops.attn_quant_k(k, ops.attn_kmean(k))
    v8t, sv = ops.attn_quant_v(v)
    q8, sq = ops.attn_quant_q(q, 0.1)
    for Sk in (400, 200):  # 512 and 256 padded keys where the codes hold 384
        with pytest.raises(ValueError, match="k8"):
            ops.attn_fwd_q(q, 0.1, k8, v8t, sk, sv, None, None, -1.0, Sk)
        with pytest.raises(ValueError, match="k8"):
            ops.attn_fwd(q8, k8, v8t, sq, sk, sv, None, None, -1.0, q, Sk)
    with pytest.raises(ValueError, match="sk"):
        ops.attn_fwd_q(q, 0.1, k8, v8t, sk.double(), sv, None, None, -1.0, S)
    with pytest.raises(ValueError, match="v8t"):
        ops.attn_fwd_q(q, 0.1, k8, v8t.transpose(2, 3), sk, sv, None, None, -1.0, S)
    with pytest.raises(ValueError, match="q8"):
        ops.attn_fwd(q8[:, :, :256], k8, v8t, sq, sk, sv, None, None, -1.0, q, S)
    torch.cuda.synchronize()
    out = ops.attn_fwd_q(q, 0.1, k8, v8t, sk, sv, None, None, -1.0, S)
    assert out.shape == q.shape
