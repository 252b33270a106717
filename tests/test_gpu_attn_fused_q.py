"""GPU parity of the fused Q quantizer + attention forward (mxf8_attn_fwd_q).

The fused launch must reproduce mxf8_attn_quant_q followed by mxf8_attn_fwd bit for bit
(same Q codes and scales, then the same kernel arithmetic), its Q scales must equal the
oracle's quantize_q (fp8_attention.py:54-77), and its output must equal, bit for bit in all
but rare cases, the oracle's forward computed with the fp8 instruction's arithmetic
(oracle.mfma: Q K^T, P V and the row sums), within 2 ulps with the repair.  For rows of
ordinary sharpness (q_std <= 1) it must also meet the attention bar against the
exact-product oracle.  In sharply peaked rows a P code whose 8 S + 56 - 8 m lies within a
few thousandths of a rounding boundary follows the instruction's rounding of the dot
product, and one such code of a dominant key moves the output by up to 4e-2 against the
exact products.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import assert_attn_close, assert_attn_model, bf16_randn, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _layout(x_np, layout, dtype):
    """[B,H,S,D] numpy -> GPU tensor: contiguous, a permuted view of [B,S,H,D] storage, or
    slot 1 of a [B,S,3,H,D] fused projection output (the DiT block's q/k/v views)."""
    if layout == "contig":
        return to_gpu(x_np, dtype)
    if layout == "perm":
        return to_gpu(np.ascontiguousarray(x_np.transpose(0, 2, 1, 3)), dtype).permute(0, 2, 1, 3)
    B, H, S, D = x_np.shape
    qkv = np.zeros((B, S, 3, H, D), np.float32)
    qkv[:, :, 1] = x_np.transpose(0, 2, 1, 3)
    return to_gpu(qkv, dtype)[:, :, 1].permute(0, 2, 1, 3)


def _bits(t):
    return t.view(torch.int16).cpu()


def _fused_abi(q, c, k8, v8t, sk, sv, km, kb, tau, Sk, nq, kv_mode):
    """mxf8_attn_fwd_q through the C ABI, with the Q scales written out."""
    from minimaxh3_amd import _native as N
    B, H, Sq, D = q.shape
    out = torch.empty_like(q)
    sq = torch.full((B, H, nq), -1.0, dtype=torch.float32, device=q.device)
    km = None if km is None else km.to(torch.uint8).contiguous()
    N.check(N.load().mxf8_attn_fwd_q(
        q.data_ptr(), N.strides4(q), float(c), k8.data_ptr(), v8t.data_ptr(), sk.data_ptr(), sv.data_ptr(),
        N.ptr(km), N.ptr(kb), float(tau), sq.data_ptr(), out.data_ptr(), N.dtype_code(out.dtype), N.strides4(out),
        B, H, Sq, Sk, D, kv_mode, N.stream_of(q)), "attn_fwd_q")
    torch.cuda.synchronize()
    return out, sq


CASES = [
    # B, H, Sq, Sk, D, dtype, layout, mask, bias, tau, q_std
    (2, 2, 300, 700, 128, torch.bfloat16, "qkv", False, False, -1.0, 1.0),
    (1, 3, 130, 200, 64, torch.float16, "perm", True, False, -1.0, 1.0),
    (2, 2, 257, 512, 128, torch.bfloat16, "contig", True, True, 0.5, 1.0),
    (1, 2, 5, 300, 128, torch.bfloat16, "contig", False, True, -1.0, 1.0),
    (1, 1, 128, 1, 64, torch.bfloat16, "qkv", False, False, 0.0, 1.0),
    (1, 2, 384, 256, 128, torch.bfloat16, "perm", False, False, -1.0, 300.0),
    # peaked rows over a long key sequence (with a key mask, rows whose few valid keys dominate)
    (1, 2, 640, 2048, 128, torch.bfloat16, "contig", False, False, -1.0, 4.0),
    (1, 2, 640, 2048, 128, torch.bfloat16, "qkv", True, False, 0.5, 4.0),
]


@pytest.mark.parametrize("B,H,Sq,Sk,D,dtype,layout,use_mask,use_bias,tau,q_std", CASES)
def test_fused_q_equals_two_calls_and_oracle(B, H, Sq, Sk, D, dtype, layout, use_mask, use_bias, tau, q_std):
    _say(f"attn fused-Q B={B} H={H} Sq={Sq} Sk={Sk} D={D} {dtype} {layout} mask={use_mask} bias={use_bias} "
         f"tau={tau} q_std={q_std}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(Sq * 13 + Sk + D)
    q = bf16_randn(rng, (B, H, Sq, D), q_std)
    if Sq >= 256:
        q[:, 0, 128:256] = 0.0  # an all-zero Q block: the scale floor, codes 0
    k, v = bf16_randn(rng, (B, H, Sk, D)), bf16_randn(rng, (B, H, Sk, D))
    if dtype == torch.float16:
        q, k, v = (t.astype(np.float16).astype(np.float32) for t in (q, k, v))
    mask = bias = None
    if use_mask:
        mask = np.ones((B, Sk), bool)
        mask[-1, Sk // 2:] = False
        mask[0, rng.choice(Sk, Sk // 10, replace=False)] = False
    if use_bias:
        bias = (rng.standard_normal((B, Sk)) * 0.5).astype(np.float32)
        bias[0, :3] = -1e9
    qg, kg, vg = (_layout(t, layout, dtype) for t in (q, k, v))
    assert ops.attn_fwd_q_supported(qg)
    c = np.float32(oa.LOG2E / math.sqrt(D))
    km = None if mask is None else to_gpu(mask.astype(np.uint8), torch.bool)
    kb = None if bias is None else to_gpu(bias, torch.float32)

    k8, sk = ops.attn_quant_k(kg, ops.attn_kmean(kg))
    v8t, sv = ops.attn_quant_v(vg)
    q8, sq = ops.attn_quant_q(qg, float(c))
    two = ops.attn_fwd(q8, k8, v8t, sq, sk, sv, km, kb, float(tau), qg, Sk)
    nq = -(-Sq // 128)
    # kv_mode 0 takes the resident-K/V kernel where K/V fit in LDS and tau < 0, 1 streams
    for kv_mode in (0, 1):
        fused, sq_f = _fused_abi(qg, c, k8, v8t, sk, sv, km, kb, tau, Sk, nq, kv_mode)
        assert fused.stride() == two.stride()
        assert torch.equal(_bits(fused), _bits(two)), kv_mode
        assert torch.equal(sq_f, sq), kv_mode
    np.testing.assert_array_equal(sq_f.cpu().numpy(), oa.quantize_q(q, c)[1])
    via_op = ops.attn_fwd_q(qg, float(c), k8, v8t, sk, sv, km, kb, float(tau), Sk)
    assert torch.equal(_bits(via_op), _bits(fused))

    out_dtype = "bf16" if dtype == torch.bfloat16 else "fp16"
    got = fused.float().cpu().numpy()
    ref_mfma, _ = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=bias, repair_tau=tau, out_dtype=out_dtype,
                                   dot="mfma")
    assert_attn_model(got, ref_mfma, out_dtype, tau)
    if q_std <= 1.0:
        ref, _ = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=bias, repair_tau=tau, out_dtype=out_dtype)
        assert_attn_close(got, ref)


def test_fp8_attention_fused_and_two_call_paths_agree():
    """fp8_attention takes the fused launch where q's layout allows it and the two-call
    path otherwise (here: a row stride of D + 4 elements); both give the same bits."""
    _say("attn fused-Q: fp8_attention paths")
    from minimaxh3_amd import ops
    from minimaxh3_amd.kernels import fp8_attention as fa
    rng = np.random.default_rng(21)
    B, H, S, D = 1, 2, 300, 128
    q, k, v = (bf16_randn(rng, (B, H, S, D)) for _ in range(3))
    mask = np.ones((B, S), bool)
    mask[0, 250:] = False
    qg, kg, vg = (_layout(t, "qkv", torch.bfloat16) for t in (q, k, v))
    km = to_gpu(mask, torch.bool)
    wide = torch.zeros((B, H, S, D + 4), dtype=torch.bfloat16, device="cuda")
    wide[..., :D] = qg
    q_odd = wide[..., :D]
    assert ops.attn_fwd_q_supported(qg) and not ops.attn_fwd_q_supported(q_odd)
    saved = fa.fuse_q_quant
    try:
        fa.fuse_q_quant = True
        fused = fa.fp8_attention(qg, kg, vg, key_mask=km)
        odd = fa.fp8_attention(q_odd, kg, vg, key_mask=km)
        fa.fuse_q_quant = False
        two = fa.fp8_attention(qg, kg, vg, key_mask=km)
    finally:
        fa.fuse_q_quant = saved
    torch.cuda.synchronize()
    assert torch.equal(_bits(fused), _bits(two))
    assert torch.equal(_bits(odd.contiguous()), _bits(two.contiguous()))
    # a view 8 bytes off a 16-byte boundary passes the layout check; the op sees the
    # pointer and runs the two launches
    flat = torch.zeros(B * H * S * D + 8, dtype=torch.bfloat16, device="cuda")
    q_off = flat[4:4 + B * H * S * D].view(B, H, S, D)
    q_off.copy_(qg)
    assert ops.attn_fwd_q_supported(q_off) and q_off.data_ptr() % 16 == 8
    fa.fuse_q_quant = True
    off = fa.fp8_attention(q_off, kg, vg, key_mask=km)
    fa.fuse_q_quant = saved
    assert torch.equal(_bits(off), _bits(two.contiguous()))
    k8, sk = ops.attn_quant_k(kg, ops.attn_kmean(kg))
    v8t, sv = ops.attn_quant_v(vg)
    with pytest.raises(ValueError, match="unit channel stride"):
        ops.attn_fwd_q(q_odd, 1.0, k8, v8t, sk, sv, km, None, -1.0, S)


@pytest.mark.parametrize("B,Sq,Sk,masked", [(1, 20280, 20280, 0), (2, 21304, 21304, 384), (2, 21304, 512, 0)])
def test_fused_q_full_size_equals_two_calls(B, Sq, Sk, masked):
    """At the workloads' full sizes (480p self-attention, the joint self-attention with
    item 1's last keys masked, text cross-attention), the fused launch and the two launches
    give the same bits on every output element."""
    _say(f"attn fused-Q full size B={B} Sq={Sq} Sk={Sk} masked={masked}")
    from minimaxh3_amd import ops
    H, D = 24, 128
    g = torch.Generator(device="cuda").manual_seed(Sq + Sk)
    q = torch.randn((B, Sq, H, D), device="cuda", generator=g).to(torch.bfloat16).permute(0, 2, 1, 3)
    kv = torch.randn((B, Sk, 2, H, D), device="cuda", generator=g).to(torch.bfloat16)
    k, v = kv[:, :, 0].permute(0, 2, 1, 3), kv[:, :, 1].permute(0, 2, 1, 3)
    km = None
    if masked:
        km = torch.ones((B, Sk), dtype=torch.bool, device="cuda")
        km[1, Sk - masked:] = False
    c = ops.softmax_c(None, D)
    k8, sk = ops.attn_quant_k(k, ops.attn_kmean(k))
    v8t, sv = ops.attn_quant_v(v)
    q8, sq = ops.attn_quant_q(q, c)
    two = ops.attn_fwd(q8, k8, v8t, sq, sk, sv, km, None, -1.0, q, Sk)
    fused = ops.attn_fwd_q(q, c, k8, v8t, sk, sv, km, None, -1.0, Sk)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))
    assert torch.isfinite(fused.float()).all()
