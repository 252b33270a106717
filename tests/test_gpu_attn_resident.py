"""GPU parity of the resident-KV attention kernel (short key sequences).

When every KV tile of a head fits in LDS (Sk <= 512 at D = 128, <= 1024 at D = 64) and no
repair is asked for, the launcher runs attn_fwd_resident_kernel.  Per Q tile it performs
attn_fwd_kernel's arithmetic in the same KV visit order, so both kernels must give the same
bits; kv_mode 1 (MXF8_ATTN_KV_STREAM) selects attn_fwd_kernel for the comparison.  With Q
as 16-bit values (mxf8_attn_fwd_q) each group quantizes its own Q block inside the resident
kernel, and the result must equal the two-call path's.  The output is also held to the
attention bar against the oracle.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import assert_attn_close, bf16_randn, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _both(fn):
    """fn(kv_mode) with the resident kernel allowed (0), then with K/V streamed (1)."""
    a = fn(0)
    b = fn(1)
    torch.cuda.synchronize()
    return a, b


CASES = [
    # B, H, Sq, Sk, D, dtype, mask, bias
    (2, 3, 1000, 512, 128, torch.bfloat16, False, False),
    (1, 5, 700, 300, 128, torch.bfloat16, True, False),
    (2, 2, 257, 77, 128, torch.float16, False, True),
    (2, 2, 390, 500, 128, torch.bfloat16, True, True),
    (1, 4, 333, 1024, 64, torch.bfloat16, True, False),
    (3, 2, 129, 900, 64, torch.float16, False, True),
    (1, 1, 5, 128, 128, torch.bfloat16, False, False),
    (1, 3, 640, 256, 64, torch.bfloat16, True, True),
]


@pytest.mark.parametrize("B,H,Sq,Sk,D,dtype,use_mask,use_bias", CASES)
def test_resident_kv_equals_streaming_kernel(B, H, Sq, Sk, D, dtype, use_mask, use_bias):
    _say(f"attn resident-KV B={B} H={H} Sq={Sq} Sk={Sk} D={D} {dtype} mask={use_mask} bias={use_bias}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(Sq * 7 + Sk * 3 + D)
    q = bf16_randn(rng, (B, H, Sq, D))
    k, v = bf16_randn(rng, (B, H, Sk, D)), bf16_randn(rng, (B, H, Sk, D))
    if dtype == torch.float16:
        q, k, v = (t.astype(np.float16).astype(np.float32) for t in (q, k, v))
    mask = bias = None
    if use_mask:
        mask = np.ones((B, Sk), bool)
        mask[-1, Sk // 3:] = False
        mask[0, rng.choice(Sk, Sk // 8, replace=False)] = False
    if use_bias:
        bias = (rng.standard_normal((B, Sk)) * 0.5).astype(np.float32)
        bias[0, :5] = -1e9
    qg = to_gpu(np.ascontiguousarray(q.transpose(0, 2, 1, 3)), dtype).permute(0, 2, 1, 3)
    kg, vg = to_gpu(k, dtype), to_gpu(v, dtype)
    km = None if mask is None else to_gpu(mask.astype(np.uint8), torch.bool)
    kb = None if bias is None else to_gpu(bias, torch.float32)
    c = np.float32(oa.LOG2E / math.sqrt(D))
    k8, sk = ops.attn_quant_k(kg, ops.attn_kmean(kg))
    v8t, sv = ops.attn_quant_v(vg)
    q8, sq = ops.attn_quant_q(qg, float(c))
    res, stream = _both(lambda m: ops.attn_fwd(q8, k8, v8t, sq, sk, sv, km, kb, -1.0, qg, Sk, m))
    assert torch.equal(res.view(torch.int16), stream.view(torch.int16))
    fres, fstream = _both(lambda m: ops.attn_fwd_q(qg, float(c), k8, v8t, sk, sv, km, kb, -1.0, Sk, m))
    assert torch.equal(fres.view(torch.int16), res.view(torch.int16))
    assert torch.equal(fstream.view(torch.int16), res.view(torch.int16))
    ref, _ = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=bias, repair_tau=-1.0,
                              out_dtype="bf16" if dtype == torch.bfloat16 else "fp16")
    assert_attn_close(res.float().cpu().numpy(), ref)


@pytest.mark.parametrize("D", [128, 64])
def test_streaming_kernel_skips_fully_masked_tiles(D):
    """Whole 128-key tiles masked out (the first, a middle and the last one, and every tile of
    one batch item): both kernels skip their products, which would only have added zeros (the
    resident kernel not on an item's last tile), so they must agree bit for bit; the item with
    no valid key gives zeros."""
    _say(f"attn fully masked tiles D={D}")
    from minimaxh3_amd import ops
    B, H, Sq, Sk = 3, 2, 300, 512
    rng = np.random.default_rng(31 + D)
    q = bf16_randn(rng, (B, H, Sq, D))
    k, v = bf16_randn(rng, (B, H, Sk, D)), bf16_randn(rng, (B, H, Sk, D))
    mask = np.ones((B, Sk), bool)
    mask[0, 128:256] = False
    mask[0, rng.choice(Sk, 40, replace=False)] = False
    mask[1, :128] = False
    mask[1, 384:] = False
    mask[1, 300:310] = False
    mask[2, :] = False
    qg = to_gpu(np.ascontiguousarray(q.transpose(0, 2, 1, 3))).permute(0, 2, 1, 3)
    kg, vg = to_gpu(k), to_gpu(v)
    km = to_gpu(mask.astype(np.uint8), torch.bool)
    c = np.float32(oa.LOG2E / math.sqrt(D))
    k8, sk = ops.attn_quant_k(kg, ops.attn_kmean(kg))
    v8t, sv = ops.attn_quant_v(vg)
    q8, sq = ops.attn_quant_q(qg, float(c))
    res, stream = _both(lambda m: ops.attn_fwd(q8, k8, v8t, sq, sk, sv, km, None, -1.0, qg, Sk, m))
    assert torch.equal(res.view(torch.int16), stream.view(torch.int16))
    fres, fstream = _both(lambda m: ops.attn_fwd_q(qg, float(c), k8, v8t, sk, sv, km, None, -1.0, Sk, m))
    assert torch.equal(fstream.view(torch.int16), res.view(torch.int16))
    assert torch.equal(fres.view(torch.int16), res.view(torch.int16))
    assert not res[2].any()
    ref, _ = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=None, repair_tau=-1.0, out_dtype="bf16")
    assert_attn_close(res[:2].float().cpu().numpy(), ref[:2])


def test_resident_kv_text_cross_attention_full_size():
    """The joint workload's text cross-attention (B=2, H=24, Sq=21304, Sk=512): both kernels,
    with Q from q8 / sq and with Q quantized inside the launch, give the same bits at full
    size."""
    _say("attn resident-KV full-size cross-attention")
    from minimaxh3_amd import ops
    B, H, Sq, Sk, D = 2, 24, 21304, 512, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((B, Sq, H, D), device="cuda", generator=g).to(torch.bfloat16).permute(0, 2, 1, 3)
    kv = torch.randn((B, Sk, 2, H, D), device="cuda", generator=g).to(torch.bfloat16)
    k, v = kv[:, :, 0].permute(0, 2, 1, 3), kv[:, :, 1].permute(0, 2, 1, 3)
    c = ops.softmax_c(None, D)
    k8, sk = ops.attn_quant_k(k, ops.attn_kmean(k))
    v8t, sv = ops.attn_quant_v(v)
    q8, sq = ops.attn_quant_q(q, c)
    res, stream = _both(lambda m: ops.attn_fwd(q8, k8, v8t, sq, sk, sv, None, None, -1.0, q, Sk, m))
    assert torch.equal(res.view(torch.int16), stream.view(torch.int16))
    fres, fstream = _both(lambda m: ops.attn_fwd_q(q, c, k8, v8t, sk, sv, None, None, -1.0, Sk, m))
    assert torch.equal(fres.view(torch.int16), res.view(torch.int16))
    assert torch.equal(fstream.view(torch.int16), res.view(torch.int16))
    assert torch.isfinite(res.float()).all()


@pytest.mark.parametrize("D,Sk", [(128, 300), (64, 1000)])
def test_resident_kv_many_tiles_per_workgroup_mask_bias(D, Sk):
    """More Q tiles than CUs (B=2, H=8, Sq=21000: 2640 work items), so each workgroup walks a
    range that crosses heads at arbitrary offsets and pairs tiles; with a key mask, a bias and
    a ragged last key tile.  Bit for bit against the streaming kernel."""
    _say(f"attn resident-KV many tiles D={D} Sk={Sk}")
    from minimaxh3_amd import ops
    B, H, Sq = 2, 8, 21000
    g = torch.Generator(device="cuda").manual_seed(D + Sk)
    q = torch.randn((B, Sq, H, D), device="cuda", generator=g).to(torch.bfloat16).permute(0, 2, 1, 3)
    kv = torch.randn((B, Sk, 2, H, D), device="cuda", generator=g).to(torch.bfloat16)
    k, v = kv[:, :, 0].permute(0, 2, 1, 3), kv[:, :, 1].permute(0, 2, 1, 3)
    km = torch.rand((B, Sk), device="cuda", generator=g) > 0.25
    km[1, Sk // 2:] = False
    kb = torch.randn((B, Sk), device="cuda", generator=g)
    kb[0, :4] = -1e9
    c = ops.softmax_c(None, D)
    k8, sk = ops.attn_quant_k(k, ops.attn_kmean(k))
    v8t, sv = ops.attn_quant_v(v)
    q8, sq = ops.attn_quant_q(q, c)
    res, stream = _both(lambda m: ops.attn_fwd(q8, k8, v8t, sq, sk, sv, km, kb, -1.0, q, Sk, m))
    assert torch.equal(res.view(torch.int16), stream.view(torch.int16))
    fres, fstream = _both(lambda m: ops.attn_fwd_q(q, c, k8, v8t, sk, sv, km, kb, -1.0, Sk, m))
    assert torch.equal(fres.view(torch.int16), res.view(torch.int16))
    assert torch.equal(fstream.view(torch.int16), res.view(torch.int16))
    assert torch.isfinite(res.float()).all()


@pytest.mark.parametrize("D", [128, 64])
def test_resident_kv_output_channel_stride(D):
    """A query whose channel stride is not 1 (a [B, D, H, S] tensor viewed as [B, H, S, D]):
    the output takes the query's strides, so the resident kernel's staged stores write it two
    bytes at a time.  Bit for bit against the streaming kernel, which writes it element by
    element, and close to the oracle."""
    _say(f"attn resident-KV output channel stride D={D}")
    from minimaxh3_amd import ops
    B, H, Sq, Sk = 1, 3, 300, 200
    rng = np.random.default_rng(D + 11)
    q = bf16_randn(rng, (B, H, Sq, D))
    k, v = bf16_randn(rng, (B, H, Sk, D)), bf16_randn(rng, (B, H, Sk, D))
    qg = to_gpu(np.ascontiguousarray(q.transpose(0, 3, 1, 2)), torch.bfloat16).permute(0, 2, 3, 1)
    assert qg.stride(-1) != 1
    kg, vg = to_gpu(k, torch.bfloat16), to_gpu(v, torch.bfloat16)
    c = np.float32(oa.LOG2E / math.sqrt(D))
    k8, sk = ops.attn_quant_k(kg, ops.attn_kmean(kg))
    v8t, sv = ops.attn_quant_v(vg)
    q8, sq = ops.attn_quant_q(qg.contiguous(), float(c))
    res, stream = _both(lambda m: ops.attn_fwd(q8, k8, v8t, sq, sk, sv, None, None, -1.0, qg, Sk, m))
    assert res.stride() == qg.stride()
    assert torch.equal(res.view(torch.int16), stream.view(torch.int16))
    ref, _ = oa.fp8_attention(q, k, v, key_mask=None, key_bias=None, repair_tau=-1.0, out_dtype="bf16")
    assert_attn_close(res.float().cpu().numpy(), ref)
