"""GPU quantizers on non-finite inputs, bit for bit against the oracle.

The reference kernels take block maxima and clamp with Triton's tl.max / tl.maximum /
tl.minimum, which skip NaN (kernels/fp8_linear.py:20-22, kernels/fp8_attention.py:54-77,
136-170): a NaN element does not enter the scale and its quotient clamps to -448; a block
maximum of inf gives the scale inf, finite elements quantize to +-0 and +-inf to -448.
The oracle states those semantics (pinned by closed forms in the CPU suite).
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import linear as ol
from oracle.numerics import bf16_round
from tests.helpers import codes, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rows_with_non_finite(rng, M, K):
    x = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    x[0, 3] = np.inf                 # row maximum inf
    x[1, 5] = -np.inf
    x[2, 7] = np.nan                 # NaN skipped by the maximum
    x[3, :] = np.nan                 # all NaN: the scale floor
    x[4, 1], x[4, 2] = np.nan, np.inf
    return x


# One wave per row with whole rows in registers (K = 3072 / 12288 bf16, 3072 fp16, 1024 fp32:
# 64 lanes x 16 bytes x NC chunks exactly), with a partial last chunk (K = 1000, 200), and the
# general path (K = 100 is not a multiple of the 16-byte chunk).  Each register path has its
# own NaN-skipping maximum per element type.
@pytest.mark.parametrize("K,dtype", [(3072, torch.bfloat16), (12288, torch.bfloat16), (1000, torch.bfloat16),
                                     (3072, torch.float16), (200, torch.float16), (1024, torch.float32),
                                     (100, torch.bfloat16)])
def test_quant_rows_non_finite(K, dtype):
    _say(f"quant_rows non-finite K={K} {dtype}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(K)
    x = _rows_with_non_finite(rng, 9, K)
    if dtype == torch.float16:
        x = x.astype(np.float16).astype(np.float32)
    x8, sa = ops.quant_rows(to_gpu(x, dtype))
    rc, rs = ol.quantize_rows(x)
    np.testing.assert_array_equal(codes(x8), rc)
    np.testing.assert_array_equal(sa.cpu().numpy(), rs)


def test_attention_quantizers_non_finite():
    _say("attention quantizers non-finite")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(7)
    B, H, S, D = 1, 2, 300, 128
    q = bf16_round(rng.standard_normal((B, H, S, D)).astype(np.float32))
    v = bf16_round(rng.standard_normal((B, H, S, D)).astype(np.float32))
    q[0, 0, 10, 4] = np.inf      # Q block 0 of head 0: scale inf
    q[0, 1, 200, 9] = np.nan     # Q block 1 of head 1: NaN skipped
    q[0, 1, 0:128, :] = np.nan   # Q block 0 of head 1: all NaN
    v[0, 0, 17, 3] = -np.inf     # V channel 3 of head 0: scale inf
    v[0, 1, 40, 8] = np.nan      # V channel 8 of head 1: NaN skipped
    c = np.float32(oa.LOG2E / math.sqrt(D))
    q8, sq = ops.attn_quant_q(to_gpu(q), float(c))
    rq8, rsq = oa.quantize_q(q, c)
    np.testing.assert_array_equal(sq.cpu().numpy(), rsq)
    np.testing.assert_array_equal(codes(q8)[:, :, :S], rq8)
    v8t, sv = ops.attn_quant_v(to_gpu(v))
    rv8t, rsv = oa.quantize_v(v)
    np.testing.assert_array_equal(sv.cpu().numpy(), rsv)
    np.testing.assert_array_equal(codes(v8t)[..., :S], rv8t)
