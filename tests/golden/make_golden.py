"""Writes the golden fixtures of the FP8 hot path (tests/golden/*.npz) from the CPU oracle.

The reference ships no tests, fixtures or known-answer vectors for this path, so these
vectors are produced by the oracle (oracle/), itself pinned by closed forms, torch CPU
casts and brute-force loops (tests/test_oracle_*.py).  They freeze the oracle's outputs
on small seeded inputs so that (a) a later change to the oracle that alters its results
is caught on the CPU, and (b) the HIP path is compared with the same fixed inputs and
outputs on the GPU.  bf16 values are stored as uint16 bit patterns, e4m3 as uint8 codes.

    python tests/golden/make_golden.py      # rewrites the .npz files next to this script

Fixtures
--------
quant_rows.npz   x bf16 [37, 1024] (outliers x20, an all-zero row, a row whose amax element
                 maps to exactly -448, a row of exact e4m3 midpoints) -> codes, scales
linear.npz       x bf16 [40, 256], W bf16 [96, 256], bias bf16 [96], LoRA A [8, 256],
                 B [96, 8], scale 0.75 -> weight codes/scales, plain, +GELU, +LoRA,
                 +LoRA+GELU outputs (bf16)
attention.npz    q bf16 [2, 1, 136, 128], k/v bf16 [2, 1, 260, 128] (non-zero key mean),
                 key mask (item 1 keeps keys < 200), key bias -> quantizer outputs and
                 the forward for (no mask, tau -1), (mask, tau -1), (mask, tau 0.5),
                 (bias, tau -1)
attention_d64.npz  q/k/v bf16 [1, 2, 150, 64], fp16 output, tau -1
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import attention as oa  # noqa: E402
from oracle import linear as ol  # noqa: E402
from oracle.numerics import bf16_bits, bf16_round  # noqa: E402


def _randn(rng, shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def quant_rows_fixture():
    rng = np.random.default_rng(101)
    M, K = 37, 1024
    x = _randn(rng, (M, K))
    idx = rng.choice(K, K // 100, replace=False)
    x[:, idx] *= 20.0
    x = bf16_round(x)
    x[3] = 0.0                                   # all-zero row: scale 1e-12/448, codes 0
    x[5, :] = 1.0
    x[5, 7] = -448.0                             # amax element maps to exactly -448 (0xFE)
    # row 9: values on e4m3 rounding midpoints once divided by scale = 1 (amax 448)
    mids = np.array([1.0625, 1.1875, 0.0087890625, 3.25 + 0.125, -1.0625, -2.375], np.float32)
    x[9, :] = 0.5
    x[9, 0] = 448.0
    x[9, 1:1 + len(mids)] = mids
    x = bf16_round(x)
    codes, scale = ol.quantize_rows(x)
    return dict(x=bf16_bits(x), codes=codes, scale=scale)


def linear_fixture():
    rng = np.random.default_rng(202)
    M, K, N, r = 40, 256, 96, 8
    x = _randn(rng, (M, K))
    w = _randn(rng, (N, K), 0.02)
    bias = _randn(rng, (N,), 0.01)
    A = _randn(rng, (r, K), 0.05)
    B = _randn(rng, (N, r), 0.05)
    lscale = 0.75
    w8, sw = ol.quantize_rows(w)
    sw = sw.reshape(-1)
    plain = ol.fp8_linear_forward(x, w8, sw, bias)
    gelu = ol.fp8_linear_forward(x, w8, sw, bias, gelu=True)
    lora = ol.fp8_linear_forward(x, w8, sw, bias, adapters=[(A, B, lscale)])
    lora_gelu = ol.fp8_linear_forward(x, w8, sw, bias, adapters=[(A, B, lscale)], gelu=True)
    return dict(x=bf16_bits(x), w=bf16_bits(w), bias=bf16_bits(bias), lora_a=bf16_bits(A), lora_b=bf16_bits(B),
                lora_scale=np.float32(lscale), w8=w8, w_scale=sw, out_plain=bf16_bits(plain),
                out_gelu=bf16_bits(gelu), out_lora=bf16_bits(lora), out_lora_gelu=bf16_bits(lora_gelu))


def attention_fixture():
    rng = np.random.default_rng(303)
    B, H, Sq, Sk, D = 2, 1, 136, 260, 128
    q = _randn(rng, (B, H, Sq, D))
    k = bf16_round(_randn(rng, (B, H, Sk, D)) + _randn(rng, (1, 1, 1, D), 2.0))
    v = _randn(rng, (B, H, Sk, D))
    mask = np.ones((B, Sk), bool)
    mask[1, 200:] = False
    bias = (rng.standard_normal((B, Sk)) * 0.5).astype(np.float32)
    bias[0, 10:20] = -1.0e9                      # masked through the bias
    out = {}
    cases = {"plain": dict(), "mask": dict(key_mask=mask), "mask_tau05": dict(key_mask=mask, repair_tau=0.5),
             "bias": dict(key_bias=bias)}
    inter = None
    for name, kw in cases.items():
        o, inter = oa.fp8_attention(q, k, v, **kw)
        out[f"out_{name}"] = bf16_bits(o)
    return dict(q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), key_mask=mask, key_bias=bias,
                c=np.float32(inter["c"]), q8=inter["q8"], sq=inter["sq"], mu=inter["mu"][:, :, 0, :],
                k8=inter["k8"], sk=inter["sk"], v8t=inter["v8t"], sv=inter["sv"], **out)


def attention_d64_fixture():
    rng = np.random.default_rng(404)
    B, H, S, D = 1, 2, 150, 64
    q, k, v = (_randn(rng, (B, H, S, D)) for _ in range(3))
    o, inter = oa.fp8_attention(q, k, v, out_dtype="fp16")
    return dict(q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), out=o.astype(np.float16),
                scale_c=np.float32(oa.LOG2E / math.sqrt(D)))


FIXTURES = {
    "quant_rows": quant_rows_fixture,
    "linear": linear_fixture,
    "attention": attention_fixture,
    "attention_d64": attention_d64_fixture,
}


def main() -> None:
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
