"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every stored output exactly from the stored inputs, so a
change to the oracle's results cannot go unnoticed.  GPU: the HIP path on the same
inputs gives bit-exact codes and scales, GEMM outputs within 1e-2 relative and attention
outputs at cosine >= 0.999 and max-abs <= 2e-2 of the stored outputs.
"""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import linear as ol
from oracle.numerics import bf16_from_bits
from tests.helpers import assert_attn_close, assert_gemm_close, codes, to_gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ---- CPU: the oracle against the fixtures -------------------------------------------------

def test_oracle_reproduces_quant_rows():
    g = _load("quant_rows")
    c, s = ol.quantize_rows(bf16_from_bits(g["x"]))
    np.testing.assert_array_equal(c, g["codes"])
    np.testing.assert_array_equal(s, g["scale"])
    # closed forms planted in the fixture
    assert g["scale"][3, 0] == np.float32(1e-12) / np.float32(448) and not g["codes"][3].any()
    assert g["codes"][5, 7] == 0xFE
    assert list(g["codes"][9, :7]) == [0x7E, 0x38, 0x3A, 0x04, 0x46, 0xB8, 0xC2]


def test_oracle_reproduces_linear():
    g = _load("linear")
    x, w, bias = (bf16_from_bits(g[n]) for n in ("x", "w", "bias"))
    A, B = bf16_from_bits(g["lora_a"]), bf16_from_bits(g["lora_b"])
    w8, sw = ol.quantize_rows(w)
    np.testing.assert_array_equal(w8, g["w8"])
    np.testing.assert_array_equal(sw.reshape(-1), g["w_scale"])
    ad = [(A, B, float(g["lora_scale"]))]
    for name, kw in (("plain", {}), ("gelu", dict(gelu=True)), ("lora", dict(adapters=ad)),
                     ("lora_gelu", dict(adapters=ad, gelu=True))):
        out = ol.fp8_linear_forward(x, w8, sw.reshape(-1), bias, **kw)
        np.testing.assert_array_equal(out, bf16_from_bits(g[f"out_{name}"]), err_msg=name)


def _attn_cases(g):
    return {"plain": {}, "mask": dict(key_mask=g["key_mask"]),
            "mask_tau05": dict(key_mask=g["key_mask"], repair_tau=0.5), "bias": dict(key_bias=g["key_bias"])}


def test_oracle_reproduces_attention():
    g = _load("attention")
    q, k, v = (bf16_from_bits(g[n]) for n in ("q", "k", "v"))
    for name, kw in _attn_cases(g).items():
        o, inter = oa.fp8_attention(q, k, v, **kw)
        np.testing.assert_array_equal(o, bf16_from_bits(g[f"out_{name}"]), err_msg=name)
    for n in ("q8", "sq", "k8", "sk", "v8t", "sv"):
        np.testing.assert_array_equal(inter[n], g[n], err_msg=n)
    np.testing.assert_array_equal(inter["mu"][:, :, 0, :], g["mu"])


def test_oracle_reproduces_attention_d64():
    g = _load("attention_d64")
    q, k, v = (bf16_from_bits(g[n]) for n in ("q", "k", "v"))
    o, _ = oa.fp8_attention(q, k, v, out_dtype="fp16")
    np.testing.assert_array_equal(o.astype(np.float16), g["out"])


# ---- GPU: the HIP path against the fixtures -----------------------------------------------

def _bf16_gpu(bits):
    return to_gpu(bf16_from_bits(bits), torch.bfloat16)


@pytest.mark.gpu
def test_gpu_quant_rows_golden():
    _say("golden quant_rows [37, 1024]")
    from minimaxh3_amd.kernels import fp8_linear as fl
    g = _load("quant_rows")
    x8, s = fl.quantize_rows(_bf16_gpu(g["x"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(codes(x8), g["codes"])
    np.testing.assert_array_equal(s.cpu().numpy(), g["scale"])


@pytest.mark.gpu
def test_gpu_linear_golden():
    _say("golden linear M=40 N=96 K=256")
    from minimaxh3_amd.kernels import fp8_linear as fl
    g = _load("linear")
    dev = torch.device("cuda")
    lin = torch.nn.Linear(256, 96, bias=True, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(_bf16_gpu(g["w"]))
        lin.bias.copy_(_bf16_gpu(g["bias"]))
    mod = fl.FP8Linear.from_linear(lin)
    np.testing.assert_array_equal(codes(mod.w8), g["w8"])
    np.testing.assert_array_equal(mod.w_scale.cpu().numpy().reshape(-1), g["w_scale"])
    x = _bf16_gpu(g["x"])
    ad = (_bf16_gpu(g["lora_a"]), _bf16_gpu(g["lora_b"]), float(g["lora_scale"]))
    for name, act, adapters in (("plain", 0, []), ("gelu", 1, []), ("lora", 0, [ad]), ("lora_gelu", 1, [ad])):
        mod.act = act
        mod.adapters = adapters
        out = mod(x).float().cpu().numpy()
        assert_gemm_close(out, bf16_from_bits(g[f"out_{name}"]))


@pytest.mark.gpu
def test_gpu_attention_golden():
    _say("golden attention B=2 H=1 Sq=136 Sk=260 D=128")
    from minimaxh3_amd import ops
    from minimaxh3_amd.kernels import fp8_attention as fa
    g = _load("attention")
    q, k, v = (_bf16_gpu(g[n]) for n in ("q", "k", "v"))
    q8, sq = ops.attn_quant_q(q, float(g["c"]))
    Sq, Sk = q.shape[2], k.shape[2]
    np.testing.assert_array_equal(codes(q8)[:, :, :Sq], g["q8"])
    np.testing.assert_array_equal(sq.cpu().numpy(), g["sq"])
    k8, sk = ops.attn_quant_k(k, to_gpu(g["mu"], torch.float32))
    np.testing.assert_array_equal(codes(k8)[:, :, :Sk], g["k8"])
    np.testing.assert_array_equal(sk.cpu().numpy(), g["sk"])
    v8t, sv = ops.attn_quant_v(v)
    np.testing.assert_array_equal(codes(v8t)[..., :Sk], g["v8t"])
    np.testing.assert_array_equal(sv.cpu().numpy(), g["sv"])
    for name, kw in _attn_cases(g).items():
        args = dict(repair_tau=kw.get("repair_tau", -1.0))
        if "key_mask" in kw:
            args["key_mask"] = to_gpu(kw["key_mask"], torch.bool)
        if "key_bias" in kw:
            args["key_bias"] = to_gpu(kw["key_bias"], torch.float32)
        o = fa.fp8_attention(q, k, v, **args)
        assert_attn_close(o.float().cpu().numpy(), bf16_from_bits(g[f"out_{name}"]))


@pytest.mark.gpu
def test_gpu_attention_d64_golden():
    _say("golden attention D=64 fp16 out")
    from minimaxh3_amd.kernels import fp8_attention as fa
    g = _load("attention_d64")
    q, k, v = (to_gpu(bf16_from_bits(g[n]), torch.float16) for n in ("q", "k", "v"))
    o = fa.fp8_attention(q, k, v)
    assert o.dtype == torch.float16
    assert_attn_close(o.float().cpu().numpy(), g["out"].astype(np.float32))
