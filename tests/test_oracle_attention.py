"""Pins the FP8 attention oracle (oracle/attention.py).

Checks are chosen so that a plausible mistake fails one of them: a wrong visit
order or max policy (hand-computed two-tile cases), a wrong P code formula
(Mitchell's closed form), a dropped mean-centring, wrong masking, a transposed V
(exact softmax through torch SDPA with tau=0), and vectorisation/indexing slips
(a scalar brute-force loop).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle.numerics import bf16_round, e4m3_decode, e4m3_encode

LOG2E = oa.LOG2E


def _cos(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def _bf16_randn(rng, shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def _dequant(inter, c):
    """Dequantized Q (undoing c), K (centred) and V from the oracle intermediates."""
    q8, sq, k8, sk, v8t, sv = (inter[n] for n in ("q8", "sq", "k8", "sk", "v8t", "sv"))
    B, H, Sq, D = q8.shape
    Sk = k8.shape[2]
    qd = e4m3_decode(q8).astype(np.float64) * np.repeat(sq, 128, axis=2)[:, :, :Sq, None] / float(c)
    kd = e4m3_decode(k8).astype(np.float64) * np.repeat(sk, 128, axis=2)[:, :, :Sk, None]
    vd = e4m3_decode(v8t).astype(np.float64).transpose(0, 1, 3, 2) * sv[:, :, None, :]
    return qd, kd, vd


def test_quantizers_match_torch_restatement():
    rng = np.random.default_rng(0)
    B, H, S, D = 1, 2, 300, 128
    q = _bf16_randn(rng, (B, H, S, D))
    k = _bf16_randn(rng, (B, H, S, D)) + 0.5
    v = _bf16_randn(rng, (B, H, S, D))
    c = np.float32(LOG2E / math.sqrt(D))
    q8, sq = oa.quantize_q(q, c)
    mu = oa.key_mean(k)
    k8, sk = oa.quantize_k(k, mu)
    v8t, sv = oa.quantize_v(v)

    def tq(x, blocks):
        xt = torch.from_numpy(x)
        out, scales = [], []
        for i in range(0, S, 128):
            t = xt[:, :, i:i + 128]
            s = t.abs().amax(dim=(2, 3), keepdim=True).clamp_min(1e-12) / 448.0
            out.append((t / s).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8))
            scales.append(s[:, :, 0, 0])
        return torch.cat(out, 2).numpy(), torch.stack(scales, 2).numpy()

    rq, rsq = tq((q * c).astype(np.float32), 128)
    np.testing.assert_array_equal(q8, rq)
    np.testing.assert_array_equal(sq, rsq)
    rk, rsk = tq((k - mu).astype(np.float32), 128)
    np.testing.assert_array_equal(k8, rk)
    np.testing.assert_array_equal(sk, rsk)
    vt = torch.from_numpy(v)
    s = vt.abs().amax(dim=2).clamp_min(1e-12) / 448.0
    rv = (vt / s[:, :, None, :]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    np.testing.assert_array_equal(v8t, rv.transpose(2, 3).numpy())
    np.testing.assert_array_equal(sv, s.numpy())
    np.testing.assert_allclose(mu, k.astype(np.float64).mean(axis=2, keepdims=True), rtol=1e-6)


def test_p_codes_are_mitchell_exp2():
    # x = s - m on a 1/8 grid: code read as e4m3 is 2**floor(x) * (1 + frac(x)); x < -6 flushes.
    x = (np.arange(-80, 65) / 8.0).astype(np.float32)
    s = x[None, :]
    m = np.zeros(1, np.float32)
    codes = oa.p_codes(s, m, np.ones_like(s, bool))[0]
    got = e4m3_decode(codes).astype(np.float64)
    fl = np.floor(x.astype(np.float64))
    want = np.where(x < -6, 0.0, np.exp2(fl) * (1.0 + (x - fl)))
    np.testing.assert_array_equal(got, want)
    # just below the flush threshold (bits in [7.5, 8)) is flushed, not rounded up to 8
    s2 = np.array([[-6.0 - 1 / 32]], np.float32)
    assert oa.p_codes(s2, m, np.ones_like(s2, bool))[0, 0] == 0
    # invalid entries always give code 0
    assert oa.p_codes(s, m, np.zeros_like(s, bool)).max() == 0


def _two_tile_case(s0_code, s1_code, D=128):
    """Sq=Sk=256: rows see score s0 on keys 0..127 and s1 on keys 128..255.

    V carries 1.0 in channel 0 for tile 0 keys and in channel 1 for tile 1 keys, so
    output channel 0 / 1 is the normalised weight of tile 0 / 1.
    """
    S = 256
    q8 = np.zeros((1, 1, S, D), np.uint8)
    q8[..., 0] = 0x38                      # 1.0
    k8 = np.zeros((1, 1, S, D), np.uint8)
    k8[0, 0, :128, 0] = s0_code
    k8[0, 0, 128:, 0] = s1_code
    v8t = np.zeros((1, 1, D, S), np.uint8)
    v8t[0, 0, 0, :128] = 0x38
    v8t[0, 0, 1, 128:] = 0x38
    ones = lambda *s: np.ones(s, np.float32)
    return oa.attn_fwd(q8, k8, v8t, ones(1, 1, 2), ones(1, 1, 2), ones(1, 1, D))


def test_visit_order_and_lazy_max_hand_computed():
    # s0 = 0.25 (0x28), s1 = 4.5 (0x49): gap 4.25 < 8, so m keeps the first tile's max.
    out = _two_tile_case(0x28, 0x49)
    # Q tile 0 visits KV tiles (0, 1): weights 1 : 2**4 * 1.25 (code 90)
    w = np.array([1.0, 20.0])
    np.testing.assert_allclose(out[0, 0, :128, :2], np.broadcast_to(w / w.sum(), (128, 2)), rtol=1e-6)
    # Q tile 1 starts at j0 = 1*2//2 = 1, visits (1, 0): weights 2**-5 * 1.75 (code 22) : 1
    w = np.array([0.0546875, 1.0])
    np.testing.assert_allclose(out[0, 0, 128:, :2], np.broadcast_to(w / w.sum(), (128, 2)), rtol=1e-6)


def test_lazy_max_update_and_flush_hand_computed():
    # s0 = 1 (0x38), s1 = 10 (0x52): gap 9 > 8.
    out = _two_tile_case(0x38, 0x52)
    # order (0, 1): m moves to 10, tile 0 weight rescaled by exp2(1 - 10) = 2**-9
    w = np.array([2.0 ** -9, 1.0])
    np.testing.assert_allclose(out[0, 0, :128, :2], np.broadcast_to(w / w.sum(), (128, 2)), rtol=1e-6)
    # order (1, 0): tile 0 has bits = 8*(1-10)+56 = -16 < 8, flushed to 0
    np.testing.assert_allclose(out[0, 0, 128:, :2], np.broadcast_to([0.0, 1.0], (128, 2)), atol=0)


def test_zero_query_gives_mean_of_v():
    rng = np.random.default_rng(1)
    B, H, Sq, Sk, D = 2, 1, 130, 300, 64
    q = np.zeros((B, H, Sq, D), np.float32)
    k = _bf16_randn(rng, (B, H, Sk, D))
    v = _bf16_randn(rng, (B, H, Sk, D))
    mask = np.ones((B, Sk), bool)
    mask[1, 200:] = False
    out, inter = oa.fp8_attention(q, k, v, key_mask=mask, out_dtype=None)
    vd = e4m3_decode(inter["v8t"]).astype(np.float64).transpose(0, 1, 3, 2) * inter["sv"][:, :, None, :]
    want0 = vd[0, 0].mean(axis=0)
    want1 = vd[1, 0, :200].mean(axis=0)
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(want0, (Sq, D)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out[1, 0], np.broadcast_to(want1, (Sq, D)), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("with_mask,with_bias", [(False, False), (True, False), (False, True)])
def test_tau_zero_is_exact_softmax(with_mask, with_bias):
    rng = np.random.default_rng(2)
    B, H, Sq, Sk, D = 2, 2, 200, 333, 128
    q = _bf16_randn(rng, (B, H, Sq, D))
    k = _bf16_randn(rng, (B, H, Sk, D))
    v = _bf16_randn(rng, (B, H, Sk, D))
    mask = bias = None
    if with_mask:
        mask = rng.uniform(size=(B, Sk)) > 0.3
    if with_bias:
        bias = rng.standard_normal((B, Sk)).astype(np.float32)
        bias[0, :50] = -1e9                     # "masked" through the bias
    out, inter = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=bias, repair_tau=0.0, out_dtype=None)
    qd, kd, vd = _dequant(inter, inter["c"])
    am = None
    if mask is not None:
        am = torch.from_numpy(mask)[:, None, None, :]
    if bias is not None:
        am = torch.from_numpy(np.where(bias > -1e8, bias, -np.inf).astype(np.float64))[:, None, None, :]
    ref = F.scaled_dot_product_attention(torch.from_numpy(qd), torch.from_numpy(kd), torch.from_numpy(vd),
                                         attn_mask=am, scale=1.0 / math.sqrt(D)).numpy()
    assert _cos(out, ref) > 0.99999
    assert np.max(np.abs(out - ref)) < 5e-3


def test_fp8_path_close_to_exact_softmax():
    # tau = -1 (no repair): the attention accuracy bar (cosine >= 0.999) against exact attention.
    rng = np.random.default_rng(3)
    B, H, S, D = 1, 2, 400, 128
    q, k, v = (_bf16_randn(rng, (B, H, S, D)) for _ in range(3))
    out, _ = oa.fp8_attention(q, k, v, out_dtype=None)
    ref = F.scaled_dot_product_attention(*(torch.from_numpy(t).double() for t in (q, k, v))).numpy()
    assert _cos(out, ref) > 0.99


def test_fully_masked_row_is_zero():
    rng = np.random.default_rng(4)
    B, H, S, D = 2, 1, 150, 64
    q, k, v = (_bf16_randn(rng, (B, H, S, D)) for _ in range(3))
    mask = np.ones((B, S), bool)
    mask[1] = False
    out, _ = oa.fp8_attention(q, k, v, key_mask=mask)
    assert np.all(out[1] == 0)
    assert np.all(np.isfinite(out[0])) and np.abs(out[0]).max() > 0


def test_key_shift_invariance():
    rng = np.random.default_rng(5)
    B, H, S, D = 1, 1, 256, 128
    q, k, v = (_bf16_randn(rng, (B, H, S, D)) for _ in range(3))
    out0, _ = oa.fp8_attention(q, k, v, out_dtype=None)
    out1, _ = oa.fp8_attention(q, k + np.float32(8.0), v, out_dtype=None)
    assert _cos(out0, out1) > 0.99999


def _scalar_reference(q8, k8, v8t, sq, sk, sv, mask, bias, tau):
    """Per-row scalar loop of the same algorithm (independent bookkeeping)."""
    B, H, Sq, D = q8.shape
    Sk = k8.shape[2]
    nq, nk = -(-Sq // 128), -(-Sk // 128)
    f = np.float32
    out = np.zeros((B, H, Sq, D))
    for b in range(B):
        for h in range(H):
            Q = e4m3_decode(q8[b, h]).astype(np.float64)
            K = e4m3_decode(k8[b, h]).astype(np.float64)
            V = e4m3_decode(v8t[b, h]).astype(np.float64).T
            for r in range(Sq):
                I = r // 128
                j0 = I * nk // nq
                m, l = f(-1e9), f(0)
                acc = np.zeros(D, np.float32)
                accr = np.zeros(D, np.float32)
                for i in range(nk):
                    j = (j0 + i) % nk
                    keys = range(j * 128, j * 128 + 128)
                    s = np.full(128, f(-1e9), np.float32)
                    val = np.zeros(128, bool)
                    for t, n in enumerate(keys):
                        if n >= Sk:
                            continue
                        ok = True
                        sc = f(f(f(Q[r] @ K[n]) * f(sq[b, h, I])) * f(sk[b, h, j]))
                        if bias is not None:
                            ok = ok and bias[b, n] > -1e8
                            sc = f(sc + f(f(bias[b, n]) * f(LOG2E)))
                        if mask is not None:
                            ok = ok and bool(mask[b, n])
                        if ok:
                            s[t], val[t] = sc, True
                    rm = f(s.max())
                    mn = rm if (rm > f(m + f(8)) or m == f(-1e9)) else m
                    al = f(np.exp2(f(m - mn)))
                    acc, accr, l, m = acc * al, accr * al, f(l * al), mn
                    for t, n in enumerate(keys):
                        bits = f(f(s[t] * f(8)) + f(f(56) - f(f(8) * m)))
                        code = 0 if (bits < 8 or not val[t]) else int(min(max(np.rint(bits), 0), 126))
                        p = float(e4m3_decode(np.uint8(code)))
                        l = f(l + f(p))
                        if n < Sk:
                            acc = (acc + p * V[n]).astype(np.float32)
                        if tau >= 0:
                            pe = float(np.exp2(f(s[t] - m))) if val[t] else 0.0
                            d = f(pe - p) if p >= tau else f(0)
                            if n < Sk:
                                accr = (accr + bf16_round(np.float32(d)).item() * V[n]).astype(np.float32)
                            l = f(l + d)
                out[b, h, r] = (acc + accr) * sv[b, h] / max(l, f(1e-12))
    return out


@pytest.mark.parametrize("tau", [-1.0, 0.5])
def test_brute_force_scalar_loop(tau):
    rng = np.random.default_rng(6)
    B, H, Sq, Sk, D = 1, 1, 130, 200, 64
    q, k, v = (_bf16_randn(rng, (B, H, S, D)) for S in (Sq, Sk, Sk))
    mask = rng.uniform(size=(B, Sk)) > 0.2
    bias = (rng.standard_normal((B, Sk)) * 0.5).astype(np.float32)
    out, inter = oa.fp8_attention(q, k, v, key_mask=mask, key_bias=bias, repair_tau=tau, out_dtype=None)
    ref = _scalar_reference(inter["q8"], inter["k8"], inter["v8t"], inter["sq"], inter["sk"], inter["sv"],
                            mask, bias, tau)
    np.testing.assert_allclose(out, ref, rtol=2e-5, atol=2e-6)
