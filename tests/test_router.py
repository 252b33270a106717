"""Routing logic of the drop-in attention router on the CPU (spies replace the kernel).

Every fallback branch of routed_sdpa is forced from the host (attention_router.py:66-102):
depth 0, disabled, dropout, causal, GQA, unsupported inputs, short sequences and
non-per-key masks all go to the original SDPA; per-key bool / float masks route with
key_mask / key_bias.
"""
import threading

import pytest
import torch
import torch.nn.functional as F

from minimaxh3_amd.kernels import attention_router as ar


@pytest.fixture()
def spy(monkeypatch):
    calls = []

    def fake_fp8(q, k, v, scale=None, key_mask=None, key_bias=None, repair_tau=-1.0):
        calls.append(dict(scale=scale, key_mask=key_mask, key_bias=key_bias, repair_tau=repair_tau))
        return torch.full_like(q, 7.0)

    monkeypatch.setattr(ar, "fp8_attention", fake_fp8)
    monkeypatch.setattr(ar, "is_supported", lambda q, k, v: q.ndim == 4 and q.shape[-1] in (64, 128))
    ar.configure(enabled=True, repair_tau=0.5, min_seq=64)
    yield calls
    ar.configure(enabled=True, repair_tau=-1.0, min_seq=4096)


def _qkv(B=2, H=2, Sq=64, Sk=80, D=64):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(B, H, Sq, D, generator=g), torch.randn(B, H, Sk, D, generator=g),
            torch.randn(B, H, Sk, D, generator=g))


def _routed(out):
    return bool((out == 7.0).all())


def test_routes_inside_scope_only(spy):
    q, k, v = _qkv()
    assert not _routed(ar.routed_sdpa(q, k, v))
    with ar.denoiser_scope():
        assert _routed(ar.routed_sdpa(q, k, v, scale=0.3))
    assert spy[-1]["scale"] == 0.3 and spy[-1]["repair_tau"] == 0.5
    assert spy[-1]["key_mask"] is None and spy[-1]["key_bias"] is None


@pytest.mark.parametrize("kw", [dict(dropout_p=0.1), dict(is_causal=True), dict(enable_gqa=True)])
def test_fallback_flags(spy, kw):
    q, k, v = _qkv()
    with ar.denoiser_scope():
        out = ar.routed_sdpa(q, k, v, **kw) if "dropout_p" not in kw else None
        if out is not None:
            assert not _routed(out)
    assert not spy


def test_disabled_and_short_sequences_fall_back(spy):
    q, k, v = _qkv()
    with ar.denoiser_scope():
        ar.configure(enabled=False, repair_tau=0.5, min_seq=64)
        assert not _routed(ar.routed_sdpa(q, k, v))
        ar.configure(enabled=True, repair_tau=0.5, min_seq=65)
        assert not _routed(ar.routed_sdpa(q, k, v))
    assert not spy


def test_unsupported_head_dim_and_mismatched_dims_fall_back(spy):
    q, k, v = _qkv(D=32)
    with ar.denoiser_scope():
        ref = F.scaled_dot_product_attention(q, k, v)
        torch.testing.assert_close(ar.routed_sdpa(q, k, v), ref)
    assert not spy


def test_per_key_masks_route(spy):
    q, k, v = _qkv()
    B, Sk = 2, 80
    bool_mask = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
    bool_mask[1, ..., 50:] = False
    with ar.denoiser_scope():
        assert _routed(ar.routed_sdpa(q, k, v, attn_mask=bool_mask))
        km = spy[-1]["key_mask"]
        assert km.shape == (B, Sk) and km.dtype == torch.bool and not km[1, 50:].any()
        fmask = torch.zeros(Sk)[None, None, None, :].expand(1, 1, 1, Sk).clone()
        fmask[..., :3] = -1e9
        assert _routed(ar.routed_sdpa(q, k, v, attn_mask=fmask))
        kb = spy[-1]["key_bias"]
        assert kb.shape == (B, Sk) and kb.dtype == torch.float32 and kb[0, 0] == -1e9
        assert _routed(ar.routed_sdpa(q, k, v, attn_mask=torch.ones(1, Sk, dtype=torch.bool)[None]))


@pytest.mark.parametrize("mask", [
    torch.ones(2, 1, 64, 80, dtype=torch.bool),   # per-query mask
    torch.ones(2, 2, 1, 80, dtype=torch.bool),    # per-head mask
    torch.ones(3, 1, 1, 80, dtype=torch.bool),    # wrong batch
    torch.ones(80, dtype=torch.bool),             # 1-D
    torch.ones(2, 1, 1, 80, dtype=torch.int32),   # integer mask
])
def test_non_per_key_masks_fall_back(spy, mask):
    q, k, v = _qkv()
    with ar.denoiser_scope():
        try:
            out = ar.routed_sdpa(q, k, v, attn_mask=mask)
        except (RuntimeError, IndexError):
            out = None  # SDPA itself may reject the mask; the router did not route it
    assert not spy
    if out is not None:
        assert not _routed(out)


def test_scope_is_thread_local_and_nests(spy):
    seen = {}

    def worker():
        seen["depth"] = ar._get_depth()

    with ar.denoiser_scope():
        with ar.denoiser_scope():
            assert ar._get_depth() == 2
            t = threading.Thread(target=worker)
            t.start()
            t.join()
        assert ar._get_depth() == 1
    assert ar._get_depth() == 0 and seen["depth"] == 0


def test_install_and_instrument(spy, monkeypatch):
    monkeypatch.setattr(ar, "_installed", False)
    orig = F.scaled_dot_product_attention
    orig_c = getattr(torch._C._nn, "scaled_dot_product_attention", None)
    try:
        ar.install()
        assert F.scaled_dot_product_attention is ar.routed_sdpa
        ar.install()  # idempotent

        class T(torch.nn.Module):
            def forward(self, q, k, v):
                return F.scaled_dot_product_attention(q, k, v)

        t = ar.instrument_transformer(T())
        assert ar.instrument_transformer(t) is t
        q, k, v = _qkv()
        assert _routed(t(q, k, v))
        assert not _routed(F.scaled_dot_product_attention(q, k, v))
    finally:
        F.scaled_dot_product_attention = orig
        if orig_c is not None:
            torch._C._nn.scaled_dot_product_attention = orig_c


def test_cpu_tensors_are_not_supported():
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention, is_supported
    q, k, v = _qkv()
    assert not is_supported(q.bfloat16(), k.bfloat16(), v.bfloat16())
    with pytest.raises(ValueError):
        fp8_attention(q.bfloat16(), k.bfloat16(), v.bfloat16())
