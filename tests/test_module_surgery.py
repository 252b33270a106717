"""Module surgery and FP8 weight checkpoints, on the CPU (no kernel launches).

find_primary_block_list and convert_transformer_to_fp8 follow the reference's
kernels/fp8_linear.py:111-162.  The weight quantization inside FP8Linear.from_linear
needs the GPU, so the selection tests replace it with a stub that records which linears
it receives and builds the module from seeded codes (FP8Linear.from_quantized).
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F
from safetensors.torch import save_file

from minimaxh3_amd.kernels import fp8_checkpoint as ck
from minimaxh3_amd.kernels import fp8_linear as fl

D = 64


class Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.to_q, self.to_k, self.to_v = nn.Linear(D, D), nn.Linear(D, D, bias=False), nn.Linear(D, D)
        self.to_out = nn.ModuleList([nn.Linear(D, D), nn.Dropout(0.0)])

    def forward(self, x):
        return self.to_out[1](self.to_out[0](self.to_q(x) + self.to_k(x) + self.to_v(x)))


class GELUProj(nn.Module):
    """diffusers-style tanh-GELU activation module: gelu_tanh(proj(x))."""

    def __init__(self, din, dout):
        super().__init__()
        self.proj = nn.Linear(din, dout)
        self.approximate = "tanh"

    def forward(self, x):
        return F.gelu(self.proj(x), approximate=self.approximate)


class FF(nn.Module):
    def __init__(self):
        super().__init__()
        self.net = nn.ModuleList([GELUProj(D, 4 * D), nn.Dropout(0.0), nn.Linear(4 * D, D)])

    def forward(self, x):
        for m in self.net:
            x = m(x)
        return x


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = Attn()
        self.ff = FF()
        self.adaln = nn.Linear(D, 24)  # 24 % 16 != 0: never converted

    def forward(self, x):
        x = x + self.attn(x)
        return x + self.ff(x)


class Toy(nn.Module):
    def __init__(self, n=6):
        super().__init__()
        self.blocks = nn.ModuleList([Block() for _ in range(n)])
        self.extra = nn.ModuleList([nn.Linear(D, D) for _ in range(2)])
        self.proj_out = nn.Linear(D, D)

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        return self.proj_out(x)


def _stub_from_linear(record):
    """from_linear replacement: seeded e4m3 codes of the right shape, no GPU."""

    def from_linear(cls, linear):
        record.append(linear)
        g = torch.Generator().manual_seed(len(record))
        codes = torch.randint(0, 0x7F, (linear.out_features, linear.in_features), generator=g, dtype=torch.uint8)
        scale = torch.rand(linear.out_features, generator=g) + 0.5
        bias = None if linear.bias is None else linear.bias.detach().to(torch.bfloat16)
        mod = fl.FP8Linear.from_quantized(codes.view(torch.float8_e4m3fn), scale, bias, "cpu")
        if isinstance(getattr(linear, "adapters", None), list):
            mod.adapters = list(linear.adapters)
        return mod

    return classmethod(from_linear)


@pytest.fixture
def stub(monkeypatch):
    record = []
    monkeypatch.setattr(fl.FP8Linear, "from_linear", _stub_from_linear(record))
    return record


# ------------------------------------------------------------------ find_primary_block_list

def test_primary_block_list_prefers_longest_homogeneous():
    toy = Toy()
    name, blocks = fl.find_primary_block_list(toy)
    assert name == "blocks" and blocks is toy.blocks

    m = nn.Module()
    m.mixed = nn.ModuleList([nn.Linear(4, 4), nn.ReLU(), nn.Linear(4, 4), nn.ReLU(), nn.Linear(4, 4)])
    m.same = nn.ModuleList([nn.Linear(4, 4) for _ in range(3)])
    assert fl.find_primary_block_list(m)[0] == "same"  # homogeneous wins over a longer mixed list


def test_primary_block_list_fallbacks_and_ties():
    m = nn.Module()
    m.a = nn.ModuleList([nn.Linear(4, 4), nn.ReLU()])
    m.b = nn.ModuleList([nn.ReLU(), nn.Linear(4, 4), nn.ReLU()])
    assert fl.find_primary_block_list(m)[0] == "b"  # no homogeneous list: the longest list
    t = nn.Module()
    t.first = nn.ModuleList([nn.Linear(4, 4) for _ in range(2)])
    t.second = nn.ModuleList([nn.Linear(4, 4) for _ in range(2)])
    assert fl.find_primary_block_list(t)[0] == "first"  # ties: the first in module order
    e = nn.Module()
    e.empty = nn.ModuleList()
    with pytest.raises(ValueError):
        fl.find_primary_block_list(e)


# ------------------------------------------------------------------ convert_transformer_to_fp8

def _converted_paths(model):
    return sorted(n for n, m in model.named_modules() if isinstance(m, fl.FP8Linear))


def test_convert_selects_inner_blocks_patterns_and_multiples_of_16(stub):
    toy = Toy()
    n = fl.convert_transformer_to_fp8(toy, "to_k, FF.NET.2", keep_edge_blocks=1)
    # blocks 1..4: to_q, to_v, to_out.0, ff.net.0.proj (to_k and ff.net.2 excluded, adaln 64->24 skipped)
    expect = sorted(f"blocks.{i}.{p}" for i in range(1, 5)
                    for p in ("attn.to_q", "attn.to_v", "attn.to_out.0", "ff.net.0.proj"))
    assert n == 16 and _converted_paths(toy) == expect and len(stub) == 16
    assert isinstance(toy.blocks[0].attn.to_q, nn.Linear) and isinstance(toy.blocks[5].ff.net[2], nn.Linear)
    assert isinstance(toy.proj_out, nn.Linear) and isinstance(toy.extra[0], nn.Linear)


def test_convert_pattern_list_and_edge_counts(stub):
    toy = Toy()
    assert fl.convert_transformer_to_fp8(toy, [" TO_Q ", "", "attn.to_out"], keep_edge_blocks=0) == 6 * 4
    assert not any(p.endswith("to_q") or "to_out" in p for p in _converted_paths(toy))
    assert fl.convert_transformer_to_fp8(Toy(), "", keep_edge_blocks=3) == 0  # range(3, 3)
    assert fl.convert_transformer_to_fp8(Toy(), "", keep_edge_blocks=9) == 0


def test_convert_replaces_blocks_that_are_linears(stub):
    m = nn.Module()
    m.layers = nn.ModuleList([nn.Linear(32, 32) for _ in range(4)])
    m.layers[1].adapters = [("A", "B", 1.0)]
    assert fl.convert_transformer_to_fp8(m, "layers.2", keep_edge_blocks=0) == 3
    assert [type(x).__name__ for x in m.layers] == ["FP8Linear", "FP8Linear", "Linear", "FP8Linear"]
    assert m.layers[1].adapters == [("A", "B", 1.0)]  # the LoRA registry's list carries over


def test_convert_fuse_gelu_folds_tanh_activation(stub):
    toy = Toy()
    fl.convert_transformer_to_fp8(toy, "", keep_edge_blocks=1, fuse_gelu=True)
    assert toy.blocks[2].ff.net[0].proj.act == fl.ACT_GELU_TANH
    assert toy.blocks[2].ff.net[0].forward == toy.blocks[2].ff.net[0].proj.forward
    assert isinstance(toy.blocks[0].ff.net[0].proj, nn.Linear)  # edge block untouched
    assert toy.blocks[2].attn.to_q.act == fl.ACT_NONE


# ------------------------------------------------------------------ FP8 checkpoints

def _buffers(model):
    out = {}
    for n, m in model.named_modules():
        if isinstance(m, fl.FP8Linear):
            out[n] = (m.w8.view(torch.uint8).cpu().clone(), m.w_scale.cpu().clone(),
                      None if m.bias is None else m.bias.cpu().clone(), int(m.act))
    return out


def _same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        for x, y in zip(a[k][:3], b[k][:3]):
            assert (x is None and y is None) or torch.equal(x, y), k
        assert a[k][3] == b[k][3], k


def test_checkpoint_roundtrip_into_bf16_model(stub, tmp_path):
    torch.manual_seed(0)
    base = Toy()
    conv = copy.deepcopy(base)
    fl.convert_transformer_to_fp8(conv, "to_k", keep_edge_blocks=1)
    path = str(tmp_path / "fp8.safetensors")
    assert ck.save_fp8_checkpoint(conv, path) == 20  # 5 linears x blocks 1..4
    fresh = copy.deepcopy(base)
    fresh.blocks[3].attn.to_v.adapters = []
    old_linear = fresh.blocks[1].attn.to_q
    assert ck.load_fp8_checkpoint(fresh, path, device="cpu") == 20
    _same(_buffers(conv), _buffers(fresh))
    assert old_linear.weight is None and old_linear.bias is None  # bf16 weight freed
    assert isinstance(fresh.blocks[3].attn.to_v, fl.FP8Linear) and fresh.blocks[3].attn.to_v.adapters == []
    assert isinstance(fresh.blocks[1].attn.to_k, nn.Linear)  # excluded at conversion: not in the file
    assert fresh.blocks[1].attn.to_k.weight is not None


def test_checkpoint_reload_in_place_keeps_fused_gelu(stub, tmp_path):
    conv = Toy()
    fl.convert_transformer_to_fp8(conv, "", keep_edge_blocks=1, fuse_gelu=True)
    path = str(tmp_path / "fp8.safetensors")
    ck.save_fp8_checkpoint(conv, path)
    # a bf16 model needs fuse_gelu=True for the modules saved with the fused activation
    with pytest.raises(ValueError, match="fuse_gelu"):
        ck.load_fp8_checkpoint(Toy(), path, device="cpu")
    fresh = Toy()
    ck.load_fp8_checkpoint(fresh, path, device="cpu", fuse_gelu=True)
    _same(_buffers(conv), _buffers(fresh))
    act = fresh.blocks[2].ff.net[0]
    assert act.proj.act == fl.ACT_GELU_TANH and act.forward == act.proj.forward
    assert fresh.blocks[0].ff.net[0].forward != fresh.blocks[0].ff.net[0].proj.forward  # edge: not fused
    # reload into the converted model: buffers replaced in place, activation still bound
    other = Toy()
    fl.convert_transformer_to_fp8(other, "", keep_edge_blocks=1, fuse_gelu=True)
    proj = other.blocks[2].ff.net[0].proj
    ck.load_fp8_checkpoint(other, path, device="cpu")
    assert other.blocks[2].ff.net[0].proj is proj and other.blocks[2].ff.net[0].forward == proj.forward
    _same(_buffers(conv), _buffers(other))


def test_checkpoint_errors_leave_model_unchanged(stub, tmp_path):
    conv = Toy()
    fl.convert_transformer_to_fp8(conv, "", keep_edge_blocks=0)
    path = str(tmp_path / "fp8.safetensors")
    ck.save_fp8_checkpoint(conv, path)
    # missing module: KeyError (strict) and nothing replaced; skipped otherwise
    small = Toy(n=4)
    with pytest.raises(KeyError):
        ck.load_fp8_checkpoint(small, path, device="cpu")
    assert not _converted_paths(small)
    assert ck.load_fp8_checkpoint(small, path, device="cpu", strict=False) == 4 * 6
    # shape mismatch
    wide = Toy()
    wide.blocks[5].attn.to_q = nn.Linear(D, 2 * D)
    with pytest.raises(ValueError, match="does not match"):
        ck.load_fp8_checkpoint(wide, path, device="cpu")
    assert not _converted_paths(wide)
    # not a checkpoint of this format
    bad = str(tmp_path / "bad.safetensors")
    save_file({"x": torch.zeros(2)}, bad, metadata={"format": "other"})
    with pytest.raises(ValueError, match="not an"):
        ck.load_fp8_checkpoint(Toy(), bad, device="cpu")
    with pytest.raises(ValueError):
        ck.save_fp8_checkpoint(Toy(), str(tmp_path / "none.safetensors"))


def test_from_quantized_validates():
    codes = torch.zeros((32, 16), dtype=torch.uint8).view(torch.float8_e4m3fn)
    m = fl.FP8Linear.from_quantized(codes, torch.ones(32), torch.zeros(32), "cpu")
    assert (m.in_features, m.out_features) == (16, 32) and m.w_scale.shape == (1, 32)
    assert m.bias.dtype == torch.bfloat16
    with pytest.raises(ValueError):
        fl.FP8Linear.from_quantized(codes.view(torch.uint8), torch.ones(32))
    with pytest.raises(ValueError):
        fl.FP8Linear.from_quantized(codes, torch.ones(31))
    with pytest.raises(ValueError):
        fl.FP8Linear.from_quantized(codes, torch.ones(32, dtype=torch.float64))
    np.testing.assert_array_equal(m.w8.view(torch.uint8).numpy(), np.zeros((32, 16), np.uint8))


def test_checkpoint_fingerprint_refuses_stale_codes(stub, tmp_path):
    """A cache keyed by the conversion fingerprint: a load expecting another fingerprint (other
    fused LoRAs, exclude patterns, kept edge blocks or base weights) is refused untouched."""
    fp = ck.conversion_fingerprint("to_k,norm", 1, fused_loras=[("lora_a.safetensors", 0.8)], source="rev1")
    assert fp == ck.conversion_fingerprint(["norm", " to_k"], 1, [("lora_a.safetensors", 0.8)], "rev1")
    others = [ck.conversion_fingerprint("to_k", 1, [("lora_a.safetensors", 0.8)], "rev1"),
              ck.conversion_fingerprint("to_k,norm", 2, [("lora_a.safetensors", 0.8)], "rev1"),
              ck.conversion_fingerprint("to_k,norm", 1, [("lora_a.safetensors", 0.9)], "rev1"),
              ck.conversion_fingerprint("to_k,norm", 1, [("lora_a.safetensors", 0.8)], "rev2"),
              ck.conversion_fingerprint("to_k,norm", 1, [("lora_a.safetensors", 0.8)], "rev1", fuse_gelu=True)]
    assert len({fp, *others}) == 6
    conv = Toy()
    fl.convert_transformer_to_fp8(conv, "", keep_edge_blocks=1)
    path = str(tmp_path / "fp8.safetensors")
    ck.save_fp8_checkpoint(conv, path, fingerprint=fp)
    fresh = Toy()
    with pytest.raises(ValueError, match="fingerprint"):
        ck.load_fp8_checkpoint(fresh, path, device="cpu", fingerprint=others[0])
    assert not _converted_paths(fresh)
    assert ck.load_fp8_checkpoint(fresh, path, device="cpu", fingerprint=fp) == 24
    # a file saved without a fingerprint does not satisfy a load that expects one
    plain = str(tmp_path / "plain.safetensors")
    ck.save_fp8_checkpoint(conv, plain)
    with pytest.raises(ValueError, match="fingerprint"):
        ck.load_fp8_checkpoint(Toy(), plain, device="cpu", fingerprint=fp)


def test_checkpoint_tensor_and_bias_checks_run_before_any_change(stub, tmp_path):
    """Missing tensors, wrong stored dtypes and a bias the target lacks (or has) are refused in
    the first pass: the transformer is left as it was."""
    from safetensors import safe_open
    conv = Toy()
    fl.convert_transformer_to_fp8(conv, "", keep_edge_blocks=0)
    path = str(tmp_path / "fp8.safetensors")
    ck.save_fp8_checkpoint(conv, path)
    with safe_open(path, framework="pt") as f:
        meta = f.metadata()
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    last = "blocks.5.attn.to_out.0"

    def variant(name, edit):
        t = dict(tensors)
        edit(t)
        p = str(tmp_path / name)
        save_file(t, p, metadata=meta)
        return p

    cases = [
        (variant("nobias.safetensors", lambda t: t.pop(f"{last}.bias")), "missing"),
        (variant("f16scale.safetensors", lambda t: t.update({f"{last}.w_scale": t[f"{last}.w_scale"].half()})),
         "w_scale"),
        (variant("u8codes.safetensors", lambda t: t.update({f"{last}.w8": t[f"{last}.w8"].view(torch.uint8)})),
         "w8"),
    ]
    for p, msg in cases:
        fresh = Toy()
        with pytest.raises(ValueError, match=msg):
            ck.load_fp8_checkpoint(fresh, p, device="cpu")
        assert not _converted_paths(fresh), p
    # the target linear lacks the stored bias (or has one the file lacks)
    nob = Toy()
    nob.blocks[5].attn.to_out[0] = nn.Linear(D, D, bias=False)
    with pytest.raises(ValueError, match="bias"):
        ck.load_fp8_checkpoint(nob, path, device="cpu")
    assert not _converted_paths(nob)
    conv_k = Toy()  # to_k has no bias in Toy: give the target one
    conv_k.blocks[0].attn.to_k = nn.Linear(D, D, bias=True)
    with pytest.raises(ValueError, match="bias"):
        ck.load_fp8_checkpoint(conv_k, path, device="cpu")
    assert not _converted_paths(conv_k)


def test_forward_quantized_validates_operands():
    codes8 = torch.zeros((32, 16), dtype=torch.uint8).view(torch.float8_e4m3fn)
    m = fl.FP8Linear.from_quantized(codes8, torch.ones(32), None, "cpu")
    x8 = torch.zeros((5, 16), dtype=torch.uint8).view(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="x_scale"):
        m.forward_quantized(x8, torch.ones(4, 1))
    with pytest.raises(ValueError, match="x_scale"):
        m.forward_quantized(x8, torch.ones(5, 1, dtype=torch.float64))
    with pytest.raises(ValueError, match="e4m3"):
        m.forward_quantized(x8.view(torch.uint8), torch.ones(5, 1))
    with pytest.raises(ValueError, match="contiguous"):
        m.forward_quantized(torch.zeros((16, 5), dtype=torch.uint8).view(torch.float8_e4m3fn).t(), torch.ones(5, 1))
