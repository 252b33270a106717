"""GPU parity of the FP8 linear path against the oracle (quantizer bit-exact, GEMM 1e-2; bit-identical
to the oracle with the fp8 instruction's accumulation)."""
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import linear as ol
from oracle.numerics import bf16_round, e4m3_decode
from tests.helpers import assert_gemm_close, assert_ln_close, bf16_randn, codes, to_gpu, with_outliers

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def fl():
    from minimaxh3_amd.kernels import fp8_linear
    return fp8_linear


# ---------------------------------------------------------------- quantize_rows (a1/a2)

@pytest.mark.parametrize("M,K,dtype", [
    (37, 3072, torch.bfloat16), (16, 12288, torch.bfloat16), (5, 64, torch.bfloat16),
    (33, 3072, torch.float16), (9, 1024, torch.float32), (7, 100, torch.bfloat16),
    (3, 20000, torch.bfloat16), (1, 16, torch.float32),
])
def test_quantize_rows_bit_exact(fl, M, K, dtype):
    _say(f"quantize_rows M={M} K={K} {dtype}")
    rng = np.random.default_rng(M * 131 + K)
    x = with_outliers(rng, bf16_randn(rng, (M, K)))
    if dtype == torch.float16:
        x = x.astype(np.float16).astype(np.float32)
    if dtype == torch.float32:
        x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    x8, sc = fl.quantize_rows(to_gpu(x, dtype))
    torch.cuda.synchronize()
    rc, rs = ol.quantize_rows(x)
    assert x8.dtype == torch.float8_e4m3fn and x8.shape == (M, K)
    assert sc.dtype == torch.float32 and sc.shape == (M, 1)
    np.testing.assert_array_equal(sc.cpu().numpy(), rs)
    np.testing.assert_array_equal(codes(x8), rc)


def test_quantize_rows_edge_cases(fl):
    _say("quantize_rows edge cases")
    x = np.zeros((6, 256), np.float32)
    x[1, 3] = -3.0
    x[1, 4] = 1.5
    x[2] = -0.0
    x[3, :] = 1e-30
    # values that land exactly on e4m3 rounding midpoints after the division (ties)
    x[4, 0] = 448.0
    x[4, 1:9] = np.array([1.0625, 1.1875, 3.25, 0.0087890625, 2.125, 6.5, 13.0, 416.0]) * 1.0
    x[5] = np.linspace(-7, 7, 256)
    x = bf16_round(x)
    x8, sc = fl.quantize_rows(to_gpu(x))
    rc, rs = ol.quantize_rows(x)
    np.testing.assert_array_equal(sc.cpu().numpy(), rs)
    np.testing.assert_array_equal(codes(x8), rc)
    # empty and non-contiguous inputs
    e8, es = fl.quantize_rows(torch.empty((0, 32), device="cuda", dtype=torch.bfloat16))
    assert e8.shape == (0, 32) and es.shape == (0, 1)
    big = to_gpu(bf16_randn(np.random.default_rng(1), (8, 512)))
    view = big[:, 128:384]
    v8, vs = fl.quantize_rows(view)
    rc, rs = ol.quantize_rows(big[:, 128:384].float().cpu().numpy())
    np.testing.assert_array_equal(codes(v8), rc)
    with pytest.raises(ValueError):
        fl.quantize_rows(torch.zeros(4, 4))            # CPU tensor
    with pytest.raises(ValueError):
        fl.quantize_rows(torch.zeros(4, 4, 4, device="cuda"))


def test_quantize_rows_ties_at_every_midpoint(fl):
    # Row amax 448 -> scale exactly 1: every e4m3 midpoint appears verbatim as x / s.
    _say("quantize_rows midpoints")
    c = np.arange(256, dtype=np.uint8)
    vals = np.unique(e4m3_decode(c[(c & 0x7F) != 0x7F]).astype(np.float64))
    mids = (vals[1:] + vals[:-1]) / 2
    mids = mids[np.abs(mids) < 448]
    row = np.concatenate([[448.0], mids]).astype(np.float32)
    x = np.zeros((1, 512), np.float32)
    x[0, :len(row)] = row
    x8, sc = fl.quantize_rows(to_gpu(x, torch.float32))
    rc, rs = ol.quantize_rows(x)
    assert sc.item() == 1.0
    np.testing.assert_array_equal(codes(x8), rc)


# ---------------------------------------------------------------- scaled GEMM (a3/a4/a6)

def _gemm_case(rng, M, N, K, bias=True):
    x = with_outliers(rng, bf16_randn(rng, (M, K)))
    w = bf16_randn(rng, (N, K), 0.02)
    b = bf16_randn(rng, (N,), 0.01) if bias else None
    x8, sa = ol.quantize_rows(x)
    w8, sw = ol.quantize_rows(w)
    return x, x8, sa, w8, sw, b


@pytest.mark.parametrize("M,N,K,bias", [
    (40, 96, 256, True), (300, 320, 400, True), (2048, 3072, 3072, True), (129, 64, 16, False),
    (1, 3072, 3072, True), (600, 1040, 1152, False),
])
def test_gemm_rowwise_matches_oracle(M, N, K, bias):
    _say(f"gemm M={M} N={N} K={K} bias={bias}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(M + N + K)
    x, x8, sa, w8, sw, b = _gemm_case(rng, M, N, K, bias)
    out = ops.gemm_rowwise(to_gpu(x8, torch.uint8).view(torch.float8_e4m3fn),
                           to_gpu(w8, torch.uint8).view(torch.float8_e4m3fn),
                           to_gpu(sa, torch.float32), to_gpu(sw.reshape(1, -1), torch.float32),
                           None if b is None else to_gpu(b), 0, None, None, 0.0)
    ref = bf16_round(ol.scaled_mm(x8, w8, sa, sw, b))
    assert out.dtype == torch.bfloat16 and out.shape == (M, N)
    assert_gemm_close(out.float().cpu().numpy(), ref)



@pytest.mark.parametrize("M,N,K,bias", [(300, 512, 1024, True), (129, 256, 3072, False)])
def test_gemm_rowwise_equals_the_instruction_model(M, N, K, bias):
    """Against the oracle with the fp8 instruction's accumulation (oracle.mfma) every output
    is bit-identical; against the exact-product oracle outputs near zero (where the group
    truncation of an outlier channel's products survives the cancellation) miss by more
    than one bf16 ulp."""
    _say(f"gemm model M={M} N={N} K={K} bias={bias}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(M * 3 + N + K)
    x, x8, sa, w8, sw, b = _gemm_case(rng, M, N, K, bias)
    out = ops.gemm_rowwise(to_gpu(x8, torch.uint8).view(torch.float8_e4m3fn),
                           to_gpu(w8, torch.uint8).view(torch.float8_e4m3fn),
                           to_gpu(sa, torch.float32), to_gpu(sw.reshape(1, -1), torch.float32),
                           None if b is None else to_gpu(b), 0, None, None, 0.0).float().cpu().numpy()
    np.testing.assert_array_equal(out, bf16_round(ol.scaled_mm(x8, w8, sa, sw, b, dot="mfma")))
    exact = bf16_round(ol.scaled_mm(x8, w8, sa, sw, b))
    mag = np.maximum(np.abs(out), np.abs(exact)).astype(np.float64)
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(mag, 2.0 ** -126))).astype(np.int64) - 7)
    assert (np.abs(out.astype(np.float64) - exact) > ulp).any()


def test_gemm_rowwise_gelu():
    _say("gemm gelu")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(5)
    M, N, K = 300, 512, 384
    x, x8, sa, w8, sw, b = _gemm_case(rng, M, N, K)
    out = ops.gemm_rowwise(to_gpu(x8, torch.uint8).view(torch.float8_e4m3fn),
                           to_gpu(w8, torch.uint8).view(torch.float8_e4m3fn),
                           to_gpu(sa, torch.float32), to_gpu(sw.reshape(1, -1), torch.float32), to_gpu(b), 1,
                           None, None, 0.0)
    ref = bf16_round(ol.gelu_tanh(bf16_round(ol.scaled_mm(x8, w8, sa, sw, b))))
    assert_gemm_close(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("ld_extra,offset", [(0, 0), (8, 0), (4, 0), (8, 4), (0, 8)])
def test_gemm_output_stride_and_alignment(ld_extra, offset):
    """The C ABI writes into a strided, possibly offset output: whole tiles take the store
    staged through LDS when rows are 16-byte aligned (ld_out % 8 == 0 and a 16-byte aligned
    base) and the direct 8-byte stores otherwise; both must give the oracle's result and
    leave the padding columns untouched."""
    _say(f"gemm ld_out=N+{ld_extra} offset={offset}")
    from minimaxh3_amd import _native as N
    rng = np.random.default_rng(11 + ld_extra + offset)
    M, Nn, K = 1024, 2048, 512  # 256 x 256 tiles do not fill the chip: 128 x 128 tiles, all whole
    x, x8, sa, w8, sw, b = _gemm_case(rng, M, Nn, K, True)
    a8g = to_gpu(x8, torch.uint8)
    w8g = to_gpu(w8, torch.uint8)
    sag, swg, bg = to_gpu(sa, torch.float32), to_gpu(sw, torch.float32), to_gpu(b)
    ld = Nn + ld_extra
    buf = torch.full((offset + M * ld,), -7.0, dtype=torch.bfloat16, device="cuda")
    lib = N.load()
    N.check(lib.mxf8_gemm_rowwise(a8g.data_ptr(), w8g.data_ptr(), sag.data_ptr(), swg.data_ptr(), bg.data_ptr(), 0,
                                  None, None, 0, 0.0, buf.data_ptr() + 2 * offset, M, Nn, K, ld,
                                  torch.cuda.current_stream().cuda_stream), "gemm_rowwise")
    torch.cuda.synchronize()
    out = buf[offset:].view(M, ld)
    ref = bf16_round(ol.scaled_mm(x8, w8, sa, sw, b))
    assert_gemm_close(out[:, :Nn].float().cpu().numpy(), ref)
    assert (buf[:offset] == -7.0).all() and (out[:, Nn:] == -7.0).all()


def test_gemm_rejects_bad_shapes():
    from minimaxh3_amd import ops
    from minimaxh3_amd._native import NativeError
    a = torch.zeros((4, 24), device="cuda", dtype=torch.float8_e4m3fn)
    w = torch.zeros((8, 24), device="cuda", dtype=torch.float8_e4m3fn)
    s = torch.ones((4, 1), device="cuda")
    with pytest.raises(NativeError):
        ops.gemm_rowwise(a, w, s, torch.ones((1, 8), device="cuda"), None, 0, None, None, 0.0)


# ---------------------------------------------------------------- FP8Linear module (a3, a5)

def test_fp8linear_forward_matches_oracle(fl):
    _say("FP8Linear forward")
    rng = np.random.default_rng(7)
    K, N = 512, 384
    lin = torch.nn.Linear(K, N, bias=True).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_gpu(bf16_randn(rng, (N, K), 0.02)))
        lin.bias.copy_(to_gpu(bf16_randn(rng, (N,), 0.01)))
    w = lin.weight.detach().float().cpu().numpy()
    b = lin.bias.detach().float().cpu().numpy()
    mod = fl.FP8Linear.from_linear(lin)
    assert lin.weight is None and mod.w8.dtype == torch.float8_e4m3fn and mod.w_scale.shape == (1, N)
    w8, sw = ol.quantize_rows(w)
    np.testing.assert_array_equal(codes(mod.w8), w8)
    np.testing.assert_array_equal(mod.w_scale.cpu().numpy().ravel(), sw.ravel())
    x = with_outliers(rng, bf16_randn(rng, (3, 77, K)))          # M = 231 (not a multiple of 16)
    with torch.no_grad():
        out = mod(to_gpu(x))
    assert out.shape == (3, 77, N) and out.dtype == torch.bfloat16
    ref = ol.fp8_linear_forward(x.reshape(-1, K), w8, sw, b).reshape(3, 77, N)
    assert_gemm_close(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("gelu", [False, True])
def test_fp8linear_lora_epilogue(fl, gelu):
    _say(f"FP8Linear lora gelu={gelu}")
    rng = np.random.default_rng(8)
    M, K, N, r = 500, 768, 640, 64
    lin = torch.nn.Linear(K, N, bias=True).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_gpu(bf16_randn(rng, (N, K), 0.02)))
        lin.bias.copy_(to_gpu(bf16_randn(rng, (N,), 0.01)))
    w, b = lin.weight.detach().float().cpu().numpy(), lin.bias.detach().float().cpu().numpy()
    mod = fl.FP8Linear.from_linear(lin)
    A = bf16_randn(rng, (r, K), 0.01 * 8)
    B = bf16_randn(rng, (N, r), 0.01 * 8)
    mod.adapters.append((to_gpu(A), to_gpu(B), 0.75))
    mod.act = 1 if gelu else 0
    x = with_outliers(rng, bf16_randn(rng, (M, K)))
    out = mod(to_gpu(x)).float().cpu().numpy()
    w8, sw = ol.quantize_rows(w)
    ref = ol.fp8_linear_forward(x, w8, sw, b, adapters=[(A, B, 0.75)], gelu=gelu)
    assert_gemm_close(out, ref)
    # the LoRA delta must be visible at this tolerance (not silently dropped)
    no_lora = ol.fp8_linear_forward(x, w8, sw, b, gelu=gelu)
    assert np.abs(ref - no_lora).max() > 5e-2 * np.abs(ref).max()


def test_fp8linear_two_adapters_odd_rank(fl):
    _say("FP8Linear two adapters")
    rng = np.random.default_rng(9)
    M, K, N = 200, 256, 256
    lin = torch.nn.Linear(K, N, bias=False).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_gpu(bf16_randn(rng, (N, K), 0.02)))
    w = lin.weight.detach().float().cpu().numpy()
    mod = fl.FP8Linear.from_linear(lin)
    ads = []
    for r, s in ((8, 1.0), (24, 0.5)):
        A, B = bf16_randn(rng, (r, K), 0.1), bf16_randn(rng, (N, r), 0.1)
        ads.append((A, B, s))
        mod.adapters.append((to_gpu(A), to_gpu(B), s))
    x = bf16_randn(rng, (M, K))
    out = mod(to_gpu(x)).float().cpu().numpy()
    w8, sw = ol.quantize_rows(w)
    ref = ol.fp8_linear_forward(x, w8, sw, None, adapters=ads)
    assert_gemm_close(out, ref)


def test_fp8_checkpoint_roundtrip_bit_identical(fl, tmp_path):
    """convert_transformer_to_fp8 on the GPU (with the GELU fold), save_fp8_checkpoint, then
    load_fp8_checkpoint into a fresh bf16 copy: bit-identical forward outputs, and every
    loaded module's codes and scales equal the oracle's per-row quantization of the
    original weight."""
    _say("fp8 checkpoint roundtrip")
    import copy
    from minimaxh3_amd.kernels import fp8_checkpoint as ck
    from tests.test_module_surgery import Toy
    torch.manual_seed(0)
    base = Toy().to("cuda", torch.bfloat16)
    conv = copy.deepcopy(base)
    n = fl.convert_transformer_to_fp8(conv, "to_k", keep_edge_blocks=1, fuse_gelu=True)
    x = torch.randn(3, 40, 64, device="cuda").to(torch.bfloat16)
    with torch.no_grad():
        y1 = conv(x)
    path = str(tmp_path / "toy_fp8.safetensors")
    assert ck.save_fp8_checkpoint(conv, path) == n == 20
    fresh = copy.deepcopy(base)
    assert ck.load_fp8_checkpoint(fresh, path, fuse_gelu=True) == n
    with torch.no_grad():
        y2 = fresh(x)
    assert torch.equal(y1, y2)
    for name, m in fresh.named_modules():
        if isinstance(m, fl.FP8Linear):
            assert m.w8.is_cuda
            w8, sw = ol.quantize_rows(base.get_submodule(name).weight.detach().float().cpu().numpy())
            np.testing.assert_array_equal(codes(m.w8), w8)
            np.testing.assert_array_equal(m.w_scale.cpu().numpy().ravel(), sw.ravel())


def test_lora_down_matches_bf16_matmul():
    _say("lora_down")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(10)
    # (M, K, r, ldx): K tails (520, 64 + 8), ranks below / above one 128-column workgroup
    # slice (192: two slices, the second half full), strided rows
    for M, K, r, ldx in ((100, 3072, 64, 3072), (33, 520, 16, 520), (257, 1024, 128, 1024), (64, 64, 48, 64),
                         (300, 72, 192, 72), (130, 256, 80, 320)):
        xf = bf16_randn(rng, (M, ldx))
        x = xf[:, :K]
        A = bf16_randn(rng, (r, K), 0.05)
        xg = to_gpu(xf)[:, :K]
        assert xg.stride(0) == ldx
        t = ops.lora_down(xg, to_gpu(A)).float().cpu().numpy()
        dot = x.astype(np.float64) @ A.astype(np.float64).T
        ref = bf16_round(dot.astype(np.float32))
        np.testing.assert_allclose(t, ref, rtol=2 ** -7, atol=1e-3 * np.abs(ref).max())


@pytest.mark.parametrize("r", [64, 96])
def test_lora_down_rows_independent_of_tile_height(r):
    """lora_down picks the rows per workgroup (64, 96, 128 or 160) from M and the CU count, so
    that the tiles fill whole rounds; a row's result must not depend on that choice.  Prefixes of
    one x (77648 rows: the 720p token count, 20280, 32768, 5000, 300) give the same rows bit for
    bit, and sampled rows of the full call match the float64 product rounded to bf16."""
    _say(f"lora_down tile heights r={r}")
    from minimaxh3_amd import ops
    torch.manual_seed(11)
    M, K = 77648, 264  # K % 64 != 0: the zeroed tail chunks take part too
    x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
    A = (torch.randn((r, K), device="cuda") * 0.05).to(torch.bfloat16)
    full = ops.lora_down(x, A)
    for m in (32768, 20280, 5000, 300):
        assert torch.equal(ops.lora_down(x[:m], A).view(torch.int16), full[:m].view(torch.int16)), m
    rows = torch.randint(0, M, (512,), generator=torch.Generator().manual_seed(1)).cuda()
    dot = x[rows].double() @ A.double().t()
    ref = dot.float().to(torch.bfloat16).float()
    got = full[rows].float()
    torch.testing.assert_close(got, ref, rtol=2 ** -7, atol=1e-3 * ref.abs().max().item())


@pytest.mark.parametrize("rank", [0, 64, 128])
def test_forward_adaln_equals_forward_of_modulation(fl, rank):
    """FP8Linear.forward_adaln(x, shift, scale) == FP8Linear.forward(y) bit for bit, with no
    adapter and with rank-64 / rank-128 adapters."""
    _say(f"forward_adaln rank={rank}")
    rng = np.random.default_rng(40 + rank)
    B, S, C, N = 2, 100, 3072, 768
    lin = torch.nn.Linear(C, N, bias=True).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_gpu(bf16_randn(rng, (N, C), 0.02)))
    mod = fl.FP8Linear.from_linear(lin)
    if rank:
        mod.adapters.append((to_gpu(bf16_randn(rng, (rank, C), 0.01)), to_gpu(bf16_randn(rng, (N, rank), 0.01)),
                             0.5))
    x = to_gpu(bf16_randn(rng, (B, S, C)))
    shift, scale = to_gpu(bf16_randn(rng, (B, C), 0.1)), to_gpu(bf16_randn(rng, (B, C), 0.1))
    out = mod.forward_adaln(x, shift, scale)
    _, _, y = fl.adaln_quantize_rows(x, shift, scale, return_modulated=True)
    ref = mod(y.view(B, S, C))
    torch.cuda.synchronize()
    assert out.shape == (B, S, N)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("M,N,K,r,gelu", [
    (300, 640, 768, 64, False),      # 128 x 128 tiles, one 64-column LoRA chunk in LDS
    (1100, 1280, 528, 128, True),    # K tail stage, two LoRA chunks, GELU on the bf16 output
    (4096, 8192, 256, 64, False),    # 256 x 256 tiles
    (500, 384, 256, 80, False),      # second chunk partly past r (zeroed in LDS)
    (200, 256, 256, 16, True),       # first chunk partly past r
    (300, 512, 256, 192, False),     # r > 128: operands read from global memory
])
def test_gemm_lora_epilogue_matches_oracle(M, N, K, r, gelu):
    """The GEMM's LoRA epilogue (t = bf16(x A^T), B, scale) against the reference branch
    bf16(bf16(bf16(t B^T) * scale) + bf16(linear)); the branch must be visible at the
    tolerance."""
    _say(f"gemm lora epilogue M={M} N={N} K={K} r={r} gelu={gelu}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(M + r)
    x = with_outliers(rng, bf16_randn(rng, (M, K)))
    w = bf16_randn(rng, (N, K), 0.02)
    b = bf16_randn(rng, (N,), 0.01)
    A, B, scale = bf16_randn(rng, (r, K), 0.08), bf16_randn(rng, (N, r), 0.08), 0.75
    xg = to_gpu(x)
    x8, sa = ops.quant_rows(xg)
    w8, sw = ops.quant_rows(to_gpu(w))
    lt = ops.lora_down(xg, to_gpu(A))
    out = ops.gemm_rowwise(x8, w8, sa, sw.view(1, -1), to_gpu(b), int(gelu), lt, to_gpu(B), scale)
    out = out.float().cpu().numpy()
    w8c, swc = ol.quantize_rows(w)
    ref = ol.fp8_linear_forward(x, w8c, swc, b, adapters=[(A, B, scale)], gelu=gelu)
    assert_gemm_close(out, ref)
    no_lora = ol.fp8_linear_forward(x, w8c, swc, b, gelu=gelu)
    assert np.abs(ref - no_lora).max() > 5e-2 * np.abs(ref).max()


@pytest.mark.parametrize("M,N,K,r,gelu", [
    (600, 3072, 3072, 64, False),   # LoRA operands in LDS, 256 x 256 tiles
    (600, 3072, 3072, 64, True),
    (300, 512, 256, 192, False),    # read from global memory in the epilogue
])
def test_gemm_lora_scale_one_equals_scaled_branch(M, N, K, r, gelu):
    """Scale 1 (what the runtime passes: alpha / rank is folded into B) skips the branch's
    product and second rounding.  Scaling by powers of two commutes with every bf16 rounding
    of the branch (normal range), so (B, scale 1) and (2 B, scale 0.5) must give the same
    bits: the skipped path against the full one."""
    _say(f"gemm lora scale one M={M} N={N} K={K} r={r} gelu={gelu}")
    from minimaxh3_amd import ops
    rng = np.random.default_rng(7 + r)
    x = to_gpu(with_outliers(rng, bf16_randn(rng, (M, K))))
    w8, sw = ops.quant_rows(to_gpu(bf16_randn(rng, (N, K), 0.02)))
    b = to_gpu(bf16_randn(rng, (N,), 0.01))
    A, B = to_gpu(bf16_randn(rng, (r, K), 0.08)), to_gpu(bf16_randn(rng, (N, r), 0.08))
    x8, sa = ops.quant_rows(x)
    lt = ops.lora_down(x, A)
    one = ops.gemm_rowwise(x8, w8, sa, sw.view(1, -1), b, int(gelu), lt, B, 1.0)
    half = ops.gemm_rowwise(x8, w8, sa, sw.view(1, -1), b, int(gelu), lt, (B * 2).contiguous(), 0.5)
    assert torch.equal(one.view(torch.int16), half.view(torch.int16))
    plain = ops.gemm_rowwise(x8, w8, sa, sw.view(1, -1), b, int(gelu), None, None, 0.0)
    assert not torch.equal(one.view(torch.int16), plain.view(torch.int16))


# ---------------------------------------------------------------- full-size shapes (properties)

@pytest.mark.parametrize("N,K", [(9216, 3072), (12288, 3072), (3072, 12288)])
def test_dit_block_linear_shapes_sampled_rows(N, K):
    """M = 20280 DiT-block linears: the whole output against the oracle on sampled rows."""
    _say(f"DiT linear M=20280 N={N} K={K}")
    from minimaxh3_amd import ops
    M = 20280
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn((N, K), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn((N,), device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    x8, sa = ops.quant_rows(x)
    w8, sw = ops.quant_rows(w)
    out = ops.gemm_rowwise(x8, w8, sa, sw.view(1, -1), b, 0, None, None, 0.0)
    torch.cuda.synchronize()
    rows = np.r_[0:64, 10000:10064, M - 64:M]
    xs = x[rows].float().cpu().numpy()
    rc, rs = ol.quantize_rows(xs)
    np.testing.assert_array_equal(codes(x8[rows]), rc)
    ref = bf16_round(ol.scaled_mm(rc, codes(w8), rs, sw.cpu().numpy(), b.float().cpu().numpy()))
    assert_gemm_close(out[rows].float().cpu().numpy(), ref)
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("N,K,gelu", [(3072, 3072, False), (12288, 3072, True)])
def test_720p_linear_lora_sampled_rows(fl, N, K, gelu):
    """720p DiT block (M = 75600 video + 2048 audio tokens): FP8Linear with a rank-64 LoRA
    (A, B ~ N(0, 0.01), scale 1) fused in the epilogue, GELU-tanh on MLP-up; the whole
    output against the oracle on sampled rows (rows are independent)."""
    _say(f"720p linear M=77648 N={N} K={K} gelu={gelu}")
    M, r = 77648, 64
    g = torch.Generator(device="cuda").manual_seed(1)
    lin = torch.nn.Linear(K, N, bias=True, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn((N, K), device="cuda", generator=g) * 0.02)
        lin.bias.copy_(torch.randn((N,), device="cuda", generator=g) * 0.01)
    w, b = lin.weight.detach().float().cpu().numpy(), lin.bias.detach().float().cpu().numpy()
    mod = fl.FP8Linear.from_linear(lin)
    A = (torch.randn((r, K), device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    B = (torch.randn((N, r), device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    mod.adapters.append((A, B, 1.0))
    mod.act = 1 if gelu else 0
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    out = mod(x)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and torch.isfinite(out).all()
    rows = np.r_[0:64, 40000:40064, M - 64:M]
    w8, sw = ol.quantize_rows(w)
    ad = [(A.float().cpu().numpy(), B.float().cpu().numpy(), 1.0)]
    xs = x[rows].float().cpu().numpy()
    ref = ol.fp8_linear_forward(xs, w8, sw, b, adapters=ad, gelu=gelu)
    assert_gemm_close(out[rows].float().cpu().numpy(), ref)
    # the LoRA delta is visible at this tolerance
    no_lora = ol.fp8_linear_forward(xs, w8, sw, b, gelu=gelu)
    assert np.abs(ref - no_lora).max() > 1e-2 * np.abs(ref).max()


# ---------------------------------------------------------------- adaLN modulation + quantization

def _eager_modulate(nb, shift_rows, scale_rows):
    """torch's eager bf16 ops after the LayerNorm output nb (bf16 values)."""
    op = bf16_round((1.0 + scale_rows.astype(np.float64)).astype(np.float32)).astype(np.float64)
    prod = bf16_round((nb.astype(np.float64) * op).astype(np.float32)).astype(np.float64)
    return bf16_round((prod + shift_rows).astype(np.float32))


def _assert_eager_from_ln_neighbours(y, nb, shift_rows, scale_rows, what):
    """Eager bar: the LayerNorm output the kernel rounded to bf16 lies within 1 bf16 ulp of
    nb, and everything after it is exact bf16 arithmetic, so y must equal the eager
    modulation of one of nb's neighbours (and of nb itself almost everywhere)."""
    bits = np.ascontiguousarray(nb, np.float32).view(np.uint32).astype(np.int64)
    ok = np.zeros(y.shape, bool)
    for d in (0, -0x10000, 0x10000):
        c = np.clip(bits + d, 0, 0xFFFFFFFF).astype(np.uint32).view(np.float32)
        hit = _eager_modulate(c, shift_rows, scale_rows) == y
        if d == 0:
            assert hit.mean() > 1 - 5e-3, (what, hit.mean())
        ok |= hit
    assert ok.all(), (what, y[~ok][:5])


@pytest.mark.parametrize("eager", [False, True])
def test_adaln_quant_closed_form_bit_exact(fl, eager):
    """Rows of +-a with eps = 0 have an exact LayerNorm (+-1): y, codes and scales are then
    fixed by the modulation and the quantizer alone and must match the oracle bit for bit."""
    _say(f"adaln closed form eager={eager}")
    rng = np.random.default_rng(2)
    B, S, C = 3, 40, 3072
    sign = np.tile(np.r_[np.ones(C // 2), -np.ones(C // 2)], (B * S, 1))
    for r in range(B * S):
        rng.shuffle(sign[r])
    a = 2.0 ** rng.integers(-3, 4, size=(B * S, 1))
    x = (sign * a).astype(np.float32).reshape(B, S, C)
    shift = bf16_randn(rng, (B, C), 0.1)
    scale = bf16_randn(rng, (B, C), 0.1)
    x8, sa, y = fl.adaln_quantize_rows(to_gpu(x), to_gpu(shift), to_gpu(scale), eps=0.0, eager_rounding=eager,
                                       return_modulated=True)
    ref_y = ol.adaln_modulate(x.reshape(-1, C), shift, scale, S, eps=0.0, eager=eager)
    np.testing.assert_array_equal(y.float().cpu().numpy(), ref_y)
    rc, rs = ol.quantize_rows(ref_y)
    np.testing.assert_array_equal(codes(x8), rc)
    np.testing.assert_array_equal(sa.cpu().numpy(), rs)


@pytest.mark.parametrize("B,S,C", [(2, 300, 3072), (1, 77, 1000), (3, 5, 8192), (2, 1, 64)])
def test_adaln_quant_general_rows(fl, B, S, C):
    """DiT-like rows (offset mean, outlier channels): y within 1 bf16 ulp of the oracle (fp32
    vs float64 LayerNorm statistics), almost always equal; codes and scales bit-exact against
    the row quantizer applied to the kernel's own y; x8 / sa independent of writing y."""
    _say(f"adaln general B={B} S={S} C={C}")
    rng = np.random.default_rng(B * S + C)
    x = bf16_randn(rng, (B, S, C), 1.5) + 0.25
    x[..., rng.choice(C, max(1, C // 100), replace=False)] *= 20.0
    x = bf16_round(x)
    shift = bf16_randn(rng, (B, C), 0.1)
    scale = bf16_randn(rng, (B, C), 0.1)
    for eager in (False, True):
        x8, sa, y = fl.adaln_quantize_rows(to_gpu(x), to_gpu(shift), to_gpu(scale), eager_rounding=eager,
                                           return_modulated=True)
        yk = y.float().cpu().numpy()
        if eager:
            x64 = x.reshape(-1, C).astype(np.float64)
            mean = x64.mean(axis=1, keepdims=True)
            n = (x64 - mean) / np.sqrt(((x64 - mean) ** 2).mean(axis=1, keepdims=True) + 1e-6)
            rows = np.arange(B * S) // S
            _assert_eager_from_ln_neighbours(yk, bf16_round(n.astype(np.float32)), shift[rows], scale[rows], eager)
        else:
            assert_ln_close(yk, ol.adaln_modulate(x.reshape(-1, C), shift, scale, S), eager)
        rc, rs = ol.quantize_rows(yk)
        np.testing.assert_array_equal(codes(x8), rc)
        np.testing.assert_array_equal(sa.cpu().numpy(), rs)
        x8b, sab = fl.adaln_quantize_rows(to_gpu(x), to_gpu(shift), to_gpu(scale), eager_rounding=eager)
        assert torch.equal(x8b.view(torch.uint8), x8.view(torch.uint8)) and torch.equal(sab, sa)
    if B > 1:
        # one shift / scale row broadcast to every batch item (stride 0) is accepted
        sh1, sc1 = to_gpu(shift[:1]).expand(B, C), to_gpu(scale[:1]).expand(B, C)
        x8c, sac = fl.adaln_quantize_rows(to_gpu(x), sh1, sc1)
        x8d, sad = fl.adaln_quantize_rows(to_gpu(x), sh1.contiguous(), sc1.contiguous())
        assert torch.equal(x8c.view(torch.uint8), x8d.view(torch.uint8)) and torch.equal(sac, sad)


def test_adaln_quant_matches_torch_gpu_ops(fl):
    """Against torch's own GPU layer_norm and bf16 ops (eager) and its fp32 form rounded once."""
    _say("adaln vs torch gpu ops")
    torch.manual_seed(3)
    B, S, C, eps = 2, 500, 3072, 1e-6
    x = (torch.randn(B, S, C, device="cuda") * 1.5 + 0.25).to(torch.bfloat16)
    shift = (torch.randn(B, C, device="cuda") * 0.1).to(torch.bfloat16)
    scale = (torch.randn(B, C, device="cuda") * 0.1).to(torch.bfloat16)
    with torch.no_grad():
        ref_e = F.layer_norm(x, (C,), eps=eps) * (1 + scale[:, None]) + shift[:, None]
        ref_f = (F.layer_norm(x.float(), (C,), eps=eps) * (1 + scale.float()[:, None])
                 + shift.float()[:, None]).to(torch.bfloat16)
    rows = np.arange(B * S) // S
    nb_torch = F.layer_norm(x, (C,), eps=eps).float().reshape(B * S, C).cpu().numpy()
    sh, sc = shift.float().cpu().numpy()[rows], scale.float().cpu().numpy()[rows]
    for eager, ref in ((True, ref_e), (False, ref_f)):
        _, _, y = fl.adaln_quantize_rows(x, shift, scale, eps=eps, eager_rounding=eager, return_modulated=True)
        yk = y.float().cpu().numpy()
        if eager:
            np.testing.assert_array_equal(_eager_modulate(nb_torch, sh, sc), ref.float().reshape(B * S, C).cpu().numpy())
            _assert_eager_from_ln_neighbours(yk, nb_torch, sh, sc, eager)
        else:
            assert_ln_close(yk, ref.float().reshape(B * S, C).cpu().numpy(), eager)


@pytest.mark.parametrize("lora", [False, True])
def test_forward_quantized_equals_forward(fl, lora):
    """FP8Linear.forward_quantized on the fused output == FP8Linear.forward on y, bit for bit."""
    _say(f"forward_quantized lora={lora}")
    rng = np.random.default_rng(4)
    B, S, C, N = 2, 150, 3072, 1024
    lin = torch.nn.Linear(C, N, bias=True).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_gpu(bf16_randn(rng, (N, C), 0.02)))
    mod = fl.FP8Linear.from_linear(lin)
    if lora:
        mod.adapters.append((to_gpu(bf16_randn(rng, (64, C), 0.01)), to_gpu(bf16_randn(rng, (N, 64), 0.01)), 1.0))
    x = to_gpu(bf16_randn(rng, (B, S, C)))
    shift, scale = to_gpu(bf16_randn(rng, (B, C), 0.1)), to_gpu(bf16_randn(rng, (B, C), 0.1))
    x8, sa, y = fl.adaln_quantize_rows(x, shift, scale, return_modulated=True)
    out_q = mod.forward_quantized(x8, sa, y)
    out = mod(y)
    assert torch.equal(out_q, out)
    if lora:
        with pytest.raises(ValueError):
            mod.forward_quantized(x8, sa)


@pytest.mark.parametrize("gelu", [False, True])
def test_fp16_input_lora_follows_reference_sequence(fl, gelu):
    """fp16 activations with a LoRA adapter: the bf16 linear output is converted to fp16 and
    the branch added in fp16, as the reference does (fp8_linear.py:105-108), then the folded
    tanh-GELU in fp16; against the oracle's fp16 statement at the GEMM bar."""
    _say(f"fp16 input LoRA gelu={gelu}")
    rng = np.random.default_rng(21)
    M, K, N, r = 300, 512, 384, 32
    x = with_outliers(rng, bf16_randn(rng, (M, K))).astype(np.float16).astype(np.float32)
    w, b = bf16_randn(rng, (N, K), 0.02), bf16_randn(rng, (N,), 0.01)
    A, B = bf16_randn(rng, (r, K), 0.08), bf16_randn(rng, (N, r), 0.08)
    lin = torch.nn.Linear(K, N, bias=True).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_gpu(w))
        lin.bias.copy_(to_gpu(b))
    mod = fl.FP8Linear.from_linear(lin)
    mod.act = 1 if gelu else 0
    mod.adapters.append((to_gpu(A), to_gpu(B), 0.75))
    out = mod(to_gpu(x, torch.float16))
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == (M, N)
    w8c, swc = ol.quantize_rows(w)
    ref = ol.fp8_linear_forward(x, w8c, swc, b, adapters=[(A, B, 0.75)], gelu=gelu, in_dtype="fp16")
    assert_gemm_close(out.float().cpu().numpy(), ref)
    no_lora = ol.fp8_linear_forward(x, w8c, swc, b, gelu=gelu, in_dtype="fp16")
    assert np.abs(ref - no_lora).max() > 5e-2 * np.abs(ref).max()
    # without adapters an fp16 input with the folded GELU also takes the reference's sequence
    # (bf16 linear output -> fp16 -> GELU in fp16), bit for bit against the same launches
    mod.adapters.clear()
    out = mod(to_gpu(x, torch.float16))
    torch.cuda.synchronize()
    assert_gemm_close(out.float().cpu().numpy(), no_lora)
    if gelu:
        from minimaxh3_amd import ops
        x16 = to_gpu(x, torch.float16)
        x8g, sag = fl.quantize_rows(x16)
        lin_out = ops.gemm_rowwise(x8g, mod.w8, sag, mod.w_scale, mod.bias, 0, None, None, 0.0).to(torch.float16)
        seq = torch.nn.functional.gelu(lin_out, approximate="tanh")
        assert torch.equal(out.view(torch.int16), seq.view(torch.int16))
