"""The C-ABI library loads, exports every symbol include/mxf8.h declares, and rejects bad
arguments on the host (no GPU needed: these checks run before any launch)."""
import ctypes
import os
import re

import pytest

from minimaxh3_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "mxf8.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mxf8_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(N.lib_path()):
        pytest.fail("libmxf8.so is not built (run __graft_entry__.build())")
    return N.load()


def test_header_declares_the_binding_table():
    assert _declared() == sorted(N.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(N.lib_path())
    for name in _declared():
        assert hasattr(raw, name), name
    assert lib.mxf8_abi_version() == 201
    assert lib.mxf8_last_error() is not None


def _err(lib):
    return lib.mxf8_last_error().decode()


def test_gemm_rejects_k_not_multiple_of_16(lib):
    dummy = ctypes.c_void_p(256)
    rc = lib.mxf8_gemm_rowwise(dummy, dummy, dummy, dummy, None, 0, None, None, 0, 0.0, dummy, 4, 8, 24, 8, None)
    assert rc == 1 and "multiple of 16" in _err(lib)


def test_gemm_rejects_bad_ld_and_act(lib):
    d = ctypes.c_void_p(256)
    assert lib.mxf8_gemm_rowwise(d, d, d, d, None, 0, None, None, 0, 0.0, d, 4, 8, 32, 4, None) == 1
    assert "ld_out" in _err(lib)
    assert lib.mxf8_gemm_rowwise(d, d, d, d, None, 7, None, None, 0, 0.0, d, 4, 8, 32, 8, None) == 1
    assert lib.mxf8_gemm_rowwise(d, d, d, d, None, 0, d, d, 20, 1.0, d, 4, 8, 32, 8, None) == 1
    assert "rank" in _err(lib)
    assert lib.mxf8_gemm_rowwise(d, d, d, d, None, 0, d, d, 4112, 1.0, d, 4, 8, 32, 8, None) == 1
    assert "rank" in _err(lib)
    assert lib.mxf8_gemm_rowwise(d, d, d, d, None, 0, d, None, 64, 1.0, d, 4, 8, 32, 8, None) == 1
    assert "lora_b" in _err(lib)
    assert lib.mxf8_gemm_rowwise(d, d, d, d, None, 0, None, None, 0, 0.0, d, 4, 8, (1 << 22) + 16, 8, None) == 1
    assert "too large" in _err(lib)


def test_empty_shapes_are_no_ops(lib):
    assert lib.mxf8_gemm_rowwise(None, None, None, None, None, 0, None, None, 0, 0.0, None, 0, 8, 32, 8, None) == 0
    assert lib.mxf8_quant_rows(None, 0, 0, 16, 16, None, None, None) == 0
    assert lib.mxf8_lora_down(None, 16, None, None, 0, 16, 16, None) == 0


def test_lora_down_argument_checks(lib):
    d = ctypes.c_void_p(256)
    assert lib.mxf8_lora_down(d, 16, d, d, 4, 16, 24, None) == 1      # r % 16
    assert lib.mxf8_lora_down(d, 16, d, d, 4, 16, 4112, None) == 1    # r > 4096
    assert lib.mxf8_lora_down(d, 16, d, d, 4, 12, 16, None) == 1      # K % 8
    assert lib.mxf8_lora_down(d, 8, d, d, 4, 16, 16, None) == 1       # ldx < K
    assert lib.mxf8_lora_down(None, 16, d, d, 4, 16, 16, None) == 1   # null x


def test_quant_rows_argument_checks(lib):
    d = ctypes.c_void_p(256)
    assert lib.mxf8_quant_rows(d, 0, 4, 16, 8, d, d, None) == 1 and "ldx" in _err(lib)
    assert lib.mxf8_quant_rows(d, 9, 4, 16, 16, d, d, None) == 1 and "dtype" in _err(lib)
    assert lib.mxf8_quant_rows(None, 0, 4, 16, 16, d, d, None) == 1


def test_attention_argument_checks(lib):
    d = ctypes.c_void_p(256)
    st = N._I64x4(1, 1, 1, 1)
    assert lib.mxf8_attn_quant_q(d, 0, st, 1, 1, 16, 96, 1.0, d, d, None) == 1 and "D must be" in _err(lib)
    assert lib.mxf8_attn_quant_q(d, 2, st, 1, 1, 16, 128, 1.0, d, d, None) == 1 and "dtype" in _err(lib)
    assert lib.mxf8_attn_kmean(d, 0, st, 1, 1, 16, 128, d, None, None) == 1
    assert lib.mxf8_attn_fwd(d, d, d, d, d, d, None, None, -1.0, d, 0, st, 1, 1, 0, 16, 128, 0, None) == 1
    assert lib.mxf8_attn_fwd(d, d, d, d, d, d, None, None, -1.0, d, 2, st, 1, 1, 8, 16, 128, 0, None) == 1
    assert lib.mxf8_attn_fwd(d, d, d, d, d, d, None, None, -1.0, d, 0, st, 1, 1, 8, 16, 128, 2, None) == 1 \
        and "kv_mode" in _err(lib)
    qs = N._I64x4(128 * 16, 128 * 16, 128, 1)
    assert lib.mxf8_attn_fwd_q(None, qs, 1.0, d, d, d, d, None, None, -1.0, None, d, 0, st, 1, 1, 16, 16, 128,
                               0, None) == 1 and "null" in _err(lib)
    bad = N._I64x4(128 * 16, 128 * 16, 128, 2)  # channel stride 2
    assert lib.mxf8_attn_fwd_q(d, bad, 1.0, d, d, d, d, None, None, -1.0, None, d, 0, st, 1, 1, 16, 16, 128,
                               0, None) == 1 and "unit channel stride" in _err(lib)
    odd = N._I64x4(128 * 16, 128 * 16, 132, 1)  # row stride not a multiple of 8
    assert lib.mxf8_attn_fwd_q(d, odd, 1.0, d, d, d, d, None, None, -1.0, None, d, 0, st, 1, 1, 16, 16, 128,
                               0, None) == 1 and "multiples of 8" in _err(lib)
    assert lib.mxf8_attn_fwd_q(ctypes.c_void_p(264), qs, 1.0, d, d, d, d, None, None, -1.0, None, d, 0, st, 1, 1,
                               16, 16, 128, 0, None) == 1 and "alignment" in _err(lib)
    assert lib.mxf8_attn_fwd_q(d, qs, 1.0, d, d, d, d, None, None, -1.0, None, d, 0, st, 1, 1, 16, 16, 96,
                               0, None) == 1 and "D must be" in _err(lib)
    assert lib.mxf8_attn_workspace_bytes(1, 24, 20280, 20280, 128) > 0
    assert lib.mxf8_attn_workspace_bytes(0, 24, 20280, 20280, 128) == 0
    # K and V together: shape, dtype and pointer checks run before any launch
    assert lib.mxf8_attn_quant_kv(d, st, d, st, 0, 1, 1, 16, 96, d, d, d, d, None, d, None) == 1 \
        and "D must be" in _err(lib)
    assert lib.mxf8_attn_quant_kv(d, st, d, st, 2, 1, 1, 16, 128, d, d, d, d, None, d, None) == 1 \
        and "dtype" in _err(lib)
    assert lib.mxf8_attn_quant_kv(d, st, None, st, 0, 1, 1, 16, 128, d, d, d, d, None, d, None) == 1 \
        and "null" in _err(lib)
    assert lib.mxf8_attn_quant_kv(d, st, d, st, 0, 1, 1, 16, 128, d, d, d, d, None, None, None) == 1 \
        and "workspace" in _err(lib)
    assert lib.mxf8_attn_quant_kv(d, st, d, st, 0, 1, 1, 0, 128, d, d, d, d, None, d, None) == 1
    assert lib.mxf8_attn_kv_workspace_bytes(1, 24, 20280, 128) > 0
    assert lib.mxf8_attn_kv_workspace_bytes(1, 0, 20280, 128) == 0


def test_kv_stats_argument_checks(lib):
    d = ctypes.c_void_p(256)
    args = lambda M=600, N=768, K=256, ld=768, S=300, kc=256, vc=512, C=256, part=d: (
        d, d, d, d, None, d, M, N, K, ld, S, kc, vc, C, part, None)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(N=640, ld=640)) == 1 and "multiples of 256" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(S=64, M=640)) == 1 and "S=64" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(S=250)) == 1 and "divide" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(C=128)) == 1 and "C=128" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(kc=-1, vc=-1)) == 1 and "neither" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(vc=640)) == 1 and "column range" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(kc=256, vc=256)) == 1 and "overlap" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(part=None)) == 1 and "null" in _err(lib)
    assert lib.mxf8_gemm_rowwise_kv_stats(*args(K=24)) == 1 and "multiple of 16" in _err(lib)
    assert lib.mxf8_gemm_kv_stats_bytes(20280, 3072) == 2 * 159 * 3072 * 4
    assert lib.mxf8_gemm_kv_stats_bytes(0, 3072) == 0
    st = N._I64x4(1, 1, 1, 1)
    assert lib.mxf8_attn_quant_kv_gemm_stats(d, st, d, st, 0, 1, 2, 100, 128, d, 1, d, d, d, d, d, None) == 1 \
        and "S=100" in _err(lib)
    assert lib.mxf8_attn_quant_kv_gemm_stats(d, st, d, st, 0, 1, 1, 300, 128, d, 1, d, d, d, d, d, None) == 1 \
        and "H*D" in _err(lib)
    assert lib.mxf8_attn_quant_kv_gemm_stats(d, st, d, st, 0, 1, 2, 300, 128, None, 1, d, d, d, d, d, None) == 1 \
        and "null" in _err(lib)
    assert lib.mxf8_attn_quant_kv_gemm_stats(d, st, d, st, 0, 1, 2, 300, 96, d, 1, d, d, d, d, d, None) == 1 \
        and "D must be" in _err(lib)
