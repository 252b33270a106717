"""ctypes binding of the C ABI in include/mxf8.h (libmxf8.so, built for gfx950).

The library is loaded lazily on first use.  There is no fallback: if it is missing or
the device is not an MI355X-class gfx950 GPU, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libmxf8.so")
_lock = threading.Lock()
_lib = None

BF16, F16, F32 = 0, 1, 2
ACT_NONE, ACT_GELU_TANH = 0, 1
KV_AUTO, KV_STREAM = 0, 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_I64x4 = _i64 * 4

# name -> (restype, argtypes); mirrors include/mxf8.h
_SIGNATURES = {
    "mxf8_abi_version": (_i32, []),
    "mxf8_last_error": (ctypes.c_char_p, []),
    "mxf8_quant_rows": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp]),
    "mxf8_adaln_quant_rows": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _f32, _i32, _vp, _vp, _vp, _vp]),
    "mxf8_gemm_rowwise": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _f32, _vp, _i64, _i64, _i64, _i64,
                                 _vp]),
    "mxf8_gemm_kv_stats_bytes": (_i64, [_i64, _i64]),
    "mxf8_gemm_rowwise_kv_stats": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                          _i64, _vp, _vp]),
    "mxf8_lora_down": (_i32, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
    "mxf8_attn_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "mxf8_attn_quant_q": (_i32, [_vp, _i32, _I64x4, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _vp]),
    "mxf8_attn_kmean": (_i32, [_vp, _i32, _I64x4, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "mxf8_attn_quant_k": (_i32, [_vp, _i32, _I64x4, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "mxf8_attn_quant_v": (_i32, [_vp, _i32, _I64x4, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "mxf8_attn_kv_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "mxf8_attn_quant_kv": (_i32, [_vp, _I64x4, _vp, _I64x4, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _vp]),
    "mxf8_attn_quant_kv_gemm_stats": (_i32, [_vp, _I64x4, _vp, _I64x4, _i32, _i64, _i64, _i64, _i64, _vp, _i32,
                                             _vp, _vp, _vp, _vp, _vp, _vp]),
    "mxf8_attn_quant_kv_noalloc":(_i32, [_vp, _I64x4, _vp, _I64x4, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                          _vp, _vp]),
    "mxf8_attn_fwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _vp, _i32, _I64x4, _i64, _i64, _i64, _i64,
                             _i64, _i32, _vp]),
    "mxf8_attn_fwd_q": (_i32, [_vp, _I64x4, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _i32, _I64x4, _i64,
                               _i64, _i64, _i64, _i64, _i32, _vp]),
}
EXPORTS = tuple(_SIGNATURES)


class NativeError(RuntimeError):
    """A call into libmxf8 returned a non-zero status."""


def lib_path() -> str:
    return _LIB_PATH


def _bind(path: str):
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load():
    """Load the in-tree libmxf8.so once (idempotent) with the argument types of every export."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"{_LIB_PATH} is missing: build the HIP library first (python -m minimaxh3_amd.build)")
            _lib = _bind(_LIB_PATH)
        return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mxf8_last_error().decode(errors="replace")
        raise NativeError(f"{what} failed (status {rc}): {msg}")


_arch_ok: dict[int, bool] = {}


def require_gfx950(device: torch.device) -> None:
    """The kernels are built for gfx950 only; refuse other devices loudly."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ok = _arch_ok.get(idx)
    if ok is None:
        name = getattr(torch.cuda.get_device_properties(idx), "gcnArchName", "")
        ok = name.split(":")[0] == "gfx950"
        _arch_ok[idx] = ok
    if not ok:
        raise RuntimeError(f"minimaxh3_amd kernels need a gfx950 (MI355X) device, got cuda:{idx}")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    if dt == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {dt}")


def strides4(t: torch.Tensor):
    return _I64x4(*[int(s) for s in t.stride()])
