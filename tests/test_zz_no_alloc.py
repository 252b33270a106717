"""The no-allocation K / V quantizer (mxf8_attn_quant_kv_noalloc) against mxf8_attn_quant_kv.

The entry point has no counterpart in the reference: it serves callers that cannot allocate
device memory, taking its scratch from a device array inside the library instead of a
workspace argument.  Through the C ABI, two calls in a row (the second on a smaller input,
so stale scratch contents from the first would show) must give the workspace entry point's
outputs bit for bit, and so must two calls issued back to back on two streams.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _packed_kv(B, H, S, D, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    kv = torch.randn((B, S, 2, H, D), device="cuda", generator=g) * 1.5 + 0.5
    kv = kv.to(torch.bfloat16)
    return kv[:, :, 0].permute(0, 2, 1, 3), kv[:, :, 1].permute(0, 2, 1, 3)


def _noalloc(k, v, with_mean=True):
    from minimaxh3_amd import _native as N
    B, H, S, D = k.shape
    nk = -(-S // 128)
    k8 = torch.empty((B, H, nk * 128, D), dtype=torch.float8_e4m3fn, device=k.device)
    sk = torch.empty((B, H, nk), dtype=torch.float32, device=k.device)
    v8t = torch.empty((B, H, D, nk * 128), dtype=torch.float8_e4m3fn, device=k.device)
    sv = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    mean = torch.empty((B, H, D), dtype=torch.float32, device=k.device)
    rc = N.load().mxf8_attn_quant_kv_noalloc(
        k.data_ptr(), N.strides4(k), v.data_ptr(), N.strides4(v), N.dtype_code(k.dtype), B, H, S, D, k8.data_ptr(),
        sk.data_ptr(), v8t.data_ptr(), sv.data_ptr(), mean.data_ptr() if with_mean else None, N.stream_of(k))
    N.check(rc, "attn_quant_kv_noalloc")
    return k8, sk, v8t, sv, mean


@pytest.mark.parametrize("first,second", [((2, 24, 3000, 128), (1, 3, 333, 64)), ((1, 24, 20280, 128), (2, 2, 200, 128))])
def test_noalloc_equals_workspace_entry_point_twice(first, second):
    from minimaxh3_amd import ops
    print(f"[no-alloc] {first} then {second}", flush=True)
    for i, shape in enumerate((first, second)):
        k, v = _packed_kv(*shape, seed=31 + i)
        ref = ops.attn_quant_kv(k, v)
        got = _noalloc(k, v)
        torch.cuda.synchronize()
        for name, r, o in zip(("k8", "sk", "v8t", "sv", "mean"), ref, got):
            if r.dtype == torch.float8_e4m3fn:
                r, o = r.view(torch.uint8), o.view(torch.uint8)
            assert torch.equal(r, o), (shape, name)
        # without a mean buffer the key mean lives in the scratch array after the partial slabs
        # (stale from the call before): the codes and scales must not change
        got = _noalloc(k, v, with_mean=False)
        torch.cuda.synchronize()
        for name, r, o in zip(("k8", "sk", "v8t", "sv"), ref[:4], got[:4]):
            if r.dtype == torch.float8_e4m3fn:
                r, o = r.view(torch.uint8), o.view(torch.uint8)
            assert torch.equal(r, o), (shape, name, "mean=NULL")


def test_noalloc_two_streams_back_to_back():
    """A large call on one stream, then at once a smaller one on another stream, both keeping
    the key mean in the scratch array: the entry point orders the second after the first (they
    share the array), so both equal the workspace entry point bit for bit."""
    from minimaxh3_amd import ops
    print("[no-alloc] two streams", flush=True)
    shapes = ((1, 24, 20280, 128), (2, 3, 3000, 128))
    inputs = [_packed_kv(*shape, seed=41 + i) for i, shape in enumerate(shapes)]
    refs = [ops.attn_quant_kv(k, v) for k, v in inputs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = []
    for st, (k, v) in zip(streams, inputs):
        with torch.cuda.stream(st):
            outs.append(_noalloc(k, v, with_mean=False))
    torch.cuda.synchronize()
    for shape, ref, got in zip(shapes, refs, outs):
        for name, r, o in zip(("k8", "sk", "v8t", "sv"), ref[:4], got[:4]):
            if r.dtype == torch.float8_e4m3fn:
                r, o = r.view(torch.uint8), o.view(torch.uint8)
            assert torch.equal(r, o), (shape, name)


def test_noalloc_rejects_shapes_beyond_its_scratch():
    from minimaxh3_amd import _native as N
    lib = N.load()
    d = ctypes.c_void_p(256)
    st = N._I64x4(1, 1, 1, 1)
    # B*H = 2000 heads at D = 128 need more than the 4 MiB array: refused before any launch
    assert lib.mxf8_attn_quant_kv_noalloc(d, st, d, st, 0, 1, 2000, 4096, 128, d, d, d, d, None, None) == 1
    assert b"scratch" in lib.mxf8_last_error()
