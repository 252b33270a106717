"""Build recipe for the native library ``minimaxh3_amd/_lib/libmxf8.so`` (gfx950 only).

Each ``csrc/*.hip`` file is compiled by hipcc in parallel and the objects are linked into
one shared library exporting the C ABI declared in ``include/mxf8.h``.

    python -m minimaxh3_amd.build            # build (always recompiles)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "_lib")
LIBNAME = "libmxf8.so"
# (source, object name, extra defines); attn_inst.hip is instantiated per (D, out dtype)
SOURCES = [
    ("capi.hip", "capi", []),
    ("quant.hip", "quant", []),
    ("gemm.hip", "gemm", []),
    ("attn.hip", "attn", []),
] + [
    ("attn_inst.hip", f"attn_d{d}_o{o}", [f"-DMXF8_ATTN_D={d}", f"-DMXF8_ATTN_ODT={o}"])
    for d in (128, 64) for o in (0, 1)
]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # keep the compiler from forming packed fp32 VALU ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # start every loop on a 64-byte boundary: where a loop happens to start otherwise moves
    # with unrelated code before it, and the attention loop ran 12% slower from an unlucky
    # start (same instructions, measured on MI355X)
    "-falign-loops=64",
    "-Wno-pass-failed",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the MI355X library cannot be built")
    return path


def _compile(src: str, obj: str, defines) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *defines, "-I", os.path.join(ROOT, "include"), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{res.stderr[-8000:]}")


def build(verbose: bool = True) -> str:
    """Compile every HIP source for gfx950 and link libmxf8.so; returns its path."""
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    jobs = []
    for name, objname, defines in SOURCES:
        jobs.append((os.path.join(CSRC, name), os.path.join(objdir, objname + ".o"), defines))
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(_compile, s, o, d) for s, o, d in jobs]
        for f in futs:
            f.result()
    out = os.path.join(LIBDIR, LIBNAME)
    tmp = out + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[o for _, o, _ in jobs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-8000:]}")
    os.replace(tmp, out)
    if verbose:
        print(f"[minimaxh3_amd] built {out}")
    return out


if __name__ == "__main__":
    build()
    sys.exit(0)
