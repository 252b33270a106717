#!/usr/bin/env python3
"""Throughput of the MI355X FP8 hot path on one DiT block (one GPU).

A step is one pass of the FP8 hot path over one DiT block's worth of synthetic inputs.
The default workload (--workload dit480) is the 480p block:

* the four FP8 linears of the block at M = 20280 tokens (13 latent frames x 30 x 52
  patches), hidden 3072: QKV 3072->9216, attention-out 3072->3072, MLP-up 3072->12288
  with the fused GELU-tanh epilogue, MLP-down 12288->3072.  Each one is the FP8Linear
  forward: per-token e4m3 activation quantization, then the row-wise scaled FP8 GEMM
  with bias.  Activations bf16 ~N(0,1) with 1% of the channels scaled x20 (outliers),
  weights ~N(0,0.02) quantized per output channel at load, bias ~N(0,0.01);
* one non-causal FP8 flash-attention forward, B=1, H=24, S=20280, D=128: Q/K/V bf16
  ~N(0,1) in the [B,S,H,D] storage of a fused QKV projection (permuted views), Q/K/V
  quantizers, then the attention kernel; softmax scale 1/sqrt(128), repair off.

Two more workloads measure the other DiT shapes the same way:

* --workload joint: joint video + audio self-attention over 20280 + 1024 tokens (B=2, the
  second item's last 384 keys masked: its audio is 640 tokens long) and text
  cross-attention of those 21304 queries against 512 context keys, H=24, D=128;
* --workload dit720: the 720p block, 75600 video + 2048 audio = 77648 tokens: the four
  FP8 linears with a rank-64 bf16 LoRA (A, B ~N(0,0.01), scale 1) fused in every
  epilogue, and self-attention at S=77648.  The QKV and MLP-up inputs are the adaLN
  modulation LayerNorm(x) * (1 + scale) + shift (shift, scale ~N(0,0.1)) of the block's
  hidden state, made with their e4m3 codes by the fused adaLN quantizer.

value = algorithmic FLOPs of the step (2*M*N*K per GEMM with the un-padded M,
4*B*H*Sq*Sk*D per attention; LoRA FLOPs are reported per kernel, not counted) / wall
time of the step, in TFLOP/s, with every input resident in HBM before the timed region.
In the timed steps only the attention launches are bracketed by HIP events on the stream
they run on (the largest gives the roofline entry); the per-kernel breakdown comes from
the same number of steps run again after the timed ones with every launch bracketed (for
--workload linear2048, whose timed steps are one replay of a HIP graph holding all of them,
from a graph of 20 copies of each launch, timed by one event pair around its replay).  The CPU baseline times the
reference's torch CPU fallbacks (fp32 dequant-matmul and SDPA) on a bounded sample and
scales those rates to the step's FLOP mix.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--workload dit480|joint|dit720]
                    [--no-cpu-baseline] [--separate-q-quant] [--repair-tau TAU]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "FP8 GEMM + FP8 attn TFLOP/s (S=20k, D=128) and % of MI355X FP8 peak, 1 GPU"
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense FP8 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
# HBM bytes per launch of the attention kernel at S=20280, H=24, D=128, measured with
# `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` over this script's dispatches and
# scaled by what the counters read for the 1 GiB streaming kernel of
# hbm_stream_reference() (FETCH_SIZE reports 0.500 of the bytes read, WRITE_SIZE 1.000 of
# the bytes written): 357606.2 KiB x 2 fetched + 121680.7 KiB written.  The algorithmic
# traffic is 249.2 MB of bf16 Q (quantized inside the launch) and K8/V8T read + 124.6 MB
# of output written.
ATTN_TRAFFIC_BYTES = 357606.2 * 1024 * 2 + 121680.7 * 1024
TOKENS = 20280                # 13 x 30 x 52
HIDDEN, MLP = 3072, 12288
HEADS, HEAD_DIM = 24, 128
# (name, in_features, out_features, fused activation)
LINEARS = (("qkv", HIDDEN, 3 * HIDDEN, 0), ("attn_out", HIDDEN, HIDDEN, 0),
           ("mlp_up", HIDDEN, MLP, 1), ("mlp_down", MLP, HIDDEN, 0))
# workload -> (description, linear tokens or 0, LoRA rank, attentions, adaLN inputs); an
# attention is (name, B, Sq, Sk, masked key tail of item 1); with adaLN the QKV and MLP-up
# inputs are LayerNorm(x) * (1 + scale) + shift, made by the fused adaLN quantizer
ADALN_LINEARS = ("qkv", "mlp_up")
WORKLOADS = {
    "dit480": ("DiT block FP8 hot path at 480p: 4 FP8 linears (M=20280, hidden 3072, MLP 12288, "
               "GELU-tanh on MLP-up) + FP8 flash-attention B=1 H=24 S=20280 D=128",
               TOKENS, 0, (("attn", 1, TOKENS, TOKENS, 0),), False),
    "joint": ("joint video+audio FP8 self-attention B=2 S=20280+1024 (item 1: last 384 keys masked) + "
              "text FP8 cross-attention B=2 Sq=21304 Sk=512, H=24 D=128",
              0, 0, (("self", 2, 21304, 21304, 384), ("cross", 2, 21304, 512, 0)), False),
    "dit720": ("DiT block FP8 hot path at 720p: adaLN (shift/scale ~N(0,0.1)) fused with the FP8 quantization "
               "of the QKV and MLP-up inputs, 4 FP8 linears (M=77648, hidden 3072, MLP 12288, GELU-tanh on "
               "MLP-up) with a rank-64 LoRA in every epilogue + FP8 flash-attention B=1 H=24 S=77648 D=128",
               77648, 64, (("attn", 1, 77648, 77648, 0),), True),
    "linear2048": ("FP8 linear x bf16 [2048,3072] ~N(0,1) (no outliers), W [3072,3072] ~N(0,0.02) e4m3 per-channel, "
                   "bias ~N(0,0.01): per-token activation quantization + row-wise scaled FP8 GEMM, bf16 out",
                   2048, 0, (), False),
}
# the linears of each workload (default: the DiT block's four) and whether 1% of the activation
# channels are scaled x20
LINEAR_SETS = {"linear2048": (("linear", HIDDEN, HIDDEN, 0),)}
NO_OUTLIERS = ("linear2048",)
# workloads whose K timed steps are captured in one HIP graph and replayed once: a step is two
# launches of ~5 and ~24 us, which neither Python launches nor a graph replay per step keep
# the GPU busy with
GRAPHED = ("linear2048",)


def linears_of(workload: str):
    return LINEAR_SETS.get(workload, LINEARS)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemm_flops(m: int, n: int, k: int) -> float:
    return 2.0 * m * n * k


def attn_flops(b: int, h: int, sq: int, sk: int, d: int) -> float:
    return 4.0 * b * h * sq * sk * d


def activations(torch, g, m: int, k: int, dev, outliers: bool = True):
    """bf16 ~N(0,1) [m, k] with floor(1% of k) channels (seeded randperm) scaled x20 (outliers)."""
    x = torch.randn((m, k), device=dev, generator=g)
    if outliers:
        idx = torch.randperm(k, device=dev, generator=g)[: k // 100]
        x[:, idx] *= 20.0
    return x.to(torch.bfloat16)


def build_workload(torch, dev, tokens: int, lora_rank: int, attns, adaln: bool = False, specs=LINEARS,
                   outliers: bool = True):
    """FP8Linear modules with their activations (and adaLN shift / scale [1, C] where the
    input is adaLN-modulated), and the Q/K/V (+ key mask) of each attention."""
    from minimaxh3_amd.kernels.fp8_linear import FP8Linear

    g = torch.Generator(device=dev).manual_seed(0)
    linears = []
    if tokens:
        for name, k, n, act in specs:
            lin = torch.nn.Linear(k, n, bias=True, device=dev, dtype=torch.bfloat16)
            with torch.no_grad():
                lin.weight.copy_(torch.randn((n, k), device=dev, generator=g) * 0.02)
                lin.bias.copy_(torch.randn((n,), device=dev, generator=g) * 0.01)
            mod = FP8Linear.from_linear(lin)
            mod.act = act
            if lora_rank:
                a = (torch.randn((lora_rank, k), device=dev, generator=g) * 0.01).to(torch.bfloat16)
                b = (torch.randn((n, lora_rank), device=dev, generator=g) * 0.01).to(torch.bfloat16)
                mod.adapters.append((a, b, 1.0))
            mod_params = None
            if adaln and name in ADALN_LINEARS:
                mod_params = tuple((torch.randn((1, k), device=dev, generator=g) * 0.1).to(torch.bfloat16)
                                   for _ in range(2))
            linears.append((name, mod, activations(torch, g, tokens, k, dev, outliers), mod_params))
    attn_inputs = []
    for name, b, sq, sk, tail in attns:
        q = torch.randn((b, sq, HEADS, HEAD_DIM), device=dev, generator=g).to(torch.bfloat16).permute(0, 2, 1, 3)
        kv = torch.randn((b, sk, 2, HEADS, HEAD_DIM), device=dev, generator=g).to(torch.bfloat16)
        k, v = (kv[:, :, i].permute(0, 2, 1, 3) for i in range(2))
        mask = None
        if tail:
            mask = torch.ones((b, sk), dtype=torch.bool, device=dev)
            mask[1, sk - tail:] = False
        attn_inputs.append((name, q, k, v, mask))
    return linears, attn_inputs


class Timers:
    """Per-kernel HIP event pairs recorded on the launching (current) stream; with `prefix`,
    only the launches whose part name starts with it are timed.

    reps = 0 brackets each launch in the step with an event pair.  reps > 0 (graph-replayed
    workloads, whose launches take ~20 us) keeps the first launch of each part and, in
    graph_times(), captures `reps` copies of it in a HIP graph of its own and times one
    replay with one event pair: an event pair around a single short launch from Python
    measures the host's launch gap, not the kernel."""

    def __init__(self, torch, prefix: str = "", reps: int = 0):
        self.torch = torch
        self.prefix = prefix
        self.reps = reps
        self.pairs: dict[str, list] = {}
        self.launches: dict[str, tuple] = {}

    def run(self, name, fn, *args):
        if not name.startswith(self.prefix):
            return fn(*args)
        if self.reps:
            self.launches.setdefault(name, (fn, args))
            return fn(*args)
        s = self.torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn(*args)
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.setdefault(name, []).append((s, e))
        return out

    def graph_times(self):
        torch = self.torch
        for name, (fn, args) in self.launches.items():
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(self.reps):
                    fn(*args)
            g.replay()
            torch.cuda.synchronize()
            for _ in range(3):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                g.replay()
                e.record()
                self.pairs.setdefault(name, []).append((s, e))
            torch.cuda.synchronize()
            del g

    def mean_ms(self):
        n = max(self.reps, 1)
        return {k: sum(s.elapsed_time(e) for s, e in v) / len(v) / n for k, v in self.pairs.items()}


def run_step(torch, ops, linears, attn_inputs, timers: Timers | None, fuse_q: bool = True, tau: float = -1.0,
             chain: str | None = None):
    """One pass of the hot path; the same kernel calls FP8Linear.forward / fp8_attention make
    (tau: the attention's repair threshold, < 0 for none).

    chain: None runs every linear on its own activations and the attention on its own Q/K/V;
    "stats" / "pass" make the (single) attention's q, k, v the [B, H, S, D] views of the QKV
    projection's output and run it right after that projection, as a DiT block does, with
    the K/V statistics from the projection's epilogue ("stats": gemm_rowwise_kv_stats +
    attn_quant_kv_gemm_stats, K and V read once) or from their own pass ("pass":
    attn_quant_kv)."""
    timed = timers.run if timers else (lambda name, fn, *args: fn(*args))
    outs = []

    def attention(name, q, k, v, mask, part=None):
        sfx = "" if name == "attn" else f"[{name}]"
        c = ops.softmax_c(None, HEAD_DIM)
        if part is None:
            k8, sk, v8t, sv, _ = timed("attn_quant_kv" + sfx, ops.attn_quant_kv, k, v)
        else:
            k8, sk, v8t, sv, _ = timed("attn_quant_kv" + sfx, ops.attn_quant_kv_gemm_stats, k, v, part, None)
        if fuse_q:
            # the Q quantizer runs inside the attention launch
            outs.append(timed("attn_fwd" + sfx, ops.attn_fwd_q, q, c, k8, v8t, sk, sv, mask, None, tau,
                              k.shape[2]))
        else:
            q8, sq = timed("attn_quant_q" + sfx, ops.attn_quant_q, q, c)
            outs.append(timed("attn_fwd" + sfx, ops.attn_fwd, q8, k8, v8t, sq, sk, sv, mask, None, tau, q,
                              k.shape[2]))

    for name, mod, x, mod_params in linears:
        if mod_params is None:
            x8, sa = timed(f"quant_rows[{name}]", ops.quant_rows, x)
        else:
            # x is the block's hidden state; the linear's input is its adaLN modulation
            x8, sa, x = timed(f"adaln_quant[{name}]", ops.adaln_quant_rows, x.unsqueeze(0), mod_params[0],
                              mod_params[1], 1e-6, False, bool(mod.adapters))
        lt, lb, ls = None, None, 0.0
        if mod.adapters:
            lt, lb, ls = timed(f"lora_down[{name}]", mod._lora_operands, x)
        if chain == "stats" and name == "qkv":
            out, part = timed(f"gemm[{name}]", ops.gemm_rowwise_kv_stats, x8, mod.w8, sa, mod.w_scale, mod.bias,
                              x.shape[0], HIDDEN, 2 * HIDDEN, HIDDEN)
        else:
            out, part = timed(f"gemm[{name}]", ops.gemm_rowwise, x8, mod.w8, sa, mod.w_scale, mod.bias,
                              int(mod.act), lt, lb, ls), None
        outs.append(out)
        if chain and name == "qkv":
            (aname, q, k, v, mask), = attn_inputs
            B, S = q.shape[0], q.shape[2]
            qkv = out.view(B, S, 3, HEADS, HEAD_DIM)
            q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
            attention(aname, q, k, v, mask, part)
    if not chain:
        for name, q, k, v, mask in attn_inputs:
            attention(name, q, k, v, mask)
    return outs


def hbm_stream_reference(torch, dev, mib: int = 1024, reps: int = 5) -> dict:
    """A plain streaming kernel of known traffic: y = -x over `mib` MiB of bf16.

    Reports the HBM rate a simple elementwise kernel reaches on this device (read + write
    bytes / kernel time), next to the quantizers' rates.  Under `rocprofv3 --pmc` its
    dispatches are the calibration point of FETCH_SIZE / WRITE_SIZE (exactly `mib` MiB
    read and written per launch).
    """
    n = mib * (1 << 20) // 2
    x = torch.ones(n, dtype=torch.bfloat16, device=dev)
    y = torch.empty_like(x)
    torch.neg(x, out=y)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        torch.neg(x, out=y)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    del x, y
    return {"kernel": "torch.neg bf16 (elementwise)", "bytes_per_launch": 2 * mib * (1 << 20),
            "ms": round(ms, 4), "GB/s": round(2 * mib * (1 << 20) / ms / 1e6, 1)}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(step_lin: float, step_att: float, specs=LINEARS, full_tokens: int = 0, runs: int = 5) -> dict:
    """Reference CPU fallbacks on a bounded sample, scaled to the step's FLOP mix
    (step_lin GEMM FLOPs of the linears `specs`, step_att attention FLOPs): the median of
    `runs` timed runs of each part after one warmup run.  With `full_tokens` the linear
    sample is the whole step's linears at that many tokens; otherwise 2048 of the DiT's
    20280 tokens."""
    import statistics

    import torch

    from oracle.cpu_baseline import dequant_linear, quantize_rows_torch, sdpa_fallback

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    ms = full_tokens or 2048
    lin = []
    for _, k, n, _ in specs:
        x = torch.randn((ms, k), generator=g).to(torch.bfloat16)
        w = (torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16)
        x8, sa = quantize_rows_torch(x)
        w8, sw = quantize_rows_torch(w)
        lin.append((x8, sa, w8, sw.view(1, -1), (torch.randn((n,), generator=g) * 0.01).to(torch.bfloat16)))
    lin_flops = sum(gemm_flops(ms, n, k) for _, k, n, _ in specs)
    hs = 2
    q, k, v = (torch.randn((1, hs, TOKENS, HEAD_DIM), generator=g) for _ in range(3))
    at_flops = attn_flops(1, hs, TOKENS, TOKENS, HEAD_DIM)

    def median_time(fn):
        fn()  # warmup
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    # a part the step does not have is not sampled
    t_lin = median_time(lambda: [dequant_linear(*a) for a in lin]) if step_lin else float("inf")
    t_att = median_time(lambda: sdpa_fallback(q, k, v)) if step_att else float("inf")
    lin_rate, att_rate = lin_flops / t_lin, at_flops / t_att
    step_s = (step_lin / lin_rate if step_lin else 0.0) + (step_att / att_rate if step_att else 0.0)
    if full_tokens and not step_att:
        sample = (f"median of {runs} runs after a warmup: torch CPU fp32 dequant-matmul of the whole step "
                  f"({len(specs)} linear(s) at {ms} tokens, {lin_flops / 1e9:.2f} GFLOP, {t_lin * 1e3:.1f} ms); "
                  f"host {cpu_model()}, {cores} threads")
    else:
        sample = (f"median of {runs} runs after a warmup: torch CPU fp32 dequant-matmul of the {len(specs)} DiT "
                  f"linears on {ms} of {TOKENS} tokens ({lin_rate / 1e12:.3f} TFLOP/s) and fp32 SDPA on {hs} of "
                  f"{HEADS} heads at S={TOKENS} ({att_rate / 1e12:.3f} TFLOP/s); value = the step's FLOPs over the "
                  f"step time these rates imply ({step_s:.1f} s, heads scaled x{HEADS // hs}); host {cpu_model()}, "
                  f"{cores} threads")
    return {
        "value": round((step_lin + step_att) / step_s / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": sample,
    }


# ---------------------------------------------------------------------------------------
# Profile summaries (no GPU needed): tables from rocprofv3's CSV output of this script's
# default workload, e.g.
#   rocprofv3 --kernel-trace --stats --output-format csv -d T -o run -- python3 bench.py ...
#   python3 bench.py --summarize-trace T
#   rocprofv3 --pmc <counters> --output-format csv -d P1 -o run -- python3 bench.py ...   (per pass)
#   python3 bench.py --summarize-counters P1 P2 P3 P4
# ---------------------------------------------------------------------------------------

def _csv_rows(directory: str, suffix: str):
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {directory}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _labels(dispatches, tokens: int = TOKENS, attn_names=("attn",), gemm_names=("qkv", "attn_out", "mlp_down")):
    """dispatch id -> part name for the DiT-block kernels of this script's steps, in dispatch
    order: the no-activation GEMMs of a step are `gemm_names` in turn (the DiT block's QKV,
    attention-out, MLP-down; MLP-up is the GELU instance); activation quantizers are told from
    the weight quantizers at set-up by their grid (one 256-thread block per 4 rows of the
    workload's tokens)."""
    act_grid = str(math.ceil(tokens / 4) * 256)
    out, k = {}, 0
    na = len(attn_names)
    ka = kq = kl = 0  # attention, K/V quantizer and LoRA-down launches so far (in step order)

    def sfx(i):
        return "" if na == 1 else f"[{attn_names[i % na]}]"
    for d, name, grid in dispatches:
        if "gemm_fp8_rowwise_kernel" in name:
            act = re.search(r"GemmCfg<[^>]*>, (\d+),", name)
            if act and act.group(1) == "1":  # the GELU-tanh epilogue
                out[d] = "gemm[mlp_up]"
            else:
                out[d] = f"gemm[{gemm_names[k % len(gemm_names)]}]"
                k += 1
        elif "quant_rows_reg_kernel" in name and grid == act_grid:
            out[d] = "quant_rows<0, 24>[mlp_down]" if "<0, 24" in name else "quant_rows<0, 6>"
        elif "adaln_quant_rows_kernel" in name:
            out[d] = "adaln_quant_rows"
        elif "lora_down_kernel" in name:  # every linear of a LoRA workload runs one, in LINEARS order
            out[d] = f"lora_down[{LINEARS[kl % len(LINEARS)][0]}]"
            kl += 1
        elif "attn_fwd_kernel" in name or "attn_fwd_resident_kernel" in name:
            out[d] = "attn_fwd" + sfx(ka)
            ka += 1
        elif "attn_kv_colreduce_kernel" in name:
            out[d] = "attn_quant_kv: colreduce" + sfx(kq)
        elif "attn_kv_fold_kernel" in name or "gemm_kv_stats_fold_kernel" in name:
            out[d] = "attn_quant_kv: fold" + sfx(kq)
        elif "attn_quant_kv_kernel" in name:
            out[d] = "attn_quant_kv: quantize" + sfx(kq)
            kq += 1
        elif "vectorized_elementwise_kernel" in name and "neg_kernel" in name:
            out[d] = "torch.neg 1 GiB (HBM reference)"
    return out


PART_ORDER = ("gemm[qkv]", "gemm[attn_out]", "gemm[mlp_up]", "gemm[mlp_down]", "quant_rows<0, 6>",
              "quant_rows<0, 24>[mlp_down]", "adaln_quant_rows", "lora_down[qkv]", "lora_down[attn_out]",
              "lora_down[mlp_up]", "lora_down[mlp_down]", "attn_quant_kv: colreduce", "attn_quant_kv: fold",
              "attn_quant_kv: quantize", "attn_fwd", "torch.neg 1 GiB (HBM reference)")


def summarize_trace(directory: str, workload: str = "dit480") -> str:
    """Kernel-trace durations of each part over every step the run made (workload: the
    --workload of the traced run), and the roofline fraction of its largest attention
    recomputed from the median launch (for several attentions per step, of all of them)."""
    _, tokens, _, attns, _ = WORKLOADS[workload]
    rows = _csv_rows(directory, "kernel_trace.csv")
    disp = sorted((int(r["Dispatch_Id"]), r["Kernel_Name"], r.get("Grid_Size", r.get("Grid_Size_X"))) for r in rows)
    names = tuple(a[0] for a in attns)
    gemm_names = tuple(n for n, _, _, act in linears_of(workload) if act == 0)
    lab = _labels(disp, tokens or TOKENS, names, gemm_names)
    dur = {}
    for r in rows:
        d = int(r["Dispatch_Id"])
        if d in lab:
            dur.setdefault(lab[d], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    def median(v):
        v = sorted(v)
        return v[len(v) // 2] if len(v) % 2 else 0.5 * (v[len(v) // 2 - 1] + v[len(v) // 2])

    order = list(PART_ORDER)
    if len(names) > 1:
        order += [f"{base}[{n}]" for n in names for base in ("attn_quant_kv: colreduce", "attn_quant_kv: fold",
                                                              "attn_quant_kv: quantize", "attn_fwd")]
    order += sorted(p for p in dur if p not in order)
    lines = ["| part | launches | median us | mean us | min us | max us |", "|---|---|---|---|---|---|"]
    for p in order:
        if p in dur:
            v = dur[p]
            lines.append(f"| `{p}` | {len(v)} | {median(v):.1f} | {sum(v) / len(v):.1f} | {min(v):.1f} | "
                         f"{max(v):.1f} |")
    lines.append("")
    for i, (name, b, sq, sk, _) in enumerate(attns):
        key = "attn_fwd" + ("" if len(attns) == 1 else f"[{name}]")
        if key not in dur:
            continue
        med = median(dur[key])
        f = attn_flops(b, HEADS, sq, sk, HEAD_DIM)
        lines.append(f"`{key}` recomputed from this trace: FLOPs 4 x {b} x 24 x {sq} x {sk} x 128 = {f / 1e12:.4f} "
                     f"TFLOP per launch / {med:.1f} us (median launch) = {f / (med * 1e-6) / 1e12:.1f} TFLOP/s = "
                     f"{f / (med * 1e-6) / 1e12 / PEAK_FP8_TFLOPS:.4f} of the {PEAK_FP8_TFLOPS:.0f} TFLOP/s dense "
                     f"FP8 peak.")
    for name, k, n, _ in (linears_of(workload) if tokens else ()):
        key = f"gemm[{name}]"
        if key in dur:
            med = median(dur[key])
            f = gemm_flops(tokens, n, k)
            lines.append(f"`{key}` recomputed from this trace: 2 x {tokens} x {n} x {k} = {f / 1e12:.4f} TFLOP / "
                         f"{med:.1f} us (median launch) = {f / (med * 1e-6) / 1e12:.1f} TFLOP/s = "
                         f"{f / (med * 1e-6) / 1e12 / PEAK_FP8_TFLOPS:.4f} of peak.")
    return "\n".join(lines)


def summarize_counters(directories: list[str], workload: str = "dit480") -> str:
    """Per part, the mean over its launches of each counter the passes collected, as busy
    fractions (SQ counters) and calibrated HBM bytes (FETCH_SIZE / WRITE_SIZE); workload: the
    --workload of the profiled runs."""
    _, tokens, _, attns, _ = WORKLOADS[workload]
    anames = tuple(a[0] for a in attns)
    gemm_names = tuple(n for n, _, _, act in linears_of(workload) if act == 0)
    per = {}
    for d in directories:
        rows = _csv_rows(d, "counter_collection.csv")
        names = {}
        vals = {}
        durs = {}
        for r in rows:
            i = int(r["Dispatch_Id"])
            names[i] = (r["Kernel_Name"], r["Grid_Size"])
            vals.setdefault(i, {}).setdefault(r["Counter_Name"], 0.0)
            vals[i][r["Counter_Name"]] += float(r["Counter_Value"])
            if r["Counter_Name"] == "SQ_BUSY_CYCLES":
                durs[i] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])  # ns
        lab = _labels([(i, n, g) for i, (n, g) in sorted(names.items())], tokens or TOKENS, anames, gemm_names)
        for i, part in lab.items():
            for c, v in vals[i].items():
                per.setdefault(part, {}).setdefault(c, []).append(v)
            if i in durs:
                per.setdefault(part, {}).setdefault("duration_ns", []).append(float(durs[i]))

    def m(part, c):
        v = per.get(part, {}).get(c)
        return sum(v) / len(v) if v else None

    ref = "torch.neg 1 GiB (HBM reference)"
    fetch_k = (1 << 30) / (m(ref, "FETCH_SIZE") * 1024) if m(ref, "FETCH_SIZE") else None
    write_k = (1 << 30) / (m(ref, "WRITE_SIZE") * 1024) if m(ref, "WRITE_SIZE") else None
    lines = []
    if fetch_k and write_k:
        lines += [f"Calibration (the 1 GiB bf16 negation reads and writes exactly 1 GiB per launch): bytes read = "
                  f"{fetch_k:.3f} x FETCH_SIZE KiB x 1024, bytes written = {write_k:.3f} x WRITE_SIZE KiB x 1024.", ""]
    lds_cols = any(m(p, "SQ_LDS_IDX_ACTIVE") is not None for p in per)
    lines += ["| part | kernel cycles (M) | clock GHz | MFMA busy | VALU busy | MFMA+VALU co-issue | LDS busy | wait | "
              "VALU instr / MFMA instr | HBM read MB | HBM write MB |" +
              (" LDS active | LDS data FIFO full |" if lds_cols else ""),
              "|---|---|---|---|---|---|---|---|---|---|---|" + ("---|---|" if lds_cols else "")]
    order = list(PART_ORDER)
    if len(anames) > 1:
        order += [f"{base}[{n}]" for n in anames for base in ("attn_quant_kv: colreduce", "attn_quant_kv: fold",
                                                               "attn_quant_kv: quantize", "attn_fwd")]
    for p in order:
        if p not in per:
            continue
        busy = m(p, "SQ_BUSY_CYCLES")
        cyc = busy / 32 if busy else None  # SQ busy cycles are summed over the 32 shader engines
        simd = 1024 * cyc if cyc else None  # 256 CUs x 4 SIMDs

        def frac(c, k=1.0):
            v = m(p, c)
            return f"{k * v / simd:.1%}" if v is not None and simd else "-"
        waves = m(p, "SQ_WAVE_CYCLES")
        wait = f"{m(p, 'SQ_WAIT_INST_ANY') / waves:.1%}" if waves and m(p, "SQ_WAIT_INST_ANY") is not None else "-"
        ratio = "-"
        if m(p, "SQ_INSTS_VALU") is not None and m(p, "SQ_INSTS_MFMA"):
            ratio = f"{m(p, 'SQ_INSTS_VALU') / m(p, 'SQ_INSTS_MFMA'):.1f}"
        rd = f"{m(p, 'FETCH_SIZE') * 1024 * fetch_k / 1e6:.1f}" if m(p, "FETCH_SIZE") is not None and fetch_k else "-"
        wr = f"{m(p, 'WRITE_SIZE') * 1024 * write_k / 1e6:.1f}" if m(p, "WRITE_SIZE") is not None and write_k else "-"
        dur = m(p, "duration_ns")
        ghz = f"{cyc / dur:.2f}" if cyc and dur else "-"
        extra = ""
        if lds_cols:
            # per-CU cycles (summed over the 256 CUs) over the kernel's cycles
            extra = f" {frac('SQ_LDS_IDX_ACTIVE', 4.0)} | {frac('SQ_LDS_DATA_FIFO_FULL', 4.0)} |"
        lines.append(f"| `{p}` | {cyc / 1e6:.2f} | {ghz} | {frac('SQ_VALU_MFMA_BUSY_CYCLES')} | "
                     f"{frac('SQ_ACTIVE_INST_VALU', 4.0)} | {frac('SQ_VALU_MFMA_COEXEC_CYCLES')} | "
                     f"{frac('SQ_ACTIVE_INST_LDS', 4.0)} | {wait} | {ratio} | {rd} | {wr} |{extra}"
                     if cyc else f"| `{p}` | - | - | - | - | - | - | - | {ratio} | {rd} | {wr} |{extra}")
    lines += ["", "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x kernel cycles); VALU busy = 4 x "
                  "SQ_ACTIVE_INST_VALU (quad-cycles) / the same; co-issue = SQ_VALU_MFMA_COEXEC_CYCLES / the same; "
                  "LDS busy = 4 x SQ_ACTIVE_INST_LDS / the same; LDS active = SQ_LDS_IDX_ACTIVE (cycles the LDS "
                  "serves indexed accesses, summed over the CUs) / (256 CUs x kernel cycles), FIFO full = "
                  "SQ_LDS_DATA_FIFO_FULL over the same; kernel cycles = SQ_BUSY_CYCLES / 32; clock = "
                  "kernel cycles / the dispatch's duration in the same pass (the 5.0 PFLOP/s peak assumes 2.4 GHz); "
                  "wait = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES."]
    return "\n".join(lines)


def compare_scaled_mm(torch, dev, workload: str, reps: int = 6, inner: int = 10) -> dict:
    """The reference's own GEMM call on this GPU against mxf8_gemm_rowwise, same operands.

    kernels/fp8_linear.py:95-102 calls torch._scaled_mm(x8, w8.t(), scale_a=x_scale [M, 1],
    scale_b=w_scale, bias=bias, out_dtype=bf16); on ROCm that is hipBLASLt's row-wise scaled
    FP8 GEMM.  For each linear of the workload (activations and weights made and quantized as
    the bench makes them, GELU off on both sides), the two launches are timed alternately,
    `inner` launches per HIP event pair, best of `reps` pairs each."""
    from minimaxh3_amd import ops
    g = torch.Generator(device=dev).manual_seed(1)
    tokens = WORKLOADS[workload][1]
    rows = []
    for name, k, n, _act in linears_of(workload):
        x = activations(torch, g, tokens, k, dev, workload not in NO_OUTLIERS)
        w = (torch.randn((n, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
        bias = (torch.randn((n,), device=dev, generator=g) * 0.01).to(torch.bfloat16)
        x8, sa = ops.quant_rows(x)
        w8, sw = ops.quant_rows(w)
        sw_row = sw.view(1, -1)
        ours = lambda: ops.gemm_rowwise(x8, w8, sa, sw_row, bias, 0, None, None, 0.0)
        ref_call = lambda: torch._scaled_mm(x8, w8.t(), scale_a=sa, scale_b=sw_row, bias=bias,
                                            out_dtype=torch.bfloat16)
        row = {"linear": name, "M": tokens, "N": n, "K": k}
        try:
            r = ref_call()
            r = r[0] if isinstance(r, tuple) else r
        except Exception as exc:  # the call the reference makes is not available here
            row["scaled_mm"] = f"unavailable: {type(exc).__name__}: {str(exc)[:160]}"
            r = None
        o = ours()
        torch.cuda.synchronize()
        best = {"mxf8": float("inf"), "scaled_mm": float("inf")}
        for _ in range(reps):
            for key, fn in (("mxf8", ours), ("scaled_mm", ref_call if r is not None else None)):
                if fn is None:
                    continue
                s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s0.record()
                for _ in range(inner):
                    fn()
                s1.record()
                torch.cuda.synchronize()
                best[key] = min(best[key], s0.elapsed_time(s1) / inner)
        flops = gemm_flops(tokens, n, k)
        for key in best:
            if best[key] != float("inf"):
                row[f"{key}_us"] = round(best[key] * 1e3, 1)
                row[f"{key}_tflops"] = round(flops / (best[key] * 1e-3) / 1e12, 1)
        if r is not None:
            row["scaled_mm_time_over_mxf8"] = round(best["scaled_mm"] / best["mxf8"], 3)
            diff = (o.float() - r.float()).abs().max().item()
            row["max_abs_diff_over_max_abs"] = round(diff / max(r.float().abs().max().item(), 1e-30), 6)
        rows.append(row)
        log(f"[bench] {row}")
    return {"compare": "torch._scaled_mm (the reference's call, fp8_linear.py:95-102) vs mxf8_gemm_rowwise",
            "workload": workload, "device": torch.cuda.get_device_name(dev), "rows": rows}


def compare_sdpa(torch, dev, workload: str, reps: int = 3, inner: int = 5) -> dict:
    """The FP8 attention call against torch's bf16 scaled_dot_product_attention on this GPU.

    bf16 SDPA is what the reference's router runs for the cases it does not send to the FP8
    kernel (kernels/attention_router.py); here it takes the same q, k, v for each unmasked
    attention of the workload.  fp8_attention is the whole call:
    K/V quantization and the attention launch.  Alternating, `inner` calls per HIP event pair,
    best of `reps` pairs each."""
    import torch.nn.functional as F
    from minimaxh3_amd.kernels.attention_router import _orig_sdpa
    from minimaxh3_amd.kernels.fp8_attention import fp8_attention
    _, _, _, attns, _ = WORKLOADS[workload]
    _, attn_inputs = build_workload(torch, dev, 0, 0, attns, False, (), True)
    rows = []
    for (name, b, sq, sk, tail), (_, q, k, v, mask) in zip(attns, attn_inputs):
        if mask is not None:
            # a boolean mask can send SDPA to its math path, which holds the whole B x H x Sq x Sk
            # score matrix (tens of GB here)
            rows.append({"attention": name, "B": b, "Sq": sq, "Sk": sk, "masked_tail": tail,
                         "skipped": "key mask: SDPA's masked path would hold the whole score matrix"})
            continue
        fns = {"fp8_attention": lambda: fp8_attention(q, k, v),
               "sdpa_bf16": lambda: _orig_sdpa(q, k, v)}
        outs = {key: fn() for key, fn in fns.items()}
        torch.cuda.synchronize()
        best = {key: float("inf") for key in fns}
        for _ in range(reps):
            for key, fn in fns.items():
                s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s0.record()
                for _ in range(inner):
                    fn()
                s1.record()
                torch.cuda.synchronize()
                best[key] = min(best[key], s0.elapsed_time(s1) / inner)
        flops = attn_flops(b, HEADS, sq, sk, HEAD_DIM)
        row = {"attention": name, "B": b, "Sq": sq, "Sk": sk, "masked_tail": tail}
        for key, ms in best.items():
            row[f"{key}_ms"] = round(ms, 4)
            row[f"{key}_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
        row["sdpa_time_over_fp8"] = round(best["sdpa_bf16"] / best["fp8_attention"], 3)
        a, r = outs["fp8_attention"].float(), outs["sdpa_bf16"].float()
        row["cosine"] = round((a * r).sum().item() / max((a.norm() * r.norm()).item(), 1e-30), 6)
        rows.append(row)
        log(f"[bench] {row}")
        del outs
    return {"compare": "torch bf16 scaled_dot_product_attention vs fp8_attention (whole call)",
            "workload": workload, "device": torch.cuda.get_device_name(dev), "rows": rows}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="dit480")
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--separate-q-quant", action="store_true",
                    help="quantize Q in its own launch instead of inside the attention launch")
    ap.add_argument("--chain", choices=("stats", "pass"),
                    help="dit480 only: the attention's q, k, v are the QKV projection's output (views of "
                         "[1, S, 3, H, D]), its K/V statistics from the projection's epilogue (stats) or from "
                         "their own pass over K and V (pass)")
    ap.add_argument("--repair-tau", type=float, default=-1.0,
                    help="exact repair of P codes >= tau in every attention (the reference's quality "
                         "profile uses 0.5); < 0 disables it (default)")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print the per-part table of a rocprofv3 --kernel-trace run of this script and exit")
    ap.add_argument("--summarize-counters", metavar="DIR", nargs="+",
                    help="print the per-part counter table of rocprofv3 --pmc runs of this script and exit")
    ap.add_argument("--no-reference-call", action="store_true",
                    help="skip the comparison with the reference's torch._scaled_mm call that follows the timed "
                         "steps of workloads with plain linears (--no-cpu-baseline skips it too)")
    ap.add_argument("--compare-sdpa", action="store_true",
                    help="time torch's bf16 scaled_dot_product_attention against the FP8 attention call on the "
                         "workload's attentions, print one JSON object and exit")
    ap.add_argument("--compare-scaled-mm", action="store_true",
                    help="time the reference's torch._scaled_mm call (hipBLASLt) against mxf8_gemm_rowwise on "
                         "the workload's linears, print one JSON object and exit")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.workload))
        return 0
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.workload))
        return 0
    if args.compare_sdpa and args.compare_scaled_mm:
        print("--compare-sdpa and --compare-scaled-mm are separate runs", file=sys.stderr)
        return 2
    if args.compare_sdpa and not WORKLOADS[args.workload][3]:
        print(f"--compare-sdpa: workload {args.workload} has no attention", file=sys.stderr)
        return 2
    if args.compare_scaled_mm and not WORKLOADS[args.workload][1]:
        print(f"--compare-scaled-mm: workload {args.workload} has no linears", file=sys.stderr)
        return 2
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the FP8 hot path runs on a single MI355X); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch

    from minimaxh3_amd import _native, ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _native.load()
    _native.require_gfx950(dev)
    if args.compare_sdpa:
        print(json.dumps(compare_sdpa(torch, dev, args.workload)), flush=True)
        return 0
    if args.compare_scaled_mm:
        print(json.dumps(compare_scaled_mm(torch, dev, args.workload)), flush=True)
        return 0
    desc, tokens, lora_rank, attns, adaln = WORKLOADS[args.workload]
    specs = linears_of(args.workload)
    fuse_q = not args.separate_q_quant
    tau = float(args.repair_tau)
    chain = args.chain
    if chain and args.workload != "dit480":
        print("--chain applies to --workload dit480 only", file=sys.stderr)
        return 2
    if chain:
        desc += (f"; chained: the attention reads the QKV projection's output, K/V statistics "
                 f"{'from its epilogue' if chain == 'stats' else 'from their own pass'}")
    log("[bench] HBM streaming reference")
    stream_ref = hbm_stream_reference(torch, dev)
    log(f"[bench] building workload {args.workload}")
    linears, attn_inputs = build_workload(torch, dev, tokens, lora_rank, attns, adaln, specs,
                                          args.workload not in NO_OUTLIERS)
    torch.cuda.synchronize()

    def step(timers=None):
        return run_step(torch, ops, linears, attn_inputs, timers, fuse_q, tau, chain)

    graphed = args.workload in GRAPHED
    with torch.inference_mode():
        for i in range(args.warmup):
            step()
        torch.cuda.synchronize()
        graph = None
        if graphed:
            # the K timed steps captured back to back in one graph (after one eager step on a
            # side stream), replayed once untimed, then once in the timed region
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(args.steps):
                    step()
            graph.replay()
            torch.cuda.synchronize()
        log(f"[bench] warmup done ({args.warmup} steps{f', then the {args.steps} captured steps replayed once' if graphed else ''})")
        # The timed steps bracket only the attention launches (the roofline kernel) with HIP
        # events: an event pair around every launch adds ~0.1 ms to a 5 ms step.
        roof_timers = Timers(torch, prefix="attn_fwd")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if graph is not None:
            graph.replay()  # the K steps
        else:
            for _ in range(args.steps):
                step(roof_timers)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        log(f"[bench] timed {args.steps} steps in {elapsed:.3f} s")
        # per-launch breakdown (not timed): the same steps again with every launch bracketed,
        # or, for a graph-replayed step, each launch timed over a graph of 20 copies of it
        if graphed:
            timers = Timers(torch, reps=20)
            step(timers)
            torch.cuda.synchronize()
            timers.graph_times()
        else:
            timers = Timers(torch)
            for _ in range(args.steps):
                step(timers)
            torch.cuda.synchronize()
    ms_step = elapsed * 1e3 / args.steps
    kern = timers.mean_ms()
    roof_kern = roof_timers.mean_ms()

    def flop_part(f, t):
        return {"ms": round(t, 4), "TFLOP/s": round(f / t / 1e9, 1), "frac": round(f / t / 1e9 / PEAK_FP8_TFLOPS, 4)}

    def byte_part(nbytes, t):
        return {"ms": round(t, 4), "GB/s": round(nbytes / t / 1e6, 1), "frac": round(nbytes / t / 1e6 / PEAK_HBM_GBS, 4)}

    parts = {}
    gemm_f = gemm_ms = 0.0
    biggest_gemm = None
    for name, k, n, _ in (specs if tokens else ()):
        f = gemm_flops(tokens, n, k)
        gemm_f += f
        gemm_ms += kern[f"gemm[{name}]"]
        parts[f"gemm[{name}]"] = flop_part(f, kern[f"gemm[{name}]"])
        if biggest_gemm is None or f > biggest_gemm[1]:
            biggest_gemm = (f"gemm[{name}]", f, kern[f"gemm[{name}]"])
        if lora_rank:
            # the rank-r up-projection runs in the GEMM epilogue (not in its FLOP count)
            parts[f"gemm[{name}]"]["lora_tflop"] = round(2.0 * tokens * lora_rank * n / 1e12, 4)
            # lora_down streams x (bf16) once and writes t (bf16)
            t_ld = kern[f"lora_down[{name}]"]
            parts[f"lora_down[{name}]"] = dict(flop_part(2.0 * tokens * lora_rank * k, t_ld),
                                               **{"GB/s": round((tokens * k * 2 + tokens * lora_rank * 2) / t_ld / 1e6, 1)})
        # bf16 read + e4m3 write + fp32 scales
        if adaln and name in ADALN_LINEARS:
            # bf16 read + e4m3 write + fp32 scales (+ the bf16 modulated copy the LoRA reads)
            nbytes = tokens * k * 3 + tokens * 4 + (tokens * k * 2 if lora_rank else 0)
            parts[f"adaln_quant[{name}]"] = byte_part(nbytes, kern[f"adaln_quant[{name}]"])
        else:
            parts[f"quant_rows[{name}]"] = byte_part(tokens * k * 3 + tokens * 4, kern[f"quant_rows[{name}]"])
    attn_f = attn_ms = 0.0
    biggest = None
    for name, b, sq, sk, _ in attns:
        sfx = "" if name == "attn" else f"[{name}]"
        f = attn_flops(b, HEADS, sq, sk, HEAD_DIM)
        t = roof_kern["attn_fwd" + sfx]  # from the timed steps
        attn_f += f
        attn_ms += t
        parts["attn_fwd" + sfx] = flop_part(f, t)
        if biggest is None or f > biggest[1]:
            biggest = ("attn_fwd" + sfx, f, t)
        # K and V: one pass over both credited (3 bytes per element) plus their scales
        for qname, nelem, nscale in (("attn_quant_q", b * HEADS * sq * HEAD_DIM, b * HEADS * math.ceil(sq / 128)),
                                     ("attn_quant_kv", 2 * b * HEADS * sk * HEAD_DIM,
                                      b * HEADS * (math.ceil(sk / 128) + HEAD_DIM))):
            if qname + sfx in kern:  # attn_quant_q only when Q is quantized in its own launch
                parts[qname + sfx] = byte_part(3 * nelem + 4 * nscale, kern[qname + sfx])
    # end-to-end wrappers over the same FLOPs: FP8Linear.forward (activation quantizer or
    # fused adaLN quantizer, LoRA down-projection, GEMM) and fp8_attention (quantizers +
    # attention), from the per-part event times
    lin_ms = sum(v for k, v in kern.items() if k.split("[")[0] in ("quant_rows", "adaln_quant", "lora_down", "gemm"))
    att_ms = attn_ms + sum(v for k, v in kern.items() if k.startswith("attn_quant"))
    step_flops = gemm_f + attn_f
    value = step_flops / (ms_step * 1e-3) / 1e12
    if biggest is not None:
        roof_name, roof_f, roof_t = biggest
        roof_kernel = f"{roof_name}: attn_fwd_kernel<128,...>"
    else:
        # no attention in the step: the largest GEMM (its per-launch time from the breakdown)
        roof_name, roof_f, roof_t = biggest_gemm
        roof_kernel = f"{roof_name}: gemm_fp8_rowwise_kernel"
    achieved = roof_f / (roof_t * 1e-3) / 1e12

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 (fp32 accumulate)",
        "data": "synthetic (seeded randn, random-init weights)",
        "config": {
            "workload": desc,
            "tokens": tokens or None, "hidden": HIDDEN, "mlp": MLP, "heads": HEADS, "head_dim": HEAD_DIM,
            "lora_rank": lora_rank or None,
            "repair_tau": tau if tau >= 0 else None,
            "chain": chain,
            "graph_replay": graphed,
            "step_tflop": round(step_flops / 1e12, 4),
        },
        "frac_of_fp8_peak": round(value / PEAK_FP8_TFLOPS, 4),
        "gemm_tflops": round(gemm_f / (gemm_ms * 1e-3) / 1e12, 1) if gemm_ms else None,
        "attn_tflops": round(attn_f / (attn_ms * 1e-3) / 1e12, 1) if attn_ms else None,
        "end_to_end": {
            "linear": {"ms": round(lin_ms, 4), "TFLOP/s": round(gemm_f / (lin_ms * 1e-3) / 1e12, 1)} if lin_ms else None,
            "attention": ({"ms": round(att_ms, 4), "TFLOP/s": round(attn_f / (att_ms * 1e-3) / 1e12, 1)}
                          if att_ms else None),
        },
        "roofline": {
            "kernel": roof_kernel,
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": PEAK_FP8_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP8_TFLOPS, 4),
            # counter-measured for the 480p attention only
            "traffic": round(ATTN_TRAFFIC_BYTES) if args.workload == "dit480" and not chain else None,
        },
        "kernels": parts,
        "hbm_stream_reference": stream_ref,
    }
    if tokens and not lora_rank and not adaln and not args.no_reference_call and not args.no_cpu_baseline:
        # the reference's own GEMM call on this GPU, timed against this GEMM after the timed
        # region (it does not enter `value`); not in profiling runs (--no-cpu-baseline), whose
        # kernel traces _labels reads in dispatch order
        log("[bench] reference GEMM call")
        try:
            cmp = compare_scaled_mm(torch, dev, args.workload, reps=3, inner=5)
            line["reference_gemm_call"] = {
                "call": "torch._scaled_mm row-wise + bias (kernels/fp8_linear.py:95-102; hipBLASLt on ROCm)",
                "scaled_mm_time_over_mxf8": {r["linear"]: r.get("scaled_mm_time_over_mxf8", r.get("scaled_mm"))
                                             for r in cmp["rows"]},
            }
        except Exception as exc:  # a failure here must not cost the bench line
            line["reference_gemm_call"] = {"error": f"{type(exc).__name__}: {str(exc)[:200]}"}
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline")
        line["cpu_baseline"] = cpu_baseline(gemm_f, attn_f, specs, tokens if args.workload in LINEAR_SETS else 0)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
