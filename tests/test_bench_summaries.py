"""CPU tests of bench.py's profile tooling: the step labeler and the --summarize-trace /
--summarize-counters tables, on small synthetic rocprofv3-style CSV files (the tables in
profiles/ are made by these functions)."""
import csv
import math

import pytest

import bench

GEMM = "void mxf8::gemm_fp8_rowwise_kernel<mxf8::GemmCfg<256, 256, 4, 2>, {act}, {lm}, false>(unsigned char const*)"
ACT_GRID = str(math.ceil(bench.TOKENS / 4) * 256)


def _step(lora: bool):
    """Kernel names and grids of one 480p step in launch order (the bench's run_step): per
    linear the activation quantizer, (lora_down,) the GEMM; then the K/V quantizer and the
    attention."""
    out = []
    for name, k, n, act in bench.LINEARS:
        out.append((f"void mxf8::quant_rows_reg_kernel<0, {24 if k == 12288 else 6}>(...)", ACT_GRID))
        if lora:
            out.append(("void mxf8::lora_down_kernel<2, 5>(...)", "1"))
        out.append((GEMM.format(act=act, lm=1 if lora else 0), "1"))
    out += [("void mxf8::attn_kv_colreduce_kernel<128>(...)", "1"), ("void mxf8::attn_kv_fold_kernel(...)", "1"),
            ("void mxf8::attn_quant_kv_kernel<128>(...)", "1"),
            ("void mxf8::attn_fwd_kernel<128, false, false, false, 0, true>(...)", "1")]
    return out


@pytest.mark.parametrize("lora", [False, True])
def test_labels_follow_the_step_order(lora):
    disp = [(i, n, g) for i, (n, g) in enumerate(_step(lora) + _step(lora))]
    lab = bench._labels(disp)
    got = [lab.get(i) for i, _, _ in disp]
    one = []
    for name, k, _, _ in bench.LINEARS:
        one.append("quant_rows<0, 24>[mlp_down]" if k == 12288 else "quant_rows<0, 6>")
        if lora:
            one.append(f"lora_down[{name}]")
        one.append(f"gemm[{name}]")
    one += ["attn_quant_kv: colreduce", "attn_quant_kv: fold", "attn_quant_kv: quantize", "attn_fwd"]
    assert got == one + one


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_summarize_trace_medians_and_attention_rate(tmp_path):
    rows, t = [], 0
    durs = {"gemm[qkv]": [400, 500, 600], "attn_fwd": [2000, 2500, 3000]}  # us, three steps
    for step in range(3):
        for name, grid in _step(False):
            i = len(rows)
            lab = bench._labels([(j, r["Kernel_Name"], r["Grid_Size"]) for j, r in enumerate(rows)] +
                                [(i, name, grid)]).get(i)
            us = durs.get(lab, [10, 10, 10])[step]
            rows.append({"Dispatch_Id": i, "Kernel_Name": name, "Grid_Size": grid,
                         "Start_Timestamp": t, "End_Timestamp": t + us * 1000})
            t += us * 1000 + 5000
    _write(tmp_path / "run_kernel_trace.csv", rows)
    table = bench.summarize_trace(str(tmp_path))
    assert "| `gemm[qkv]` | 3 | 500.0 | 500.0 | 400.0 | 600.0 |" in table
    assert "| `attn_fwd` | 3 | 2500.0 | 2500.0 | 2000.0 | 3000.0 |" in table
    flops = bench.attn_flops(1, bench.HEADS, bench.TOKENS, bench.TOKENS, bench.HEAD_DIM)
    assert f"= {flops / 2500e-6 / 1e12 / bench.PEAK_FP8_TFLOPS:.4f} of the" in table


def test_summarize_counters_fractions_clock_and_calibration(tmp_path):
    cyc = 4.0e6                          # kernel cycles of the attention
    counters = {
        "attn_fwd": {"SQ_BUSY_CYCLES": 32 * cyc, "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * 1024 * cyc,
                     "SQ_ACTIVE_INST_VALU": 0.6 * 1024 * cyc / 4, "SQ_VALU_MFMA_COEXEC_CYCLES": 0.2 * 1024 * cyc,
                     "SQ_ACTIVE_INST_LDS": 0.05 * 1024 * cyc / 4, "SQ_WAVE_CYCLES": 1000.0, "SQ_WAIT_INST_ANY": 400.0,
                     "FETCH_SIZE": 100000.0, "WRITE_SIZE": 50000.0},
        "torch.neg 1 GiB (HBM reference)": {"FETCH_SIZE": (1 << 30) / 1024 / 2, "WRITE_SIZE": (1 << 30) / 1024},
    }
    names = {"attn_fwd": ("void mxf8::attn_fwd_kernel<128, false, false, false, 0, true>(...)", "1"),
             "torch.neg 1 GiB (HBM reference)": ("void at::native::vectorized_elementwise_kernel<neg_kernel>(...)", "1")}
    rows = []
    for i, (part, cs) in enumerate(counters.items()):
        for c, v in cs.items():
            rows.append({"Dispatch_Id": i, "Kernel_Name": names[part][0], "Grid_Size": names[part][1],
                         "Counter_Name": c, "Counter_Value": v, "Start_Timestamp": 0,
                         "End_Timestamp": 2_000_000 if part == "attn_fwd" else 500_000})
    _write(tmp_path / "run_counter_collection.csv", rows)
    table = bench.summarize_counters([str(tmp_path)])
    assert "bytes read = 2.000 x FETCH_SIZE KiB x 1024, bytes written = 1.000 x WRITE_SIZE KiB x 1024" in table
    row = next(line for line in table.splitlines() if line.startswith("| `attn_fwd`"))
    cells = [c.strip() for c in row.split("|")[2:-1]]
    # cycles, clock (4e6 cycles in 2 ms), MFMA, VALU, co-issue, LDS, wait, ratio, read MB, write MB
    assert cells[:7] == ["4.00", "2.00", "50.0%", "60.0%", "20.0%", "5.0%", "40.0%"]
    assert cells[8] == f"{100000 * 1024 * 2 / 1e6:.1f}" and cells[9] == f"{50000 * 1024 / 1e6:.1f}"


def test_summarize_counters_per_attention_of_the_joint_workload(tmp_path):
    """--workload joint: the two attention launches of a step (self, then cross) and their K/V
    quantizers get rows of their own."""
    step = [("void mxf8::attn_kv_colreduce_kernel<128>(...)", "1"), ("void mxf8::attn_kv_fold_kernel(...)", "1"),
            ("void mxf8::attn_quant_kv_kernel<128>(...)", "1"),
            ("void mxf8::attn_fwd_kernel<128, true, false, false, 0, true>(...)", "1"),
            ("void mxf8::attn_kv_colreduce_kernel<128>(...)", "1"), ("void mxf8::attn_kv_fold_kernel(...)", "1"),
            ("void mxf8::attn_quant_kv_kernel<128>(...)", "1"),
            ("void mxf8::attn_fwd_resident_kernel<128, false, false, 0, true>(...)", "1")]
    busy = {3: 0.5, 7: 0.25}  # MFMA busy of the self and the cross attention
    rows = []
    for i, (name, grid) in enumerate(step):
        cs = {"SQ_BUSY_CYCLES": 32 * 1.0e6, "SQ_VALU_MFMA_BUSY_CYCLES": busy.get(i, 0.0) * 1024 * 1.0e6}
        for c, v in cs.items():
            rows.append({"Dispatch_Id": i, "Kernel_Name": name, "Grid_Size": grid, "Counter_Name": c,
                         "Counter_Value": v, "Start_Timestamp": 0, "End_Timestamp": 1_000_000})
    _write(tmp_path / "run_counter_collection.csv", rows)
    table = bench.summarize_counters([str(tmp_path)], "joint")
    cell = {line.split("|")[1].strip(): [c.strip() for c in line.split("|")[2:-1]]
            for line in table.splitlines() if line.startswith("| `")}
    assert cell["`attn_fwd[self]`"][2] == "50.0%" and cell["`attn_fwd[cross]`"][2] == "25.0%"
    assert "`attn_quant_kv: quantize[cross]`" in cell and "`attn_fwd`" not in cell
