"""bench.py's command-line contract that needs no GPU: one GPU only, and its flags parse."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode != 0
    assert "--gpus 2 is not supported" in r.stderr


def test_help_lists_the_workloads_and_switches():
    r = _run("--help")
    assert r.returncode == 0
    for flag in ("--steps", "--warmup", "--workload", "--no-cpu-baseline", "--separate-q-quant"):
        assert flag in r.stdout
    for workload in ("dit480", "joint", "dit720"):
        assert workload in r.stdout


def test_comparison_modes_reject_workloads_without_the_compared_part():
    r = _run("--compare-sdpa", "--workload", "linear2048")
    assert r.returncode == 2 and "has no attention" in r.stderr
    r = _run("--compare-scaled-mm", "--workload", "joint")
    assert r.returncode == 2 and "has no linears" in r.stderr
    r = _run("--compare-sdpa", "--compare-scaled-mm")
    assert r.returncode == 2 and "separate runs" in r.stderr
    r = _run("--help")
    assert "--compare-sdpa" in r.stdout and "--compare-scaled-mm" in r.stdout
