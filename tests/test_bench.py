"""The bench.py contract parts that need no GPU: the one-GPU refusal, the
traffic figures it reads from the committed rocprofv3 summary, and the CPU
baseline record (cfg1, both forms of the oracle)."""
import os
import subprocess
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and "--gpus 2" in proc.stderr
    assert proc.stdout == ""  # no JSON line for a configuration that was not measured


def test_traffic_figures_come_from_the_committed_summary():
    dense, sparse = bench.profiled_traffic()
    text = open(os.path.join(ROOT, "profiles", "hbm_traffic_cfg2_dense_cfg4_sparse.md")).read()
    assert f"traffic dense_step_bytes={dense}" in text
    assert f"traffic sparse_step_bytes={sparse}" in text
    # the sparse path reads every visible K block once: within 1% above its
    # algorithmic bytes (K scan plus the unique selected K/V slabs)
    assert 2_684_878_848 <= sparse < 1.01 * 2_684_878_848


def test_cpu_baseline_record_names_cfg1_and_both_forms():
    line = bench.cpu_baseline(0.0, torch)  # no budget: cfg1 only, no cfg2 head sample
    assert line["kind"] == "port" and line["unit"] == "TFLOP/s"
    assert line["cores"] == len(os.sched_getaffinity(0))
    assert "cfg1" in line["sample"] and "median of 10" in line["sample"]
    assert line["value"] > 0 and line["seconds_per_step"] > 0
    assert line["flop_per_step"] == 941_359_104  # cfg1's causal forward+backward FLOP
    chunked = line["chunked"]
    assert chunked["q_chunk"] == 32 and chunked["kv_chunk"] == 1024 and chunked["value"] > 0
    assert "cfg2_one_head" not in line
