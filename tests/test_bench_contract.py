"""bench.py's contract on the CPU: the one-GPU refusal, the metric naming BASELINE.json's, the
roofline / prefill objects built from a measurement record, and the recorded HBM traffic ratio
the bench line reads from profiles/."""

import json
import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


def test_metric_is_the_baseline_metric():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        assert bench.METRIC == json.load(f)["metric"]


def test_roofline_object_from_a_record():
    r = {"attn_bytes": 8.0e8, "attn_ms": 0.125, "decode_nb": 2, "n_split": 1,
         "attn_launches": 80}
    roof = bench.roofline_of(r)
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert roof["achieved"] == pytest.approx(6400.0)       # 0.8 GB in 0.125 ms
    assert roof["frac"] == pytest.approx(0.8)
    assert roof["bytes_per_launch"] == 800_000_000
    assert "32-slot" in roof["kernel"]


def test_prefill_attention_and_prefill_objects():
    pa = bench.prefill_attention_of({"pa_ms": 0.8, "pa_flops": 0.5e12})
    assert pa["bound"] == "mfma" and pa["unit"] == "TFLOP/s"
    assert pa["achieved"] == pytest.approx(625.0)
    assert pa["frac"] == pytest.approx(0.25)
    assert "hbm" not in pa
    pa = bench.prefill_attention_of({"pa_ms": 0.8, "pa_flops": 0.5e12, "pa_bytes": 2.0e9})
    assert pa["hbm"]["unit"] == "GB/s" and pa["hbm"]["peak"] == 8000.0
    assert pa["hbm"]["achieved"] == pytest.approx(2500.0)     # 2 GB in 0.8 ms
    assert pa["hbm"]["frac"] == pytest.approx(0.3125)
    r = {"n_valid": torch.tensor([300, 700]), "prefill_ms": 2.0, "B": 2, "S": 700,
         "prefill_flops": 3.0e12}
    pf = bench.prefill_of(r)
    assert pf["tokens"] == 1000 and pf["padded_tokens"] == 1400
    assert pf["tokens_per_s"] == pytest.approx(500_000.0)


def test_recorded_traffic_ratio_parses_the_committed_profile():
    ratio, src = bench.recorded_traffic_ratio("attn_decode_kernel", "small_b256")
    assert src == os.path.join("profiles", "pmc_traffic_small_b256.md")
    assert 0.99 < ratio < 1.1
    assert bench.recorded_traffic_ratio("attn_decode_kernel", "no_such_workload") == (None, None)
