"""The committed profile summaries the benchmark's rooflines cite (profiles/traffic.json): for each
decode kernel at batch 1 and 64, its HBM traffic a launch (FETCH_SIZE and WRITE_SIZE, scaled by
the copy calibration) and its traced average duration; for each prefill GEMM at 8 x 2048, its
traced duration. bench.py looks them up by kernel label; a record missing (as when a kernel's
template arguments change and a summary no longer finds it) leaves the line without them. Every
record names a summary file that is committed beside it and the commit it was measured at."""

import json
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PROFILES = ROOT / "profiles"
DECODE = ("gemv_qkv_rope", "attention_decode", "o_proj", "gemv_gate_up", "down_proj")
PREFILL = ("prefill_qkv", "prefill_o", "prefill_gate_up", "prefill_down")


def records():
    return json.loads((PROFILES / "traffic.json").read_text())


def check_file(path: str, commit: str):
    f = ROOT / path
    assert f.exists(), path
    assert commit in f.read_text(), f"{path} does not name commit {commit}"


@pytest.mark.parametrize("workload", ["batch 1", "batch 64"])
def test_every_decode_kernel_has_its_traffic_and_trace_on_record(workload):
    data = records()
    table = data if workload == "batch 1" else data["batch64"]
    for label in DECODE:
        rec = table.get(label)
        assert isinstance(rec, dict), f"{label} at {workload}: no record"
        assert rec["workload"] == workload
        assert rec["bytes_per_launch"] > 0 and rec["trace_avg_us"] > 0, (label, rec)
        assert rec["fetch_scale"] > 0 and rec["write_scale"] > 0
        check_file(rec["source"], rec["commit"])
        check_file(rec["trace_file"], rec["commit"])


def test_every_prefill_gemm_has_its_trace_on_record():
    data = records()["prefill_8x2048"]
    for label in PREFILL:
        rec = data.get(label)
        assert isinstance(rec, dict), f"{label}: no record"
        assert rec["workload"] == "8 x 2048 prefill" and rec["trace_avg_us"] > 0, (label, rec)
        check_file(rec["trace_file"], rec["commit"])


def test_the_benchmark_finds_the_records_of_its_rooflines():
    import sys

    sys.path.insert(0, str(ROOT))
    import bench

    for label in DECODE:
        assert bench.trace_figure(label, "batch 1") is not None, label
        traffic, source = bench.measured_traffic(label, "batch 1")
        assert traffic and source["measured_in_this_run"] is False, label
    assert bench.trace_figure("prefill_gate_up", "8 x 2048 prefill") is not None
