"""bench.py's output contract: one JSON line with the headline metric, its roofline and CPU baseline blocks, and a
clear refusal of more than one GPU."""
import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args, timeout=300):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args], cwd=REPO, capture_output=True,
                          text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused_with_a_message():
    """--gpus N > 1 (or a WORLD_SIZE above 1) exits with status 2 and says why, before touching a device."""
    r = _bench("--gpus", "2", timeout=120)
    assert r.returncode == 2
    assert "single MI355X" in r.stdout and "--gpus 2" in r.stdout


@pytest.mark.gpu
def test_bench_prints_one_json_line_with_the_contract_keys():
    """A short headline run: exactly one JSON line on stdout with the metric, the throughput and the measurement
    blocks, their units and the workload named."""
    r = _bench("--steps", "2", "--warmup", "1", "--cpu-boards", "8", "--evaluator-steps", "2")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, lines
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 2 and d["warmup"] == 1
    assert d["unit"] == "board-evals/s" and d["higher_is_better"] is True and d["value"] > 0
    # dtype is the arithmetic type (float32 sums and updates); the fp16 deviation state is a storage format
    assert d["dtype"] == "f32" and d["data"] == "synthetic" and "workload" in d["config"]
    assert "fp16 deviation" in d["config"]["state"]
    rf = d["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in rf, key
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    cb = d["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in cb, key
    assert cb["kind"] == "port" and cb["value"] > 0 and cb["cores"] >= 1
