"""bench.py's output contract on a short run (ViT-B/16 q2 at batch 16):
one JSON line with the metric, whole-job images/s, the step counts and a
roofline over the packed launches of the recorded steps (every 4th timed
step, from the first)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_bench_json_line():
    steps, warmup = 5, 1
    cmd = [sys.executable, os.path.join(ROOT, "bench.py"), "--steps", str(steps), "--warmup", str(warmup),
           "--batch", "16", "--no-cpu-baseline", "--no-stream-line", "--no-bf16-line"]
    out = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = [ln for ln in out.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, out.stdout[-2000:]
    rec = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in rec, key
    assert rec["unit"] == "images/s" and rec["n_gpus"] == 1
    assert rec["steps"] == steps and rec["warmup"] == warmup
    assert rec["value"] > 0 and rec["ms_per_step"] > 0
    # value is the batch over the measured step time
    assert abs(rec["value"] - 16 / (rec["ms_per_step"] / 1e3)) <= 1e-3 * rec["value"]
    rf = rec["roofline"]
    assert rf["bound"] == "mfma" and rf["unit"] == "TFLOP/s" and rf["peak"] == 2500.0
    assert 0 < rf["frac"] < 1 and abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    assert rf["recorded_steps"] == 2  # steps 0 and 4 of 5
    assert rec["config"]["packed_layers_per_step"] == 49
    assert rf["launches"] > 0 and rf["launches"] % rf["recorded_steps"] == 0
    assert sum(v["launches"] for v in rf["by_kernel"].values()) == 49 * rf["recorded_steps"]
