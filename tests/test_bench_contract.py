"""The benchmark's output contract, checked on the CPU.

`bench.py` prints one JSON line that the round's driver parses: fixed keys, the metric of
BASELINE.json, a roofline object for the dominant kernel and a CPU-baseline object. The
committed bench line in profiles/ is checked against that contract, and a request for more
than one GPU must be refused before any GPU work.
"""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
LINE = ROOT / "profiles" / "bench_layer_step_m16384.json"
TRAFFIC = ROOT / "profiles" / "hbm_traffic_layer_step_m16384.md"


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_committed_bench_line_keeps_the_contract():
    line = json.loads(LINE.read_text())
    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["metric"] == baseline["metric"]
    assert line["unit"] == "TFLOP/s" and line["higher_is_better"] is True
    assert line["n_gpus"] == 1 and line["dtype"] == "bf16" and line["scaling"] == "weak"
    assert "workload" in line["config"] and "model" not in line["config"]
    # value is the step's FLOPs over its wall time.
    flops = line["config"]["step_gflop"] * 1e9
    assert abs(flops / (line["ms_per_step"] * 1e-3) / 1e12 - line["value"]) < 0.01 * line["value"]

    roof = line["roofline"]
    assert roof["bound"] in ("hbm", "mfma") and roof["unit"] in ("GB/s", "TFLOP/s")
    assert roof["peak"] == 2516.6 and roof["unit"] == "TFLOP/s"
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert roof["kernel"] in line["kernels"]
    # The dominant kernel is the slowest measured region of the step. The hipBLASLt
    # yardstick and the adapter operator are timed outside the step and do not compete.
    step_regions = [k for k in line["kernels"] if not k.endswith((".hipblaslt", ".adapter_op"))]
    assert roof["kernel"] == max(step_regions, key=lambda k: line["kernels"][k]["ms"])
    traffic_lines = {p[1]: int(p[2]) for p in
                     (l.split() for l in TRAFFIC.read_text().splitlines())
                     if len(p) == 3 and p[0] == "traffic_bytes"}
    assert roof["kernel"] in traffic_lines
    assert roof["traffic"] is None or abs(roof["traffic"] - traffic_lines[roof["kernel"]]) < \
        0.01 * traffic_lines[roof["kernel"]]

    cpu = line["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in cpu, key
    assert cpu["kind"] in ("reference", "port") and cpu["cores"] >= 1 and cpu["value"] > 0
