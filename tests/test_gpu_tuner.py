"""A tiny end-to-end tuner run on the GPU: every candidate is timed against ATen controls,
checked against the control's output, and the winners form a loadable plan."""
import json
import shutil
import uuid

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["mm", "swiglu"])
def test_tuner_writes_results_and_a_loadable_policy(kind, monkeypatch):
    from ops import tune_matmul
    from ops.matmul_execution import matmul_plan_from_dict

    # The tuner requires its temporary and cache directories inside the workspace.
    scratch = tune_matmul.PACKAGE / "work" / f"tuner-scratch-{uuid.uuid4().hex[:8]}"
    scratch.mkdir(parents=True, exist_ok=True)
    monkeypatch.setenv("TMPDIR", str(scratch))
    monkeypatch.setenv("XDG_CACHE_HOME", str(scratch))
    out = tune_matmul.PACKAGE / "work" / f"benchmark-test-{kind}-{uuid.uuid4().hex[:8]}"
    flags = ["--kind", kind, "--rows", "512", "--ffn", "1024", "--width", "256",
             "--repeats", "3", "--trials", "2", "--warmup", "1", "--burnin-seconds", "0",
             "--minimum-gain", "0", "--tile", "128,128,32,8,3", "--output-dir", str(out)]
    try:
        tune_matmul.main(flags)
        report = json.loads((out / "results.json").read_text())
        policy = json.loads((out / "candidate-policy.json").read_text())
        operations = ["fwd", "dw"] if kind == "mm" else ["fwd"]
        algorithms = ["tiled", "persistent"] + (["persistent_tma"] if kind == "mm" else [])
        assert len(report["results"]) == len(operations) * len(algorithms)
        assert report["device"]["arch"].startswith("gfx950")
        for row in report["results"]:
            assert row["status"] == "ok", row.get("error")
            assert row["relative_rms_error"] <= 3e-3
            assert len(row["trials"]) == 2
        winners = {r["case"]["operation"] for r in report["results"] if r["eligible"]}
        assert {e["name"] for e in policy["entries"]} == winners
        plan = matmul_plan_from_dict(policy)
        assert all(entry.kind == kind for entry in plan.entries)
    finally:
        shutil.rmtree(out, ignore_errors=True)
        shutil.rmtree(scratch, ignore_errors=True)
