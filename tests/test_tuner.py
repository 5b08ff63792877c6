"""Host logic of the gfx950 tile tuner: options, case layouts, output and timing metrics.

These follow the reference's tuner tests (test_matmul_kernels.py:51-118); no GPU is used.
"""
import math

import pytest
import torch

from ops.tune_matmul import arguments, cases, output_metrics, paired_timing_metrics


def test_kind_defaults_and_selected_tiles():
    generic = arguments(["--list-cases"])
    assert generic.operations == ["fwd", "dw"]
    assert generic.algorithms == ["tiled", "persistent", "persistent_tma"]
    fused = arguments(["--list-cases", "--kind", "swiglu", "--tile", "128,128,32,8,3"])
    assert fused.operations == ["fwd"]
    assert fused.algorithms == ["tiled", "persistent"]
    assert fused.tile == [(128, 128, 32, 8, 3)]


def test_case_layouts_match_the_projection_and_its_weight_gradient():
    forward, dw = cases(8192, ["fwd", "dw"])
    # X [8192, 2048] row-major times W^T with W [14336, 2048] row-major (nn.Linear).
    assert (forward["m"], forward["n"], forward["k"]) == (8192, 14336, 2048)
    assert forward["a_stride"] == [2048, 1] and forward["b_stride"] == [1, 2048]
    # dP^T [14336, 8192] (a transposed view of dP [8192, 14336]) times X [8192, 2048].
    assert (dw["m"], dw["n"], dw["k"]) == (14336, 2048, 8192)
    assert dw["a_stride"] == [1, 14336] and dw["b_stride"] == [2048, 1]
    # The strides are those of real tensors of that layout.
    x = torch.empty(8192, 2048)
    w = torch.empty(14336, 2048)
    dp = torch.empty(8192, 14336)
    assert list(w.T.stride()) == forward["b_stride"] and list(x.stride()) == forward["a_stride"]
    assert list(dp.T.stride()) == dw["a_stride"] and list(x.stride()) == dw["b_stride"]
    only_dw = cases(16, ["dw"], ffn=64, width=32)
    assert [c["operation"] for c in only_dw] == ["ffn_up_gate.dw"]
    assert only_dw[0]["a_stride"] == [1, 64] and only_dw[0]["b_stride"] == [32, 1]


@pytest.mark.parametrize("flags", [
    ["--kind", "swiglu", "--operations", "dw"],
    ["--kind", "swiglu", "--algorithms", "persistent_tma"],
    ["--kind", "swiglu", "--tile", "256,256,32,8,3"],
    ["--tile", "128,128,32,4"],
    ["--tile", "120,128,32,4,3"],
    ["--input-scale", "nan"], ["--input-scale", "0"], ["--input-scale", "-1"],
    ["--burnin-seconds", "inf"], ["--minimum-gain", "-0.1"],
    ["--maximum-relative-rms", "nan"],
    ["--rows", "0"], ["--trials", "0"], ["--repeats", "-2"], ["--warmup", "0"],
    ["--operations", "fwd", "fwd"],
    ["--algorithms", "tiled", "tiled"],
    ["--tile", "128,128,32,4,3", "--tile", "128,128,32,4,3"],
    ["--output-dir", "/tmp/outside-workspace"],
])
def test_rejects_unsupported_kind_or_unsafe_output(flags):
    with pytest.raises(SystemExit):
        arguments(["--list-cases", *flags])


def test_output_directory_must_be_a_benchmark_folder_in_the_package_work_area():
    from ops import tune_matmul

    work = tune_matmul.PACKAGE / "work"
    ok = arguments(["--list-cases", "--output-dir", str(work / "benchmark-x")])
    assert ok.output_dir == (work / "benchmark-x").resolve()
    for bad in (work, work / "other", work / "benchmark-x" / ".." / ".." / "benchmark-y"):
        with pytest.raises(SystemExit):
            arguments(["--list-cases", "--output-dir", str(bad)])


def test_real_runs_require_workspace_scratch_directories(monkeypatch, tmp_path):
    from ops import tune_matmul

    monkeypatch.setenv("TMPDIR", "/tmp")
    monkeypatch.setenv("XDG_CACHE_HOME", str(tune_matmul.WORKSPACE / "_cache"))
    with pytest.raises(SystemExit):
        arguments([])
    monkeypatch.setenv("TMPDIR", str(tune_matmul.WORKSPACE / "_tmp"))
    assert arguments([]).operations == ["fwd", "dw"]


def test_checks_all_outputs_and_preserves_bf16():
    expected = torch.ones((4, 8), dtype=torch.bfloat16)
    metrics = output_metrics((expected.clone(), expected * 2), (expected, expected))
    assert metrics["output_metrics"][0]["relative_rms_error"] == 0
    # |2 - 1| over an RMS of 1 on the second output.
    assert metrics["relative_rms_error"] == 1
    assert metrics["max_abs_error"] == 1
    with pytest.raises(ValueError, match="BF16"):
        output_metrics(expected.float(), expected)
    with pytest.raises(ValueError, match="BF16"):
        output_metrics(expected[:2], expected)
    with pytest.raises(ValueError, match="Nonfinite"):
        output_metrics((expected, expected * float("nan")), (expected, expected))
    with pytest.raises(ValueError, match="same number"):
        output_metrics((expected,), (expected, expected))


def test_relative_rms_against_a_hand_computed_value():
    want = torch.tensor([[3.0, 4.0]], dtype=torch.bfloat16)
    got = torch.tensor([[3.0, 5.0]], dtype=torch.bfloat16)
    # sqrt(mean([0, 1])) / sqrt(mean([9, 16])) = sqrt(0.5) / sqrt(12.5) = 0.2
    assert output_metrics(got, want)["relative_rms_error"] == pytest.approx(0.2, rel=1e-6)


def test_cannot_select_a_median_winner_with_a_losing_trial():
    trials = [{"aten_before_ms": 2.0, "candidate_ms": candidate, "aten_after_ms": 2.0}
              for candidate in (1.5, 1.5, 2.1)]
    metrics = paired_timing_metrics(trials, minimum_gain=0.01)
    assert metrics["paired_gain"] == pytest.approx(2.0 / 1.5 - 1.0)
    assert metrics["minimum_trial_gain"] == pytest.approx(2.0 / 2.1 - 1.0)
    assert not metrics["timing_eligible"]
    assert metrics["median_ms"] == 1.5 and metrics["median_control_ms"] == 2.0
    drifted = [{"aten_before_ms": 1.0, "candidate_ms": 1.4, "aten_after_ms": 2.0}]
    metrics = paired_timing_metrics(drifted, minimum_gain=0.01)
    assert metrics["timing_eligible"]
    assert metrics["maximum_control_drift_fraction"] == pytest.approx(2 / 3)


@pytest.mark.parametrize("timing", [0, -1, float("nan"), float("inf")])
def test_rejects_invalid_timing_metrics(timing):
    with pytest.raises(ValueError, match="finite and positive"):
        paired_timing_metrics([{"aten_before_ms": 1, "candidate_ms": timing,
                                "aten_after_ms": 1}], minimum_gain=0.01)
    with pytest.raises(ValueError, match="finite and positive"):
        paired_timing_metrics([], minimum_gain=0.01)


def test_list_cases_prints_json_without_a_gpu(capsys):
    import json

    from ops.tune_matmul import main

    main(["--list-cases", "--rows", "64", "--operations", "dw"])
    listed = json.loads(capsys.readouterr().out)
    assert listed == cases(64, ["dw"])
    assert math.isfinite(listed[0]["k"])
