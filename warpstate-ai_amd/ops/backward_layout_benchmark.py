#!/usr/bin/env python3
"""Time the packed attention-backward gradient layout on one gfx950 GPU against its
two-kernel scratch baseline (the counterpart of ops/backward_layout_benchmark.py).

Every candidate ("paired", "single") is checked bit for bit against the "profile"
baseline, then timed in trials bracketed by baseline runs. The profile shape's inputs are
synthetic; no model, checkpoint or token file is opened.
"""

from __future__ import annotations

import argparse
import datetime as dt
import hashlib
import json
import math
import os
from pathlib import Path
import statistics
import sys
import time

PACKAGE = Path(__file__).resolve().parents[1]
WORKSPACE = PACKAGE.parent
if str(PACKAGE) not in sys.path:
    sys.path.insert(0, str(PACKAGE))
_UTC = dt.timezone.utc
SECTIONS = ("q", "k", "v", "gate", "u")


def arguments(argv=None):
    """Options of ops/backward_layout_benchmark.py:22-49 (block/warps kept for the
    command line; on gfx950 they do not change the launch)."""
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--algorithms", nargs="+", choices=["paired", "single"],
                        default=["paired", "single"])
    parser.add_argument("--blocks", nargs="+", type=int, choices=[128, 256, 512, 1024],
                        default=[512])
    parser.add_argument("--warps", nargs="+", type=int, choices=[4, 8], default=[4])
    parser.add_argument("--trials", type=int, default=5)
    parser.add_argument("--repeats", type=int, default=40)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--burnin-seconds", type=float, default=0.5)
    parser.add_argument("--seed", type=int, default=817)
    parser.add_argument("--output-dir", type=Path, required=True)
    args = parser.parse_args(argv)
    for name in ("trials", "repeats", "warmup"):
        if getattr(args, name) < 1:
            parser.error(name + " must be positive")
    if not math.isfinite(args.burnin_seconds) or args.burnin_seconds < 0:
        parser.error("burnin-seconds must be finite and nonnegative")
    args.output_dir = args.output_dir.expanduser().resolve()
    work = PACKAGE / "work"
    if (not args.output_dir.is_relative_to(work) or args.output_dir == work
            or not args.output_dir.relative_to(work).parts[0].startswith("benchmark-")):
        parser.error("output-dir must be below warpstate-ai_amd/work/benchmark-*")
    for name in ("TMPDIR", "XDG_CACHE_HOME"):
        value = os.environ.get(name)
        if not value or not Path(value).resolve().is_relative_to(WORKSPACE):
            parser.error(name + " must be set to a directory inside the workspace")
    return args


def output_errors(actual, expected):
    """Per-section agreement, so one wrong derivative cannot hide behind the others
    (ops/backward_layout_benchmark.py:52-66). ``unequal`` compares values (+0 == -0);
    ``bitwise_unequal`` compares BF16 bit patterns."""
    import torch

    result = {}
    for name, value, wanted in zip(SECTIONS, actual.chunk(5, -1), expected.chunk(5, -1),
                                   strict=True):
        finite = bool(torch.isfinite(value).all())
        delta = value.float() - wanted.float()
        result[name] = {
            "finite": finite,
            "unequal": int((value != wanted).sum()),
            "bitwise_unequal": int((value.view(torch.int16) != wanted.view(torch.int16)).sum()),
            "relative_rms": (float(delta.norm() / wanted.float().norm().clamp_min(1e-30))
                             if finite else None),
            "max_abs": float(delta.abs().max()) if finite else None,
        }
    return result


def main(argv=None):
    args = arguments(argv)
    import torch

    from ops.backward_layout import PROFILE_SHAPE, make_inputs, prepare_layout, reference_layout

    if not torch.cuda.is_available():
        raise RuntimeError("A GPU is required")
    torch.cuda.set_device(0)
    inputs = make_inputs(PROFILE_SHAPE, device="cuda", seed=args.seed)
    b, n, h, c, d = PROFILE_SHAPE
    baseline_output = torch.empty((b, n * c, 5 * h * d), device="cuda", dtype=torch.bfloat16)
    candidate_output = torch.empty_like(baseline_output)
    scratch = tuple(torch.empty_like(inputs.q_memory) for _ in range(2))
    baseline = prepare_layout(inputs, "profile", output=baseline_output, scratch=scratch)
    baseline()
    baseline_errors = output_errors(baseline_output, reference_layout(inputs))
    if any(not v["finite"] or v["relative_rms"] > 0.002 for v in baseline_errors.values()):
        raise RuntimeError("Profile baseline disagrees with the independent tensor expression")
    args.output_dir.mkdir(parents=True, exist_ok=False)
    elements = inputs.q_memory.numel()
    sources = ["ops/backward_layout.py", "ops/backward_layout_benchmark.py", "csrc/layout.hip"]
    report = {
        "format": "warpstate-backward-layout-v1",
        "started_utc": dt.datetime.now(_UTC).isoformat(),
        "arguments": {k: str(v) if isinstance(v, Path) else v for k, v in vars(args).items()},
        "shape_b_n_h_c_d": PROFILE_SHAPE, "dtype": "bfloat16", "rope_dtype": "float32",
        "torch": torch.__version__, "hip": torch.version.hip,
        "device": torch.cuda.get_device_name(0),
        "source_sha256": {name: hashlib.sha256((PACKAGE / name).read_bytes()).hexdigest()
                          for name in sources},
        "baseline_reference_errors": baseline_errors,
        # 12 BF16 inputs read and 5 BF16 sections written per element, once each.
        "algorithmic_bytes_per_call": 34 * elements,
        "static_removed_scratch_store_and_read_bytes_per_call": elements * 2 * 4,
        "limitations": ["Isolated backward region, not a measured training speedup.",
                        "Preallocated outputs and scratch; event times include launch gaps.",
                        "Synthetic saved inputs are reused across calls."],
        "results": [],
    }

    def save():
        path = args.output_dir / "results.json"
        partial = path.with_suffix(".json.partial")
        partial.write_text(json.dumps(report, indent=2, allow_nan=False) + "\n")
        partial.replace(path)

    def elapsed_ms(operation):
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(args.repeats):
            operation()
        end.record()
        end.synchronize()
        return begin.elapsed_time(end) / args.repeats

    for algorithm in args.algorithms:
        for block in args.blocks:
            for warps in args.warps:
                row = {"algorithm": algorithm, "block": block, "warps": warps}
                try:
                    candidate = prepare_layout(inputs, algorithm, block=block, warps=warps,
                                               output=candidate_output)
                    candidate()
                    row["errors"] = output_errors(candidate_output, baseline_output)
                    row["bitwise_equal"] = all(v["bitwise_unequal"] == 0
                                               for v in row["errors"].values())
                    for _ in range(args.warmup):
                        baseline()
                        candidate()
                    torch.cuda.synchronize()
                    begin = time.monotonic()
                    while time.monotonic() - begin < args.burnin_seconds:
                        for _ in range(10):
                            baseline()
                            candidate()
                        torch.cuda.synchronize()
                    trials = [{"baseline_before_ms": elapsed_ms(baseline),
                               "candidate_ms": elapsed_ms(candidate),
                               "baseline_after_ms": elapsed_ms(baseline)}
                              for _ in range(args.trials)]
                    controls = [(t["baseline_before_ms"] + t["baseline_after_ms"]) / 2
                                for t in trials]
                    gains = [(ctl / t["candidate_ms"] - 1) * 100
                             for ctl, t in zip(controls, trials, strict=True)]
                    median_ms = statistics.median(t["candidate_ms"] for t in trials)
                    row.update(status="ok", trials=trials, median_candidate_ms=median_ms,
                               median_baseline_ms=statistics.median(controls),
                               median_gain_percent=statistics.median(gains),
                               minimum_gain_percent=min(gains),
                               candidate_gbs=34 * elements / (median_ms * 1e6))
                except Exception as error:  # recorded; the sweep continues
                    row.update(status="error", error=type(error).__name__ + ": " + str(error)[:4000])
                report["results"].append(row)
                save()
                print(json.dumps({k: v for k, v in row.items() if k not in ("errors", "trials")}),
                      flush=True)
    report["finished_utc"] = dt.datetime.now(_UTC).isoformat()
    save()
    if not any(row["status"] == "ok" for row in report["results"]):
        raise RuntimeError("No candidate completed")


if __name__ == "__main__":
    main()
