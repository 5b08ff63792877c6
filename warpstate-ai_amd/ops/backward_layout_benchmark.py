#!/usr/bin/env python3
"""Screen the packed attention-backward gradient layouts on one gfx950 GPU.

The options, the per-section error report (``output_errors``) and ``results.json`` follow
WarpState's ``ops/backward_layout_benchmark.py``. The two-pass ``profile`` layout is the
control: it is first checked against the independent tensor expression
(``reference_layout``), then every candidate (``paired``, ``single``) is compared with it
bit for bit and timed in control / candidate / control trials (``ops.bracketed_timing``).
The profile shape's inputs are synthetic; no model, checkpoint or token file is opened.
"""

from __future__ import annotations

import argparse
import datetime as dt
import hashlib
import json
from pathlib import Path
import statistics
import sys

PACKAGE = Path(__file__).resolve().parents[1]
WORKSPACE = PACKAGE.parent
if str(PACKAGE) not in sys.path:
    sys.path.insert(0, str(PACKAGE))

from ops.bracketed_timing import (AtomicJson, Bracket, bracket_summary,  # noqa: E402
                                  check_finite, check_output_dir, check_workspace_env)

_UTC = dt.timezone.utc
SECTIONS = ("q", "k", "v", "gate", "u")
# Algorithmic bytes per element of the profile shape: 12 BF16 inputs read and 5 BF16
# sections written, once each.
BYTES_PER_ELEMENT = 34


def arguments(argv=None):
    """Options of ops/backward_layout_benchmark.py:22-49. ``--blocks`` and ``--warps``
    are accepted for the same command lines and recorded; the gfx950 launch does not
    depend on them."""
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--algorithms", nargs="+", choices=["paired", "single"],
                   default=["paired", "single"])
    p.add_argument("--blocks", nargs="+", type=int, choices=[128, 256, 512, 1024], default=[512])
    p.add_argument("--warps", nargs="+", type=int, choices=[4, 8], default=[4])
    for name, default in (("trials", 5), ("repeats", 40), ("warmup", 20), ("seed", 817)):
        p.add_argument("--" + name, type=int, default=default)
    p.add_argument("--burnin-seconds", type=float, default=0.5)
    p.add_argument("--output-dir", type=Path, required=True)
    args = p.parse_args(argv)
    for name in ("trials", "repeats", "warmup"):
        if getattr(args, name) < 1:
            p.error(name + " must be positive")
    check_finite(p, args, ("burnin_seconds",))
    args.output_dir = check_output_dir(p, args.output_dir, PACKAGE / "work", PACKAGE.name)
    check_workspace_env(p, ("TMPDIR", "XDG_CACHE_HOME"), WORKSPACE)
    return args


def output_errors(actual, expected):
    """Agreement of each of the five packed sections on its own (so one wrong derivative
    cannot hide behind the other four; ops/backward_layout_benchmark.py:52-66).
    ``unequal`` counts values that differ (+0 equals -0), ``bitwise_unequal`` BF16 bit
    patterns that differ."""
    import torch

    report = {}
    pieces = zip(SECTIONS, actual.chunk(5, -1), expected.chunk(5, -1))
    for name, value, wanted in pieces:
        finite = bool(torch.isfinite(value).all())
        error = value.float() - wanted.float()
        report[name] = {
            "finite": finite,
            "unequal": int((value != wanted).sum()),
            "bitwise_unequal": int((value.view(torch.int16) != wanted.view(torch.int16)).sum()),
            "relative_rms": (float(error.norm() / wanted.float().norm().clamp_min(1e-30))
                             if finite else None),
            "max_abs": float(error.abs().max()) if finite else None,
        }
    return report


def _checked_control(torch, inputs, shape):
    """The profile layout, after checking it against the tensor expression."""
    from ops.backward_layout import prepare_layout, reference_layout

    b, n, h, c, d = shape
    output = torch.empty((b, n * c, 5 * h * d), device="cuda", dtype=torch.bfloat16)
    scratch = tuple(torch.empty_like(inputs.q_memory) for _ in range(2))
    control = prepare_layout(inputs, "profile", output=output, scratch=scratch)
    control()
    errors = output_errors(output, reference_layout(inputs))
    if any(not e["finite"] or e["relative_rms"] > 0.002 for e in errors.values()):
        raise RuntimeError("Profile baseline disagrees with the independent tensor expression")
    return control, output, errors


def _screen(bracket, control, control_output, candidate, candidate_output, trials, elements):
    """One candidate: bitwise comparison, warm-up, bracketed trials and the summary."""
    candidate()
    row = {"errors": output_errors(candidate_output, control_output)}
    row["bitwise_equal"] = all(e["bitwise_unequal"] == 0 for e in row["errors"].values())
    bracket.warm(control, candidate)
    names = ("baseline_before_ms", "candidate_ms", "baseline_after_ms")
    row["trials"] = [bracket.trial(control, candidate, names) for _ in range(trials)]
    s = bracket_summary(row["trials"], *names)
    percent = [100 * g for g in s["gains"]]
    row.update(status="ok", median_candidate_ms=s["median_candidate"],
               median_baseline_ms=s["median_control"],
               median_gain_percent=statistics.median(percent),
               minimum_gain_percent=min(percent),
               candidate_gbs=BYTES_PER_ELEMENT * elements / (s["median_candidate"] * 1e6))
    return row


def main(argv=None):
    args = arguments(argv)
    import torch

    from ops.backward_layout import PROFILE_SHAPE, make_inputs, prepare_layout

    if not torch.cuda.is_available():
        raise RuntimeError("A GPU is required")
    torch.cuda.set_device(0)
    inputs = make_inputs(PROFILE_SHAPE, device="cuda", seed=args.seed)
    control, control_output, control_errors = _checked_control(torch, inputs, PROFILE_SHAPE)
    candidate_output = torch.empty_like(control_output)
    args.output_dir.mkdir(parents=True, exist_ok=False)
    files = AtomicJson(args.output_dir)
    elements = inputs.q_memory.numel()
    sources = ["ops/backward_layout.py", "ops/backward_layout_benchmark.py",
               "ops/bracketed_timing.py", "csrc/layout.hip"]
    report = {
        "format": "warpstate-backward-layout-v1",
        "started_utc": dt.datetime.now(_UTC).isoformat(),
        "arguments": {k: str(v) if isinstance(v, Path) else v for k, v in vars(args).items()},
        "shape_b_n_h_c_d": PROFILE_SHAPE, "dtype": "bfloat16", "rope_dtype": "float32",
        "torch": torch.__version__, "hip": torch.version.hip,
        "device": torch.cuda.get_device_name(0),
        "source_sha256": {n: hashlib.sha256((PACKAGE / n).read_bytes()).hexdigest()
                          for n in sources},
        "baseline_reference_errors": control_errors,
        "algorithmic_bytes_per_call": BYTES_PER_ELEMENT * elements,
        "static_removed_scratch_store_and_read_bytes_per_call": elements * 2 * 4,
        "limitations": ["Isolated backward region, not a measured training speedup.",
                        "Preallocated outputs and scratch; event times include launch gaps.",
                        "Synthetic saved inputs are reused across calls."],
        "results": [],
    }
    bracket = Bracket(args.repeats, args.warmup, args.burnin_seconds)
    for algorithm in args.algorithms:
        for block in args.blocks:
            for warps in args.warps:
                row = {"algorithm": algorithm, "block": block, "warps": warps}
                try:
                    candidate = prepare_layout(inputs, algorithm, block=block, warps=warps,
                                               output=candidate_output)
                    row.update(_screen(bracket, control, control_output, candidate,
                                       candidate_output, args.trials, elements))
                except Exception as error:  # recorded; the screen goes on
                    row.update(status="error", error=f"{type(error).__name__}: {str(error)[:4000]}")
                report["results"].append(row)
                files.save("results.json", report)
                print(json.dumps({k: v for k, v in row.items() if k not in ("errors", "trials")}),
                      flush=True)
    report["finished_utc"] = dt.datetime.now(_UTC).isoformat()
    files.save("results.json", report)
    if not any(row["status"] == "ok" for row in report["results"]):
        raise RuntimeError("No candidate completed")


if __name__ == "__main__":
    main()
