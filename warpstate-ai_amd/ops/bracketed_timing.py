"""Shared harness of the isolated-kernel screens (``tune_matmul``, ``backward_layout_benchmark``).

A screen compares candidates with a control on one GPU. Each trial times the control, the
candidate and the control again back to back, so that clock and thermal drift shows up as
a difference between the two control readings instead of as a gain. Times come from HIP
events on the current stream around ``repeats`` back-to-back calls. Results are written as
JSON through a temporary file and a rename, so an interrupted screen leaves the last
complete report.
"""

from __future__ import annotations

import json
import math
import os
from pathlib import Path
import statistics
import time
from typing import Callable

Operation = Callable[[], object]


def check_output_dir(parser, path: Path, work: Path, package_name: str) -> Path:
    """``path`` resolved; it must be a ``benchmark-*`` directory below ``work``."""
    path = path.expanduser().resolve()
    inside = path.is_relative_to(work) and path != work
    if not inside or not path.relative_to(work).parts[0].startswith("benchmark-"):
        parser.error(f"output-dir must be below {package_name}/work/benchmark-*")
    return path


def check_workspace_env(parser, names, workspace: Path) -> None:
    """Scratch and cache directories must be set and lie inside the workspace."""
    for name in names:
        value = os.environ.get(name)
        if not value or not Path(value).resolve().is_relative_to(workspace):
            parser.error(name + " must be set to a directory inside the workspace")


def check_finite(parser, args, names, *, positive: bool = False) -> None:
    for name in names:
        value = getattr(args, name)
        bad = not math.isfinite(value) or (value <= 0 if positive else value < 0)
        if bad:
            parser.error(name.replace("_", "-") + (" must be finite and positive" if positive
                                                   else " must be finite and nonnegative"))


class AtomicJson:
    """JSON files in one directory, each replaced whole on every save."""

    def __init__(self, directory: Path):
        self.directory = directory

    def save(self, name: str, value) -> None:
        final = self.directory / name
        partial = final.with_name(name + ".partial")
        partial.write_text(json.dumps(value, indent=2, allow_nan=False) + "\n")
        partial.replace(final)


class Bracket:
    """Event timing of a control and candidates on the calling thread's current stream."""

    def __init__(self, repeats: int, warmup: int, burnin_seconds: float):
        import torch

        self.torch = torch
        self.repeats, self.warmup, self.burnin = repeats, warmup, burnin_seconds

    def ms(self, operation: Operation) -> float:
        """Mean milliseconds per call over ``repeats`` back-to-back calls."""
        torch = self.torch
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(self.repeats):
            operation()
        end.record()
        end.synchronize()
        return begin.elapsed_time(end) / self.repeats

    def warm(self, *operations: Operation) -> None:
        """``warmup`` calls of each, then alternating calls for ``burnin`` seconds so that
        the clocks settle under this load."""
        for _ in range(self.warmup):
            for operation in operations:
                operation()
        self.torch.cuda.synchronize()
        started = time.monotonic()
        while time.monotonic() - started < self.burnin:
            for _ in range(10):
                for operation in operations:
                    operation()
            self.torch.cuda.synchronize()

    def trial(self, control: Operation, candidate: Operation, names=("before", "candidate",
                                                                     "after")) -> dict:
        before = self.ms(control)
        middle = self.ms(candidate)
        after = self.ms(control)
        return dict(zip(names, (before, middle, after)))


def bracket_summary(trials, before: str, candidate: str, after: str) -> dict:
    """Per-trial gain of the candidate over the mean of its two controls, and the worst
    control drift. Every timing must be finite and positive."""
    if not trials:
        raise ValueError("Paired GPU timings must be finite and positive")
    for trial in trials:
        for value in trial.values():
            if not (math.isfinite(value) and value > 0):
                raise ValueError("Paired GPU timings must be finite and positive")
    controls = [(t[before] + t[after]) / 2 for t in trials]
    gains = [c / t[candidate] - 1.0 for c, t in zip(controls, trials, strict=True)]
    return {"controls": controls, "gains": gains,
            "median_candidate": statistics.median(t[candidate] for t in trials),
            "median_control": statistics.median(controls),
            "drift": max(abs(t[after] - t[before]) / c
                         for c, t in zip(controls, trials, strict=True))}
