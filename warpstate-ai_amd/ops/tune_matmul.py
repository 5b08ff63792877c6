#!/usr/bin/env python3
"""Screen gfx950 BF16 FFN GEMM / paired-SwiGLU candidates against warmed ATen controls.

The command line, the case layouts, the metrics and the two output files
(``results.json``, ``candidate-policy.json``) are those of WarpState's
``ops/tune_matmul.py``, so that its plan-generation workflow runs unchanged: every
candidate trial is bracketed by ATen controls (``ops.bracketed_timing``), a candidate
qualifies only when its worst trial still gains ``--minimum-gain`` and every output it
returns matches the control within ``--maximum-relative-rms``, and each case's best
qualifying candidate becomes a ``warpstate-matmul-plan-v1`` entry. Winners are isolated
kernel results that need full-model validation before promotion. No model, checkpoint or
token file is opened.
"""

from __future__ import annotations

import argparse
import datetime as dt
import hashlib
import json
import math
from pathlib import Path
import statistics
import subprocess
import sys
import time

PACKAGE = Path(__file__).resolve().parents[1]
WORKSPACE = PACKAGE.parent
if str(PACKAGE) not in sys.path:
    sys.path.insert(0, str(PACKAGE))

from ops.bracketed_timing import (AtomicJson, Bracket, bracket_summary,  # noqa: E402
                                  check_finite, check_output_dir, check_workspace_env)

_UTC = dt.timezone.utc
# Scratch and cache directories a real screen keeps inside the workspace.
_SCRATCH_ENV = ("TMPDIR", "XDG_CACHE_HOME")
_OPERATIONS = {"mm": ("fwd", "dw"), "swiglu": ("fwd",)}
_ALGORITHMS = {"mm": ("tiled", "persistent", "persistent_tma"), "swiglu": ("tiled", "persistent")}
_PAIRED_BUDGET = 96 * 1024


def _parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--kind", choices=sorted(_OPERATIONS), default="mm")
    p.add_argument("--operations", nargs="+", choices=["fwd", "dw"])
    p.add_argument("--algorithms", nargs="+", choices=list(_ALGORITHMS["mm"]),
                   help="defaults to every algorithm the selected kind supports")
    p.add_argument("--tile", action="append", metavar="BM,BN,BK,WARPS,STAGES",
                   help="repeat to choose explicit tiles instead of the default sweep")
    for name, default in (("rows", 8192), ("ffn", 14336), ("width", 2048), ("repeats", 30),
                          ("trials", 3), ("warmup", 10), ("seed", 1337), ("device", 0)):
        p.add_argument("--" + name, type=int, default=default)
    for name, default in (("burnin-seconds", 1.0), ("minimum-gain", 0.01),
                          ("maximum-relative-rms", 0.003), ("input-scale", 1.0)):
        p.add_argument("--" + name, type=float, default=default)
    p.add_argument("--list-cases", action="store_true")
    p.add_argument("--output-dir", type=Path, default=None)
    return p


def _tiles(parser, kind: str, texts: list[str]) -> list[tuple]:
    from ops.matmul_kernels import normalize_tile

    try:
        tiles = [normalize_tile(tuple(int(v) for v in text.split(","))) for text in texts]
        if len(set(tiles)) != len(tiles):
            raise ValueError("tile must not contain duplicate selections; use --trials for repeats")
        if kind == "swiglu":
            for bm, bn, bk, _warps, stages in tiles:
                if (bm + 2 * bn) * bk * 2 * stages > _PAIRED_BUDGET:
                    raise ValueError("Paired SwiGLU pipeline exceeds the conservative 96 KiB budget")
    except ValueError as error:
        parser.error(str(error))
    return tiles


def arguments(argv=None):
    """Parse and validate the options (ops/tune_matmul.py:27-93); invalid choices exit
    through ``parser.error``."""
    parser = _parser()
    args = parser.parse_args(argv)
    kind = args.kind
    args.operations = list(args.operations or _OPERATIONS[kind])
    if not set(args.operations) <= set(_OPERATIONS[kind]):
        parser.error("swiglu supports only --operations fwd")
    args.algorithms = list(args.algorithms or _ALGORITHMS[kind])
    if not set(args.algorithms) <= set(_ALGORITHMS[kind]):
        parser.error("persistent_tma is implemented for mm only")
    for name in ("operations", "algorithms"):
        values = getattr(args, name)
        if len(set(values)) != len(values):
            parser.error(name + " must not contain duplicate selections")
    if args.tile:
        args.tile = _tiles(parser, kind, args.tile)
    for name in ("rows", "ffn", "width", "repeats", "trials", "warmup"):
        if getattr(args, name) < 1:
            parser.error(name + " must be positive")
    check_finite(parser, args, ("burnin_seconds", "minimum_gain", "maximum_relative_rms"))
    if args.device < 0:
        parser.error("device must be nonnegative")
    check_finite(parser, args, ("input_scale",), positive=True)
    work = PACKAGE / "work"
    if args.output_dir is None:
        stamp = dt.datetime.now(_UTC).strftime("%Y%m%dT%H%M%S")
        args.output_dir = work / ("benchmark-matmul-tiles-" + stamp)
    args.output_dir = check_output_dir(parser, args.output_dir, work, PACKAGE.name)
    if not args.list_cases:
        check_workspace_env(parser, _SCRATCH_ENV, WORKSPACE)
    return args


def cases(rows, operations, ffn=14336, width=2048):
    """GEMM layouts of the packed up/gate projection (ops/tune_matmul.py:96-105):
    ``fwd`` = X [rows, width] @ W^T with W [ffn, width] in nn.Linear layout;
    ``dw`` = dP^T [ffn, rows] @ X [rows, width]."""
    def layout(operation):
        if operation == "fwd":
            return {"m": rows, "n": ffn, "k": width, "a_transposed": False,
                    "b_transposed": True, "a_stride": [width, 1], "b_stride": [1, width]}
        return {"m": ffn, "n": width, "k": rows, "a_transposed": True,
                "b_transposed": False, "a_stride": [1, ffn], "b_stride": [width, 1]}

    return [{"operation": "ffn_up_gate." + op, **layout(op), "dtype": "bfloat16"}
            for op in operations]


def telemetry():
    """GPU clocks, power and temperature as reported by amd-smi (rocm-smi if absent)."""
    failure = {"error": "no telemetry tool ran"}
    for command in (["amd-smi", "metric", "--json"],
                    ["rocm-smi", "--showpower", "--showclocks", "--showtemp", "--json"]):
        try:
            done = subprocess.run(command, capture_output=True, text=True, timeout=10)
        except (OSError, subprocess.TimeoutExpired) as error:
            failure = {"error": f"{command[0]}: {error}"}
            continue
        return {"timestamp": time.time(), "tool": command[0], "returncode": done.returncode,
                "output": done.stdout.strip()[:20000]}
    return failure


def output_metrics(output, reference):
    """Max-abs and relative-RMS error of each returned BF16 tensor against the control's
    (ops/tune_matmul.py:119-140). Every output is checked, so one bad epilogue output
    cannot hide behind a good one; a wrong count, shape or dtype, or a non-finite value,
    is an error."""
    import torch

    got = output if isinstance(output, tuple) else (output,)
    want = reference if isinstance(reference, tuple) else (reference,)
    if len(got) != len(want):
        raise ValueError("Candidate and reference must return the same number of tensors")
    rows = []
    for value, expected in zip(got, want):
        if value.dtype != torch.bfloat16 or value.shape != expected.shape:
            raise ValueError("Candidate output must preserve the reference shape and BF16 dtype")
        error = value.float() - expected.float()
        scale = expected.float().square().mean().sqrt().clamp_min(1e-30)
        relative = (error.square().mean().sqrt() / scale).item()
        if not (math.isfinite(relative) and bool(torch.isfinite(value).all())):
            raise ValueError("Nonfinite candidate output or error metric")
        rows.append({"max_abs_error": error.abs().max().item(), "relative_rms_error": relative})
    return {"output_metrics": rows, "finite": True,
            "max_abs_error": max(r["max_abs_error"] for r in rows),
            "relative_rms_error": max(r["relative_rms_error"] for r in rows)}


def paired_timing_metrics(trials, minimum_gain):
    """Timing verdict of one candidate (ops/tune_matmul.py:143-157): the median gain over
    the bracketing controls, the worst trial's gain (which must reach ``minimum_gain``)
    and the largest control drift."""
    s = bracket_summary(trials, "aten_before_ms", "candidate_ms", "aten_after_ms")
    return {"median_ms": s["median_candidate"], "median_control_ms": s["median_control"],
            "paired_gain": statistics.median(s["gains"]), "minimum_trial_gain": min(s["gains"]),
            "timing_eligible": min(s["gains"]) >= minimum_gain,
            "maximum_control_drift_fraction": s["drift"]}


class _Screen:
    """One tuner run: the report, the policy being built and the timing harness."""

    def __init__(self, args, torch, device, sources):
        self.args, self.torch, self.device = args, torch, device
        self.files = AtomicJson(args.output_dir)
        self.bracket = Bracket(args.repeats, args.warmup, args.burnin_seconds)
        props = torch.cuda.get_device_properties(device)
        self.report = {
            "format": "warpstate-matmul-tuning-v1",
            "started_utc": dt.datetime.now(_UTC).isoformat(),
            "arguments": {k: str(v) if isinstance(v, Path) else v for k, v in vars(args).items()},
            "torch_version": torch.__version__, "hip_version": torch.version.hip,
            "device": {"name": props.name, "arch": getattr(props, "gcnArchName", ""),
                       "compute_units": props.multi_processor_count},
            "input_dtype": "bfloat16", "output_dtype": "bfloat16",
            "accumulation_dtype": "float32",
            "source_sha256": {n: hashlib.sha256((PACKAGE / n).read_bytes()).hexdigest()
                              for n in sources},
            "control": "torch.mm" if args.kind == "mm" else "torch.mm + eager SwiGLU",
            "output_names": (["matrix"] if args.kind == "mm"
                             else ["packed_projection", "activation"]),
            "results": [],
            "limitations": [
                "Isolated kernels, not measured training speedups.",
                "Inputs are reused; timing includes output allocation and launch.",
                "Every candidate trial has a preceding and following warmed ATen control.",
                "Correctness compares BF16 outputs with the control, not exact arithmetic.",
                "On gfx950 a tile request selects the 256x256 or 128x128 macro-tile."],
        }
        self.policy = {"format": "warpstate-matmul-plan-v1",
                       "description": "Isolated gfx950 BF16 winners; require full-model "
                                      "validation before promotion. Unmatched shapes retain "
                                      "ATen.",
                       "entries": []}

    def save(self):
        self.files.save("results.json", self.report)
        self.files.save("candidate-policy.json", self.policy)

    def operands(self, case, seed):
        torch, args = self.torch, self.args
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def draw(rows, cols, transposed):
            value = torch.randn((cols, rows) if transposed else (rows, cols),
                                device=self.device, dtype=torch.bfloat16, generator=gen)
            if args.input_scale != 1.0:
                value.mul_(args.input_scale)
            return value.T if transposed else value

        return (draw(case["m"], case["k"], case["a_transposed"]),
                draw(case["k"], case["n"], case["b_transposed"]))

    def launchers(self, a, b):
        """(control, candidate factory) for this kind."""
        if self.args.kind == "mm":
            from ops.matmul_kernels import launch_mm

            return (lambda: launch_mm(a, b, "aten"),
                    lambda algorithm, tile: (lambda: launch_mm(a, b, algorithm, tile)))
        from ops.matmul_epilogue import launch_swiglu_mm

        return (lambda: launch_swiglu_mm(a, b, "aten", eager_rounding=False),
                lambda algorithm, tile: (
                    lambda: launch_swiglu_mm(a, b, algorithm, tile, eager_rounding=False)))

    def measure(self, row, control, candidate, reference):
        torch, args = self.torch, self.args
        started = time.monotonic()
        output = candidate()
        torch.cuda.synchronize(self.device)
        row["first_call_seconds"] = time.monotonic() - started
        row.update(output_metrics(output, reference))
        del output
        self.bracket.warm(control)
        self.bracket.warm(candidate)
        row["telemetry_before"] = telemetry()
        names = ("aten_before_ms", "candidate_ms", "aten_after_ms")
        row["trials"] = [self.bracket.trial(control, candidate, names)
                         for _ in range(args.trials)]
        row["telemetry_after"] = telemetry()
        row.update(paired_timing_metrics(row["trials"], args.minimum_gain))
        case = row["case"]
        row["tflops"] = 2 * case["m"] * case["n"] * case["k"] / (row["median_ms"] * 1e9)
        row["status"] = "ok"
        row["eligible"] = (row["relative_rms_error"] <= args.maximum_relative_rms
                           and row["timing_eligible"])

    def run_case(self, index, case, tiles):
        from ops.matmul_kernels import matrix_signature, policy_key, tile_dict

        a, b = self.operands(case, self.args.seed + index)
        control, make = self.launchers(a, b)
        reference = control()
        winner = None
        for tile in tiles:
            for algorithm in self.args.algorithms:
                row = {"case": case, "signature": matrix_signature(a, b),
                       "key": policy_key(a, b), "algorithm": algorithm,
                       "tile": tile_dict(tile), "status": "running"}
                print(json.dumps({"operation": case["operation"], "algorithm": algorithm,
                                  "tile": tile, "status": "starting"}), flush=True)
                try:
                    self.measure(row, control, make(algorithm, tile), reference)
                except Exception as error:  # recorded; the screen goes on
                    row["status"] = "error"
                    row["error"] = f"{type(error).__name__}: {str(error)[:4000]}"
                self.report["results"].append(row)
                self.save()
                print(json.dumps({k: row[k] for k in ("algorithm", "tile", "status",
                                                      "median_ms", "paired_gain",
                                                      "relative_rms_error", "error")
                                  if k in row}), flush=True)
                if row.get("eligible") and (winner is None
                                            or row["paired_gain"] > winner["paired_gain"]):
                    winner = row
        if winner is not None:
            self.policy["entries"].append({"kind": self.args.kind, "name": case["operation"],
                                           **winner["signature"],
                                           "algorithm": winner["algorithm"],
                                           "tile": winner["tile"]})
        self.save()


def main(argv=None):
    args = arguments(argv)
    selected = cases(args.rows, args.operations, args.ffn, args.width)
    if args.list_cases:
        print(json.dumps(selected, indent=2))
        return
    import torch

    from ops.matmul_kernels import TUNING_TILES

    sources = ["ops/tune_matmul.py", "ops/bracketed_timing.py", "ops/matmul_kernels.py",
               "csrc/gemm.h", "csrc/gemm_fast.h"]
    tiles = args.tile or list(TUNING_TILES)
    if args.kind == "swiglu":
        from ops.matmul_epilogue import SUPPORTED_TILES

        tiles = args.tile or list(SUPPORTED_TILES)
        sources.append("ops/matmul_epilogue.py")
    if not torch.cuda.is_available():
        raise RuntimeError("A GPU is required; --list-cases runs without one")
    torch.cuda.set_device(args.device)
    device = torch.device("cuda", args.device)
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"This tuning run targets gfx950 (MI355X), found {arch or 'unknown'}")
    args.output_dir.mkdir(parents=True, exist_ok=False)
    screen = _Screen(args, torch, device, sources)
    screen.save()
    with torch.inference_mode():
        for index, case in enumerate(selected):
            screen.run_case(index, case, tiles)
    screen.report["finished_utc"] = dt.datetime.now(_UTC).isoformat()
    screen.save()


if __name__ == "__main__":
    main()
