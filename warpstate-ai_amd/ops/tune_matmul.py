#!/usr/bin/env python3
"""Screen BF16 FFN GEMM / SwiGLU-epilogue candidates on gfx950 against warmed ATen controls.

The gfx950 counterpart of WarpState's ``ops/tune_matmul.py`` (same command line, case
shapes, metrics and output files). Every candidate trial is bracketed by an ATen control
run before and after it, and a candidate qualifies only if it wins in every trial and
matches the control within the relative-RMS bound. Winners go into a
``warpstate-matmul-plan-v1`` policy (``candidate-policy.json``) that
``ops.matmul_execution.load_matmul_plan`` accepts; like the reference's, these are
isolated-kernel results that need full-model validation before promotion. No model,
checkpoint or token file is opened.
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
import subprocess
import sys
import time

PACKAGE = Path(__file__).resolve().parents[1]
WORKSPACE = PACKAGE.parent
if str(PACKAGE) not in sys.path:
    sys.path.insert(0, str(PACKAGE))

_UTC = dt.timezone.utc
# Environment paths that must point inside the workspace for a real (non --list-cases)
# run, so that scratch and cache files stay with the results.
_WORKSPACE_ENV = ("TMPDIR", "XDG_CACHE_HOME")


def _default_output_dir() -> Path:
    stamp = dt.datetime.now(_UTC).strftime("%Y%m%dT%H%M%S")
    return PACKAGE / "work" / ("benchmark-matmul-tiles-" + stamp)


def arguments(argv=None):
    """Parse and validate the tuner's options (ops/tune_matmul.py:27-93)."""
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--kind", choices=["mm", "swiglu"], default="mm")
    parser.add_argument("--operations", nargs="+", choices=["fwd", "dw"])
    parser.add_argument("--algorithms", nargs="+", choices=["tiled", "persistent", "persistent_tma"],
                        help="defaults to every algorithm the selected kind supports")
    parser.add_argument("--tile", action="append", metavar="BM,BN,BK,WARPS,STAGES",
                        help="repeat to choose explicit tiles instead of the default sweep")
    parser.add_argument("--rows", type=int, default=8192)
    parser.add_argument("--ffn", type=int, default=14336, help="packed up/gate width")
    parser.add_argument("--width", type=int, default=2048, help="model width (reduction dim)")
    parser.add_argument("--repeats", type=int, default=30)
    parser.add_argument("--trials", type=int, default=3)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--burnin-seconds", type=float, default=1.0)
    parser.add_argument("--minimum-gain", type=float, default=0.01)
    parser.add_argument("--maximum-relative-rms", type=float, default=0.003)
    parser.add_argument("--seed", type=int, default=1337)
    parser.add_argument("--input-scale", type=float, default=1.0,
                        help="multiply both BF16 random operands by this positive scalar")
    parser.add_argument("--device", type=int, default=0)
    parser.add_argument("--list-cases", action="store_true")
    parser.add_argument("--output-dir", type=Path, default=None)
    args = parser.parse_args(argv)

    kinds_ops = {"mm": ["fwd", "dw"], "swiglu": ["fwd"]}
    if args.operations is None:
        args.operations = list(kinds_ops[args.kind])
    if set(args.operations) - set(kinds_ops[args.kind]):
        parser.error("swiglu supports only --operations fwd")
    if args.algorithms is None:
        args.algorithms = ["tiled", "persistent"] + (["persistent_tma"] if args.kind == "mm" else [])
    if args.kind == "swiglu" and "persistent_tma" in args.algorithms:
        parser.error("persistent_tma is implemented for mm only")
    for key in ("operations", "algorithms"):
        values = getattr(args, key)
        if len(values) != len(set(values)):
            parser.error(key + " must not contain duplicate selections")
    if args.tile:
        from ops.matmul_kernels import normalize_tile
        try:
            tiles = [normalize_tile(tuple(int(v) for v in tile.split(","))) for tile in args.tile]
            if len(tiles) != len(set(tiles)):
                raise ValueError("tile must not contain duplicate selections; use --trials for repeats")
            if args.kind == "swiglu" and any((bm + 2 * bn) * bk * 2 * stages > 96 * 1024
                                             for bm, bn, bk, _w, stages in tiles):
                raise ValueError("Paired SwiGLU pipeline exceeds the conservative 96 KiB budget")
        except ValueError as error:
            parser.error(str(error))
        args.tile = tiles
    for key in ("rows", "ffn", "width", "repeats", "trials", "warmup"):
        if getattr(args, key) < 1:
            parser.error(key + " must be positive")
    for key in ("burnin_seconds", "minimum_gain", "maximum_relative_rms"):
        value = getattr(args, key)
        if not math.isfinite(value) or value < 0:
            parser.error(key + " must be finite and nonnegative")
    if args.device < 0:
        parser.error("device must be nonnegative")
    if not math.isfinite(args.input_scale) or args.input_scale <= 0:
        parser.error("input-scale must be finite and positive")
    work = PACKAGE / "work"
    args.output_dir = (args.output_dir or _default_output_dir()).expanduser().resolve()
    inside = args.output_dir.is_relative_to(work) and args.output_dir != work
    if not inside or not args.output_dir.relative_to(work).parts[0].startswith("benchmark-"):
        parser.error("output-dir must be below warpstate-ai_amd/work/benchmark-*")
    if not args.list_cases:
        for key in _WORKSPACE_ENV:
            value = os.environ.get(key)
            if not value or not Path(value).resolve().is_relative_to(WORKSPACE):
                parser.error(key + " must be set to a directory inside the workspace")
    return args


def cases(rows, operations, ffn=14336, width=2048):
    """The up/gate projection's forward and weight-gradient GEMM layouts
    (ops/tune_matmul.py:96-105): fwd = X [rows, width] @ W^T, W [ffn, width] nn.Linear;
    dw = dP^T [ffn, rows] @ X [rows, width]."""
    layouts = {"fwd": (rows, ffn, width, False, True), "dw": (ffn, width, rows, True, False)}
    result = []
    for operation in operations:
        m, n, k, a_t, b_t = layouts[operation]
        result.append({"operation": "ffn_up_gate." + operation, "m": m, "n": n, "k": k,
                       "a_transposed": a_t, "b_transposed": b_t,
                       "a_stride": [1, m] if a_t else [k, 1],
                       "b_stride": [1, k] if b_t else [n, 1], "dtype": "bfloat16"})
    return result


def telemetry():
    """Clocks, power and temperature of the GPUs from amd-smi (rocm-smi as a fallback)."""
    for command in (["amd-smi", "metric", "--json"],
                    ["rocm-smi", "--showpower", "--showclocks", "--showtemp", "--json"]):
        try:
            result = subprocess.run(command, capture_output=True, text=True, timeout=10)
        except (OSError, subprocess.TimeoutExpired) as error:
            last = {"error": f"{command[0]}: {error}"}
            continue
        return {"timestamp": time.time(), "tool": command[0], "returncode": result.returncode,
                "output": result.stdout.strip()[:20000]}
    return last


def output_metrics(output, reference):
    """Max-abs and relative-RMS error of every returned BF16 tensor against the control;
    any non-BF16, misshapen or non-finite output is an error (ops/tune_matmul.py:119-140)."""
    import torch

    outputs = output if isinstance(output, tuple) else (output,)
    references = reference if isinstance(reference, tuple) else (reference,)
    if len(outputs) != len(references):
        raise ValueError("Candidate and reference must return the same number of tensors")
    per_output = []
    for got, want in zip(outputs, references, strict=True):
        if got.shape != want.shape or got.dtype != torch.bfloat16:
            raise ValueError("Candidate output must preserve the reference shape and BF16 dtype")
        delta = got.float() - want.float()
        rms = delta.square().mean().sqrt() / want.float().square().mean().sqrt().clamp_min(1e-30)
        relative = rms.item()
        if not bool(torch.isfinite(got).all()) or not math.isfinite(relative):
            raise ValueError("Nonfinite candidate output or error metric")
        per_output.append({"max_abs_error": delta.abs().max().item(), "relative_rms_error": relative})
    return {"output_metrics": per_output, "finite": True,
            "max_abs_error": max(m["max_abs_error"] for m in per_output),
            "relative_rms_error": max(m["relative_rms_error"] for m in per_output)}


def paired_timing_metrics(trials, minimum_gain):
    """Each trial's gain over the mean of its two adjacent controls; a candidate is
    timing-eligible only if its worst trial gains at least ``minimum_gain``
    (ops/tune_matmul.py:143-157)."""
    values = [v for trial in trials for v in trial.values()]
    if not trials or any(not math.isfinite(v) or v <= 0 for v in values):
        raise ValueError("Paired GPU timings must be finite and positive")
    controls = [0.5 * (t["aten_before_ms"] + t["aten_after_ms"]) for t in trials]
    gains = [c / t["candidate_ms"] - 1.0 for c, t in zip(controls, trials, strict=True)]
    drift = [abs(t["aten_after_ms"] - t["aten_before_ms"]) / c
             for c, t in zip(controls, trials, strict=True)]
    return {"median_ms": statistics.median(t["candidate_ms"] for t in trials),
            "median_control_ms": statistics.median(controls),
            "paired_gain": statistics.median(gains), "minimum_trial_gain": min(gains),
            "timing_eligible": min(gains) >= minimum_gain,
            "maximum_control_drift_fraction": max(drift)}


def main(argv=None):
    args = arguments(argv)
    selected = cases(args.rows, args.operations, args.ffn, args.width)
    if args.list_cases:
        print(json.dumps(selected, indent=2))
        return
    import torch

    from ops.matmul_kernels import TUNING_TILES, launch_mm, matrix_signature, policy_key, tile_dict

    tiles = args.tile or list(TUNING_TILES)
    sources = ["ops/tune_matmul.py", "ops/matmul_kernels.py", "csrc/gemm.h", "csrc/gemm_fast.h"]
    if args.kind == "swiglu":
        from ops.matmul_epilogue import SUPPORTED_TILES, launch_swiglu_mm
        tiles = args.tile or list(SUPPORTED_TILES)
        sources.append("ops/matmul_epilogue.py")

    if not torch.cuda.is_available():
        raise RuntimeError("A GPU is required; --list-cases runs without one")
    torch.cuda.set_device(args.device)
    device = torch.device("cuda", args.device)
    properties = torch.cuda.get_device_properties(device)
    arch = getattr(properties, "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"This tuning run targets gfx950 (MI355X), found {arch or properties.name}")
    args.output_dir.mkdir(parents=True, exist_ok=False)
    report = {
        "format": "warpstate-matmul-tuning-v1", "started_utc": dt.datetime.now(_UTC).isoformat(),
        "arguments": {k: str(v) if isinstance(v, Path) else v for k, v in vars(args).items()},
        "torch_version": torch.__version__, "hip_version": torch.version.hip,
        "device": {"name": properties.name, "arch": arch,
                   "compute_units": properties.multi_processor_count},
        "input_dtype": "bfloat16", "output_dtype": "bfloat16", "accumulation_dtype": "float32",
        "source_sha256": {name: hashlib.sha256((PACKAGE / name).read_bytes()).hexdigest()
                          for name in sources},
        "control": "torch.mm" if args.kind == "mm" else "torch.mm + eager SwiGLU",
        "output_names": ["matrix"] if args.kind == "mm" else ["packed_projection", "activation"],
        "results": [],
        "limitations": ["Isolated kernels, not measured training speedups.",
                        "Inputs are reused; timing includes output allocation and launch.",
                        "Every candidate trial has a preceding and following warmed ATen control.",
                        "Correctness compares BF16 outputs with the control, not exact arithmetic.",
                        "On gfx950 a tile request selects the 256x256 or 128x128 macro-tile."],
    }
    policy = {"format": "warpstate-matmul-plan-v1",
              "description": "Isolated gfx950 BF16 winners; require full-model validation before "
                             "promotion. Unmatched shapes retain ATen.", "entries": []}

    def save():
        for name, value in (("results.json", report), ("candidate-policy.json", policy)):
            partial = args.output_dir / (name + ".partial")
            partial.write_text(json.dumps(value, indent=2, allow_nan=False) + "\n")
            partial.replace(args.output_dir / name)

    def elapsed_ms(operation):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.repeats):
            operation()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / args.repeats

    def warm(operation):
        for _ in range(args.warmup):
            operation()
        torch.cuda.synchronize(device)
        start = time.monotonic()
        while time.monotonic() - start < args.burnin_seconds:
            for _ in range(10):
                operation()
            torch.cuda.synchronize(device)

    save()
    with torch.inference_mode():
        for index, case in enumerate(selected):
            gen = torch.Generator(device=device).manual_seed(args.seed + index)

            def operand(rows, cols, transposed):
                shape = (cols, rows) if transposed else (rows, cols)
                value = torch.randn(shape, device=device, dtype=torch.bfloat16, generator=gen)
                if args.input_scale != 1.0:
                    value.mul_(args.input_scale)
                return value.T if transposed else value

            a = operand(case["m"], case["k"], case["a_transposed"])
            b = operand(case["k"], case["n"], case["b_transposed"])
            if args.kind == "mm":
                control = lambda: launch_mm(a, b, "aten")  # noqa: E731
            else:
                control = lambda: launch_swiglu_mm(a, b, "aten", eager_rounding=False)  # noqa: E731
            reference = control()
            eligible = []
            for tile in tiles:
                for algorithm in args.algorithms:
                    row = {"case": case, "signature": matrix_signature(a, b), "key": policy_key(a, b),
                           "algorithm": algorithm, "tile": tile_dict(tile), "status": "running"}
                    print(json.dumps({"operation": case["operation"], "algorithm": algorithm,
                                      "tile": tile, "status": "starting"}), flush=True)
                    if args.kind == "mm":
                        operation = (lambda t=tile, al=algorithm: launch_mm(a, b, al, t))
                    else:
                        operation = (lambda t=tile, al=algorithm:
                                     launch_swiglu_mm(a, b, al, t, eager_rounding=False))
                    try:
                        start = time.monotonic()
                        output = operation()
                        torch.cuda.synchronize(device)
                        row["first_call_seconds"] = time.monotonic() - start
                        row.update(output_metrics(output, reference))
                        del output
                        warm(control)
                        warm(operation)
                        row["telemetry_before"] = telemetry()
                        row["trials"] = [{"aten_before_ms": elapsed_ms(control),
                                          "candidate_ms": elapsed_ms(operation),
                                          "aten_after_ms": elapsed_ms(control)}
                                         for _ in range(args.trials)]
                        row["telemetry_after"] = telemetry()
                        row.update(paired_timing_metrics(row["trials"], args.minimum_gain))
                        row["tflops"] = 2 * case["m"] * case["n"] * case["k"] / (row["median_ms"] * 1e9)
                        row["status"] = "ok"
                        row["eligible"] = (row["relative_rms_error"] <= args.maximum_relative_rms
                                           and row["timing_eligible"])
                        if row["eligible"]:
                            eligible.append(row)
                    except Exception as error:  # recorded, the sweep continues
                        row["status"] = "error"
                        row["error"] = type(error).__name__ + ": " + str(error)[:4000]
                    report["results"].append(row)
                    save()
                    print(json.dumps({k: row[k] for k in ("algorithm", "tile", "status", "median_ms",
                                                          "paired_gain", "relative_rms_error",
                                                          "error") if k in row}), flush=True)
            if eligible:
                best = max(eligible, key=lambda r: r["paired_gain"])
                policy["entries"].append({"kind": args.kind, "name": case["operation"],
                                          **best["signature"], "algorithm": best["algorithm"],
                                          "tile": best["tile"]})
            save()
            del a, b, reference
    report["finished_utc"] = dt.datetime.now(_UTC).isoformat()
    save()


if __name__ == "__main__":
    main()
