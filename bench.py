"""Benchmark of the fused BF16 GEMM hot path on one MI355X.

One step is one pass of the hot path of a WarpState layer at training shape, M = 16384
tokens (batch 8 x seq 2048), d = 2048, ffn = 5632, on synthetic seeded inputs resident in
HBM:

  qkv_fwd      RMSNorm-prologue fused projection [16384,2048] x [2048,9216], sigmoid on
               the gate slice                                                 (config 2)
  swiglu_fwd   paired up/gate GEMM [16384,2048] x [2048,11264] with SwiGLU epilogue
  down_fwd     down projection [16384,5632] x [5632,2048] with residual add  (config 3)
  mlp_bwd      SwiGLU MLP backward: dH with fused SwiGLU backward, dX, and FP32-
               accumulated wgrad of W_down and W_upgate                      (config 4)
  qkv_bwd      backward of qkv_fwd: gradient through the gate sigmoid, dX of the
               projection [16384,9216] x [9216,2048], FP32-accumulated wgrad
               [9216,16384] x [16384,2048], RMSNorm backward

``value`` is the step's algorithmic FLOPs over its wall time (TFLOP/s). The other two
configurations are timed beside it and reported under ``per_config``: config 1 (SwiGLU
4096 x 1024 -> 2 x 2816) and config 5 (LM head with fused cross-entropy, 16384 x 2048 ->
32768: the one-pass fused loss, whose logits exist one 8192-row chunk at a time, and the
two-pass variant that keeps the logits only in registers and recomputes them). The
HBM-bound passes (the RMSNorm row pass, the RMSNorm backward, the LM-head combine and
logit-gradient passes, the attention-backward layout) are timed alone under
``hbm_parts``, each as back-to-back calls queued behind a spin kernel between one event
pair, so the short kernels' time carries no host launch gaps.

``roofline`` describes the dominant kernel of the step (the FP32-accumulating wgrad GEMM
of the MLP backward by default); its average launch time comes from HIP events around
each launch on the stream it runs on. ``cpu_baseline`` times the CPU oracle (the
reference's eager PyTorch path restated) on a row sample of the same step.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _path in (ROOT, ROOT / "warpstate-ai_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

import torch  # noqa: E402

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 4096 dense BF16 FLOP/clk/CU x 2.4 GHz
PEAK_HBM_GBS = 8000.0
METRIC = "fused-epilogue BF16 GEMM TFLOP/s + % MFMA peak, M=16384 SwiGLU/QKV fwd+bwd"

M, D, FFN, NQKV, VOCAB = 16384, 2048, 5632, 9216, 32768
GATE = (6144, 8192)


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--rows", type=int, default=M, help="tokens per step (default 16384)")
    p.add_argument("--cpu-rows", type=int, default=2048,
                   help="row sample of the CPU-baseline step")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="skip configs 1 and 5")
    return p.parse_args()


def flops_step(m):
    qkv = 2 * m * D * NQKV
    swiglu = 2 * m * D * 2 * FFN
    down = 2 * m * FFN * D
    mlp_bwd = 2 * m * D * FFN + 2 * m * 2 * FFN * D + 2 * D * FFN * m + 2 * 2 * FFN * D * m
    qkv_bwd = 2 * m * NQKV * D + 2 * NQKV * m * D
    return {"qkv_fwd": qkv, "swiglu_fwd": swiglu, "down_fwd": down, "mlp_bwd": mlp_bwd,
            "qkv_bwd": qkv_bwd}


class Timer:
    """HIP-event timing of named regions on the current stream."""

    def __init__(self):
        self.events = {}

    def region(self, name):
        timer = self

        class _Region:
            def __enter__(self):
                self.start = torch.cuda.Event(enable_timing=True)
                self.end = torch.cuda.Event(enable_timing=True)
                self.start.record()

            def __exit__(self, *exc):
                self.end.record()
                timer.events.setdefault(name, []).append((self.start, self.end))

        return _Region()

    def mean_ms(self, name):
        pairs = self.events.get(name, [])
        return sum(s.elapsed_time(e) for s, e in pairs) / max(1, len(pairs))

    def reset(self):
        self.events = {}


def queued_ms(fn, calls):
    """Mean ms per call of ``calls`` back-to-back calls of ``fn`` between one HIP-event pair
    on the current stream. A bounded spin kernel launched first keeps the GPU busy while the
    host queues the calls, so host launch overhead opens no gaps between short kernels and
    the figure is the kernels' own time (as a kernel trace reports it)."""
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(10_000_000)
    start.record()
    for _ in range(calls):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / calls


def gpu_inputs(m, device):
    from ops.benchmark_configs import (down_residual_inputs, mlp_backward_inputs,
                                       rms_projection_inputs)

    qkv = rms_projection_inputs(m=m, d=D, n=NQKV, gate=GATE, seed=0)
    down = down_residual_inputs(m=m, ffn=FFN, d=D, seed=0)
    mlp = mlp_backward_inputs(m=m, d=D, ffn=FFN, seed=0)
    dev = {}
    for prefix, group in (("qkv", qkv), ("down", down), ("mlp", mlp)):
        for key, value in group.items():
            dev[f"{prefix}_{key}"] = value.to(device) if torch.is_tensor(value) else value
    # Upstream gradient of the input projection (bf16 ~N(0, 1e-2)) and its FP32 wgrad buffer.
    gen = torch.Generator("cpu").manual_seed(1)
    dev["qkv_dp"] = (torch.randn((m, NQKV), generator=gen) * 1e-2).bfloat16().to(device)
    dev["qkv_g"] = (torch.randn((NQKV, D), generator=gen) * 1e-4).to(device)
    return dev


def run_step(inp, out, dp, timer=None):
    """One hot-path pass on the current stream: every kernel is this library's and
    launches through the C ABI.

    ``dp`` is this step's incoming gradient of the input projection's output. The QKV
    backward applies the gate-sigmoid backward to it in place (rmsnorm_gate_mm_backward
    with in_place=True: autograd hands the gradient over and frees it after this use), so
    every step gets its own fresh copy (``fresh_gradients``)."""
    from contextlib import nullcontext

    from ops.activation_execution import _rms_backward
    from ops.fused_execution import (dgrad_mm, mm_accumulate_, mm_accumulate_group_,
                                     residual_mm, rmsnorm_gate_mm, sigmoid_backward_cols,
                                     swiglu_backward_mm)
    from ops.matmul_epilogue import launch_swiglu_mm

    reg = timer.region if timer else (lambda name: nullcontext())
    with reg("qkv_fwd"):
        rmsnorm_gate_mm(inp["qkv_x"], inp["qkv_norm_weight"], inp["qkv_eps"], inp["qkv_w"],
                        GATE, out=out["qkv"], rstd=out["rstd"], normed=out["qkv_z"])
    with reg("swiglu_fwd"):
        packed, act = launch_swiglu_mm(inp["mlp_x"], inp["mlp_w_upgate"].T, "persistent",
                                       (128, 128, 32, 8, 3), True)
    with reg("down_fwd"):
        residual_mm(inp["down_h"], inp["down_w_down"], inp["down_residual"], out=out["down"])
    with reg("mlp_bwd"):
        with reg("mlp_bwd.dact_swiglu"):
            dpacked = swiglu_backward_mm(inp["mlp_dy"], inp["mlp_w_down"], packed, True,
                                         out=out["dpacked"])
        with reg("mlp_bwd.dx"):
            dgrad_mm(dpacked, inp["mlp_w_upgate"])
        with reg("mlp_bwd.wgrad"):
            # W_down's and W_upgate's gradients in one launch (both reduce over tokens).
            mm_accumulate_group_([(inp["mlp_g_down"], inp["mlp_dy"].T, act),
                                  (inp["mlp_g_upgate"], dpacked.T, inp["mlp_x"])], True)
    with reg("qkv_bwd"):
        # Backward of RMSNorm -> projection -> gate sigmoid (rmsnorm_gate_mm_backward with
        # in_place=True): the incoming gradient of the projection output has no other
        # consumer, so the sigmoid backward rewrites its gate columns in place.
        dp = sigmoid_backward_cols(dp, out["qkv"], GATE, dp)
        with reg("qkv_bwd.dx"):
            dy = dgrad_mm(dp, inp["qkv_w"])
        with reg("qkv_bwd.wgrad"):
            mm_accumulate_(inp["qkv_g"], dp.T, out["qkv_z"], True)
        _rms_backward(inp["qkv_x"], inp["qkv_norm_weight"], out["rstd"], dy, True)


def fresh_gradients(inp, count):
    """``count`` copies of the pristine incoming gradient, made before a timed loop so
    that each step's in-place sigmoid backward starts from the same values."""
    return [inp["qkv_dp"].clone() for _ in range(count)]


def bench_gpu(args):
    device = torch.device("cuda:0")
    m = args.rows
    inp = gpu_inputs(m, device)
    out = {"qkv": torch.empty((m, NQKV), dtype=torch.bfloat16, device=device),
           "rstd": torch.empty((m,), dtype=torch.float32, device=device),
           "down": torch.empty((m, D), dtype=torch.bfloat16, device=device),
           "dpacked": torch.empty((m, 2 * FFN), dtype=torch.bfloat16, device=device),
           # The normalized input the forward saves for the wgrad of the input projection.
           "qkv_z": torch.empty((m, D), dtype=torch.bfloat16, device=device)}
    for dp in fresh_gradients(inp, args.warmup):
        run_step(inp, out, dp)
    grads = fresh_gradients(inp, args.steps)
    torch.cuda.synchronize()
    # Timed region: exactly `steps` steps, synchronised on both sides.
    t0 = time.perf_counter()
    for dp in grads:
        run_step(inp, out, dp)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # Per-region HIP-event times over separate steps (not part of the timed region).
    timer = Timer()
    grads = fresh_gradients(inp, args.steps)
    for dp in grads:
        run_step(inp, out, dp, timer)
    torch.cuda.synchronize()
    del grads
    flops = flops_step(m)
    regions = {}
    for name, f in flops.items():
        ms = timer.mean_ms(name)
        regions[name] = {"ms": round(ms, 4), "tflops": round(f / ms / 1e9, 1),
                         "pct_peak": round(100 * f / ms / 1e9 / PEAK_BF16_TFLOPS, 2)}
    sub = {"mlp_bwd.dact_swiglu": 2 * m * D * FFN, "mlp_bwd.dx": 2 * m * 2 * FFN * D,
           "mlp_bwd.wgrad": 2 * D * FFN * m + 2 * 2 * FFN * D * m,
           "qkv_bwd.dx": 2 * m * NQKV * D, "qkv_bwd.wgrad": 2 * NQKV * m * D}
    kernels = {}
    for name, f in sub.items():
        ms = timer.mean_ms(name)
        kernels[name] = {"ms": round(ms, 4), "tflops": round(f / ms / 1e9, 1),
                         "pct_peak": round(100 * f / ms / 1e9 / PEAK_BF16_TFLOPS, 2),
                         "flops": f}
    # hipBLASLt (torch.mm) as a yardstick, outside the step, timed the same way:
    # - on the two input-gradient products, after the same weight transpose (the same
    #   work as this library's kernels there);
    # - on the plain product of every other GEMM region, the operands as the step holds
    #   them, without the work this library fuses into it (RMSNorm row pass and gate
    #   sigmoid, SwiGLU, residual add, SwiGLU backward, the FP32 accumulation of the weight
    #   gradients: hipBLASLt writes BF16 instead).
    from ops.fused_execution import k_contiguous_b
    from ops.matmul_epilogue import launch_swiglu_mm

    packed, act = launch_swiglu_mm(inp["mlp_x"], inp["mlp_w_upgate"].T, "persistent",
                                   (128, 128, 32, 8, 3), True)
    products = {
        "qkv_fwd": lambda: torch.mm(out["qkv_z"], inp["qkv_w"].T),
        "swiglu_fwd": lambda: torch.mm(inp["mlp_x"], inp["mlp_w_upgate"].T),
        "down_fwd": lambda: torch.mm(inp["down_h"], inp["down_w_down"].T),
        "mlp_bwd.dact_swiglu": lambda: torch.mm(inp["mlp_dy"], inp["mlp_w_down"]),
        "mlp_bwd.dx": lambda: torch.mm(out["dpacked"], k_contiguous_b(inp["mlp_w_upgate"], m)),
        "mlp_bwd.wgrad": lambda: (torch.mm(inp["mlp_dy"].T, act),
                                  torch.mm(out["dpacked"].T, inp["mlp_x"])),
        "qkv_bwd.dx": lambda: torch.mm(inp["qkv_dp"], k_contiguous_b(inp["qkv_w"], m)),
        "qkv_bwd.wgrad": lambda: torch.mm(inp["qkv_dp"].T, out["qkv_z"]),
    }
    vendor = Timer()
    for _ in range(max(2, args.warmup)):  # hipBLASLt picks its kernel on a shape's first call
        for fn in products.values():
            fn()
    for _ in range(args.steps):
        for name, fn in products.items():
            with vendor.region(name):
                fn()
    torch.cuda.synchronize()
    plain = {"qkv_fwd": 2 * m * NQKV * D, "swiglu_fwd": 2 * m * 2 * FFN * D,
             "down_fwd": 2 * m * D * FFN, **sub}
    for name in products:
        ms, f = vendor.mean_ms(name), plain[name]
        kernels[name + ".hipblaslt"] = {"ms": round(ms, 4), "tflops": round(f / ms / 1e9, 1),
                                        "pct_peak": round(100 * f / ms / 1e9 / PEAK_BF16_TFLOPS, 2),
                                        "flops": f}
    # The training adapter's MLP backward operator on the same tensors: the same kernels
    # as mlp_bwd, with the two weight gradients written into fresh FP32 buffers (returned
    # through autograd) instead of accumulated into resident ones.
    from ops.fused_training import fused_swiglu_block_backward

    adapter = Timer()
    for i in range(args.warmup + args.steps):
        with adapter.region("run" if i >= args.warmup else "warm"):
            fused_swiglu_block_backward(inp["mlp_dy"], inp["mlp_x"], packed, act,
                                        inp["mlp_w_upgate"], inp["mlp_w_down"])
    torch.cuda.synchronize()
    f = sub["mlp_bwd.dact_swiglu"] + sub["mlp_bwd.dx"] + sub["mlp_bwd.wgrad"]
    ms = adapter.mean_ms("run")
    kernels["mlp_bwd.adapter_op"] = {"ms": round(ms, 4), "tflops": round(f / ms / 1e9, 1),
                                     "pct_peak": round(100 * f / ms / 1e9 / PEAK_BF16_TFLOPS, 2),
                                     "flops": f}
    del packed, act
    # The RMSNorm row pass of qkv_fwd (HBM-bound): x read once, the normalized rows y and
    # rstd written. The eager standalone forward launches the same kernel
    # (rmsnorm_rows_reg_kernel) as rmsnorm_gate_mm's row pass.
    from ops.activation_execution import bf16_rmsnorm

    rows_ms = queued_ms(lambda: bf16_rmsnorm(inp["qkv_x"], inp["qkv_norm_weight"],
                                             float(inp["qkv_eps"]), True), args.steps)
    rows_bytes = 2 * m * D * 2 + m * 4 + D * 4
    hbm = {"rmsnorm_rows": {"ms": round(rows_ms, 4), "bytes": rows_bytes,
                            "gbs": round(rows_bytes / rows_ms / 1e6, 1),
                            "frac_hbm": round(rows_bytes / rows_ms / 1e6 / PEAK_HBM_GBS, 4),
                            "kernel": "rmsnorm_rows_reg_kernel<4, true> (qkv_fwd row pass)"}}
    # RMSNorm backward of the step (dX and the weight gradient, both launches): x and the
    # incoming gradient read, dX written, rstd read and the FP32 weight gradient written
    # once each (the per-block partials are not counted).
    from ops.activation_execution import _rms_backward

    bwd_ms = queued_ms(lambda: _rms_backward(inp["qkv_x"], inp["qkv_norm_weight"], out["rstd"],
                                             out["qkv_z"], True), args.steps)
    bwd_bytes = 3 * m * D * 2 + m * 4 + D * 4
    hbm["rmsnorm_backward"] = {"ms": round(bwd_ms, 4), "bytes": bwd_bytes,
                               "gbs": round(bwd_bytes / bwd_ms / 1e6, 1),
                               "frac_hbm": round(bwd_bytes / bwd_ms / 1e6 / PEAK_HBM_GBS, 4)}
    return wall_ms, sum(flops.values()), regions, kernels, hbm, inp, out


def bench_layout(args, device):
    """Packed attention-backward gradient layout at the reference's profile shape
    (4, 16, 32, 128, 64): HBM-bound, 12 BF16 inputs read and 5 BF16 sections written per
    element. "single" is the product path; "profile" is the two-pass scratch baseline."""
    from ops.backward_layout import PROFILE_SHAPE, make_inputs, prepare_layout

    inputs = make_inputs(PROFILE_SHAPE, device=device, seed=817)
    b, n, h, c, d = PROFILE_SHAPE
    out = torch.empty((b, n * c, 5 * h * d), dtype=torch.bfloat16, device=device)
    ops = {"single": prepare_layout(inputs, "single", output=out),
           "profile": prepare_layout(inputs, "profile", output=out)}
    times = {}
    for name, operation in ops.items():
        for _ in range(args.warmup):
            operation()
        times[name] = queued_ms(operation, args.steps)
    nbytes = 34 * inputs.q_memory.numel()
    ms = times["single"]
    return {"ms": round(ms, 4), "bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
            "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
            "profile_baseline_ms": round(times["profile"], 4)}


def bench_extra(args, device):
    """Configs 1 and 5, and configs 1-3 with weights stored [K, N], each timed over `steps`
    launches with HIP events."""
    from ops.benchmark_configs import lm_head_inputs, swiglu_forward_inputs
    from ops.fused_execution import (CrossEntropyState, linear_cross_entropy_backward,
                                     linear_cross_entropy_forward)
    from ops.matmul_epilogue import launch_swiglu_mm

    res = {}
    c1 = swiglu_forward_inputs(seed=0)
    x, w = c1["x"].to(device), c1["w_upgate"].to(device)
    for _ in range(args.warmup):
        launch_swiglu_mm(x, w.T, "persistent", (128, 128, 32, 8, 3), True)
    t = Timer()
    for _ in range(args.steps):
        with t.region("c1"):
            launch_swiglu_mm(x, w.T, "persistent", (128, 128, 32, 8, 3), True)
    torch.cuda.synchronize()
    f1 = 2 * 4096 * 1024 * 5632
    ms = t.mean_ms("c1")
    res["config1_swiglu_4096x1024x5632"] = {"ms": round(ms, 4), "tflops": round(f1 / ms / 1e9, 1),
                                            "pct_peak": round(100 * f1 / ms / 1e9 / PEAK_BF16_TFLOPS, 2)}
    # Configs 1-3 with the weight stored [K, N] row-major, the reference's second measured
    # layout (an N-contiguous B; the launchers copy it K-contiguous first). Configs 2 and 3
    # in the native layout are the step's qkv_fwd and down_fwd regions.
    from ops.benchmark_configs import down_residual_inputs, rms_projection_inputs
    from ops.fused_execution import residual_mm, rmsnorm_gate_mm

    w_kn = w.T.contiguous()
    c2 = rms_projection_inputs(seed=0)
    x2, nw2, w2_kn = c2["x"].to(device), c2["norm_weight"].to(device), c2["w"].to(device).T.contiguous()
    c3 = down_residual_inputs(seed=0)
    h3, r3, w3_kn = c3["h"].to(device), c3["residual"].to(device), c3["w_down"].to(device).T.contiguous()
    o2 = torch.empty((M, NQKV), dtype=torch.bfloat16, device=device)
    rs2 = torch.empty((M,), dtype=torch.float32, device=device)
    z2 = torch.empty((M, D), dtype=torch.bfloat16, device=device)
    o3 = torch.empty((M, D), dtype=torch.bfloat16, device=device)
    w2, w3 = c2["w"].to(device), c3["w_down"].to(device)
    kn = {  # (FLOPs, native-layout call, [K, N]-layout call), alternated call by call
        "config1_swiglu_4096x1024x5632_kn_weight": (
            f1, lambda: launch_swiglu_mm(x, w.T, "persistent", (128, 128, 32, 8, 3), True),
            lambda: launch_swiglu_mm(x, w_kn, "persistent", (128, 128, 32, 8, 3), True)),
        "config2_rmsnorm_qkv_16384x2048x9216_kn_weight": (
            2 * M * NQKV * D,
            lambda: rmsnorm_gate_mm(x2, nw2, c2["eps"], w2, c2["gate"], out=o2, rstd=rs2,
                                    normed=z2),
            lambda: rmsnorm_gate_mm(x2, nw2, c2["eps"], w2_kn.T, c2["gate"], out=o2, rstd=rs2,
                                    normed=z2)),
        "config3_down_residual_16384x5632x2048_kn_weight": (
            2 * M * D * FFN, lambda: residual_mm(h3, w3, r3, out=o3),
            lambda: residual_mm(h3, w3_kn.T, r3, out=o3)),
    }
    for key, (f, native, stored_kn) in kn.items():
        for _ in range(args.warmup):
            native()
            stored_kn()
        t = Timer()
        for _ in range(args.steps):
            with t.region("native"):
                native()
            with t.region("kn"):
                stored_kn()
        torch.cuda.synchronize()
        ms, ms_native = t.mean_ms("kn"), t.mean_ms("native")
        res[key] = {"ms": round(ms, 4), "tflops": round(f / ms / 1e9, 1),
                    "pct_peak": round(100 * f / ms / 1e9 / PEAK_BF16_TFLOPS, 2),
                    "native_layout_ms": round(ms_native, 4),
                    "flops_note": "weight stored [K, N]; its K-contiguous copy is timed; the "
                                  "native [N, K] layout alternated with it call by call"}
    del x, w, w_kn, x2, nw2, w2, w2_kn, h3, r3, w3, w3_kn, o2, rs2, z2, o3
    c5 = lm_head_inputs(seed=0)
    hidden, weight, targets = (c5[k].to(device) for k in ("hidden", "weight", "targets"))
    dh = torch.empty((M, D), dtype=torch.bfloat16, device=device)
    one = torch.ones((), device=device)
    f5 = 4 * M * D * VOCAB
    # Config 5 is the one-pass fused loss: each 8192-row chunk's BF16 logits exist only in
    # the chunk workspace (512 MiB; the full [16384, 32768] logits never do), and the
    # chunk's dHidden is formed while they are there; the backward scales by the upstream
    # gradient. The two-pass variant (logits only in registers, recomputed by the
    # backward) is timed beside it. So is the one-pass loss under an upstream gradient that
    # is not a power of two (1/3, e.g. a loss averaged over three micro-batches): its
    # backward then falls back to the two-pass recompute, after the forward has already
    # formed the unit gradients.
    third = torch.full((), 1.0 / 3.0, device=device)
    fused_state = None
    for key, fused, g, note in (
            ("config5_lm_head_ce_16384x2048x32768", True, one,
             "logits fwd + dHidden, one pass (ws_linear_ce_fused) + upstream scale"),
            ("config5_two_pass_recompute_16384x2048x32768", False, one,
             "logits fwd + dHidden; the backward recomputes the logits GEMM (not counted)"),
            ("config5_one_pass_upstream_third_16384x2048x32768", True, third,
             "one-pass loss with upstream gradient 1/3: the backward falls back to the "
             "two-pass recompute (its extra GEMMs not counted)")):
        state = CrossEntropyState(M, VOCAB, device, d=D, fused=fused)
        for _ in range(args.warmup):
            linear_cross_entropy_forward(hidden, weight, targets, state)
            linear_cross_entropy_backward(hidden, weight, targets, state, g, out=dh)
        t = Timer()
        for _ in range(args.steps):
            with t.region("fwd"):
                linear_cross_entropy_forward(hidden, weight, targets, state)
            with t.region("bwd"):
                linear_cross_entropy_backward(hidden, weight, targets, state, g, out=dh)
        torch.cuda.synchronize()
        ms = t.mean_ms("fwd") + t.mean_ms("bwd")
        res[key] = {
            "ms": round(ms, 4), "fwd_ms": round(t.mean_ms("fwd"), 4),
            "bwd_ms": round(t.mean_ms("bwd"), 4), "tflops": round(f5 / ms / 1e9, 1),
            "pct_peak": round(100 * f5 / ms / 1e9 / PEAK_BF16_TFLOPS, 2), "flops_note": note}
        if fused and fused_state is None:
            fused_state = state
        else:
            del state
    res["_hbm"] = lm_head_hbm_parts(args, fused_state, targets, device)
    del fused_state
    return res


def lm_head_hbm_parts(args, state, targets, device):
    """The LM-head loss's HBM-bound passes at config 5, each timed alone (``queued_ms``):
    the row combine + mean (part_max / part_sum / target logit / targets read, lse and loss
    written, then loss and targets read again), and the elementwise logit-gradient pass over
    one 8192-row chunk, in place (BF16 logits read and gradients written)."""
    from ops import _hip

    parts = state.part_max.shape[1]
    stream = _hip.stream(targets)
    scale = torch.full((1,), 1.0 / M, device=device)
    chunk = torch.empty((8192, VOCAB), dtype=torch.bfloat16, device=device).normal_()

    def combine():
        _hip.call("ws_linear_ce_combine", state.part_max.data_ptr(), state.part_sum.data_ptr(),
                  state.target_logit.data_ptr(), targets.data_ptr(), state.lse.data_ptr(),
                  state.loss.data_ptr(), state.mean.data_ptr(), state.count.data_ptr(), M,
                  VOCAB, stream)

    def logit_grad():
        _hip.call("ws_linear_ce_logit_grad", chunk.data_ptr(), VOCAB, targets.data_ptr(),
                  state.lse.data_ptr(), scale.data_ptr(), chunk.data_ptr(), VOCAB, 8192, VOCAB,
                  stream)

    out = {}
    for name, fn, nbytes, kernels in (
            ("ce_combine_mean", combine, M * (2 * parts * 4 + 4 + 8 + 4 + 4) + M * (4 + 8),
             "ce_combine_kernel + ce_mean_kernel"),
            ("ce_logit_grad_chunk", logit_grad, 2 * 8192 * VOCAB * 2 + 8192 * (8 + 4),
             "ce_grad_logits_kernel, 8192 x 32768 in place")):
        for _ in range(args.warmup):
            fn()
        ms = queued_ms(fn, args.steps)
        out[name] = {"ms": round(ms, 4), "bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
                     "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
                     "kernel": kernels}
    del chunk
    return out


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (the platform string if absent)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _median_seconds(fn, min_runs=3, budget_s=4.0, max_runs=10):
    """Median wall time of ``fn`` over at least ``min_runs`` runs after one warmup, more
    while ``budget_s`` lasts."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s
                                    and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline(rows):
    """The CPU oracle (the reference's eager PyTorch path restated, BF16 CPU tensors) on
    the host's cores: the layer step on a ``rows``-token sample, and each of the five
    configurations, config 1 at its full size and configs 2-5 on a ``rows``-row sample of
    their 16384 rows (every GEMM row, and every loss row, depends only on its own input
    row, so throughput per row is the same). Returns (step TFLOP/s, step seconds, threads,
    per-config dict)."""
    from oracle import reference as oracle
    from ops import benchmark_configs as cfg

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    qkv = cfg.rms_projection_inputs(m=rows, d=D, n=NQKV, gate=GATE, seed=0)
    down = cfg.down_residual_inputs(m=rows, ffn=FFN, d=D, seed=0)
    mlp = cfg.mlp_backward_inputs(m=rows, d=D, ffn=FFN, seed=0)
    gen = torch.Generator("cpu").manual_seed(1)
    dp = (torch.randn((rows, NQKV), generator=gen) * 1e-2).bfloat16()
    g_qkv = torch.randn((NQKV, D), generator=gen) * 1e-4

    def step():
        oracle.rmsnorm_gate_projection(qkv["x"], qkv["norm_weight"], qkv["eps"], qkv["w"], GATE)
        packed, act = oracle.swiglu_mm(mlp["x"], mlp["w_upgate"].T, True)
        oracle.residual_projection(down["h"], down["w_down"], down["residual"])
        oracle.mlp_backward(mlp["x"], mlp["w_upgate"], mlp["w_down"], packed, act, mlp["dy"],
                            mlp["g_upgate"], mlp["g_down"])
        oracle.rmsnorm_gate_projection_backward(qkv["x"], qkv["norm_weight"], qkv["eps"],
                                                qkv["w"], GATE, dp, g_qkv)

    sec = _median_seconds(step, budget_s=10.0, max_runs=20)
    step_tflops = sum(flops_step(rows).values()) / sec / 1e12

    c1 = cfg.swiglu_forward_inputs(seed=0)
    packed, act = oracle.swiglu_mm(mlp["x"], mlp["w_upgate"].T, True)
    lm = cfg.lm_head_inputs(m=rows, seed=0)
    cases = {
        "config1_swiglu_4096x1024x5632": (
            4096, cfg.flops_swiglu_forward(4096, 1024, 2816),
            lambda: oracle.swiglu_mm(c1["x"], c1["w_upgate"].T, False)),
        "config2_rmsnorm_qkv_16384x2048x9216": (
            rows, cfg.flops_rms_projection(rows, D, NQKV),
            lambda: oracle.rmsnorm_gate_projection(qkv["x"], qkv["norm_weight"], qkv["eps"],
                                                   qkv["w"], GATE)),
        "config3_down_residual_16384x5632x2048": (
            rows, cfg.flops_down_residual(rows, FFN, D),
            lambda: oracle.residual_projection(down["h"], down["w_down"], down["residual"])),
        "config4_mlp_backward_16384x2048x5632": (
            rows, cfg.flops_mlp_backward(rows, D, FFN),
            lambda: oracle.mlp_backward(mlp["x"], mlp["w_upgate"], mlp["w_down"], packed, act,
                                        mlp["dy"], mlp["g_upgate"], mlp["g_down"])),
        "config5_lm_head_ce_16384x2048x32768": (
            rows, cfg.flops_lm_head(rows, D, VOCAB),
            lambda: oracle.linear_cross_entropy(lm["hidden"], lm["weight"], lm["targets"])),
    }
    per_config = {}
    for name, (sample_rows, flops, fn) in cases.items():
        t = _median_seconds(fn)
        per_config[name] = {"ms": round(t * 1e3, 2), "tflops": round(flops / t / 1e12, 4),
                            "rows": sample_rows,
                            "sample": "full size" if name.startswith("config1")
                            else f"{sample_rows} of 16384 rows"}
    return step_tflops, sec, torch.get_num_threads(), per_config


TRAFFIC_PROFILE = ROOT / "profiles" / "hbm_traffic_layer_step_m16384.md"


TRACE_PROFILE = ROOT / "profiles" / "gemm_kernels_layer_step_m16384.md"


def _profile_value(path: Path, tag: str, region: str):
    """The number recorded on a ``<tag> <region> <value>`` line of a committed profile
    summary, or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == tag and parts[1] == region:
            return float(parts[2])
    return None


def measured_traffic(region: str):
    """HBM bytes per launch of a bench region, measured with rocprofv3 FETCH_SIZE and
    WRITE_SIZE (scaled by a plain copy's readings) and recorded in the traffic profile;
    None when the region has no measurement there."""
    value = _profile_value(TRAFFIC_PROFILE, "traffic_bytes", region)
    return None if value is None else int(value)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the hot path shards over tokens; see the design notes). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda:0")
    wall_ms, step_flops, regions, kernels, hbm, inp, out = bench_gpu(args)
    del inp, out
    torch.cuda.empty_cache()
    per_config = {} if args.no_extra else bench_extra(args, device)
    if not args.no_extra:
        hbm.update(per_config.pop("_hbm"))
        hbm["attention_bwd_layout_4x16x32x128x64"] = bench_layout(args, device)
    value = step_flops / wall_ms / 1e9
    # The dominant kernel of the step (the hipBLASLt yardstick lines are not in the step).
    dom_name = max((k for k in kernels if not k.endswith((".hipblaslt", ".adapter_op"))),
                   key=lambda k: kernels[k]["ms"])
    dom = kernels[dom_name]
    roofline = {"bound": "mfma", "kernel": dom_name,
                "achieved": round(dom["flops"] / dom["ms"] / 1e9, 1),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(dom["flops"] / dom["ms"] / 1e9 / PEAK_BF16_TFLOPS, 4),
                "frac_source": "HIP events around each launch of the region in this run",
                "traffic": measured_traffic(dom_name),
                "traffic_source": f"profiles/{TRAFFIC_PROFILE.name} (rocprofv3 FETCH_SIZE + "
                                  "WRITE_SIZE, committed; not measured in this run)"}
    # The same region's kernels in the committed rocprofv3 trace (sum of their average
    # durations), for comparison with the HIP-event figure above.
    trace_us = _profile_value(TRACE_PROFILE, "trace_us", dom_name)
    if trace_us:
        roofline["trace_source"] = (f"profiles/{TRACE_PROFILE.name} (rocprofv3 kernel trace, "
                                    "committed; not measured in this run)")
        roofline["trace_us"] = trace_us
        roofline["trace_achieved"] = round(dom["flops"] / trace_us / 1e6, 1)
        roofline["trace_frac"] = round(dom["flops"] / trace_us / 1e6 / PEAK_BF16_TFLOPS, 4)
    cpu = None
    if not args.no_cpu:
        tflops, sec, threads, per_config_cpu = cpu_baseline(args.cpu_rows)
        cpu = {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": threads,
               "kind": "port",
               "sample": f"the same step at M={args.cpu_rows} tokens (of {args.rows}), "
                         f"median of >=3 runs, {sec:.2f} s/step; per_config: each "
                         f"configuration's oracle path, config 1 in full, configs 2-5 on "
                         f"{args.cpu_rows} of their 16384 rows",
               "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
               "torch_threads": threads, "per_config": per_config_cpu}
    line = {"metric": METRIC, "value": round(value, 1), "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,s) inputs, random-init weights)",
            "config": {"workload": "WarpState layer hot path fwd+bwd: RMSNorm-QKV/gate "
                                   "projection, SwiGLU up/gate, down+residual, MLP backward, "
                                   "QKV backward",
                       "tokens": args.rows, "d_model": D, "ffn_hidden": FFN,
                       "qkv_width": NQKV, "step_gflop": round(step_flops / 1e9, 1)},
            "pct_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
            "roofline": roofline, "cpu_baseline": cpu, "regions": regions,
            "kernels": kernels, "per_config": per_config, "hbm_parts": hbm}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
