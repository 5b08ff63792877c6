"""The drop-in operator surface on the GPU: plan-selected operators, their autograd, model
patching and the fused training adapter, each checked to run the HIP kernels.

Restates test_matmul_execution.py:143-300 (forward/dX/dW with FP32 leaf gradients for every
algorithm, eager and compiled; ATen fallback of unaligned aligned-load operands; a patched
model through BF16 autocast, backward, an AdamW step and a state-dict reload; the fused
projection under compiled autograd with and without recomputation). Compiled runs use the
``aot_eager`` backend: Dynamo capture, AOTAutograd and the operators' fake and autograd
registrations are exercised without generated kernels. Bars: the reference's own
(forward rtol/atol 0.015, gradient rel-L2 0.005 or 0.02, model loss rtol 1e-3 and gradient
cosine > 0.999), plus the oracle bars of tests/metrics.py where a CPU oracle applies.
"""
import copy
import math

import pytest
import torch

from metrics import assert_bf16_close, assert_f32_close
from oracle import reference as oracle

pytestmark = pytest.mark.gpu


@pytest.fixture
def hip_calls(monkeypatch):
    """Names of the C-ABI entry points called during the test."""
    from ops import _hip

    seen = []
    real = _hip.call

    def spy(name, *args):
        seen.append(name)
        return real(name, *args)

    monkeypatch.setattr(_hip, "call", spy)
    return seen


def _entry(*, kind="mm", m=8, n=32, k=16, algorithm="tiled", a_stride=None, b_stride=None):
    return {"kind": kind, "m": m, "n": n, "k": k,
            "a_stride": a_stride or [k, 1], "b_stride": b_stride or [1, k],
            "dtype": "bfloat16", "algorithm": algorithm,
            "tile": {"block_m": 32, "block_n": 32, "block_k": 32, "num_warps": 4,
                     "num_stages": 3}}


def _plan(entries):
    from ops.matmul_execution import PLAN_FORMAT, matmul_plan_from_dict

    return matmul_plan_from_dict({"format": PLAN_FORMAT, "entries": entries})


def _model(**overrides):
    from warpstate import WarpStateConfig, WarpStateLM

    torch.manual_seed(492)
    cfg = dict(vocab_size=48, d_model=16, n_heads=2, n_cores=1, logical_depth=1,
               ffn_hidden=32, chunk_size=4, parallel_memory=True, gradient_checkpointing=False)
    cfg.update(overrides)
    return WarpStateLM(WarpStateConfig(**cfg)).train()


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30)).item()


# --- planned_matmul: forward, dX, dW -----------------------------------------------------

@pytest.mark.parametrize("algorithm", ["tiled", "persistent", "persistent_tma"])
@pytest.mark.parametrize("compiled", [False, True])
def test_selected_forward_dx_dw_keep_fp32_leaf_gradients(algorithm, compiled, hip_calls):
    """test_matmul_execution.py:143-178: the plan selects the forward, the dW-oriented
    weight gradient (dY^T @ X) and the input gradient; every one runs the HIP GEMM."""
    from ops.matmul_execution import planned_matmul

    torch.manual_seed(497)
    forward = _entry(m=64, n=128, k=64, algorithm=algorithm)
    weight_grad = _entry(m=128, n=64, k=64, algorithm=algorithm, a_stride=[1, 128],
                         b_stride=[64, 1])
    input_grad = _entry(m=64, n=64, k=128, algorithm=algorithm, b_stride=[64, 1])
    plan = _plan([forward, weight_grad, input_grad])
    reference = torch.nn.Parameter(torch.randn(128, 64, device="cuda") * 0.02)
    actual = torch.nn.Parameter(reference.detach().clone())

    def expected_fn(x, w):
        return x.to(torch.bfloat16) @ w.to(torch.bfloat16).T

    def selected_fn(x, w):
        return planned_matmul(x.to(torch.bfloat16), w.to(torch.bfloat16).T, plan)

    if compiled:
        expected_fn = torch.compile(expected_fn, backend="aot_eager", fullgraph=True, dynamic=False)
        selected_fn = torch.compile(selected_fn, backend="aot_eager", fullgraph=True, dynamic=False)
    for step in range(8):
        x = torch.randn(64, 64, device="cuda", requires_grad=True)
        selected_x = x.detach().clone().requires_grad_(True)
        dy = torch.randn(64, 128, device="cuda", dtype=torch.bfloat16)
        expected = expected_fn(x, reference)
        before = len(hip_calls)
        result = selected_fn(selected_x, actual)
        assert hip_calls[before:].count("ws_mm") == 1, hip_calls[before:]
        torch.testing.assert_close(result, expected, rtol=0.015, atol=0.015)
        if step == 0:
            want = oracle.mm(x.detach().bfloat16().cpu(), reference.detach().bfloat16().T.cpu())
            assert_bf16_close(result, want, "planned_mm forward vs oracle")
        expected.backward(dy)
        before = len(hip_calls)
        result.backward(dy)
        # dX and dW both through the selected HIP GEMM.
        assert hip_calls[before:].count("ws_mm") == 2, hip_calls[before:]
        assert selected_x.grad.dtype == torch.float32
        assert _rel(selected_x.grad, x.grad) < 0.005
    assert actual.dtype == actual.grad.dtype == torch.float32
    assert _rel(actual.grad, reference.grad) < 0.005


def test_unsupported_aligned_load_layout_falls_back_to_aten(hip_calls):
    """test_matmul_execution.py:181-188: a column-strided B cannot take the aligned-load
    kernel, so the plan entry is not used and ATen computes the product exactly."""
    from ops.matmul_execution import planned_matmul

    a = torch.randn(32, 32, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(32, 64, device="cuda", dtype=torch.bfloat16)[:, ::2]
    plan = _plan([_entry(m=32, n=32, k=32, algorithm="persistent_tma",
                         b_stride=list(b.stride()))])
    torch.testing.assert_close(planned_matmul(a, b, plan), a @ b, rtol=0, atol=0)
    assert "ws_mm" not in hip_calls


@pytest.mark.parametrize("misaligned", ["a", "b"])
def test_aligned_load_rechecks_storage_offset_before_launch(misaligned, hip_calls):
    """test_matmul_execution.py:190-211: same shape and strides, but a storage offset that
    breaks 16-byte alignment sends the call to ATen, eager and compiled."""
    from ops.matmul_execution import planned_matmul

    a = torch.randn(64, 64, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(128, 64, device="cuda", dtype=torch.bfloat16).T
    plan = _plan([_entry(m=64, n=128, k=64, algorithm="persistent_tma")])
    compiled = torch.compile(lambda x, y: planned_matmul(x, y, plan), backend="aot_eager",
                             fullgraph=True, dynamic=False)
    torch.testing.assert_close(compiled(a, b), a @ b, rtol=0.015, atol=0.015)
    assert "ws_mm" in hip_calls
    original = a if misaligned == "a" else b
    storage = torch.randn(original.numel() + 1, device="cuda", dtype=torch.bfloat16)
    shifted = storage.as_strided(original.shape, original.stride(), storage_offset=1)
    assert shifted.data_ptr() % 16 == 2
    a, b = (shifted, b) if misaligned == "a" else (a, shifted)
    hip_calls.clear()
    torch.testing.assert_close(planned_matmul(a, b, plan), a @ b, rtol=0, atol=0)
    assert "ws_mm" not in hip_calls


# --- patched model: BF16 autocast, backward, AdamW, reload --------------------------------

@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("compiled", [False, True])
def test_patched_model_matches_and_keeps_fp32_adam_and_reload(fused, compiled, hip_calls):
    """test_matmul_execution.py:216-253 with the shim model and BF16 residuals: the plan
    serves the SwiGLU up/gate projection (fused or plain), loss and gradients match the
    unpatched model, FP32 masters, gradients and AdamW state stay FP32, and a reload gives
    the same evaluation outputs."""
    from ops.matmul_execution import apply_matmul_execution
    from ops.residual_experiment import apply_bf16_residuals

    reference = _model().cuda()
    actual = copy.deepcopy(reference)
    plan = _plan([_entry(kind="swiglu" if fused else "mm", m=16, n=64, k=16)])
    keys = tuple(actual.state_dict())
    masters = tuple(actual.parameters())
    apply_matmul_execution(actual, plan)
    for model in (reference, actual):
        if compiled:
            for core in model.cores:
                core.compile(backend="aot_eager", dynamic=False)
        apply_bf16_residuals(model)
    optimizer = torch.optim.AdamW(actual.parameters(), lr=1e-4)
    inputs = torch.randint(48, (2, 8), device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        expected = reference(inputs, inputs, return_logits=False)[1]
        hip_calls.clear()
        result = actual(inputs, inputs, return_logits=False)[1]
    assert ("ws_swiglu_mm" if fused else "ws_mm") in hip_calls, hip_calls
    expected.backward()
    result.backward()
    torch.testing.assert_close(result, expected, rtol=0.001, atol=0.001)
    grads = torch.cat([p.grad.flatten() for p in actual.parameters()])
    ref_grads = torch.cat([p.grad.flatten() for p in reference.parameters()])
    assert torch.nn.functional.cosine_similarity(grads, ref_grads, dim=0).item() > 0.999
    assert _rel(grads, ref_grads) < 0.02
    optimizer.step()
    assert tuple(actual.state_dict()) == keys
    assert all(a is b for a, b in zip(masters, actual.parameters(), strict=True))
    assert all(p.dtype == p.grad.dtype == optimizer.state[p]["exp_avg"].dtype
               == optimizer.state[p]["exp_avg_sq"].dtype == torch.float32 for p in masters)
    restored = _model().cuda().eval()
    restored.load_state_dict(actual.state_dict(), strict=True)
    actual.eval()
    with torch.no_grad():
        torch.testing.assert_close(actual(inputs), restored(inputs), rtol=0, atol=0)


@pytest.mark.parametrize("algorithm", ["tiled", "persistent", "persistent_tma"])
@pytest.mark.parametrize("recompute", [False, True])
def test_compiled_autograd_fused_projection_dx_dw_and_recomputation(algorithm, recompute,
                                                                     hip_calls):
    """test_matmul_execution.py:256-300: the SwiGLU module patched with a fused entry and
    its dX / dW entries, compiled, backward under compiled autograd (which re-traces the
    operators' backward), with and without activation checkpointing."""
    from torch._dynamo import compiled_autograd
    from torch.utils.checkpoint import checkpoint

    from ops.matmul_execution import apply_matmul_execution

    torch._dynamo.reset()
    reference_model = _model().cuda()
    selected_model = copy.deepcopy(reference_model)
    fused = _entry(kind="swiglu", m=16, n=64, k=16, algorithm="persistent")
    dx = _entry(m=16, n=16, k=64, algorithm=algorithm, b_stride=[16, 1])
    dw = _entry(m=64, n=16, k=16, algorithm=algorithm, a_stride=[1, 64], b_stride=[16, 1])
    apply_matmul_execution(selected_model, _plan([fused, dx, dw]))
    reference = reference_model.cores[0].ffn
    selected = selected_model.cores[0].ffn

    def wrap(module):
        return (lambda x: checkpoint(module, x, use_reentrant=False)) if recompute else module

    wanted_fn = torch.compile(wrap(reference), backend="aot_eager", fullgraph=True, dynamic=False)
    actual_fn = torch.compile(wrap(selected), backend="aot_eager", fullgraph=True, dynamic=False)
    backward_compiler = torch.compile(backend="aot_eager")
    try:
        for _ in range(2):
            x = torch.randn(16, 16, device="cuda", requires_grad=True)
            actual_x = x.detach().clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                wanted = wanted_fn(x)
                hip_calls.clear()
                actual = actual_fn(actual_x)
            assert "ws_swiglu_mm" in hip_calls, hip_calls
            torch.testing.assert_close(actual, wanted, rtol=0.015, atol=0.0001)
            wanted.float().square().mean().backward()
            hip_calls.clear()
            with compiled_autograd._enable(backward_compiler):
                actual.float().square().mean().backward()
            assert "ws_swiglu_backward" in hip_calls and "ws_mm" in hip_calls, hip_calls
            pairs = [(x, actual_x), *zip(reference.parameters(), selected.parameters(), strict=True)]
            for p, q in pairs:
                assert q.grad.dtype == torch.float32
                assert _rel(q.grad, p.grad) < 0.02
    finally:
        torch._dynamo.reset()


# --- the fused training adapter ------------------------------------------------------------

def _compile_training_cores(model, backend):
    """Each core's forward compiled whole (fullgraph) for training calls, as the reference's
    compile_training_cores does (run_40b.py:430-438)."""
    for core in model.cores:
        eager = core.forward
        compiled = torch.compile(eager, fullgraph=True, dynamic=False, backend=backend)

        def forward(*args, _core=core, _eager=eager, _compiled=compiled, **kwargs):
            fn = _compiled if _core.training and torch.is_grad_enabled() else _eager
            return fn(*args, **kwargs)

        core.forward = forward


@pytest.mark.parametrize("size", ["tiny", "medium", "medium_checkpointed",
                                  "medium_compiled_cores", "medium_compiled_model"])
def test_fused_adapter_matches_unpatched_model(size, hip_calls):
    """apply_fused_execution routes norm1 -> in_proj -> gate sigmoid, the residual
    projections, the SwiGLU block and the chunked tied-head loss through the fused
    kernels; loss and every parameter gradient agree with the unpatched model under BF16
    autocast with BF16 residuals, the weight gradients reach autograd's hooks, an AdamW
    step keeps FP32 state and the state dict is untouched. The compiled variants compile
    the patched cores with fullgraph=True (the fused pieces are registered operators) or
    the whole model (the loss then runs eagerly)."""
    try:
        _fused_adapter_case(size, hip_calls)
    finally:
        torch._dynamo.reset()


def _fused_adapter_case(size, hip_calls):
    from ops.fused_training import apply_fused_execution
    from ops.residual_experiment import apply_bf16_residuals

    if size == "tiny":
        reference, tokens, vocab = _model(), (2, 8), 48
    else:
        vocab = 2048
        reference = _model(vocab_size=vocab, d_model=256, n_heads=4, n_cores=2,
                           logical_depth=3, ffn_hidden=512, loss_chunk_size=96,
                           gradient_checkpointing=size == "medium_checkpointed")
        tokens = (4, 64)
    reference = reference.cuda()
    actual = copy.deepcopy(reference)
    keys = tuple(actual.state_dict())
    masters = tuple(actual.parameters())
    apply_fused_execution(actual)
    for model in (reference, actual):
        apply_bf16_residuals(model)
    run = actual
    if size == "medium_compiled_cores":
        _compile_training_cores(actual, "aot_eager")
    elif size == "medium_compiled_model":
        run = torch.compile(actual, backend="aot_eager")
    hooked = []
    actual.cores[0].in_proj.weight.register_hook(lambda g: hooked.append(g.dtype))
    gen = torch.Generator("cpu").manual_seed(11)
    inputs = torch.randint(vocab, tokens, generator=gen).cuda()
    labels = torch.randint(vocab, tokens, generator=gen)
    labels.view(-1)[::7] = -100
    labels = labels.cuda()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        expected = reference(inputs, labels, return_logits=False)[1]
        hip_calls.clear()
        result = run(inputs, labels, return_logits=False)[1]
    for name in ("ws_rmsnorm_gate_mm", "ws_residual_mm", "ws_swiglu_mm", "ws_linear_ce_fused"):
        assert name in hip_calls, (name, hip_calls)
    expected.backward()
    hip_calls.clear()
    result.backward()
    # The projection weight's gradient went through autograd (where DDP's hooks sit).
    assert hooked and all(dtype == torch.float32 for dtype in hooked), hooked
    for name in ("ws_linear_ce_fused_backward", "ws_sigmoid_backward_cols", "ws_swiglu_backward_mm",
                 "ws_mm_store_f32", "ws_rmsnorm_backward"):
        assert any(call.startswith(name) for call in hip_calls), (name, hip_calls)
    assert math.isclose(result.item(), expected.item(), rel_tol=1e-3)
    for (name, p), q in zip(reference.named_parameters(), actual.parameters(), strict=True):
        assert q.grad is not None and q.grad.dtype == torch.float32, name
        cos = torch.nn.functional.cosine_similarity(q.grad.flatten().double(),
                                                    p.grad.flatten().double(), dim=0).item()
        assert cos > 0.999 and _rel(q.grad, p.grad) < 0.02, (name, cos, _rel(q.grad, p.grad))
    optimizer = torch.optim.AdamW(actual.parameters(), lr=1e-4)
    optimizer.step()
    assert tuple(actual.state_dict()) == keys
    assert all(a is b for a, b in zip(masters, actual.parameters(), strict=True))
    assert all(optimizer.state[p]["exp_avg"].dtype == torch.float32 for p in masters)
    # Evaluation and CPU-free inference keep the original path.
    reference.eval()
    actual.eval()
    with torch.no_grad():
        hip_calls.clear()
        logits = actual(inputs)
        assert not hip_calls
        assert logits.shape == (*tokens, vocab)


@pytest.mark.parametrize("dims", [(256, 512, 2048), (100, 250, 1030)],
                         ids=["d256", "d100_ffn250_vocab1030"])
@pytest.mark.parametrize("variant", ["eager", "checkpointed", "compiled_cores", "compiled_model"])
def test_fused_adapter_on_the_reference_core_layout(variant, dims, hip_calls):
    """A model in the reference's own layout (one WarpStateCore.forward with _split, the
    inline gate sigmoid and residual adds, and the inline chunked loss; no seams): the
    adapter attaches its RMSNorm, Linear and SwiGLU modules and the loss (through a forward
    wrap that stops at final_norm), and loss and every parameter gradient agree with the
    unpatched model at the reference's bars (loss rtol 1e-3, gradient cosine > 0.999)
    under BF16 autocast with BF16 residuals. No weight gradient is formed in a cleared
    buffer: every one comes from the FP32 store GEMMs, through autograd. The second width
    set (model width 100, hidden 250, vocabulary 1030: none a multiple of 8) takes the
    library's generic loaders and row kernels throughout."""
    from inline_layout_model import InlineLM
    from warpstate.config import WarpStateConfig

    from ops.fused_training import apply_fused_execution
    from ops.residual_experiment import apply_bf16_residuals

    try:
        torch.manual_seed(733)
        d_model, ffn, vocab = dims
        tokens = (4, 64)
        reference = InlineLM(WarpStateConfig(
            vocab_size=vocab, d_model=d_model, n_heads=4, n_cores=2, logical_depth=3,
            ffn_hidden=ffn, loss_chunk_size=96,
            gradient_checkpointing=variant == "checkpointed")).train().cuda()
        actual = copy.deepcopy(reference)
        keys = tuple(actual.state_dict())
        apply_fused_execution(actual)
        for model in (reference, actual):
            apply_bf16_residuals(model)
        run = actual
        if variant == "compiled_cores":
            _compile_training_cores(actual, "aot_eager")
        elif variant == "compiled_model":
            run = torch.compile(actual, backend="aot_eager")
        gen = torch.Generator("cpu").manual_seed(12)
        inputs = torch.randint(vocab, tokens, generator=gen).cuda()
        labels = torch.randint(vocab, tokens, generator=gen)
        labels.view(-1)[::7] = -100
        labels = labels.cuda()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            expected = reference(inputs, labels, return_logits=False)[1]
            hip_calls.clear()
            result = run(inputs, labels, return_logits=False)[1]
        for name in ("ws_rmsnorm_forward", "ws_mm", "ws_swiglu_mm", "ws_linear_ce_fused"):
            assert name in hip_calls, (name, hip_calls)
        # The seams' fusions are not available here.
        assert "ws_rmsnorm_gate_mm" not in hip_calls and "ws_residual_mm" not in hip_calls
        expected.backward()
        hip_calls.clear()
        result.backward()
        for name in ("ws_linear_ce_fused_backward", "ws_swiglu_backward_mm", "ws_mm_store_f32",
                     "ws_mm_store_f32_group", "ws_rmsnorm_backward"):
            assert name in hip_calls, (name, hip_calls)
        assert not any(call.startswith("ws_mm_accumulate") for call in hip_calls), hip_calls
        assert math.isclose(result.item(), expected.item(), rel_tol=1e-3)
        for (name, p), q in zip(reference.named_parameters(), actual.parameters(), strict=True):
            assert q.grad is not None and q.grad.dtype == torch.float32, name
            cos = torch.nn.functional.cosine_similarity(q.grad.flatten().double(),
                                                        p.grad.flatten().double(), dim=0).item()
            assert cos > 0.999 and _rel(q.grad, p.grad) < 0.02, (name, cos, _rel(q.grad, p.grad))
        assert tuple(actual.state_dict()) == keys
        actual.eval()
        with torch.no_grad():
            hip_calls.clear()
            assert actual(inputs).shape == (*tokens, vocab)
            assert not hip_calls
    finally:
        torch._dynamo.reset()


def test_fused_adapter_refuses_second_application_and_bf16_masters():
    from ops.fused_training import apply_fused_execution

    model = _model().cuda()
    apply_fused_execution(model)
    with pytest.raises(ValueError, match="already been applied"):
        apply_fused_execution(model)
    with pytest.raises(ValueError, match="FP32 master"):
        apply_fused_execution(_model().cuda().bfloat16())


# --- LM-head autograd and state checks ----------------------------------------------------

@pytest.mark.parametrize("weight_dtype", [torch.float32, torch.bfloat16])
def test_linear_cross_entropy_autograd_gives_hidden_and_weight_gradients(weight_dtype):
    from ops.benchmark_configs import lm_head_inputs
    from ops.fused_execution import linear_cross_entropy

    inp = lm_head_inputs(m=384, d=256, vocab=2048, seed=3)
    h = inp["hidden"].cuda().requires_grad_(True)
    w = inp["weight"].to(weight_dtype).cuda().requires_grad_(True)
    t = inp["targets"].cuda()
    mean, loss = linear_cross_entropy(h, w, t, 128)
    mean.backward()
    torch.cuda.synchronize()
    want_loss, want_mean, _count, want_dh = oracle.linear_cross_entropy(
        inp["hidden"], inp["weight"], inp["targets"], chunk=128)
    assert torch.allclose(loss.cpu(), want_loss, rtol=1e-4, atol=1e-4)
    assert math.isclose(mean.item(), want_mean.item(), rel_tol=1e-5)
    assert h.grad.dtype == torch.bfloat16
    assert_bf16_close(h.grad, want_dh, "dHidden through autograd")
    want_dw = oracle.linear_cross_entropy_weight_grad(inp["hidden"], inp["weight"],
                                                      inp["targets"], chunk=128)
    assert w.grad.dtype == weight_dtype
    if weight_dtype == torch.float32:
        assert_f32_close(w.grad.cpu(), want_dw, "head weight gradient (FP32 master)")
    else:
        assert_bf16_close(w.grad, want_dw.bfloat16(), "head weight gradient (BF16)")


def test_cross_entropy_state_of_another_shape_is_rejected_before_launch(hip_calls):
    from ops.fused_execution import CrossEntropyState, linear_cross_entropy_forward

    h = torch.zeros(64, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(512, 128, dtype=torch.bfloat16, device="cuda")
    t = torch.zeros(64, dtype=torch.int64, device="cuda")
    for state in (CrossEntropyState(32, 512, h.device), CrossEntropyState(64, 256, h.device)):
        with pytest.raises(ValueError, match="CrossEntropyState"):
            linear_cross_entropy_forward(h, w, t, state)
    assert not hip_calls
