"""Host-side behaviour of the operator surface, restating the reference's CPU tests.

test_matmul_kernels.py:16-48,121-135 (tile validation, dispatch signatures, no CPU or
unknown-algorithm fallback, TMA alignment errors raised before any launch),
test_matmul_epilogue.py:12-47 (aten numerics, argument errors before a launch),
test_matmul_execution.py:36-138 (plan schema, hashing, exact selection, CPU autograd,
model patching) and test_activation_execution.py:24-63 (CPU paths unchanged). None of
these touch a GPU.
"""
import copy
import json

import pytest
import torch
import torch.nn.functional as F

from ops.matmul_epilogue import SUPPORTED_TILES, launch_swiglu_mm
from ops.matmul_execution import (PLAN_FORMAT, apply_matmul_execution, load_matmul_plan,
                                  matmul_plan_from_dict, planned_matmul)
from ops.matmul_kernels import (DEFAULT_TILE, TUNING_TILES, launch_mm, matrix_signature,
                                normalize_tile, policy_key, tile_dict)
from warpstate import WarpStateConfig, WarpStateLM


# --- ops.matmul_kernels ---------------------------------------------------------------

@pytest.mark.parametrize("tile", [
    [], (128, 128, 32, 4), (128, 128, 32, True, 3), (120, 128, 32, 4, 3),
    (128, 128, 32, 2, 3), (128, 128, 32, 4, 8), (256, 256, 128, 8, 4),
    {"block_m": 128},
])
def test_invalid_or_oversized_tiles_fail(tile):
    with pytest.raises(ValueError):
        normalize_tile(tile)


def test_tuning_tiles_and_json_round_trip():
    for tile in TUNING_TILES:
        assert normalize_tile(json.loads(json.dumps(tile_dict(tile)))) == tile
    assert normalize_tile() == DEFAULT_TILE


def test_signature_distinguishes_strides_even_when_shapes_match():
    a = torch.empty((16, 32), dtype=torch.bfloat16)
    b = torch.empty((64, 32), dtype=torch.bfloat16).T
    signature = matrix_signature(a, b)
    assert signature == {"m": 16, "n": 64, "k": 32, "a_stride": [32, 1],
                         "b_stride": [1, 32], "dtype": "bfloat16"}
    assert json.loads(policy_key(a, b)) == signature
    assert policy_key(a, b) != policy_key(a, b.contiguous())


def test_no_cpu_or_unknown_algorithm_fallback():
    a = torch.empty((16, 32), dtype=torch.bfloat16)
    b = torch.empty((32, 16), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        launch_mm(a, b)
    with pytest.raises(ValueError, match="Unknown"):
        launch_mm(a, b, "fp8")


@pytest.mark.parametrize("offset_operand", ["a", "b"])
def test_tma_rejects_misaligned_offset_without_launching(offset_operand):
    from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode

    mode = FakeTensorMode()
    tensors = []
    for name, shape in (("a", (32, 64)), ("b", (64, 32))):
        offset = 1 if name == offset_operand else 0
        storage = torch.empty(shape[0] * shape[1] + offset, device="meta", dtype=torch.bfloat16)
        view = storage.as_strided(shape, (shape[1], 1), offset)
        tensors.append(FakeTensor(mode, view, torch.device("cuda:0")))
    with pytest.raises(ValueError, match="16-byte-aligned storage offsets"):
        launch_mm(*tensors, "persistent_tma")


# --- ops.matmul_epilogue --------------------------------------------------------------

@pytest.mark.parametrize("eager_rounding", [False, True])
def test_aten_swiglu_preserves_projection_and_activation_rounding(eager_rounding):
    torch.manual_seed(554)
    a = torch.randn(7, 31, dtype=torch.bfloat16)
    b = torch.randn(46, 31, dtype=torch.bfloat16).T
    packed, activation = launch_swiglu_mm(a, b, "aten", SUPPORTED_TILES[0], eager_rounding)
    expected = a @ b
    up, gate = expected.chunk(2, dim=-1)
    wanted = F.silu(gate) * up if eager_rounding else (F.silu(gate.float()) * up.float()).bfloat16()
    assert torch.equal(packed, expected) and torch.equal(activation, wanted)
    assert packed.is_contiguous() and activation.is_contiguous()
    assert packed.untyped_storage().data_ptr() != activation.untyped_storage().data_ptr()


@pytest.mark.parametrize("case", ["dtype", "shape", "odd_width", "empty", "cpu", "tile", "algorithm"])
def test_unsupported_swiglu_execution_fails_before_a_kernel_launch(case):
    a = torch.ones(4, 8, dtype=torch.bfloat16)
    b = torch.ones(8, 16, dtype=torch.bfloat16)
    algorithm, tile = "aten", SUPPORTED_TILES[0]
    if case == "dtype":
        a = a.float()
    elif case == "shape":
        b = b[:7]
    elif case == "odd_width":
        b = b[:, :15]
    elif case == "empty":
        a = a[:0]
    elif case == "cpu":
        algorithm = "tiled"
    elif case == "tile":
        tile = (256, 256, 64, 8, 4)
    elif case == "algorithm":
        algorithm = "unsupported"
    with pytest.raises(ValueError):
        launch_swiglu_mm(a, b, algorithm, tile)


# --- ops.matmul_execution -------------------------------------------------------------

def _entry(*, kind="mm", m=8, n=32, k=16, algorithm="tiled"):
    return {"kind": kind, "m": m, "n": n, "k": k, "a_stride": [k, 1], "b_stride": [1, k],
            "dtype": "bfloat16", "algorithm": algorithm,
            "tile": {"block_m": 32, "block_n": 32, "block_k": 32, "num_warps": 4,
                     "num_stages": 3}}


def _document(entries=None):
    return {"format": PLAN_FORMAT, "entries": entries if entries is not None else [_entry()]}


def _model():
    torch.manual_seed(492)
    return WarpStateLM(WarpStateConfig(vocab_size=48, d_model=16, n_heads=2, n_cores=1,
                                       logical_depth=1, ffn_hidden=32, chunk_size=4,
                                       parallel_memory=True,
                                       gradient_checkpointing=False)).train()


def test_plan_exact_shape_stride_key_and_source_provenance(tmp_path, monkeypatch):
    monkeypatch.setenv("WARPSTATE_WORKSPACE", str(tmp_path))
    path = tmp_path / "plan.json"
    path.write_text(json.dumps(_document()))
    plan = load_matmul_plan(path)
    assert plan.select("mm", 8, 32, 16, (16, 1), (1, 16)).algorithm == "tiled"
    assert plan.select("mm", 8, 32, 16, (16, 1), (32, 1)) is None
    assert plan.select("mm", 7, 32, 16, (16, 1), (1, 16)) is None
    assert plan.select("swiglu", 8, 32, 16, (16, 1), (1, 16)) is None
    assert len(plan.metadata["sha256"]) == 64
    assert "ops/matmul_execution.py" in plan.metadata["source_sha256"]
    assert "ops/matmul_kernels.py" in plan.metadata["source_sha256"]
    path.write_text(json.dumps(_document(), indent=4))
    assert load_matmul_plan(path).metadata == plan.metadata
    altered = _document()
    altered["entries"][0]["tile"]["block_m"] = 64
    assert matmul_plan_from_dict(altered).sha256 != plan.sha256
    fused = matmul_plan_from_dict(_document([_entry(kind="swiglu")]))
    assert "ops/matmul_epilogue.py" in fused.metadata["source_sha256"]
    assert "ops/activation_execution.py" in fused.metadata["source_sha256"]


def test_plan_outside_workspace_is_rejected(tmp_path, monkeypatch):
    monkeypatch.setenv("WARPSTATE_WORKSPACE", str(tmp_path / "inner"))
    path = tmp_path / "plan.json"
    path.write_text(json.dumps(_document()))
    with pytest.raises(ValueError, match="workspace"):
        load_matmul_plan(path)


@pytest.mark.parametrize("mutation", [
    lambda d: d.update(format="other"),
    lambda d: d.update(unknown=True),
    lambda d: d["entries"][0].update(dtype="float16"),
    lambda d: d["entries"][0].update(algorithm="unknown"),
    lambda d: d["entries"][0].update(m=True),
    lambda d: d["entries"][0].update(n=0),
    lambda d: d["entries"][0].update(a_stride=[0, 1]),
    lambda d: d["entries"][0].update(b_stride=[1]),
    lambda d: d["entries"][0].update(kind="swiglu", n=31),
    lambda d: d["entries"][0].update(kind="swiglu", algorithm="persistent_tma"),
    lambda d: d["entries"][0]["tile"].update(block_k=0),
    lambda d: d["entries"].append(copy.deepcopy(d["entries"][0])),
])
def test_invalid_plan_fails_before_model_or_gpu_work(mutation):
    document = _document()
    mutation(document)
    with pytest.raises(ValueError):
        matmul_plan_from_dict(document)


def test_duplicate_json_keys_rejected(tmp_path, monkeypatch):
    monkeypatch.setenv("WARPSTATE_WORKSPACE", str(tmp_path))
    path = tmp_path / "duplicate.json"
    path.write_text('{"format":"warpstate-matmul-plan-v1","entries":[],"entries":[]}')
    with pytest.raises(ValueError, match="Duplicate JSON"):
        load_matmul_plan(path)


@pytest.mark.parametrize("compiled", [False, True])
def test_unsupported_cpu_matmul_retains_cast_and_fp32_gradient_accumulation(compiled):
    torch.manual_seed(495)
    plan = matmul_plan_from_dict(_document())
    expected = torch.nn.Parameter(torch.randn(32, 16))
    actual = torch.nn.Parameter(expected.detach().clone())
    original = lambda x, weight: torch.mm(x, weight.to(torch.bfloat16).T)  # noqa: E731
    selected = lambda x, weight: planned_matmul(x, weight.to(torch.bfloat16).T, plan)  # noqa: E731
    if compiled:
        original = torch.compile(original, backend="aot_eager", fullgraph=True)
        selected = torch.compile(selected, backend="aot_eager", fullgraph=True)
    for _ in range(4):
        x = torch.randn(8, 16, dtype=torch.bfloat16)
        grad = torch.randn(8, 32, dtype=torch.bfloat16)
        y = original(x, expected)
        z = selected(x, actual)
        assert torch.equal(z, y)
        y.backward(grad)
        z.backward(grad)
        assert actual.grad.dtype == torch.float32
        assert torch.equal(actual.grad, expected.grad)


def test_model_patch_preserves_parameters_state_and_cpu_eval():
    reference = _model()
    actual = copy.deepcopy(reference)
    masters = tuple(actual.parameters())
    keys = tuple(actual.state_dict())
    apply_matmul_execution(actual, matmul_plan_from_dict(_document([_entry(kind="swiglu")])))
    inputs = torch.randint(48, (2, 8))
    for training in [True, False]:
        reference.train(training)
        actual.train(training)
        with torch.set_grad_enabled(training):
            assert torch.equal(actual(inputs), reference(inputs))
    assert tuple(actual.state_dict()) == keys
    assert all(a is b for a, b in zip(masters, actual.parameters(), strict=True))
    with pytest.raises(ValueError, match="already been applied"):
        apply_matmul_execution(actual, matmul_plan_from_dict(_document()))
    with pytest.raises(ValueError, match="FP32 master"):
        apply_matmul_execution(_model().bfloat16(), matmul_plan_from_dict(_document()))


def test_shape_policy_only_patches_relevant_projection_modules():
    model = _model()
    core = model.cores[0]
    originals = {name: module.forward for name, module in core.named_modules()
                 if isinstance(module, torch.nn.Linear)}
    apply_matmul_execution(model, matmul_plan_from_dict(_document([_entry(m=16, n=64, k=16)])))
    assert core.ffn.up_gate.forward != originals["ffn.up_gate"]
    assert core.ffn.down.forward == originals["ffn.down"]
    assert core.in_proj.forward == originals["in_proj"]
    assert core.out_proj.forward == originals["out_proj"]


# --- ops.activation_execution ---------------------------------------------------------

@pytest.mark.parametrize("mode", ["baseline", "swiglu", "rmsnorm", "all"])
def test_activation_cpu_path_retains_parameters_and_outputs(mode):
    from ops.activation_execution import apply_activation_execution

    torch.manual_seed(943)
    reference = WarpStateLM(WarpStateConfig(vocab_size=48, d_model=32, n_heads=2, n_cores=1,
                                            logical_depth=2, ffn_hidden=56, chunk_size=4,
                                            gradient_checkpointing=False,
                                            parallel_memory=True)).train()
    actual = copy.deepcopy(reference)
    parameters = tuple(actual.parameters())
    apply_activation_execution(actual, mode)
    tokens = torch.randint(48, (2, 8))
    with torch.autocast("cpu", dtype=torch.bfloat16):
        expected, result = reference(tokens), actual(tokens)
    assert torch.equal(result, expected)
    assert all(a is b for a, b in zip(actual.parameters(), parameters, strict=True))
    if mode != "baseline":
        with pytest.raises(ValueError, match="already been applied"):
            apply_activation_execution(actual, "all")
    with pytest.raises(ValueError, match="Unknown activation"):
        apply_activation_execution(copy.deepcopy(reference), "invalid")


# --- fused entry points: argument errors before any launch --------------------------

def test_fused_entry_points_reject_cpu_tensors():
    from ops import fused_execution as fx

    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    w = torch.zeros(6, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        fx.rmsnorm_gate_mm(x, torch.ones(8), 1e-6, w, (0, 2))
    with pytest.raises(ValueError, match="CUDA"):
        fx.residual_mm(x, w, torch.zeros(4, 6, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA"):
        fx.linear_cross_entropy_forward(x, w, torch.zeros(4, dtype=torch.int64))


def test_cross_entropy_state_must_match_the_operands():
    """A state built for another row count or vocabulary is refused before any launch
    (its buffers are indexed by the operands' rows and vocabulary)."""
    from ops.fused_execution import CrossEntropyState, _check_state

    state = CrossEntropyState(8, 64, "cpu")
    _check_state(state, 8, 64, torch.device("cpu"))
    for rows, vocab in ((16, 64), (8, 128), (4, 64)):
        with pytest.raises(ValueError, match="CrossEntropyState"):
            _check_state(state, rows, vocab, torch.device("cpu"))
    state.lse = torch.empty(4)
    with pytest.raises(ValueError, match="state.lse"):
        _check_state(state, 8, 64, torch.device("cpu"))
    with pytest.raises(TypeError):
        _check_state(object(), 8, 64, torch.device("cpu"))


def test_fused_output_buffers_are_checked_before_launch():
    from ops.fused_execution import _check_buffer

    good = torch.empty(4, 6, dtype=torch.bfloat16)
    _check_buffer(good, (4, 6), torch.bfloat16, good.device, "out")
    for bad in (torch.empty(4, 5, dtype=torch.bfloat16), torch.empty(4, 6),
                torch.empty(6, 4, dtype=torch.bfloat16).T):
        with pytest.raises(ValueError):
            _check_buffer(bad, (4, 6), torch.bfloat16, good.device, "out")
    # A row-strided view is fine where only a unit column stride is needed.
    _check_buffer(torch.empty(4, 8, dtype=torch.bfloat16)[:, :6], (4, 6), torch.bfloat16,
                  good.device, "out", contiguous=False)


def _small_lm(**overrides):
    torch.manual_seed(572)
    cfg = dict(vocab_size=32, d_model=16, n_heads=2, n_cores=1, logical_depth=2,
               ffn_hidden=24, chunk_size=4, gradient_checkpointing=False,
               parallel_memory=True, loss_chunk_size=3)
    cfg.update(overrides)
    return WarpStateLM(WarpStateConfig(**cfg)).train()


def test_fused_adapter_keeps_cpu_and_eval_paths_and_state():
    """On the CPU (and in evaluation) the adapted model runs the original forwards: same
    loss, same gradients, same parameters and state dict."""
    from ops.fused_training import apply_fused_execution

    reference = _small_lm()
    adapted = copy.deepcopy(reference)
    keys, params = tuple(adapted.state_dict()), tuple(adapted.parameters())
    apply_fused_execution(adapted)
    assert tuple(adapted.state_dict()) == keys
    assert all(a is b for a, b in zip(params, adapted.parameters(), strict=True))
    tokens = torch.randint(32, (2, 8))
    labels = torch.randint(32, (2, 8))
    labels.view(-1)[3:9] = -100
    with torch.autocast("cpu", dtype=torch.bfloat16):
        _, want = reference(tokens, labels, return_logits=False)
        _, got = adapted(tokens, labels, return_logits=False)
    assert torch.equal(got, want)
    want.backward()
    got.backward()
    for p, q in zip(reference.parameters(), adapted.parameters(), strict=True):
        assert torch.equal(p.grad, q.grad)
    with pytest.raises(ValueError, match="already been applied"):
        apply_fused_execution(adapted)
    with pytest.raises(ValueError, match="FP32 master"):
        apply_fused_execution(_small_lm().bfloat16())


def test_fused_adapter_on_the_inline_layout_keeps_cpu_paths_and_state():
    """A model in the reference's own core layout (no seams) takes the module-level
    attachment; on the CPU every patched module and the wrapped forward run the original
    code: same loss and gradients bit for bit, same parameters and state dict."""
    from inline_layout_model import InlineLM
    from warpstate.config import WarpStateConfig

    from ops.fused_training import apply_fused_execution

    torch.manual_seed(574)
    reference = InlineLM(WarpStateConfig(vocab_size=32, d_model=16, n_heads=2, n_cores=1,
                                         logical_depth=2, ffn_hidden=24,
                                         gradient_checkpointing=False,
                                         loss_chunk_size=3)).train()
    adapted = copy.deepcopy(reference)
    keys, params = tuple(adapted.state_dict()), tuple(adapted.parameters())
    apply_fused_execution(adapted)
    assert tuple(adapted.state_dict()) == keys
    assert all(a is b for a, b in zip(params, adapted.parameters(), strict=True))
    # The module-level routes were installed (the core has no project / mix seams).
    core = adapted.cores[0]
    for module in (core.norm1, core.in_proj, core.out_proj, core.norm2, core.ffn, adapted.final_norm):
        assert "forward" in vars(module), module
    tokens = torch.randint(32, (2, 8))
    labels = torch.randint(32, (2, 8))
    labels.view(-1)[3:9] = -100
    with torch.autocast("cpu", dtype=torch.bfloat16):
        _, want = reference(tokens, labels, return_logits=False)
        _, got = adapted(tokens, labels, return_logits=False)
    assert torch.equal(got, want)
    want.backward()
    got.backward()
    for p, q in zip(reference.parameters(), adapted.parameters(), strict=True):
        assert torch.equal(p.grad, q.grad)
    assert torch.equal(adapted(tokens), reference(tokens))


def test_bf16_residuals_make_the_stream_bf16_only_under_autocast():
    from ops.residual_experiment import apply_bf16_residuals

    reference = _small_lm()
    model = copy.deepcopy(reference)
    keys, params = tuple(model.state_dict()), tuple(model.parameters())
    apply_bf16_residuals(model)
    assert tuple(model.state_dict()) == keys
    assert all(a is b for a, b in zip(params, model.parameters(), strict=True))
    tokens = torch.randint(32, (2, 8))
    # Outside autocast: the original forward, bit for bit.
    assert torch.equal(model(tokens), reference(tokens))
    seen = []
    hook = model.cores[0].register_forward_pre_hook(lambda m, args: seen.append(args[0].dtype))
    with torch.autocast("cpu", dtype=torch.bfloat16):
        _, loss = model(tokens, tokens, return_logits=False)
    hook.remove()
    assert seen and all(dtype == torch.bfloat16 for dtype in seen)
    loss.backward()
    # Gradients reach the FP32 masters through the casts.
    for name in ("embed.weight", "depth_scale", "depth_bias"):
        grad = model.get_parameter(name).grad
        assert grad is not None and grad.dtype == torch.float32
    with pytest.raises(ValueError, match="already been applied"):
        apply_bf16_residuals(model)
