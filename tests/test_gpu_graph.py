"""The hot path under HIP graph capture.

The library launches kernels only: no allocation, memset or synchronisation happens inside
an entry point, and every scratch buffer comes from the caller. A layer step's forward and
backward therefore capture into one graph. The graph is replayed several times with eager
work and synchronisations between replays. Every replay must reproduce the eager step bit
for bit: the kernels are deterministic, and the split-K and stream-K reductions sum in a
fixed order.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

M, D, H, NQKV, GATE = 512, 256, 384, 768, (512, 640)


def _inputs():
    g = torch.Generator().manual_seed(11)

    def bf(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).bfloat16().cuda()

    return {
        "x": bf(M, D), "norm_w": (1 + 0.1 * torch.randn(D, generator=g)).float().cuda(),
        "w_qkv": bf(NQKV, D, s=0.05), "mlp_x": bf(M, D), "w_upgate": bf(2 * H, D, s=0.05),
        "w_down": bf(D, H, s=0.05), "residual": bf(M, D), "dy": bf(M, D),
        "dqkv": bf(M, NQKV),
        "g_qkv0": (torch.randn(NQKV, D, generator=g) * 1e-4).cuda(),
        "g_down0": (torch.randn(D, H, generator=g) * 1e-4).cuda(),
        "g_upgate0": (torch.randn(2 * H, D, generator=g) * 1e-4).cuda(),
    }


def _step(t, g_qkv, g_down, g_upgate):
    """One layer step of the hot path: forward projections, then their backward with FP32
    weight-gradient accumulation into the given buffers."""
    from ops.fused_execution import (mm, mm_accumulate_, residual_mm, rmsnorm_gate_mm,
                                     rmsnorm_gate_mm_backward, swiglu_backward_mm)
    from ops.matmul_epilogue import launch_swiglu_mm

    normed = torch.empty_like(t["x"])
    qkv, rstd = rmsnorm_gate_mm(t["x"], t["norm_w"], 1e-6, t["w_qkv"], GATE, normed=normed)
    packed, act = launch_swiglu_mm(t["mlp_x"], t["w_upgate"].T, "tiled", (128, 128, 32, 8, 3),
                                   True)
    down = residual_mm(act, t["w_down"], t["residual"])
    dpacked = swiglu_backward_mm(t["dy"], t["w_down"], packed, True)
    dx_mlp = mm(dpacked, t["w_upgate"])
    mm_accumulate_(g_down, t["dy"].T, act, True)
    mm_accumulate_(g_upgate, dpacked.T, t["mlp_x"], True)
    dx_qkv, dnorm = rmsnorm_gate_mm_backward(t["x"], t["norm_w"], rstd, normed, t["w_qkv"],
                                             GATE, qkv, t["dqkv"], g_qkv, True, False)
    return [qkv, rstd, normed, packed, act, down, dpacked, dx_mlp, dx_qkv, dnorm]


def test_layer_step_replays_bitwise_under_graph_capture():
    t = _inputs()
    grads = [t["g_qkv0"].clone(), t["g_down0"].clone(), t["g_upgate0"].clone()]
    eager = [o.clone() for o in _step(t, *grads)]
    eager_grads = [g.clone() for g in grads]
    torch.cuda.synchronize()

    for g, g0 in zip(grads, (t["g_qkv0"], t["g_down0"], t["g_upgate0"])):
        g.copy_(g0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(t, *grads)
    torch.cuda.synchronize()

    scratch = torch.randn(1024, 1024, device="cuda")
    for replay in range(3):
        # Eager work and a reset of the in-place accumulators between replays.
        scratch = scratch @ scratch.T.contiguous() / 1024
        for g, g0 in zip(grads, (t["g_qkv0"], t["g_down0"], t["g_upgate0"])):
            g.copy_(g0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {replay}: output {i} differs from the eager step"
        for i, (g, e) in enumerate(zip(grads, eager_grads)):
            assert torch.equal(g, e), f"replay {replay}: weight gradient {i} differs"


@pytest.mark.parametrize("mode", ["two_pass", "fused"])
def test_lm_head_cross_entropy_replays_bitwise_under_graph_capture(mode):
    """The LM-head loss and its gradients captured once and replayed: every replay equals the
    eager step bit for bit. For the fused loss the upstream gradient changes between replays
    (1.0, 0.75, 1.0): the backward's choice between scaling the unit gradients and the
    two-pass recompute is made on the device, so one captured graph serves both."""
    from ops.fused_execution import (CrossEntropyState, linear_cross_entropy_backward,
                                     linear_cross_entropy_forward)

    rows, d, vocab = 512, 256, 4096
    g = torch.Generator().manual_seed(5)
    hidden = torch.randn(rows, d, generator=g).bfloat16().cuda()
    weight = (torch.randn(vocab, d, generator=g) * 0.05).bfloat16().cuda()
    targets = torch.randint(0, vocab, (rows,), generator=g)
    targets[::7] = -100
    targets = targets.cuda()
    grad_mean = torch.ones((), device="cuda")
    wgrad0 = (torch.randn(vocab, d, generator=g) * 1e-4).cuda()
    fused = mode == "fused"
    state = CrossEntropyState(rows, vocab, hidden.device, d=d, fused=fused, weight_grad=fused)
    dh = torch.empty(rows, d, dtype=torch.bfloat16, device="cuda")
    wgrad = wgrad0.clone()

    def step():
        linear_cross_entropy_forward(hidden, weight, targets, state)
        linear_cross_entropy_backward(hidden, weight, targets, state, grad_mean, out=dh,
                                      weight_grad=wgrad)

    grads = (1.0, 0.75, 1.0) if fused else (1.0, 1.0, 1.0)
    eager = {}
    for value in sorted(set(grads)):
        grad_mean.fill_(value)
        wgrad.copy_(wgrad0)
        step()
        torch.cuda.synchronize()
        eager[value] = [state.loss.clone(), state.lse.clone(), state.mean.clone(),
                        state.count.clone(), dh.clone(), wgrad.clone()]
    wgrad.copy_(wgrad0)
    grad_mean.fill_(1.0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for replay, value in enumerate(grads):
        state.loss.zero_()
        dh.zero_()
        wgrad.copy_(wgrad0)
        grad_mean.fill_(value)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [state.loss, state.lse, state.mean, state.count, dh, wgrad]
        for i, (o, e) in enumerate(zip(got, eager[value])):
            assert torch.equal(o, e), f"replay {replay} (grad {value}): output {i} differs"


@pytest.mark.parametrize("m,n,k", [(16384, 11264, 2048), (16384, 9216, 2048), (512, 768, 256)])
def test_input_gradient_gemm_replays_bitwise_under_graph_capture(m, n, k):
    """dgrad_mm (the weight transpose, then this library's GEMM) captured once at the
    layer's shapes and replayed three times with other work and a cleared output between
    replays: every replay equals the eager call bit for bit."""
    from ops.fused_execution import dgrad_mm

    g = torch.Generator().manual_seed(m + n)
    grad = torch.randn(m, n, generator=g).bfloat16().cuda()
    weight = (torch.randn(n, k, generator=g) * 0.05).bfloat16().cuda()
    eager = dgrad_mm(grad, weight).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = dgrad_mm(grad, weight)
    torch.cuda.synchronize()
    scratch = torch.randn(2048, 2048, device="cuda").bfloat16()
    for replay in range(3):
        out.zero_()
        scratch = torch.mm(scratch, scratch.T.contiguous()) / 2048
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {replay} differs from the eager call"
