"""The allocation-free RMSNorm backward (``ws_rmsnorm_backward_static``) against the
workspace entry point it shares kernels with: the same dX and weight gradient bit for bit,
on two calls in a row (the second smaller, so stale partials of the first call would show),
plus the size limit and an oracle check of the first call."""
import pytest
import torch

from metrics import assert_bf16_close, assert_f32_close
from oracle import reference as oracle

pytestmark = pytest.mark.gpu


def _inputs(rows, d, seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn((rows, d), generator=gen).bfloat16()
    w = 1.0 + 0.1 * torch.randn((d,), generator=gen)
    dy = (torch.randn((rows, d), generator=gen) * 0.1).bfloat16()
    return x, w, dy


def _static(x, w, rstd, dy, eager):
    from ops import _hip

    rows, d = x.shape
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    _hip.call("ws_rmsnorm_backward_static", x.data_ptr(), w.data_ptr(), rstd.data_ptr(),
              dy.data_ptr(), dx.data_ptr(), dw.data_ptr(), rows, d, int(eager), _hip.stream(x))
    return dx, dw


def _workspace(x, w, rstd, dy, eager):
    from ops import _hip

    rows, d = x.shape
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    partial = torch.empty(_hip.query("ws_rmsnorm_backward_partial_floats", rows, d),
                          dtype=torch.float32, device=x.device)
    _hip.call("ws_rmsnorm_backward", x.data_ptr(), w.data_ptr(), rstd.data_ptr(),
              dy.data_ptr(), dx.data_ptr(), dw.data_ptr(), partial.data_ptr(), rows, d,
              int(eager), _hip.stream(x))
    return dx, dw


@pytest.mark.parametrize("eager", [True, False])
def test_static_scratch_matches_workspace_entry_point_twice(eager):
    # Each call smaller than the one before; the second takes the wide-row kernel.
    shapes = [(16384, 2048), (600, 6000), (1000, 1024)]
    for index, (rows, d) in enumerate(shapes):
        x, w, dy = _inputs(rows, d, 31 + index)
        gx, gw, gdy = x.cuda(), w.cuda(), dy.cuda()
        rstd = oracle.rms_rstd(x, 1e-6).cuda()
        got_dx, got_dw = _static(gx, gw, rstd, gdy, eager)
        want_dx, want_dw = _workspace(gx, gw, rstd, gdy, eager)
        torch.cuda.synchronize()
        assert torch.equal(got_dx, want_dx), (rows, d)
        assert torch.equal(got_dw, want_dw), (rows, d)
        if index == 2 and eager:
            xl = x.clone().requires_grad_(True)
            wl = w.clone().requires_grad_(True)
            y = oracle.rmsnorm(xl, wl, 1e-6)
            y.backward(dy)
            assert_bf16_close(got_dx, xl.grad, "static RMSNorm dX vs oracle")
            assert_f32_close(got_dw.cpu(), wl.grad, "static RMSNorm dW vs oracle")


def test_static_scratch_rejects_sizes_beyond_its_limit():
    from ops import _hip

    limit = _hip.query("ws_rmsnorm_backward_static_max_partial_floats")
    assert limit == 1 << 20
    rows, d = 32 * (limit // 2048 + 1), 2048  # ceil(rows / 32) * d > limit
    assert _hip.query("ws_rmsnorm_backward_partial_floats", rows, d) > limit
    x = torch.zeros((rows, d), dtype=torch.bfloat16, device="cuda")
    w = torch.ones(d, device="cuda")
    rstd = torch.ones(rows, device="cuda")
    with pytest.raises(RuntimeError, match="static scratch"):
        _static(x, w, rstd, x, True)
