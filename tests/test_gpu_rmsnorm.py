"""RMSNorm forward/backward on the GPU against the float64 oracle and Popcorn's reference at native dtype."""

import numpy as np
import pytest
import torch

from oracle import reference as O
from popcorn_amd import impls
from popcorn_amd.compat import references as R
from tests._parity import close_to_reference, gauge_ok, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _weights(cols, dtype, seed):
    return (1 + 0.1 * seeded((cols,), seed, torch.float32)).to(dtype)


def _run(shape, dtype, eps, with_bias, seed, wdtype=None):
    """x in `dtype`; weight, bias, the output and its cotangent in `wdtype` (default `dtype`)."""
    wdtype = dtype if wdtype is None else wdtype
    cols = shape[-1]
    x = seeded(shape, seed, dtype)
    w = _weights(cols, wdtype, seed + 1)
    bias = seeded((cols,), seed + 2, wdtype) if with_bias else None
    g = seeded(shape, 1000 + seed, wdtype)

    b64 = bias.double().numpy() if with_bias else None
    y64 = O.rms_norm(x.double().numpy(), w.double().numpy(), b64, eps)
    dx64, dw64, db64 = O.rms_norm_bwd(x.double().numpy(), w.double().numpy(), g.double().numpy(), eps)

    leaves = [x.clone().requires_grad_(), w.clone().requires_grad_()]
    if with_bias:
        leaves.append(bias.clone().requires_grad_())
    yr = R.rms_norm(leaves[0], leaves[1], leaves[2] if with_bias else None, eps)
    grads_r = torch.autograd.grad(yr, leaves, g)

    mine = [t.to(DEV).requires_grad_() for t in ([x, w] + ([bias] if with_bias else []))]
    ym = impls.rms_norm(mine[0], mine[1], mine[2] if with_bias else None, eps)
    grads_m = torch.autograd.grad(ym, mine, g.to(DEV))

    assert ym.shape == x.shape and ym.dtype == yr.dtype == wdtype
    assert [t.dtype for t in grads_m] == [t.dtype for t in grads_r]
    gauge_ok(ym, y64, yr, wdtype, "y")
    close_to_reference(ym, yr, "y", rounding=dtype)
    gauge_ok(grads_m[0], dx64, grads_r[0], dtype, "dx")
    gauge_ok(grads_m[1], dw64, grads_r[1], wdtype, "dw")
    if with_bias:
        gauge_ok(grads_m[2], db64, grads_r[2], wdtype, "db")


# (3000, 4096) and (9001, 256) run the persistent forward grid over several
# row strides with a ragged last stride (one row per block and four per block).
SHAPES = [(1, 64), (4, 4096), (3, 1000), (17, 8192), (2, 3, 512), (5, 16384), (2, 20000), (300, 128), (1, 7),
          (3, 3000), (2, 40000), (1030, 2048), (3000, 4096), (9001, 256)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_rmsnorm(shape, dtype):
    for seed in range(2):
        _run(shape, dtype, 1e-6, False, 10 * seed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("shape", [(4, 4096), (3, 1000), (64, 8192)], ids=str)
def test_rmsnorm_bias_eps(shape, dtype):
    _run(shape, dtype, 1e-5, True, 3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", [(4, 4096), (3, 1000), (17, 8192), (2, 3, 512), (1, 7), (5, 16384), (3000, 4096),
                                   (9001, 256)], ids=str)
def test_rmsnorm_16bit_x_fp32_weight(shape, dtype):
    """16-bit x with an fp32 weight (kernels/rms_norm.py:29): the normalized x rounds to x's dtype, the
    product promotes to fp32; dx has x's dtype, dweight fp32."""
    _run(shape, dtype, 1e-6, False, 5, wdtype=torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_rmsnorm_16bit_x_fp32_weight_and_bias(dtype):
    _run((64, 8192), dtype, 1e-5, True, 7, wdtype=torch.float32)


def test_rmsnorm_mixed_pair_outside_the_kernels_raises():
    x = torch.zeros(2, 64, dtype=torch.float32, device=DEV)
    with pytest.raises(TypeError, match="not supported"):
        impls.rms_norm(x, torch.ones(64, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(TypeError, match="bias dtype"):
        impls.rms_norm(x.bfloat16(), torch.ones(64, device=DEV), torch.ones(64, dtype=torch.bfloat16, device=DEV))


def test_rmsnorm_zero_rows_and_empty():
    x = torch.zeros(3, 256, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(256, dtype=torch.bfloat16, device=DEV)
    assert torch.count_nonzero(impls.rms_norm(x, w)).item() == 0
    e = torch.empty(0, 256, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    we = w.clone().requires_grad_()
    y = impls.rms_norm(e, we)
    (dw,) = torch.autograd.grad(y.sum(), (we,))
    assert y.shape == (0, 256) and torch.count_nonzero(dw).item() == 0


def test_rmsnorm_c1_full_size():
    """x [4096, 4096] fp32, w = 1 + 0.1 N(0,1), eps 1e-6, whole output vs oracle."""
    x = seeded((4096, 4096), 0, torch.float32)
    w = _weights(4096, torch.float32, 1)
    y64 = O.rms_norm(x.double().numpy(), w.double().numpy(), None, 1e-6)
    yr = R.rms_norm(x, w, None, 1e-6)
    with torch.no_grad():
        ym = impls.rms_norm(x.to(DEV), w.to(DEV), None, 1e-6)
    gauge_ok(ym, y64, yr, torch.float32, "y")
    close_to_reference(ym, yr, "y")


def test_rmsnorm_c4_full_size():
    """x, dy [65536, 8192] bf16 fwd+bwd. Whole y/dx against
    torch's native-dtype reference run on the GPU; dw against the float64
    oracle summed in row chunks; sampled rows of y/dx against the oracle."""
    rows, cols = 65536, 8192
    gen = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(rows, cols, generator=gen, device=DEV).to(torch.bfloat16)
    dy = torch.randn(rows, cols, generator=gen, device=DEV).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(cols, generator=gen, device=DEV)).to(torch.bfloat16)

    xm, wm = x.clone().requires_grad_(), w.clone().requires_grad_()
    ym = impls.rms_norm(xm, wm, None, 1e-6)
    dxm, dwm = torch.autograd.grad(ym, (xm, wm), dy)

    xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
    yr = R.rms_norm(xr, wr, None, 1e-6)
    dxr, dwr = torch.autograd.grad(yr, (xr, wr), dy)
    close_to_reference(ym, yr, "y")
    close_to_reference(dxm, dxr, "dx")
    del xr, wr, yr

    w64 = w.double().cpu().numpy()
    dw64 = np.zeros(cols)
    for r0 in range(0, rows, 8192):
        xs, gs = x[r0 : r0 + 8192].double().cpu().numpy(), dy[r0 : r0 + 8192].double().cpu().numpy()
        dw64 += O.rms_norm_bwd(xs, w64, gs, 1e-6)[1]
    gauge_ok(dwm, dw64, dwr, torch.bfloat16, "dw")

    sample = torch.tensor([0, 1, 4097, 65535])
    xs, gs = x[sample].double().cpu().numpy(), dy[sample].double().cpu().numpy()
    y_budget = R.rms_norm(x[sample].cpu(), w.cpu(), None, 1e-6)
    gauge_ok(ym[sample], O.rms_norm(xs, w64, None, 1e-6), y_budget, torch.bfloat16, "y rows")
    dx_rows = O.rms_norm_bwd(xs, w64, gs, 1e-6)[0]
    gauge_ok(dxm[sample], dx_rows, dxr[sample], torch.bfloat16, "dx rows")
