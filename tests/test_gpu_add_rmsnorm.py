"""Residual add + RMSNorm on the GPU against the float64 oracle and Popcorn's reference at native dtype."""

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


def _run(shape, dtype, eps, offset, seed, with_ds=True, wdtype=None):
    """x, residual and s in `dtype`; weight, y and y's cotangent in `wdtype` (default `dtype`)."""
    wdtype = dtype if wdtype is None else wdtype
    cols = shape[-1]
    x = seeded(shape, seed, dtype)
    res = seeded(shape, seed + 1, dtype)
    w = (1 + 0.1 * seeded((cols,), seed + 2, torch.float32)).to(wdtype)
    dy = seeded(shape, 1000 + seed, wdtype)
    ds = seeded(shape, 2000 + seed, dtype) if with_ds else None

    n64 = [t.double().numpy() for t in (x, res, w, dy)]
    y64, s64 = O.add_rms_norm(n64[0], n64[1], n64[2], eps, offset)
    dx64, dres64, dw64 = O.add_rms_norm_bwd(*n64, ds.double().numpy() if with_ds else None, eps, offset)

    leaves = [t.clone().requires_grad_() for t in (x, res, w)]
    yr, sr = R.add_rms_norm(*leaves, eps, offset)
    outs, cots = ([yr, sr], [dy, ds]) if with_ds else ([yr], [dy])
    grads_r = torch.autograd.grad(outs, leaves, cots)

    mine = [t.to(DEV).requires_grad_() for t in (x, res, w)]
    ym, sm = impls.add_rms_norm(*mine, eps, offset)
    outs_m, cots_m = ([ym, sm], [dy.to(DEV), ds.to(DEV)]) if with_ds else ([ym], [dy.to(DEV)])
    grads_m = torch.autograd.grad(outs_m, mine, cots_m)

    assert ym.shape == x.shape and ym.dtype == yr.dtype == wdtype and sm.shape == x.shape and sm.dtype == dtype
    assert [t.dtype for t in grads_m] == [t.dtype for t in grads_r] == [dtype, dtype, wdtype]
    # s is torch's own add at the native dtype: bit for bit
    assert torch.equal(sm.cpu(), (x + res)), "s differs from x + residual"
    gauge_ok(ym, y64, yr, wdtype, "y")
    close_to_reference(ym, yr, "y", rounding=dtype)
    gauge_ok(sm, s64, sr, dtype, "s")
    for got, truth, ref, name, dt in zip(grads_m, (dx64, dres64, dw64), grads_r, ("dx", "dresidual", "dweight"),
                                         (dtype, dtype, wdtype)):
        gauge_ok(got, truth, ref, dt, name)
    assert torch.equal(grads_m[0], grads_m[1]), "x and residual must receive the same gradient"


# (3000, 4096) and (9001, 256) run the persistent forward grid over several
# strides; (3, 1000) and (1, 7) widths take the any-width kernels.
SHAPES = [(1, 64), (4, 4096), (3, 1000), (17, 8192), (2, 3, 512), (300, 128), (1, 7), (1030, 2048), (3000, 4096),
          (9001, 256)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_add_rms_norm(shape, dtype):
    _run(shape, dtype, 1e-6, 0.0, 3)
    _run(shape, dtype, 1e-5, 1.0, 5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", [(1, 64), (4, 4096), (3, 1000), (17, 8192), (1, 7), (1030, 2048), (9001, 256)],
                         ids=str)
def test_add_rms_norm_16bit_x_fp32_weight(shape, dtype):
    """Autocast's mix: 16-bit x and residual with an fp32 weight; y promotes to fp32, s keeps x's dtype."""
    _run(shape, dtype, 1e-6, 0.0, 21, wdtype=torch.float32)
    _run(shape, dtype, 1e-5, 1.0, 23, wdtype=torch.float32)
    _run(shape, dtype, 1e-6, 1.0, 25, with_ds=False, wdtype=torch.float32)


def test_add_rms_norm_mixed_pairs_outside_the_kernels_raise():
    x = torch.ones(2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(TypeError):
        impls.add_rms_norm(x, x.float(), torch.ones(64, device=DEV))  # residual of another dtype
    with pytest.raises(TypeError):
        impls.add_rms_norm(x, x, torch.ones(64, dtype=torch.float16, device=DEV))  # bf16 x, fp16 weight


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_add_rms_norm_only_y_used(dtype):
    """No gradient reaches s directly (ds = None in the backward)."""
    _run((64, 8192), dtype, 1e-6, 1.0, 7, with_ds=False)


def test_add_rms_norm_only_s_used():
    """Only the residual stream is used downstream: d(x) = d(residual) = ds and dweight = 0."""
    x = seeded((8, 256), 11, torch.bfloat16).to(DEV).requires_grad_()
    res = seeded((8, 256), 12, torch.bfloat16).to(DEV).requires_grad_()
    w = torch.ones(256, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    _, s = impls.add_rms_norm(x, res, w)
    ds = seeded((8, 256), 13, torch.bfloat16).to(DEV)
    gx, gr, gw = torch.autograd.grad(s, (x, res, w), ds)
    assert torch.equal(gx, ds) and torch.equal(gr, ds) and torch.count_nonzero(gw).item() == 0


def test_add_rms_norm_large_rows_bf16():
    """A C4-sized call (65536 x 8192 bf16): sampled rows of y / s / grads against the oracle."""
    rows, cols = 65536, 8192
    gen = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(rows, cols, generator=gen, device=DEV).to(torch.bfloat16)
    res = torch.randn(rows, cols, generator=gen, device=DEV).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(cols, generator=gen, device=DEV)).to(torch.bfloat16)
    dy = torch.randn(rows, cols, generator=gen, device=DEV).to(torch.bfloat16)
    xm, rm, wm = (t.clone().requires_grad_() for t in (x, res, w))
    ym, sm = impls.add_rms_norm(xm, rm, wm, 1e-6, 1.0)
    dxm, _, dwm = torch.autograd.grad(ym, (xm, rm, wm), dy)
    assert torch.equal(sm, x + res)
    pick = np.array([0, 1, 4095, 4096, 32768, 65535])
    xs, rs, ws, dys = (t.double().cpu().numpy() for t in (x[pick], res[pick], w, dy[pick]))
    y64, _ = O.add_rms_norm(xs, rs, ws, 1e-6, 1.0)
    dx64, _, _ = O.add_rms_norm_bwd(xs, rs, ws, dys, None, 1e-6, 1.0)
    assert np.abs(ym[pick].detach().double().cpu().numpy() - y64).max() < 2e-2 * max(1.0, np.abs(y64).max())
    assert np.abs(dxm[pick].double().cpu().numpy() - dx64).max() < 2e-2 * max(1.0, np.abs(dx64).max())
    # dweight over all rows, float64 from the kernel's own saved s in row chunks
    s64 = sm.detach().double()
    r = torch.rsqrt(s64.square().mean(-1, keepdim=True) + 1e-6)
    dw64 = (dy.double() * s64 * r).sum(0)
    rel = ((dwm.double() - dw64).abs().max() / dw64.abs().max()).item()
    assert rel < 1e-2, rel
