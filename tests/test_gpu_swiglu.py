"""SwiGLU on the GPU against the float64 oracle (truth) and Popcorn's reference at native dtype (budget)."""

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


def _case(shape, dtype, seed):
    a, b = seeded(shape, 2 * seed, dtype), seeded(shape, 2 * seed + 1, dtype)
    g = seeded(shape, 1000 + seed, dtype)
    return a, b, g


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", [(1,), (7,), (3, 1000), (5, 3, 333), (64, 4096), (128, 14336)], ids=str)
def test_swiglu_fwd_bwd(shape, dtype):
    for seed in range(3):
        a, b, g = _case(shape, dtype, seed)
        # truth: float64 oracle on the native-dtype inputs
        y64 = O.swiglu(a.double().numpy(), b.double().numpy())
        da64, db64 = O.swiglu_bwd(g.double().numpy(), a.double().numpy(), b.double().numpy())
        # budget: the reference at native dtype (CPU eager), with autograd
        ar, br = a.clone().requires_grad_(), b.clone().requires_grad_()
        yr = R.swiglu(ar, br)
        dar, dbr = torch.autograd.grad(yr, (ar, br), g)
        # ours
        am, bm = a.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
        ym = impls.swiglu(am, bm)
        dam, dbm = torch.autograd.grad(ym, (am, bm), g.to(DEV))
        assert ym.dtype == dtype and ym.shape == a.shape
        gauge_ok(ym, y64, yr, dtype, "y")
        gauge_ok(dam, da64, dar, dtype, "da")
        gauge_ok(dbm, db64, dbr, dtype, "db")
        close_to_reference(ym, yr, "y")


def test_swiglu_unaligned_views():
    """Offset views (not 16-byte aligned) take the scalar kernel and still agree."""
    base_a, base_b = seeded((4097,), 0, torch.bfloat16), seeded((4097,), 1, torch.bfloat16)
    a, b = base_a[1:], base_b[1:]
    ym = impls.swiglu(base_a.to(DEV)[1:], base_b.to(DEV)[1:])
    gauge_ok(ym, O.swiglu(a.double().numpy(), b.double().numpy()), R.swiglu(a, b), torch.bfloat16)


def test_swiglu_empty():
    a = torch.empty(0, 16, dtype=torch.bfloat16, device=DEV)
    assert impls.swiglu(a, a).shape == (0, 16)


def test_swiglu_c2_full_size():
    """a, b [16384, 14336] bf16. Whole output against the
    reference evaluated by torch on the GPU at native dtype (same rounding
    sequence), plus sampled rows against the float64 oracle."""
    shape = (16384, 14336)
    gen = torch.Generator(device=DEV).manual_seed(0)
    a = torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16)
    b = torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        ym = impls.swiglu(a, b)
        yr = R.swiglu(a, b)
    close_to_reference(ym, yr, "y")
    mismatch = (ym != yr).sum().item() / ym.numel()
    assert mismatch < 1e-3, f"{mismatch:.2e} of elements differ from torch's own bf16 rounding"
    rows = torch.tensor([0, 1, 8191, 16383])
    a64, b64 = a[rows].double().cpu().numpy(), b[rows].double().cpu().numpy()
    gauge_ok(ym[rows], O.swiglu(a64, b64), yr[rows], torch.bfloat16, "y rows")
    assert np.isfinite(ym.float().cpu().numpy()).all()
