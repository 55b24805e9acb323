"""Rotary embedding on the GPU against the float64 oracle and Popcorn's reference at native dtype."""

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


def tables(seq, half, theta=500000.0, dtype=torch.float32):
    """cos/sin [seq, half] for positions 0..seq-1, inv_freq_j = theta^(-2j/(2 half))."""
    inv = theta ** (-torch.arange(half, dtype=torch.float64) * 2 / (2 * half))
    ang = torch.arange(seq, dtype=torch.float64)[:, None] * inv[None, :]
    return ang.cos().to(dtype), ang.sin().to(dtype)


def _check(x, cos, sin, interleaved, seed=0):
    dtype = x.dtype
    g = seeded(tuple(x.shape), 500 + seed, dtype)
    y64 = O.rotary_embedding(x.double().numpy(), cos.double().numpy(), sin.double().numpy(), interleaved)
    dx64 = O.rotary_embedding_bwd(g.double().numpy(), cos.double().numpy(), sin.double().numpy(), interleaved)
    xr = x.clone().requires_grad_()
    yr = R.rotary_embedding(xr, cos, sin, interleaved)
    (dxr,) = torch.autograd.grad(yr, (xr,), g)
    xm = x.to(DEV).requires_grad_()
    ym = impls.rotary_embedding(xm, cos.to(DEV), sin.to(DEV), interleaved)
    (dxm,) = torch.autograd.grad(ym, (xm,), g.to(DEV))
    assert ym.shape == x.shape and ym.dtype == dtype
    gauge_ok(ym, y64, yr, dtype, "y")
    gauge_ok(dxm, dx64, dxr, dtype, "dx")
    close_to_reference(ym, yr, "y")
    return ym, yr


CASES = [
    # (batch, seq, heads, head_dim, half)
    (2, 16, 4, 128, 64),
    (1, 33, 3, 64, 32),
    (2, 8, 2, 128, 32),  # partial rotary, passthrough tail
    (1, 5, 2, 8, 3),  # odd half -> scalar path
    (1, 7, 1, 10, 4),  # passthrough width 2
    (3, 4, 8, 64, 16),
]


@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "gptj"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=str)
def test_rotary(case, dtype, interleaved):
    batch, seq, heads, head_dim, half = case
    x = seeded((batch, seq, heads, head_dim), 1, dtype)
    # Popcorn's harness draws cos/sin as N(0,1) like every other float input
    cos, sin = seeded((seq, half), 2, dtype), seeded((seq, half), 3, dtype)
    _check(x, cos, sin, interleaved)
    # and real unit tables in fp32
    c32, s32 = tables(seq, half)
    _check(x, c32, s32, interleaved, seed=1)


def test_rotary_strided_view_and_inplace():
    """q sliced from a packed qkv buffer (non-contiguous heads) and the in-place variant."""
    b, s, h, d = 2, 64, 4, 128
    qkv = seeded((b, s, 3 * h, d), 7, torch.bfloat16)
    cos, sin = tables(s, d // 2)
    q = qkv[:, :, :h]
    ym, yr = _check(q, cos, sin, False)
    dev = qkv.to(DEV)
    qd = dev[:, :, :h]
    out = impls.rotary_embedding(qd, cos.to(DEV), sin.to(DEV))
    assert torch.equal(out.cpu(), ym.cpu())
    with torch.no_grad():
        impls.rotary_embedding_(qd, cos.to(DEV), sin.to(DEV))
    assert torch.equal(qd.cpu(), ym.cpu())
    assert torch.equal(dev[:, :, h:].cpu(), qkv[:, :, h:])  # k/v parts untouched


def test_rotary_c3_full_size():
    """q [8,4096,32,128], k [8,4096,8,128] bf16, fp32 tables
    (theta 500000). The kernel performs the reference's fp32 op sequence, so it
    equals the reference evaluated by torch on the GPU bit for bit; sampled
    positions are also checked against the float64 oracle."""
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(8, 4096, 32, 128, generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn(8, 4096, 8, 128, generator=gen, device=DEV).to(torch.bfloat16)
    cos, sin = tables(4096, 64)
    cos, sin = cos.to(DEV), sin.to(DEV)
    with torch.no_grad():
        for x in (q, k):
            ym = impls.rotary_embedding(x, cos, sin)
            yr = R.rotary_embedding(x, cos, sin)
            assert torch.equal(ym, yr)
            pos = [0, 1, 2047, 4095]
            xs = x[:, pos].double().cpu().numpy()
            y64 = O.rotary_embedding(xs, cos[pos].double().cpu().numpy(), sin[pos].double().cpu().numpy())
            gauge_ok(ym[:, pos], y64, yr[:, pos], torch.bfloat16, "y positions")
            impls.rotary_embedding_(x, cos, sin)  # in place: same values
            assert torch.equal(x, ym)
