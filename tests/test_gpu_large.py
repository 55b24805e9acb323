"""Tensors past 2^31 elements: 64-bit indexing in every streaming kernel.

An MI355X holds 288 GB, so a single activation of more than 2^31 elements (4.3 GB in bf16) is an
ordinary size. Each case builds such a tensor on the device, runs the kernel once, and checks
slices at the start, across the 2^31-element boundary and at the end against Popcorn's torch
reference on the CPU (the slices only, so the host does little work). A 32-bit index would wrap
at the boundary and write or read the wrong elements there.
"""

import pytest
import torch

from popcorn_amd import impls
from popcorn_amd.compat import references as R
from tests._parity import close_to_reference

pytestmark = pytest.mark.gpu
DEV = "cuda"
TWO31 = 2 ** 31


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    yield
    torch.cuda.empty_cache()


def _randn(n, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(n, generator=g, device=DEV, dtype=torch.float32).to(dtype) if n < 2 ** 28 else \
        torch.cat([torch.randn(min(2 ** 28, n - i), generator=g, device=DEV).to(dtype) for i in range(0, n, 2 ** 28)])


def test_swiglu_past_2_31_elements():
    n = TWO31 + 4096 + 3  # the odd tail also takes the scalar path
    a, b = _randn(n, torch.bfloat16, 1), _randn(n, torch.bfloat16, 2)
    with torch.no_grad():
        y = impls.swiglu(a, b)
    for lo, hi in ((0, 4096), (TWO31 - 2048, TWO31 + 2048), (n - 4096, n)):
        close_to_reference(y[lo:hi], R.swiglu(a[lo:hi].cpu(), b[lo:hi].cpu()), f"swiglu [{lo}, {hi})")
    del a, b, y


def test_rms_norm_forward_and_backward_past_2_31_elements():
    cols = 8192
    rows = TWO31 // cols + 3  # row TWO31 // cols starts at element 2^31
    x = _randn(rows * cols, torch.bfloat16, 3).view(rows, cols).requires_grad_()
    w = (1 + 0.1 * _randn(cols, torch.float32, 4)).bfloat16().requires_grad_()
    y = impls.rms_norm(x, w, None, 1e-6)
    gy = _randn(rows * cols, torch.bfloat16, 5).view(rows, cols)
    dx, _ = torch.autograd.grad(y, (x, w), gy)
    edge = TWO31 // cols
    for r0, r1 in ((0, 2), (edge - 2, edge + 2), (rows - 2, rows)):
        xs = x[r0:r1].detach().cpu().requires_grad_()
        ws = w.detach().cpu().requires_grad_()
        ys = R.rms_norm(xs, ws, None, 1e-6)
        close_to_reference(y[r0:r1], ys, f"rms_norm y rows [{r0}, {r1})")
        (dxs,) = torch.autograd.grad(ys, (xs,), gy[r0:r1].cpu())
        close_to_reference(dx[r0:r1], dxs, f"rms_norm dx rows [{r0}, {r1})")
    del x, y, gy, dx


def test_rotary_past_2_31_elements():
    b, s, h, d = 4, 65536 + 8, 64, 128  # 4 * 65544 positions * 8192 elements > 2^31
    x = _randn(b * s * h * d, torch.bfloat16, 6).view(b, s, h, d)
    ang = _randn(s * 64, torch.float32, 7).view(s, 64)
    cos, sin = ang.cos(), ang.sin()
    with torch.no_grad():
        y = impls.rotary_embedding(x, cos, sin, False)
    edge = TWO31 // (h * d)  # flat position whose first element is element 2^31
    eb, es = divmod(edge, s)
    for bi, s0, s1 in ((0, 0, 2), (eb, es - 1, es + 2), (b - 1, s - 2, s)):
        ref = R.rotary_embedding(x[bi:bi + 1, s0:s1].cpu(), cos[s0:s1].cpu(), sin[s0:s1].cpu(), False)
        close_to_reference(y[bi:bi + 1, s0:s1], ref, f"rotary batch {bi} positions [{s0}, {s1})")
    del x, y


def test_attn_forward_past_2_31_elements_of_q():
    """q [4097, 32, 128, 128] holds more than 2^31 elements (short sequences, many batch rows, 16 kv
    heads): batch rows 0 and 4096, whose first element is element 2^31, against the reference."""
    b, s, hq, hkv, d = 4097, 32, 128, 16, 128
    q = _randn(b * s * hq * d, torch.bfloat16, 11).view(b, s, hq, d)
    k = _randn(b * s * hkv * d, torch.bfloat16, 12).view(b, s, hkv, d)
    v = _randn(b * s * hkv * d, torch.bfloat16, 13).view(b, s, hkv, d)
    with torch.no_grad():
        o = impls.attn(q, k, v, True)
    assert (TWO31 // (s * hq * d)) * s * hq * d == TWO31
    for bi in (0, TWO31 // (s * hq * d)):
        ref = R.attn(q[bi:bi + 1].cpu(), k[bi:bi + 1].cpu(), v[bi:bi + 1].cpu(), True)
        close_to_reference(o[bi:bi + 1], ref, f"attn batch row {bi}")
    del q, k, v, o
