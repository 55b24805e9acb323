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


def test_attn_forward_and_backward_past_2_31_elements_of_q():
    """q [4097, 32, 128, 128] holds more than 2^31 elements (short sequences, many batch rows, 16 kv
    heads): batch rows 0 and 4096, whose first element is element 2^31, against the reference,
    forward and gradients."""
    b, s, hq, hkv, d = 4097, 32, 128, 16, 128
    q = _randn(b * s * hq * d, torch.bfloat16, 11).view(b, s, hq, d).requires_grad_()
    k = _randn(b * s * hkv * d, torch.bfloat16, 12).view(b, s, hkv, d).requires_grad_()
    v = _randn(b * s * hkv * d, torch.bfloat16, 13).view(b, s, hkv, d).requires_grad_()
    o = impls.attn(q, k, v, True)
    go = _randn(b * s * hq * d, torch.bfloat16, 25).view(b, s, hq, d)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), go)
    assert (TWO31 // (s * hq * d)) * s * hq * d == TWO31
    for bi in (0, TWO31 // (s * hq * d)):
        leaves = [t[bi:bi + 1].detach().cpu().float().requires_grad_() for t in (q, k, v)]
        ref = R.attn(*leaves, True)  # fp32 on the CPU: the reference's gradients without bf16 products
        close_to_reference(o[bi:bi + 1], ref.bfloat16(), f"attn o, batch row {bi}")
        grads = torch.autograd.grad(ref, leaves, go[bi:bi + 1].cpu().float())
        for name, mine, want in zip(("dq", "dk", "dv"), (dq, dk, dv), grads):
            close_to_reference(mine[bi:bi + 1], want.bfloat16(), f"attn {name}, batch row {bi}")
    del q, k, v, o, go, dq, dk, dv


def test_attn_varlen_past_2_31_elements_of_q():
    """Packed q [257 * 512 tokens, 128 heads, 128] (more than 2^31 elements) in sequences of 512:
    the sequence holding element 2^31 and the last one against the reference."""
    seq, n = 512, 257
    total = seq * n
    hq, hkv, d = 128, 8, 128
    assert total * hq * d > TWO31
    q = _randn(total * hq * d, torch.bfloat16, 26).view(total, hq, d)
    k = _randn(total * hkv * d, torch.bfloat16, 27).view(total, hkv, d)
    v = _randn(total * hkv * d, torch.bfloat16, 28).view(total, hkv, d)
    cu = torch.arange(0, total + 1, seq, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        o = impls.attn_varlen(q, k, v, cu, True)
    for i in (TWO31 // (hq * d) // seq, n - 1):
        lo, hi = i * seq, (i + 1) * seq
        ref = R.attn(q[None, lo:hi].cpu(), k[None, lo:hi].cpu(), v[None, lo:hi].cpu(), True)[0]
        close_to_reference(o[lo:hi], ref, f"attn_varlen sequence {i}")
    del q, k, v, o


def test_add_rms_norm_past_2_31_elements():
    cols = 8192
    rows = TWO31 // cols + 3
    x = _randn(rows * cols, torch.bfloat16, 14).view(rows, cols).requires_grad_()
    r = _randn(rows * cols, torch.bfloat16, 15).view(rows, cols).requires_grad_()
    w = (1 + 0.1 * _randn(cols, torch.float32, 16)).bfloat16()
    y, s = impls.add_rms_norm(x, r, w, 1e-6, 0.0)
    gy = _randn(rows * cols, torch.bfloat16, 17).view(rows, cols)
    (dx,) = torch.autograd.grad(y, (x,), gy)
    edge = TWO31 // cols
    for r0, r1 in ((0, 2), (edge - 2, edge + 2), (rows - 2, rows)):
        xs, rs = (t[r0:r1].detach().cpu().requires_grad_() for t in (x, r))
        ys, ss = R.add_rms_norm(xs, rs, w.cpu(), 1e-6, 0.0)
        close_to_reference(s[r0:r1], ss, f"add_rms_norm s rows [{r0}, {r1})")
        close_to_reference(y[r0:r1], ys, f"add_rms_norm y rows [{r0}, {r1})")
        (dxs,) = torch.autograd.grad(ys, (xs,), gy[r0:r1].cpu())
        close_to_reference(dx[r0:r1], dxs, f"add_rms_norm dx rows [{r0}, {r1})")
    del x, r, y, s, gy, dx


def _head_rows_across_the_boundary(heads, seq, d):
    """(batch, head, first position) of a 10-row window of q [b, heads, seq, d] around element 2^31."""
    row = TWO31 // d
    bh, pos = divmod(row, seq)
    return bh // heads, bh % heads, pos - 5


@pytest.mark.parametrize("fused_norm", [False, True], ids=["rope", "qk_norm_rope"])
def test_rope_and_qk_norm_rope_past_2_31_elements(fused_norm):
    b, hq, hkv, s, d = 4, 64, 8, 65536 + 8, 128  # q holds 4 * 64 * 65544 * 128 > 2^31 elements
    q = _randn(b * hq * s * d, torch.bfloat16, 18).view(b, hq, s, d).requires_grad_()
    k = _randn(b * hkv * s * d, torch.bfloat16, 19).view(b, hkv, s, d).requires_grad_()
    ang = _randn(s * d // 2, torch.float32, 20).view(1, s, d // 2).repeat(1, 1, 2)
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    qw = (1 + 0.1 * _randn(d, torch.float32, 21)).bfloat16()
    kw = (1 + 0.1 * _randn(d, torch.float32, 22)).bfloat16()
    if fused_norm:
        yq, yk = impls.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6)
    else:
        yq, yk = impls.rope(q, k, cos, sin)
    gq = _randn(b * hq * s * d, torch.bfloat16, 23).view(b, hq, s, d)
    gk = _randn(b * hkv * s * d, torch.bfloat16, 24).view(b, hkv, s, d)
    dq, dk = torch.autograd.grad((yq, yk), (q, k), (gq, gk))
    eb, eh, p0 = _head_rows_across_the_boundary(hq, s, d)
    for bi, hi, s0 in ((0, 0, 0), (eb, eh, p0), (b - 1, hq - 1, s - 10)):
        qs = q[bi:bi + 1, hi:hi + 1, s0:s0 + 10].detach().cpu().requires_grad_()
        ks = k[bi:bi + 1, hi % hkv:hi % hkv + 1, s0:s0 + 10].detach().cpu().requires_grad_()
        cs, sn = cos[:, s0:s0 + 10].cpu(), sin[:, s0:s0 + 10].cpu()
        if fused_norm:
            rq, rk = R.qk_norm_rope(qs, ks, qw.cpu(), kw.cpu(), cs, sn, 1e-6)
        else:
            rq, rk = R.rope(qs, ks, cs, sn)
        what = f"{'qk_norm_rope' if fused_norm else 'rope'} q[{bi}, {hi}, {s0}:{s0 + 10}]"
        close_to_reference(yq[bi:bi + 1, hi:hi + 1, s0:s0 + 10], rq, what)
        dqs, _ = torch.autograd.grad((rq, rk), (qs, ks), (gq[bi:bi + 1, hi:hi + 1, s0:s0 + 10].cpu(),
                                                          gk[bi:bi + 1, hi % hkv:hi % hkv + 1, s0:s0 + 10].cpu()))
        close_to_reference(dq[bi:bi + 1, hi:hi + 1, s0:s0 + 10], dqs, "d" + what)
    del q, k, yq, yk, gq, gk, dq, dk
