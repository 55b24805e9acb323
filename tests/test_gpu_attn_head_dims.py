"""Attention at every head_dim of Popcorn's grid (core/dims.py:74), forward and backward, on the GPU.

The kernels lay rows out at 32, 96 and 192 (16-bit), 64, 128 or 256 dims and
read zeros past the tensors' head_dim, so any multiple of 8 up to 256
is served forward and backward. Each case is graded against the float64 oracle
with Popcorn's pass rule (budget: the registered reference at native dtype, on
the CPU), and the layouts are checked against each other directly: a
head_dim-96 call (the 96-dim layouts) gives the same bits as the head_dim-128
kernels on the same rows zero-padded to 128.
"""

import numpy as np
import pytest
import torch

from oracle import reference as O
from popcorn_amd import impls
from popcorn_amd.compat import references as R
from tests._parity import gauge_ok, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
FWD_DIMS = [16, 32, 48, 80, 96, 192, 256]  # Popcorn's grid beyond the 64 and 128 the other files cover
BWD_DIMS = [16, 32, 48, 80, 96]


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _qkv(batch, seq, hq, hkv, d, dtype, seed):
    return (seeded((batch, seq, hq, d), seed, dtype), seeded((batch, seq, hkv, d), seed + 1, dtype),
            seeded((batch, seq, hkv, d), seed + 2, dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", FWD_DIMS)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq,hq,hkv", [(1, 8, 8), (77, 8, 2), (200, 8, 1)], ids=["s1-g1", "s77-g4", "s200-g8"])
def test_attn_forward_head_dims(seq, hq, hkv, causal, d, dtype):
    print(f"[head_dim fwd] d={d} seq={seq} hq={hq} hkv={hkv} causal={causal} {dtype}", flush=True)
    q, k, v = _qkv(2, seq, hq, hkv, d, dtype, seed=d)
    o64, lse64 = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal)
    with torch.no_grad():
        oref = R.attn(q, k, v, causal)
        om, lse = impls.attn_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), causal)
    assert om.shape == q.shape and om.dtype == dtype
    gauge_ok(om, o64, oref, dtype, f"o (d {d})")
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse64, rtol=0, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", BWD_DIMS)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq,hq,hkv", [(33, 8, 8), (150, 8, 2), (257, 8, 1)], ids=["s33-g1", "s150-g4", "s257-g8"])
def test_attn_backward_head_dims(seq, hq, hkv, causal, d, dtype):
    print(f"[head_dim bwd] d={d} seq={seq} hq={hq} hkv={hkv} causal={causal} {dtype}", flush=True)
    q, k, v = _qkv(1, seq, hq, hkv, d, dtype, seed=3 * d)
    do = seeded((1, seq, hq, d), 3 * d + 5, dtype)
    truth = O.attention_bwd(*(t.double().numpy() for t in (q, k, v, do)), causal)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    ref = torch.autograd.grad(R.attn(*leaves, causal), leaves, do)
    dev = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    mine = torch.autograd.grad(impls.attn(*dev, causal), dev, do.to(DEV))
    for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
        assert got.shape == r.shape and got.dtype == dtype
        gauge_ok(got, want, r, dtype, f"{name} (d {d})")


def test_attn_head_dim_96_is_the_128_kernel_on_zero_padded_rows():
    """Forward and backward bits of head_dim 96 equal those of head_dim 128 on inputs zero-padded
    to 128 (with the 96-dim scale), and the padded dims of the 128 call's gradients are zero: the
    96-dim layouts skip only products of zeros."""
    b, s, hq, hkv, d = 2, 190, 8, 2, 96
    q, k, v = (t.to(DEV) for t in _qkv(b, s, hq, hkv, d, torch.bfloat16, seed=21))
    do = seeded((b, s, hq, d), 25, torch.bfloat16).to(DEV)
    pad = lambda t: torch.nn.functional.pad(t, (0, 128 - d))  # noqa: E731
    scale = d**-0.5
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, True)
        o2, lse2 = impls.attn_with_lse(pad(q), pad(k), pad(v), True, scale)
    assert torch.equal(o, o2[..., :d]) and torch.equal(lse, lse2)
    assert torch.equal(o2[..., d:], torch.zeros_like(o2[..., d:]))
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    g96 = torch.autograd.grad(impls.attn(*leaves, True), leaves, do)
    leaves = [pad(t).requires_grad_() for t in (q, k, v)]
    g128 = torch.autograd.grad(impls.attn(*leaves, True, scale), leaves, pad(do))
    for a, b_ in zip(g96, g128):
        assert torch.equal(a, b_[..., :d])
        assert torch.equal(b_[..., d:], torch.zeros_like(b_[..., d:]))


@pytest.mark.parametrize("d", [16, 32, 80, 96, 192, 256])
def test_attn_varlen_head_dims(d):
    total, hq, hkv = 300, 8, 2
    cu = R.cuts(torch.zeros(4, dtype=torch.int64), {"total": total}, torch.Generator().manual_seed(d))
    q, k, v = (seeded((total, h, d), d + i, torch.bfloat16) for i, h in enumerate((hq, hkv, hkv)))
    o64, _ = O.attention_varlen(q.double().numpy(), k.double().numpy(), v.double().numpy(), cu.numpy(), True)
    with torch.no_grad():
        om = impls.attn_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), True)
    gauge_ok(om, o64, R.attn_varlen(q, k, v, cu, True), torch.bfloat16, f"varlen o (d {d})")
    if d <= 128:
        do = seeded((total, hq, d), d + 7, torch.bfloat16)
        truth = O.attention_varlen_bwd(*(t.double().numpy() for t in (q, k, v, do)), cu.numpy(), True)
        leaves = [t.clone().requires_grad_() for t in (q, k, v)]
        ref = torch.autograd.grad(R.attn_varlen(*leaves, cu, True), leaves, do)
        dev = [t.to(DEV).requires_grad_() for t in (q, k, v)]
        mine = torch.autograd.grad(impls.attn_varlen(*dev, cu.to(DEV), True), dev, do.to(DEV))
        for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
            gauge_ok(got, want, r, torch.bfloat16, f"varlen {name} (d {d})")


def test_attn_head_dim_256_at_c5_scale():
    """head_dim 256 (Gemma-2 attention) at B=1, S=4096, 16 q heads over 8 kv heads, causal: sampled rows
    against the float64 oracle."""
    B, S, HQ, HKV, D = 1, 4096, 16, 8, 256
    gen = torch.Generator(device=DEV).manual_seed(2)
    q, k, v = (torch.randn(B, S, h, D, generator=gen, device=DEV).to(torch.bfloat16) for h in (HQ, HKV, HKV))
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, True)
    assert torch.isfinite(o.float()).all()
    qc, kc, vc = (t.cpu() for t in (q, k, v))
    for row in (0, 1, 31, 32, 2047, 4095):
        for h in (0, 5, 15):
            kv = h // (HQ // HKV)
            s = (qc[0, row, h].double() @ kc[0, : row + 1, kv].double().T) * D**-0.5
            p = torch.softmax(s, -1)
            want = p @ vc[0, : row + 1, kv].double()
            assert (o[0, row, h].cpu().double() - want).abs().max().item() < 2e-2
            assert abs(lse[0, h, row].item() - torch.logsumexp(s, -1).item()) < 1e-3
