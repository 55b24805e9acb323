"""fp32 attention backward (the fp32 matrix-core kernels) against the float64 oracle.

Popcorn grids attention over float32 as well as the 16-bit dtypes
(bench/grid.py:43). Gradients are held to Popcorn's fp32 rule (err <= max(2 *
budget, 2e-5 * scale), the budget from torch autograd of the registered
reference in fp32 on the CPU), the same gauge as the 16-bit backward tests.
"""

import numpy as np
import pytest
import torch

from oracle import reference as O
from popcorn_amd import _lib, impls
from popcorn_amd.compat import references as R
from tests._parity import gauge_ok, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = torch.float32


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _grads(fn, inputs, do):
    leaves = [t.clone().requires_grad_() for t in inputs]
    out = fn(*leaves)
    return out, torch.autograd.grad(out, leaves, do)


def _math_attn(q, k, v, causal, scale):
    """softmax(q k^T scale + mask) v in fp32, one explicit product at a time: the reference for negative
    scales, where torch's CPU fp32 SDPA returns NaN rows."""
    b, s, hq, d = q.shape
    g = hq // k.shape[2]
    kk, vv = k.repeat_interleave(g, dim=2), v.repeat_interleave(g, dim=2)
    sc = torch.einsum("bqhd,bkhd->bhqk", q, kk) * (d**-0.5 if scale is None else scale)
    if causal:
        sc = sc.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    return torch.einsum("bhqk,bkhd->bqhd", torch.softmax(sc, dim=-1), vv)


def _check(batch, seq, hq, hkv, d, causal, scale, seed=0):
    q = seeded((batch, seq, hq, d), seed, F32)
    k = seeded((batch, seq, hkv, d), seed + 1, F32)
    v = seeded((batch, seq, hkv, d), seed + 2, F32)
    do = seeded((batch, seq, hq, d), seed + 3, F32)
    print(f"[attn bwd f32] b={batch} s={seq} hq={hq} hkv={hkv} d={d} causal={causal} scale={scale}", flush=True)
    truth = O.attention_bwd(*(t.double().numpy() for t in (q, k, v, do)), causal, scale)
    ref_fn = (lambda a, b, c: R.attn(a, b, c, causal, scale)) if scale is None or scale > 0 else \
        (lambda a, b, c: _math_attn(a, b, c, causal, scale))
    _, ref = _grads(ref_fn, (q, k, v), do)
    _, mine = _grads(lambda a, b, c: impls.attn(a, b, c, causal, scale), (q.to(DEV), k.to(DEV), v.to(DEV)),
                     do.to(DEV))
    for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
        assert got.shape == r.shape and got.dtype == F32
        gauge_ok(got, want, r, F32, f"{name} (seq {seq}, d {d}, causal {causal}, scale {scale})")


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq", [1, 17, 64, 130, 257])
def test_attn_bwd_f32_shapes(seq, causal, d):
    _check(2, seq, 8, 2, d, causal, None)


@pytest.mark.parametrize("d", [16, 40, 96, 120, 136, 192, 248])
def test_attn_bwd_f32_head_dims_laid_out_wider(d):
    """head_dim below the 64-, 128- or 256-dim layout: the dims past it read as zeros and are never stored
    (at 136 the second half of the dk/dv output dims is a block that stores nothing past 136)."""
    _check(1, 77, 4, 1, d, True, None, seed=4)


@pytest.mark.parametrize("heads", [(8, 8), (8, 1), (6, 2), (6, 1), (12, 2)], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_bwd_f32_groups(heads, causal):
    _check(2, 150, heads[0], heads[1], 64 if heads[0] % 3 == 0 else 128, causal, None, seed=11)


@pytest.mark.parametrize("heads", [(8, 1), (6, 2)], ids=str)
def test_attn_bwd_f32_wide_groups(heads):
    _check(2, 130, heads[0], heads[1], 256, True, None, seed=13)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("scale", [0.25, -0.3, 1e-3])
def test_attn_bwd_f32_scales(scale, d):
    """A negative scale negates q on load in the dq kernel and signs the exponent in the dk/dv kernel."""
    _check(1, 96, 4, 2, d, False, scale, seed=9)


def test_attn_bwd_f32_noncontiguous_inputs_and_cotangent():
    b, s, hq, hkv, d = 2, 130, 8, 2, 128
    packed = seeded((b, s, hq + 2 * hkv, d), 11, F32).to(DEV)
    do_full = seeded((b, s, 2 * hq, d), 12, F32).to(DEV)
    do = do_full[:, :, ::2]  # stride-2 heads
    q, k, v = packed[:, :, :hq], packed[:, :, hq:hq + hkv], packed[:, :, hq + hkv:]
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v)]
    mine = torch.autograd.grad(impls.attn(*leaves, True), leaves, do)
    dense = [t.contiguous().requires_grad_() for t in (q.detach(), k.detach(), v.detach())]
    again = torch.autograd.grad(impls.attn(*dense, True), dense, do.contiguous())
    for a, b_ in zip(mine, again):
        assert torch.equal(a, b_)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("total,segments", [(37, 1), (300, 3), (129, 129)])
def test_attn_varlen_bwd_f32(total, segments, causal, d):
    cu = R.cuts(torch.zeros(segments + 1, dtype=torch.int64), {"total": total}, torch.Generator().manual_seed(0))
    hq, hkv = 8, 2
    q = seeded((total, hq, d), 0, F32)
    k = seeded((total, hkv, d), 1, F32)
    v = seeded((total, hkv, d), 2, F32)
    do = seeded((total, hq, d), 3, F32)
    print(f"[attn bwd f32] varlen {cu.tolist()[:6]} causal={causal}", flush=True)
    truth = O.attention_varlen_bwd(*(t.double().numpy() for t in (q, k, v, do)), cu.numpy(), causal)
    _, ref = _grads(lambda a, b, c: R.attn_varlen(a, b, c, cu, causal), (q, k, v), do)
    _, mine = _grads(lambda a, b, c: impls.attn_varlen(a, b, c, cu.to(DEV), causal),
                     (q.to(DEV), k.to(DEV), v.to(DEV)), do.to(DEV))
    for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
        gauge_ok(got, want, r, F32, f"{name} (varlen {cu.tolist()[:6]}, causal {causal})")


def test_attn_bwd_f32_special_case_uniform_queries():
    """q = 0 and dO = 1 row-wise constant: P is uniform over the visible keys, so dV_j = sum over rows
    i >= j of 1 / (i + 1) (causal, per q head, summed over the group), and dS = P (dP - D) = 0 when every
    visible v_j . dO_i is the same; here v = 1 gives dP = D, so dQ = dK = 0 exactly up to rounding."""
    b, s, hq, hkv, d = 1, 300, 4, 2, 64
    q = torch.zeros(b, s, hq, d, device=DEV)
    k = seeded((b, s, hkv, d), 8, F32).to(DEV)
    v = torch.ones(b, s, hkv, d, device=DEV)
    do = torch.ones(b, s, hq, d, device=DEV)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    dq, dk, dv = torch.autograd.grad(impls.attn(*leaves, True), leaves, do)
    harmonic = torch.flip(torch.cumsum(torch.flip(1.0 / torch.arange(1, s + 1, dtype=torch.float64), [0]), 0), [0])
    expect = (hq // hkv) * harmonic.to(DEV)[None, :, None, None].expand(b, s, hkv, d)
    assert (dv.double() - expect).abs().max().item() < 2e-5
    assert dq.abs().max().item() < 2e-5 and dk.abs().max().item() < 2e-5


def _splits(ws_bytes, lse_n, rows, hkv, d):
    lse = -(-2 * lse_n * 4 // 256) * 256
    return (ws_bytes - lse) // (2 * rows * hkv * d * 4) if ws_bytes > lse else 1


@pytest.mark.parametrize("b,s,hq,hkv,d,causal,splits", [
    (4, 1024, 32, 16, 64, True, 1),    # 512 blocks: direct, two q heads per block
    (8, 1024, 32, 8, 128, False, 1),   # 512 blocks: direct, four q heads per block
    (4, 1024, 32, 8, 128, True, 2),    # 256 blocks: two splits of two q heads
    (8, 1024, 32, 8, 256, True, 1),    # 512 key blocks (1024 dk/dv blocks, two per 128 keys): direct
    (2, 1024, 16, 2, 192, False, 8),   # 32 key blocks, group 8: one q head per block
], ids=["direct-d64-causal", "direct-d128-full", "split2-d128-causal", "direct-d256-causal", "split8-d192-full"])
def test_attn_bwd_f32_dkdv_direct_and_partial_splits(b, s, hq, hkv, d, causal, splits):
    """Full-size grids on each dk/dv path; sampled (batch, kv group) slices against the float64 oracle (a kv
    group's gradients depend only on its own q heads, so a slice is an exact subproblem)."""
    lib = _lib.load()
    width = 64 if d <= 64 else (128 if d <= 128 else 256)
    assert _splits(lib.pk_attn_bwd_workspace(b, s, hq, hkv, d), b * hq * s, b * s, hkv, width) == splits
    print(f"[attn bwd f32] grid b={b} s={s} hq={hq} hkv={hkv} d={d} causal={causal} splits={splits}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(17)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV) for _ in range(2))
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    grads = torch.autograd.grad(impls.attn(*leaves, causal), leaves, do)
    group = hq // hkv
    for bi, g in [(0, 0), (b - 1, hkv - 1)]:
        heads = slice(g * group, (g + 1) * group)
        qs, ks, vs, dos = q[bi:bi + 1, :, heads], k[bi:bi + 1, :, g:g + 1], v[bi:bi + 1, :, g:g + 1], do[bi:bi + 1, :, heads]
        truth = O.attention_bwd(*(t.double().cpu().numpy() for t in (qs, ks, vs, dos)), causal, None)
        _, ref = _grads(lambda x, y, z: R.attn(x, y, z, causal, None), [t.cpu() for t in (qs, ks, vs)], dos.cpu())
        mine = (grads[0][bi:bi + 1, :, heads], grads[1][bi:bi + 1, :, g:g + 1], grads[2][bi:bi + 1, :, g:g + 1])
        for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
            gauge_ok(got, want, r, F32, f"{name} ({splits} split(s), batch {bi}, kv group {g})")


def test_attn_bwd_f32_long_causal_against_float64_on_device():
    """B=1, S=4096, Hq=8, Hkv=2, D=128 causal: one kv group's dq / dk / dv against float64 autograd, to the
    north star's fp32 tolerance scaled by the gradient's size."""
    b, s, hq, hkv, d = 1, 4096, 8, 2, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV) for _ in range(2))
    print("[attn bwd f32] long causal S=4096", flush=True)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    dq, dk, dv = torch.autograd.grad(impls.attn(*leaves, True), leaves, do)
    grp = 1  # kv head 1 and its q heads 4..7
    qh = q[0, :, 4 * grp:4 * grp + 4].double().permute(1, 0, 2).requires_grad_()
    kh = k[0, :, grp].double().requires_grad_()
    vh = v[0, :, grp].double().requires_grad_()
    z = (qh @ kh.T) * d**-0.5
    z = z.masked_fill(torch.ones(s, s, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
    o = torch.softmax(z, -1) @ vh
    gq, gk, gv = torch.autograd.grad(o, (qh, kh, vh), do[0, :, 4 * grp:4 * grp + 4].double().permute(1, 0, 2))
    for name, got, want in (("dq", dq[0, :, 4 * grp:4 * grp + 4].permute(1, 0, 2), gq), ("dk", dk[0, :, grp], gk),
                            ("dv", dv[0, :, grp], gv)):
        err = (got.double() - want).abs().max().item()
        scale = max(1.0, want.abs().max().item())
        assert err <= 1e-4 * scale, f"{name}: {err:.3e} vs {scale:.2f}"
