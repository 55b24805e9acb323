"""Attention backward (dense and packed) on the GPU against the float64 oracle and Popcorn's reference.

The native-dtype reference gradients come from torch autograd of the
registered reference on the CPU (its GPU path would issue batched 16-bit
products on transposed views).
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


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _grads(fn, inputs, do):
    leaves = [t.clone().requires_grad_() for t in inputs]
    out = fn(*leaves)
    return out, torch.autograd.grad(out, leaves, do)


def _check(batch, seq, hq, hkv, d, causal, scale, dtype, seed=0):
    q = seeded((batch, seq, hq, d), seed, dtype)
    k = seeded((batch, seq, hkv, d), seed + 1, dtype)
    v = seeded((batch, seq, hkv, d), seed + 2, dtype)
    do = seeded((batch, seq, hq, d), seed + 3, dtype)
    truth = O.attention_bwd(*(t.double().numpy() for t in (q, k, v, do)), causal, scale)
    _, ref = _grads(lambda a, b, c: R.attn(a, b, c, causal, scale), (q, k, v), do)
    om, mine = _grads(lambda a, b, c: impls.attn(a, b, c, causal, scale), (q.to(DEV), k.to(DEV), v.to(DEV)),
                      do.to(DEV))
    o64, _ = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal, scale)
    gauge_ok(om, o64, R.attn(q, k, v, causal, scale), dtype, "o")
    for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
        assert got.shape == r.shape and got.dtype == dtype
        gauge_ok(got, want, r, dtype, f"{name} (seq {seq}, d {d}, causal {causal}, scale {scale})")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq", [1, 17, 64, 130, 257])
def test_attn_bwd_shapes(seq, causal, d, dtype):
    _check(2, seq, 8, 2, d, causal, None, dtype)


@pytest.mark.parametrize("heads", [(6, 2), (6, 1), (12, 2)], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_bwd_uneven_group_sizes(heads, causal):
    """Group sizes 3 and 6: the dq kernel's blocks hold one or two q heads over several row groups."""
    _check(2, 150, heads[0], heads[1], 64, causal, None, torch.bfloat16, seed=11)


@pytest.mark.parametrize("hkv", [8, 4, 1])
@pytest.mark.parametrize("scale", [None, 0.25])
def test_attn_bwd_groups_and_scale(hkv, scale):
    _check(1, 200, 8, hkv, 128, True, scale, torch.bfloat16, seed=7)


def test_attn_bwd_negative_scale():
    """A negative scale negates q on load in the kernels: dk uses |scale|, dq the signed one."""
    _check(1, 96, 4, 2, 128, False, -0.3, torch.bfloat16, seed=9)


def test_attn_bwd_noncontiguous_inputs_and_cotangent():
    b, s, hq, hkv, d = 2, 130, 8, 2, 128
    packed = seeded((b, s, hq + 2 * hkv, d), 11, torch.bfloat16).to(DEV)
    do_full = seeded((b, s, 2 * hq, d), 12, torch.bfloat16).to(DEV)
    do = do_full[:, :, ::2]  # stride-2 heads
    q, k, v = packed[:, :, :hq], packed[:, :, hq:hq + hkv], packed[:, :, hq + hkv:]
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v)]
    mine = torch.autograd.grad(impls.attn(*leaves, True), leaves, do)
    dense = [t.contiguous().requires_grad_() for t in (q.detach(), k.detach(), v.detach())]
    again = torch.autograd.grad(impls.attn(*dense, True), dense, do.contiguous())
    for a, b_ in zip(mine, again):
        assert torch.equal(a, b_)


def _check_varlen(total, segments, d, causal, dtype, seed=0):
    cu = R.cuts(torch.zeros(segments + 1, dtype=torch.int64), {"total": total}, torch.Generator().manual_seed(seed))
    hq, hkv = 8, 2
    q = seeded((total, hq, d), seed, dtype)
    k = seeded((total, hkv, d), seed + 1, dtype)
    v = seeded((total, hkv, d), seed + 2, dtype)
    do = seeded((total, hq, d), seed + 3, dtype)
    truth = O.attention_varlen_bwd(*(t.double().numpy() for t in (q, k, v, do)), cu.numpy(), causal)
    _, ref = _grads(lambda a, b, c: R.attn_varlen(a, b, c, cu, causal), (q, k, v), do)
    _, mine = _grads(lambda a, b, c: impls.attn_varlen(a, b, c, cu.to(DEV), causal),
                     (q.to(DEV), k.to(DEV), v.to(DEV)), do.to(DEV))
    for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
        gauge_ok(got, want, r, dtype, f"{name} (varlen {cu.tolist()[:6]}, d {d}, causal {causal})")


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("total,segments", [(37, 1), (300, 3), (700, 7), (129, 129)])
def test_attn_varlen_bwd(total, segments, d, causal):
    _check_varlen(total, segments, d, causal, torch.bfloat16)


def test_attn_varlen_bwd_fp16():
    _check_varlen(500, 4, 128, True, torch.float16, seed=5)


def test_attn_varlen_bwd_equal_segments_match_dense():
    b, s, hq, hkv, d = 3, 200, 8, 2, 128
    q, k, v, do = (seeded((b, s, h, d), i, torch.bfloat16).to(DEV) for i, h in enumerate((hq, hkv, hkv, hq)))
    cu = torch.arange(0, (b + 1) * s, s, dtype=torch.int32, device=DEV)
    for causal in (False, True):
        ld = [t.clone().requires_grad_() for t in (q, k, v)]
        gd = torch.autograd.grad(impls.attn(*ld, causal), ld, do)
        lv = [t.reshape(b * s, t.shape[2], d).clone().requires_grad_() for t in (q, k, v)]
        gv = torch.autograd.grad(impls.attn_varlen(*lv, cu, causal), lv, do.reshape(b * s, hq, d))
        for a, c in zip(gd, gv):
            assert torch.equal(a, c.reshape(a.shape))


def test_attn_bwd_long_causal_against_float64_on_device():
    """B=1, S=4096, Hq=16, Hkv=4, D=128 causal bf16: one kv group's dq / dk / dv against float64 autograd."""
    b, s, hq, hkv, d = 1, 4096, 16, 4, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2))
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    dq, dk, dv = torch.autograd.grad(impls.attn(*leaves, True), leaves, do)
    grp = 2  # kv head 2 and its q heads 8..11
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
        assert err <= 2e-2 * scale, f"{name}: {err:.3e} vs {scale:.2f}"


def _lse_bytes(b, s, hq):
    return -(-2 * b * hq * s * 4 // 256) * 256  # D and lse2, rounded up to 256 bytes


def test_attn_bwd_split_and_direct_paths_agree():
    """B=8, S=1024, 32 q heads over 8 kv heads fills the device (512 dk/dv blocks), so dk/dv are written
    directly; sequence 0 alone (64 blocks) takes the q-head split, whose four fp32 partials are added in
    order. Both round once to bf16, so they agree to within one bf16 unit."""
    b, s, hq, hkv, d = 8, 1024, 32, 8, 128
    lib = _lib.load()
    assert lib.pk_attn_bwd_workspace(b, s, hq, hkv, d) == _lse_bytes(b, s, hq)  # no partials: direct path
    assert lib.pk_attn_bwd_workspace(1, s, hq, hkv, d) > _lse_bytes(1, s, hq)  # partials: split path
    gen = torch.Generator(device=DEV).manual_seed(5)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2))
    full = [t.clone().requires_grad_() for t in (q, k, v)]
    g_full = torch.autograd.grad(impls.attn(*full, True), full, do)
    one = [t[:1].clone().requires_grad_() for t in (q, k, v)]
    g_one = torch.autograd.grad(impls.attn(*one, True), one, do[:1])
    for name, a, c in zip(("dq", "dk", "dv"), g_full, g_one):
        torch.testing.assert_close(a[:1].float(), c.float(), rtol=2**-7, atol=1e-5, msg=name)


def test_attn_bwd_rejects_a_short_workspace():
    b, s, hq, hkv, d = 1, 256, 8, 2, 128
    lib = _lib.load()
    need = lib.pk_attn_bwd_workspace(b, s, hq, hkv, d)
    assert need > _lse_bytes(b, s, hq)
    q, k, v, do = (seeded((b, s, h, d), i, torch.bfloat16).to(DEV) for i, h in enumerate((hq, hkv, hkv, hq)))
    o, lse = impls.attn_with_lse(q, k, v, True)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    st = (_lib._i64 * 24)(*(x for t in (q, k, v, o, do, dq, dk, dv) for x in t.stride()[:3]))
    rc = lib.pk_attn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
                         ws.data_ptr(), need - 1, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), st, b, s, hq, hkv, d,
                         d**-0.5, 1, _lib.BF16, _lib.stream_handle(q.device))
    assert rc != 0 and b"workspace" in lib.pk_last_error()


# --------------------------------------------------------------------------- dk/dv launch paths
# The dk/dv kernel walks every q head of its kv group in one block (the direct
# path, nsplit = 1) when the grid of 128-key blocks fills the device twice
# over; otherwise it splits the group's q heads over nsplit blocks that leave
# fp32 partials. These cases pin each path on full-size grids, checking
# sampled (batch, kv group) slices against the float64 oracle: a kv group's
# gradients depend only on its own q heads, so a slice is an exact subproblem.


def _splits(ws_bytes, lse_n, rows, hkv, d):
    lse = -(-2 * lse_n * 4 // 256) * 256
    return (ws_bytes - lse) // (2 * rows * hkv * d * 4) if ws_bytes > lse else 1


def _check_group_slices(q, k, v, do, grads, causal, dtype, picks, what):
    group = q.shape[2] // k.shape[2]
    for b, g in picks:
        heads = slice(g * group, (g + 1) * group)
        qs, ks, vs, dos = q[b:b + 1, :, heads], k[b:b + 1, :, g:g + 1], v[b:b + 1, :, g:g + 1], do[b:b + 1, :, heads]
        truth = O.attention_bwd(*(t.double().cpu().numpy() for t in (qs, ks, vs, dos)), causal, None)
        _, ref = _grads(lambda a, c, e: R.attn(a, c, e, causal, None), [t.cpu() for t in (qs, ks, vs)], dos.cpu())
        mine = (grads[0][b:b + 1, :, heads], grads[1][b:b + 1, :, g:g + 1], grads[2][b:b + 1, :, g:g + 1])
        for name, got, want, r in zip(("dq", "dk", "dv"), mine, truth, ref):
            gauge_ok(got, want, r, dtype, f"{name} ({what}, batch {b}, kv group {g})")


@pytest.mark.parametrize("b,s,hq,hkv,d,dtype,causal,splits", [
    (4, 1024, 32, 16, 64, torch.bfloat16, True, 1),    # 512 blocks: direct, two q heads per block
    (8, 1024, 32, 8, 128, torch.float16, False, 1),    # 512 blocks: direct, four q heads per block
    (4, 1024, 32, 8, 64, torch.bfloat16, False, 2),    # 256 blocks: two splits of two q heads
    (4, 1024, 32, 8, 128, torch.float16, True, 2),
    (2, 1024, 64, 8, 128, torch.bfloat16, True, 4),    # 128 blocks, group 8: four splits of two heads
], ids=["direct-d64-bf16-causal", "direct-d128-fp16-full", "split2-d64-bf16-full", "split2-d128-fp16-causal",
        "split4of8-d128-bf16-causal"])
def test_attn_bwd_dkdv_direct_and_partial_splits(b, s, hq, hkv, d, dtype, causal, splits):
    lib = _lib.load()
    assert _splits(lib.pk_attn_bwd_workspace(b, s, hq, hkv, d), b * hq * s, b * s, hkv, d) == splits
    gen = torch.Generator(device=DEV).manual_seed(17)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV).to(dtype) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(dtype) for _ in range(2))
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    grads = torch.autograd.grad(impls.attn(*leaves, causal), leaves, do)
    _check_group_slices(q, k, v, do, grads, causal, dtype, [(0, 0), (b - 1, hkv - 1)], f"{splits} split(s)")


@pytest.mark.parametrize("seqs,length,splits", [(8, 1024, 1), (4, 1024, 2)], ids=["direct", "split2"])
def test_attn_varlen_bwd_dkdv_direct_and_partial_splits(seqs, length, splits):
    """Packed sequences write dk/dv directly into their token rows, or sum partials per token."""
    hq, hkv, d, dtype = 32, 8, 128, torch.bfloat16
    lens = [length - 37 * i for i in range(seqs)]  # ragged, the longest sizes the grid
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    total = int(cu[-1])
    lib = _lib.load()
    ws = lib.pk_attn_varlen_bwd_workspace(seqs, total, max(lens), hq, hkv, d)
    assert _splits(ws, hq * total, total, hkv, d) == splits
    gen = torch.Generator(device=DEV).manual_seed(23)
    q, do = (torch.randn(total, hq, d, generator=gen, device=DEV).to(dtype) for _ in range(2))
    k, v = (torch.randn(total, hkv, d, generator=gen, device=DEV).to(dtype) for _ in range(2))
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    grads = torch.autograd.grad(impls.attn_varlen(*leaves, cu.to(DEV), True), leaves, do)
    for seg in (0, seqs - 1):
        rows = slice(int(cu[seg]), int(cu[seg + 1]))
        seg_view = [t[rows].unsqueeze(0) for t in (q, k, v, do)]
        seg_grads = [g[rows].unsqueeze(0) for g in grads]
        _check_group_slices(*seg_view, seg_grads, True, dtype, [(0, 0), (0, hkv - 1)],
                            f"varlen {splits} split(s), sequence {seg}")


# --------------------------------------------------------------------------- head_dim 136-256
# Rows past 128 dims take the wide path (a dq kernel and the single-role dk/dv
# kernel): 16-bit head_dim 136-192 is laid out at 192 dims, 200-256 at 256.


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", [256, 192])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq", [1, 17, 130, 257])
def test_attn_bwd_wide_head_dims(seq, causal, d, dtype):
    _check(2, seq, 8, 2, d, causal, None, dtype)


@pytest.mark.parametrize("d", [136, 160, 184, 200, 248])
def test_attn_bwd_wide_head_dims_padded_layouts(d):
    """head_dim inside the 192- or 256-dim layout: the dims past it read as zeros and are never stored."""
    _check(1, 77, 4, 1, d, True, None, torch.bfloat16, seed=4)


@pytest.mark.parametrize("heads", [(8, 8), (8, 1), (6, 2), (12, 2)], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_bwd_wide_groups(heads, causal):
    _check(2, 150, heads[0], heads[1], 256, causal, None, torch.bfloat16, seed=11)


@pytest.mark.parametrize("scale", [0.25, -0.3])
def test_attn_bwd_wide_scales(scale):
    _check(1, 96, 4, 2, 256, False, scale, torch.bfloat16, seed=9)


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("total,segments", [(300, 3), (129, 129)])
def test_attn_varlen_bwd_wide(total, segments, causal):
    _check_varlen(total, segments, 256, causal, torch.bfloat16)


@pytest.mark.parametrize("b,s,hq,hkv,d,dtype,causal,splits", [
    (8, 1024, 32, 8, 256, torch.bfloat16, True, 1),    # 512 blocks: direct
    (4, 1024, 32, 8, 256, torch.float16, False, 2),    # 256 blocks: two splits of two q heads
    (2, 1024, 16, 2, 192, torch.bfloat16, True, 8),    # 32 blocks, group 8: one q head per block
], ids=["direct-d256-bf16-causal", "split2-d256-fp16-full", "split8-d192-bf16-causal"])
def test_attn_bwd_wide_dkdv_direct_and_partial_splits(b, s, hq, hkv, d, dtype, causal, splits):
    lib = _lib.load()
    assert _splits(lib.pk_attn_bwd_workspace(b, s, hq, hkv, d), b * hq * s, b * s, hkv, 256) == splits
    print(f"[attn bwd wide] b={b} s={s} hq={hq} hkv={hkv} d={d} {dtype} causal={causal} splits={splits}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(17)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV).to(dtype) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(dtype) for _ in range(2))
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    grads = torch.autograd.grad(impls.attn(*leaves, causal), leaves, do)
    _check_group_slices(q, k, v, do, grads, causal, dtype, [(0, 0), (b - 1, hkv - 1)], f"{splits} split(s)")


def test_attn_bwd_wide_long_causal_against_float64_on_device():
    """B=1, S=4096, Hq=8, Hkv=2, D=256 causal bf16: one kv group's dq / dk / dv against float64 autograd."""
    b, s, hq, hkv, d = 1, 4096, 8, 2, 256
    gen = torch.Generator(device=DEV).manual_seed(0)
    q, do = (torch.randn(b, s, hq, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(b, s, hkv, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2))
    print("[attn bwd wide] long causal S=4096 D=256", flush=True)
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
        assert err <= 2e-2 * scale, f"{name}: {err:.3e} vs {scale:.2f}"
