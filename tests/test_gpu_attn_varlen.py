"""Packed variable-length attention forward on the GPU against the float64 oracle and Popcorn's reference."""

import numpy as np
import pytest
import torch

from oracle import reference as O
from popcorn_amd import impls
from popcorn_amd.compat import references as R
from tests._parity import gauge_ok, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _cuts(total, segments, seed):
    return R.cuts(torch.zeros(segments + 1, dtype=torch.int64), {"total": total}, torch.Generator().manual_seed(seed))


def _check(total, segments, hq, hkv, d, causal, scale, dtype, seed=0):
    cu = _cuts(total, segments, seed)
    q = seeded((total, hq, d), seed, dtype)
    k = seeded((total, hkv, d), seed + 1, dtype)
    v = seeded((total, hkv, d), seed + 2, dtype)
    o64, lse64 = O.attention_varlen(q.double().numpy(), k.double().numpy(), v.double().numpy(), cu.numpy(), causal,
                                    scale)
    with torch.no_grad():
        oref = R.attn_varlen(q, k, v, cu, causal, scale)
        om, lse = impls.attn_varlen_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), causal, scale)
    assert om.shape == q.shape and om.dtype == dtype
    gauge_ok(om, o64, oref, dtype, f"o cu={cu.tolist()[:6]}")
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse64, rtol=0, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("total,segments", [(37, 1), (300, 3), (1000, 7), (513, 513)])
def test_attn_varlen_shapes(total, segments, causal, d, dtype):
    _check(total, segments, 8, 2, d, causal, None, dtype)


@pytest.mark.parametrize("scale", [None, 0.25])
@pytest.mark.parametrize("hkv", [8, 1])
def test_attn_varlen_groups_and_scale(hkv, scale):
    _check(700, 5, 8, hkv, 128, True, scale, torch.bfloat16, seed=4)


@pytest.mark.parametrize("heads", [(6, 2), (12, 2)], ids=str)
def test_attn_varlen_uneven_group_sizes(heads):
    """Group sizes 3 and 6 over packed segments of unequal lengths."""
    _check(700, 5, heads[0], heads[1], 64, True, None, torch.bfloat16, seed=6)


def test_attn_varlen_equal_segments_match_the_dense_kernel():
    """B sequences of one length packed back to back give the dense kernel's result bit for bit."""
    b, s, hq, hkv, d = 3, 333, 8, 2, 128
    q = seeded((b, s, hq, d), 1, torch.bfloat16).to(DEV)
    k = seeded((b, s, hkv, d), 2, torch.bfloat16).to(DEV)
    v = seeded((b, s, hkv, d), 3, torch.bfloat16).to(DEV)
    cu = torch.arange(0, (b + 1) * s, s, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        for causal in (False, True):
            od, ld = impls.attn_with_lse(q, k, v, causal)
            ov, lv = impls.attn_varlen_with_lse(q.reshape(b * s, hq, d), k.reshape(b * s, hkv, d),
                                                v.reshape(b * s, hkv, d), cu, causal)
            assert torch.equal(ov.reshape(b, s, hq, d), od)
            assert torch.equal(lv.reshape(hq, b, s).transpose(0, 1), ld)


def test_attn_varlen_rejects_bad_offsets():
    q = torch.zeros(10, 2, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(10, 1, 64, dtype=torch.bfloat16, device=DEV)
    with torch.no_grad():
        for bad in ([0, 4, 3, 10], [1, 10], [0, 9]):
            with pytest.raises(ValueError):
                impls.attn_varlen(q, k, k, torch.tensor(bad, dtype=torch.int32, device=DEV))


def test_attn_varlen_long_packed_batch():
    """Eight sequences of 128..4096 tokens (16k total), causal, bf16: sampled rows against the oracle."""
    lens = [4096, 128, 2048, 1000, 3000, 777, 4096, 1239]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    total, hq, hkv, d = int(cu[-1]), 16, 4, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(total, hq, d, generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn(total, hkv, d, generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn(total, hkv, d, generator=gen, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        o, lse = impls.attn_varlen_with_lse(q, k, v, cu.to(DEV), True)
    assert torch.isfinite(o.float()).all()
    for seg in (0, 2, 6, 7):
        lo, hi = int(cu[seg]), int(cu[seg + 1])
        rows = np.array([0, 1, 127, hi - lo - 1])
        for h in (0, 7, 15):
            qh, kh, vh = (t[lo:hi, hh].cpu().double().numpy() for t, hh in ((q, h), (k, h // 4), (v, h // 4)))
            o64, lse64 = O.attention_rows(qh, kh, vh, rows, True)
            got = o[lo:hi, h].cpu().double().numpy()[rows]
            assert np.abs(got - o64).max() < 2e-2 * max(1.0, np.abs(o64).max())
            np.testing.assert_allclose(lse[h, lo:hi].cpu().double().numpy()[rows], lse64, rtol=0, atol=1e-3)


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_varlen_empty_segments(causal):
    """Zero-length sequences (repeated offsets) produce nothing and leave the others exact, forward and backward."""
    cu = torch.tensor([0, 0, 5, 5, 5, 40, 41, 41], dtype=torch.int32)
    total, hq, hkv, d = 41, 4, 2, 64
    q = seeded((total, hq, d), 61, torch.bfloat16).to(DEV)
    k = seeded((total, hkv, d), 62, torch.bfloat16).to(DEV)
    v = seeded((total, hkv, d), 63, torch.bfloat16).to(DEV)
    do = seeded((total, hq, d), 64, torch.bfloat16).to(DEV)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    o = impls.attn_varlen(*leaves, cu.to(DEV), causal)
    grads = torch.autograd.grad(o, leaves, do)
    bounds = cu.tolist()
    for lo, hi in zip(bounds, bounds[1:]):
        if hi == lo:
            continue
        seg = [t[lo:hi][None].clone().requires_grad_() for t in (q, k, v)]
        ref = impls.attn(*seg, causal)
        ref_grads = torch.autograd.grad(ref, seg, do[lo:hi][None])
        assert torch.equal(o[lo:hi], ref[0]), (lo, hi)
        for g, r in zip(grads, ref_grads):
            assert torch.equal(g[lo:hi], r[0]), (lo, hi)
