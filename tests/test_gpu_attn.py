"""Attention forward on the GPU against the float64 oracle and Popcorn's reference at native dtype.

torch's attention reference is only ever evaluated on the CPU here (its math
path issues batched bf16 products on transposed views).
"""

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


def _check(batch, seq, hq, hkv, d, causal, scale, dtype, seed=0):
    q = seeded((batch, seq, hq, d), seed, dtype)
    k = seeded((batch, seq, hkv, d), seed + 1, dtype)
    v = seeded((batch, seq, hkv, d), seed + 2, dtype)
    o64, lse64 = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal, scale)
    with torch.no_grad():
        oref = R.attn(q, k, v, causal, scale)
        om, lse = impls.attn_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), causal, scale)
    assert om.shape == q.shape and om.dtype == dtype
    gauge_ok(om, o64, oref, dtype, "o")
    close_to_reference(om, oref, "o")
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse64, rtol=0, atol=1e-3)
    return om


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq", [1, 17, 64, 128, 200, 257])
def test_attn_shapes(seq, causal, d, dtype):
    _check(2, seq, 8, 2, d, causal, None, dtype)


@pytest.mark.parametrize("hkv", [8, 4, 1])
@pytest.mark.parametrize("scale", [None, 0.25])
def test_attn_groups_and_scale(hkv, scale):
    _check(1, 96, 8, hkv, 128, True, scale, torch.bfloat16, seed=3)


@pytest.mark.parametrize("heads", [(6, 2), (6, 1), (12, 2), (2, 1)], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("d", [64, 128])
def test_attn_uneven_group_sizes(heads, causal, d):
    """Group sizes 3, 6, 6 and 2: a block holds one or two q heads of a group over several
    32-row groups (four heads per block only when 4 divides the group size)."""
    hq, hkv = heads
    _check(2, 200, hq, hkv, d, causal, None, torch.bfloat16, seed=7)


def test_attn_popcorn_smoke_case():
    """The case Popcorn's per-backend smoke runs for attn (tests/kernels/test_kernels.py:107-123)."""
    _check(2, 64, 8, 2, 64, True, None, torch.bfloat16, seed=5)


def test_attn_special_cases():
    """q = 0: every query attends uniformly, o_t = mean(v_0..v_t), lse_t = log(t+1) (causal)."""
    b, s, hq, hkv, d = 1, 300, 4, 2, 128
    q = torch.zeros(b, s, hq, d, dtype=torch.bfloat16, device=DEV)
    v = seeded((b, s, hkv, d), 9, torch.bfloat16).to(DEV)
    k = seeded((b, s, hkv, d), 8, torch.bfloat16).to(DEV)
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, True)
    prefix = torch.cumsum(v.double(), dim=1) / torch.arange(1, s + 1, device=DEV, dtype=torch.float64)[None, :, None, None]
    expect = prefix.repeat_interleave(hq // hkv, dim=2)
    assert (o.double() - expect).abs().max().item() < 2e-2
    want = torch.log(torch.arange(1, s + 1, dtype=torch.float64))
    assert (lse[0].cpu().double() - want[None]).abs().max().item() < 1e-4


def test_attn_strided_qkv():
    """q, k, v as views of one packed buffer [b, s, hq + 2 hkv, d]."""
    b, s, hq, hkv, d = 2, 130, 8, 2, 128
    packed = seeded((b, s, hq + 2 * hkv, d), 11, torch.bfloat16)
    q, k, v = packed[:, :, :hq], packed[:, :, hq : hq + hkv], packed[:, :, hq + hkv :]
    o64, _ = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), True)
    dev = packed.to(DEV)
    with torch.no_grad():
        om = impls.attn(dev[:, :, :hq], dev[:, :, hq : hq + hkv], dev[:, :, hq + hkv :], True)
        oref = R.attn(q, k, v, True)
    gauge_ok(om, o64, oref, torch.bfloat16, "o")


def test_attn_c5_full_size():
    """B=4, S=8192, Hq=32, Hkv=8, D=128, causal, bf16.
    Sampled (batch, head, row) triples against the float64 oracle, with the
    budget from the reference at native dtype (CPU SDPA on the same rows)."""
    B, S, HQ, HKV, D = 4, 8192, 32, 8, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(B, S, HQ, D, generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, S, HKV, D, generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, S, HKV, D, generator=gen, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, True)
    assert torch.isfinite(o.float()).all()
    rows = np.array([0, 1, 63, 64, 127, 128, 4095, 4096, 8190, 8191])
    for b, h in [(0, 0), (1, 5), (2, 17), (3, 31)]:
        qh = q[b, :, h].cpu()
        kh, vh = k[b, :, h // 4].cpu(), v[b, :, h // 4].cpu()
        o64, lse64 = O.attention_rows(qh.double().numpy(), kh.double().numpy(), vh.double().numpy(), rows, True)
        # native-dtype reference for the same rows: SDPA with the causal mask made explicit
        mask = torch.arange(S)[None, :] <= torch.as_tensor(rows)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            qh[rows][None], kh[None], vh[None], attn_mask=mask[None]
        )[0]
        gauge_ok(o[b, rows, h], o64, ref, torch.bfloat16, f"o[{b},:,{h}]")
        np.testing.assert_allclose(lse[b, h, rows].cpu().double().numpy(), lse64, rtol=0, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq", [100, 777])
def test_attn_late_large_scores(seq, causal, dtype):
    """Scores far above the first key tile's max (boosted keys at 60..69 and
    boosted queries from row 80 on): the fixed-max sweep's row sums leave its
    range, and those blocks must sweep again with the online max."""
    b, hq, hkv, d = 2, 8, 2, 128
    q = seeded((b, seq, hq, d), 21, torch.float32)
    k = seeded((b, seq, hkv, d), 22, torch.float32)
    v = seeded((b, seq, hkv, d), 23, torch.float32)
    k[:, 60:70] *= 6.0
    q[:, 80:] *= 3.0
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    o64, lse64 = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal, None)
    with torch.no_grad():
        oref = R.attn(q, k, v, causal, None)
        om, lse = impls.attn_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), causal, None)
    assert torch.isfinite(om.float()).all()
    gauge_ok(om, o64, oref, dtype, "o")
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse64, rtol=0, atol=1e-3)


def test_attn_fp16_long_uniform_rows():
    """fp16, q = 0 over 40000 keys: every row sum is 40000 > 2^15, so the
    fixed-max sweep hands every block to the exact sweep; o = mean(v), lse = log(S)."""
    b, s, hq, hkv, d = 1, 40000, 2, 1, 64
    q = torch.zeros(b, s, hq, d, dtype=torch.float16, device=DEV)
    k = seeded((b, s, hkv, d), 31, torch.float16).to(DEV)
    v = seeded((b, s, hkv, d), 32, torch.float16).to(DEV)
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, False)
    mean = v.double().mean(dim=1, keepdim=True).expand(b, s, hkv, d).repeat_interleave(hq // hkv, dim=2)
    assert (o.double() - mean).abs().max().item() < 2e-3
    assert (lse.double() - np.log(s)).abs().max().item() < 1e-4


def test_attn_contiguous_views_at_odd_offsets():
    """A contiguous tensor starting 2 bytes into its buffer is not 16-byte aligned: the wrapper copies it."""
    b, s, hq, hkv, d = 1, 70, 4, 2, 128
    flat = seeded((b * s * (hq + 2 * hkv) * d + 3,), 31, torch.bfloat16).to(DEV)
    n_q, n_kv = b * s * hq * d, b * s * hkv * d
    q = flat[1:1 + n_q].view(b, s, hq, d)
    k = flat[1 + n_q:1 + n_q + n_kv].view(b, s, hkv, d)
    v = flat[1 + n_q + n_kv:1 + n_q + 2 * n_kv].view(b, s, hkv, d)
    assert q.is_contiguous() and q.data_ptr() % 16 != 0
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]  # aligned copies
    want = impls.attn(*leaves, True)
    want_grads = torch.autograd.grad(want, leaves, torch.ones_like(want))
    odd = [t.detach().requires_grad_() for t in (q, k, v)]
    got = impls.attn(*odd, True)
    got_grads = torch.autograd.grad(got, odd, torch.ones_like(got))
    assert torch.equal(got, want)
    for a, c in zip(got_grads, want_grads):
        assert torch.equal(a, c)
