"""fp32 attention forward (the fp32 matrix-core kernel) against the float64 oracle.

Popcorn grids attention over float32 as well as the 16-bit dtypes
(bench/grid.py:43). The fp32 kernel runs an exact online softmax, so it is held
to Popcorn's fp32 rule (err <= max(2 * budget, 2e-5 * scale), the budget from
torch's fp32 SDPA on the CPU) and to the north star's fp32 tolerance against
that reference, with the log-sum-exp to 1e-5.
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
F32 = torch.float32


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _math_ref(q, k, v, causal, scale):
    """softmax(q k^T scale + mask) v in fp32 on the CPU, one explicit product at a time. torch's CPU
    fp32 SDPA returns NaN rows for a negative scale (a float64 oracle check shows the kernel right),
    so negative scales take their native-dtype reference from this instead."""
    b, s, hq, d = q.shape
    g = hq // k.shape[2]
    kk, vv = k.repeat_interleave(g, dim=2), v.repeat_interleave(g, dim=2)
    sc = torch.einsum("bqhd,bkhd->bhqk", q, kk) * (d**-0.5 if scale is None else scale)
    if causal:
        sc = sc.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    return torch.einsum("bhqk,bkhd->bqhd", torch.softmax(sc, dim=-1), vv)


def _check(batch, seq, hq, hkv, d, causal, scale, seed=0, views=False):
    q = seeded((batch, seq, hq, d), seed, F32)
    k = seeded((batch, seq, hkv, d), seed + 1, F32)
    v = seeded((batch, seq, hkv, d), seed + 2, F32)
    print(f"[attn f32] b={batch} s={seq} hq={hq} hkv={hkv} d={d} causal={causal} scale={scale} views={views}", flush=True)
    o64, lse64 = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal, scale)
    with torch.no_grad():
        oref = R.attn(q, k, v, causal, scale) if scale is None or scale > 0 else _math_ref(q, k, v, causal, scale)
        if views:  # q, k, v as strided views into one packed [b, s, hq + 2 hkv, d] buffer
            packed = torch.cat([q, k, v], dim=2).to(DEV)
            qg, kg, vg = packed.split([hq, hkv, hkv], dim=2)
        else:
            qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
        om, lse = impls.attn_with_lse(qg, kg, vg, causal, scale)
    assert om.shape == q.shape and om.dtype == F32
    gauge_ok(om, o64, oref, F32, "o")
    close_to_reference(om, oref, "o")
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse64, rtol=0, atol=1e-5)
    return om


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("seq", [1, 17, 64, 200, 257])
def test_attn_f32_shapes(seq, causal, d):
    _check(2, seq, 8, 2, d, causal, None)


@pytest.mark.parametrize("d", [16, 32, 48, 80, 96, 120, 136, 192, 248])
def test_attn_f32_head_dims_laid_out_wider(d):
    """head_dim below the 64-, 128- or 256-dim layout: the dims past it read as zeros and are never stored."""
    _check(1, 77, 4, 1, d, True, None, seed=4)


@pytest.mark.parametrize("heads", [(8, 8), (8, 1), (6, 2), (12, 2), (2, 1)], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_f32_groups(heads, causal):
    hq, hkv = heads
    _check(2, 130, hq, hkv, 128, causal, None, seed=7)


@pytest.mark.parametrize("scale", [0.25, -0.3, 1e-3])
def test_attn_f32_scales(scale):
    _check(1, 96, 8, 2, 64, True, scale, seed=3)


def test_attn_f32_strided_views():
    _check(2, 100, 8, 2, 64, False, None, seed=11, views=True)


def test_attn_f32_large_scores_need_the_online_max():
    """Keys boosted far above the first tile's scores: the online max must rescale the earlier tiles."""
    b, s, hq, hkv, d = 1, 300, 4, 1, 128
    q = seeded((b, s, hq, d), 21, F32)
    k = seeded((b, s, hkv, d), 22, F32)
    v = seeded((b, s, hkv, d), 23, F32)
    k[:, 200:210] *= 8.0
    o64, lse64 = O.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), True)
    with torch.no_grad():
        oref = R.attn(q, k, v, True)
        om, lse = impls.attn_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), True)
    gauge_ok(om, o64, oref, F32, "o")
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse64, rtol=1e-6, atol=1e-5)


def test_attn_f32_special_case_uniform_queries():
    """q = 0: every query attends uniformly, o_t = mean(v_0..v_t) and lse_t = log(t + 1) (causal)."""
    b, s, hq, hkv, d = 1, 300, 4, 2, 128
    q = torch.zeros(b, s, hq, d, dtype=F32, device=DEV)
    k = seeded((b, s, hkv, d), 8, F32).to(DEV)
    v = seeded((b, s, hkv, d), 9, F32).to(DEV)
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, True)
    prefix = torch.cumsum(v.double(), dim=1) / torch.arange(1, s + 1, device=DEV, dtype=torch.float64)[None, :, None, None]
    expect = prefix.repeat_interleave(hq // hkv, dim=2)
    assert (o.double() - expect).abs().max().item() < 1e-5
    logs = torch.log(torch.arange(1, s + 1, dtype=torch.float64, device=DEV))
    assert (lse.double() - logs[None, None, :]).abs().max().item() < 1e-5


def test_attn_varlen_f32():
    """Packed sequences of uneven length: each segment against the oracle on its own."""
    lens = [5, 64, 1, 130, 33]
    hq, hkv, d = 8, 2, 64
    total = sum(lens)
    q = seeded((total, hq, d), 31, F32)
    k = seeded((total, hkv, d), 32, F32)
    v = seeded((total, hkv, d), 33, F32)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    print(f"[attn f32] varlen lens={lens}", flush=True)
    with torch.no_grad():
        om, lse = impls.attn_varlen_with_lse(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), True)
    for i, (a, e) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        o64, lse64 = O.attention(q[None, a:e].double().numpy(), k[None, a:e].double().numpy(),
                                 v[None, a:e].double().numpy(), True)
        with torch.no_grad():
            oref = R.attn(q[None, a:e], k[None, a:e], v[None, a:e], True)
        gauge_ok(om[a:e][None], o64, oref, F32, f"segment {i}")
        np.testing.assert_allclose(lse[:, a:e].cpu().double().numpy(), lse64[0], rtol=0, atol=1e-5)


def test_attn_f32_long_sequence_sampled_rows():
    """B=1, S=4096, Hq=8, Hkv=2, D=128, causal: sampled rows of two heads against the float64 oracle."""
    B, S, HQ, HKV, D = 1, 4096, 8, 2, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(B, S, HQ, D, generator=gen, device=DEV)
    k = torch.randn(B, S, HKV, D, generator=gen, device=DEV)
    v = torch.randn(B, S, HKV, D, generator=gen, device=DEV)
    print(f"[attn f32] long sequence S={S}", flush=True)
    with torch.no_grad():
        o, lse = impls.attn_with_lse(q, k, v, True)
    rows = np.array([0, 1, 31, 32, 127, 2047, 2048, 4094, 4095])
    for h in (0, 7):
        qh, kh, vh = q[0, :, h].cpu(), k[0, :, h // 4].cpu(), v[0, :, h // 4].cpu()
        o64, lse64 = O.attention_rows(qh.double().numpy(), kh.double().numpy(), vh.double().numpy(), rows, True)
        mask = torch.arange(S)[None, :] <= torch.as_tensor(rows)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qh[rows][None], kh[None], vh[None], attn_mask=mask[None])[0]
        gauge_ok(o[0, rows, h], o64, ref, F32, f"o[0,:,{h}]")
        np.testing.assert_allclose(lse[0, h, rows].cpu().double().numpy(), lse64, rtol=0, atol=1e-5)


@pytest.mark.parametrize("heads", [(8, 1), (6, 2)], ids=str)
def test_attn_f32_wide_groups(heads):
    _check(2, 130, heads[0], heads[1], 256, True, None, seed=13)
