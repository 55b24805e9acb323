"""Paired q/k rotary embedding (`rope`) on the GPU against the float64 oracle and Popcorn's reference."""

import ctypes

import pytest
import torch

from oracle import reference as O
from popcorn_amd import _lib, impls
from popcorn_amd.compat import references as R
from tests._parity import close_to_reference, gauge_ok, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def tables(cos_batch, seq, head_dim, seed, duplicated=True):
    """Popcorn's rope test tables: cos/sin of an N(0,1) draw, first half repeated (or full-width random)."""
    draw = seeded((cos_batch, seq, head_dim), seed, torch.float32)
    if duplicated:
        return R.rope_table(torch.cos)(draw), R.rope_table(torch.sin)(draw)
    return draw.cos(), seeded((cos_batch, seq, head_dim), seed + 1, torch.float32).sin()


def _check(batch, hq, hkv, seq, d, cos_batch, dtype, seed=0, duplicated=True, table_dtype=None):
    """q, k in `dtype`, tables in `table_dtype` (default `dtype`); outputs and cotangents in their promotion."""
    table_dtype = dtype if table_dtype is None else table_dtype
    out_dtype = torch.promote_types(dtype, table_dtype)
    q = seeded((batch, hq, seq, d), seed, dtype)
    k = seeded((batch, hkv, seq, d), seed + 1, dtype)
    cos, sin = (t.to(table_dtype) for t in tables(cos_batch, seq, d, seed + 2, duplicated))
    gq, gk = seeded(tuple(q.shape), seed + 4, out_dtype), seeded(tuple(k.shape), seed + 5, out_dtype)
    n64 = lambda t: t.double().numpy()  # noqa: E731
    y64 = O.rope(n64(q), n64(k), n64(cos), n64(sin))
    d64 = O.rope_bwd(n64(gq), n64(gk), n64(cos), n64(sin))
    qr, kr = q.clone().requires_grad_(), k.clone().requires_grad_()
    yr = R.rope(qr, kr, cos, sin)
    dr = torch.autograd.grad(yr, (qr, kr), (gq, gk))
    qm, km = q.to(DEV).requires_grad_(), k.to(DEV).requires_grad_()
    ym = impls.rope(qm, km, cos.to(DEV), sin.to(DEV))
    dm = torch.autograd.grad(ym, (qm, km), (gq.to(DEV), gk.to(DEV)))
    what = f"(b {batch}, hq {hq}, hkv {hkv}, s {seq}, d {d}, cos_batch {cos_batch}, tables {table_dtype})"
    for name, mine, truth, ref in zip(("yq", "yk", "dq", "dk"), (*ym, *dm), (*y64, *d64), (*yr, *dr)):
        want = out_dtype if name.startswith("y") else dtype
        assert mine.shape == ref.shape and mine.dtype == ref.dtype == want, name
        gauge_ok(mine, truth, ref, want, f"{name} {what}")
    for name, mine, ref in zip(("yq", "yk"), ym, yr):
        close_to_reference(mine, ref, f"{name} {what}")
    return ym


CASES = [
    # (batch, q_heads, kv_heads, seq, head_dim, cos_batch)
    (2, 4, 2, 16, 128, 1),
    (2, 4, 2, 16, 128, 2),
    (1, 8, 1, 33, 64, 1),
    (3, 2, 2, 5, 80, 3),  # half 40: 16-byte packs only for fp32
    (1, 3, 1, 7, 6, 1),  # half 3: element path
    (2, 1, 1, 1, 2, 2),  # one pair
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=str)
def test_rope(case, dtype):
    _check(*case, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=str)
def test_rope_fp32_tables(case, dtype):
    """16-bit q/k with fp32 tables (the model's fp32 cos/sin buffers): fp32 outputs, 16-bit gradients."""
    _check(*case, dtype, table_dtype=torch.float32)


@pytest.mark.parametrize("pair", [(torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16),
                                  (torch.float32, torch.bfloat16)], ids=str)
def test_rope_other_table_dtypes(pair):
    """Tables of another dtype: the outputs take the promotion (fp32 for bf16 beside fp16)."""
    dtype, table_dtype = pair
    _check(2, 4, 2, 16, 128, 1, dtype, seed=9, table_dtype=table_dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_rope_unequal_table_halves(dtype):
    """The kernel reads both halves of each table row; tables whose halves differ follow the same formula."""
    _check(2, 4, 2, 24, 64, 2, dtype, seed=3, duplicated=False)


def test_rope_strided_views_match_contiguous():
    """q, k as [b, s, h, d] buffers viewed as [b, h, s, d] (the model layout) give the contiguous result bit for bit."""
    b, s, hq, hkv, d = 2, 50, 8, 2, 128
    qkv = seeded((b, s, hq + 2 * hkv, d), 21, torch.bfloat16).to(DEV)
    q, k = qkv[:, :, :hq].transpose(1, 2), qkv[:, :, hq:hq + hkv].transpose(1, 2)
    cos, sin = (t.to(torch.bfloat16).to(DEV) for t in tables(1, s, d, 22))
    with torch.no_grad():
        a = impls.rope(q, k, cos, sin)
        c = impls.rope(q.contiguous(), k.contiguous(), cos, sin)
    for x, y in zip(a, c):
        assert x.is_contiguous() and torch.equal(x, y)


def test_rope_gradient_of_one_output():
    """Only yq reaches the loss: dk is zero and dq matches the two-output gradient."""
    b, hq, hkv, s, d = 1, 4, 2, 32, 64
    q = seeded((b, hq, s, d), 31, torch.bfloat16).to(DEV).requires_grad_()
    k = seeded((b, hkv, s, d), 32, torch.bfloat16).to(DEV).requires_grad_()
    cos, sin = (t.to(torch.bfloat16).to(DEV) for t in tables(1, s, d, 33))
    g = seeded((b, hq, s, d), 34, torch.bfloat16).to(DEV)
    yq, _ = impls.rope(q, k, cos, sin)
    dq, dk = torch.autograd.grad(yq, (q, k), g, allow_unused=True)
    assert dk is None or not dk.any()
    yq2, yk2 = impls.rope(q, k, cos, sin)
    dq2, _ = torch.autograd.grad((yq2, yk2), (q, k), (g, torch.zeros_like(yk2)))
    assert torch.equal(dq, dq2)


def test_rope_fp32_tables_with_bf16_inputs_through_the_c_abi():
    """Table dtype may differ from x's at the C ABI: fp32 tables, bf16 q/k, one rounding to bf16."""
    b, hq, hkv, s, d = 2, 4, 1, 40, 128
    q = seeded((b, hq, s, d), 41, torch.bfloat16).to(DEV)
    k = seeded((b, hkv, s, d), 42, torch.bfloat16).to(DEV)
    cos, sin = (t.to(DEV).contiguous() for t in tables(b, s, d, 43))
    yq, yk = torch.empty_like(q), torch.empty_like(k)
    lib = _lib.load()
    st = (ctypes.c_int64 * 12)(*(x for t in (q, k, yq, yk) for x in t.stride()[:3]))
    _lib.check(lib.pk_rope(q.data_ptr(), k.data_ptr(), cos.data_ptr(), sin.data_ptr(), yq.data_ptr(), yk.data_ptr(),
                           st, b, hq, hkv, s, d, b, _lib.BF16, _lib.BF16, _lib.F32, 0, _lib.stream_handle(q.device)), lib)
    want = O.rope(q.cpu().double().numpy(), k.cpu().double().numpy(), cos.cpu().double().numpy(),
                  sin.cpu().double().numpy())
    for got, w in zip((yq, yk), want):
        exact = torch.from_numpy(w).to(torch.bfloat16)  # the correctly rounded result
        diff = (got.cpu().float() - exact.float()).abs()
        # fp32 arithmetic (error below 1e-5 for these magnitudes) then one rounding:
        # within one bf16 ulp of the correctly rounded value
        assert (diff <= exact.float().abs() * 2**-7 + 1e-5).all()


def test_rope_long_sequence_model_shape():
    """q [4, 32, 4096, 128], k [4, 8, 4096, 128] bf16 (the fused qk-norm+rope notebook's shape) against fp32 torch."""
    b, hq, hkv, s, d = 4, 32, 8, 4096, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(b, hq, s, d, generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, hkv, s, d, generator=gen, device=DEV).to(torch.bfloat16)
    inv = 500000.0 ** (-torch.arange(d // 2, device=DEV, dtype=torch.float64) * 2 / d)
    ang = torch.arange(s, device=DEV, dtype=torch.float64)[:, None] * inv
    ang = torch.cat([ang, ang], -1)[None]
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    with torch.no_grad():
        yq, yk = impls.rope(q, k, cos, sin)
        for x, y in ((q, yq), (k, yk)):
            xf, c, sn = x.float(), cos.float()[:, None], sin.float()[:, None]
            want = xf * c + R.rotate_half(xf) * sn
            err = (y.float() - want).abs().max().item()
            assert err <= 2 ** -8 * want.abs().max().item(), err
