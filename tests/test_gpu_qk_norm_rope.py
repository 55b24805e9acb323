"""Fused per-head RMSNorm + rope (`qk_norm_rope`) on the GPU against the float64 oracle and the reference."""

import pytest
import torch

from oracle import reference as O
from popcorn_amd import backend, impls
from popcorn_amd.compat import references as R
from tests._parity import close_to_reference, gauge_ok, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def tables(cos_batch, seq, head_dim, seed, duplicated=True):
    draw = seeded((cos_batch, seq, head_dim), seed, torch.float32)
    if duplicated:
        return R.rope_table(torch.cos)(draw), R.rope_table(torch.sin)(draw)
    return draw.cos(), seeded((cos_batch, seq, head_dim), seed + 1, torch.float32).sin()


def _check(batch, hq, hkv, seq, d, cos_batch, dtype, eps=1e-6, seed=0, duplicated=True, table_dtype=None,
           weight_dtype=None):
    """q, k in `dtype`, weights in `weight_dtype` and tables in `table_dtype` (both default `dtype`); outputs and
    cotangents in the promotion of all three, weight gradients in the weights' dtype."""
    table_dtype = dtype if table_dtype is None else table_dtype
    weight_dtype = dtype if weight_dtype is None else weight_dtype
    out_dtype = torch.promote_types(torch.promote_types(dtype, weight_dtype), table_dtype)
    q = seeded((batch, hq, seq, d), seed, dtype)
    k = seeded((batch, hkv, seq, d), seed + 1, dtype)
    qw = seeded((d,), seed + 6, weight_dtype)
    kw = seeded((d,), seed + 7, weight_dtype)
    cos, sin = (t.to(table_dtype) for t in tables(cos_batch, seq, d, seed + 2, duplicated))
    gq, gk = seeded(tuple(q.shape), seed + 4, out_dtype), seeded(tuple(k.shape), seed + 5, out_dtype)
    n64 = lambda t: t.double().numpy()  # noqa: E731
    y64 = O.qk_norm_rope(n64(q), n64(k), n64(qw), n64(kw), n64(cos), n64(sin), eps)
    d64 = O.qk_norm_rope_bwd(n64(q), n64(k), n64(qw), n64(kw), n64(cos), n64(sin), n64(gq), n64(gk), eps)
    leaves = [t.clone().requires_grad_() for t in (q, k, qw, kw)]
    yr = R.qk_norm_rope(*leaves, cos, sin, eps)
    dr = torch.autograd.grad(yr, leaves, (gq, gk))
    mine = [t.to(DEV).requires_grad_() for t in (q, k, qw, kw)]
    ym = impls.qk_norm_rope(*mine, cos.to(DEV), sin.to(DEV), eps)
    dm = torch.autograd.grad(ym, mine, (gq.to(DEV), gk.to(DEV)))
    what = f"(b {batch}, hq {hq}, hkv {hkv}, s {seq}, d {d}, cos_batch {cos_batch}, eps {eps})"
    names = ("yq", "yk", "dq", "dk", "dq_weight", "dk_weight")
    for name, got, truth, ref in zip(names, (*ym, *dm), (*y64, *d64), (*yr, *dr)):
        want = out_dtype if name.startswith("y") else weight_dtype if name.endswith("weight") else dtype
        assert got.shape == ref.shape and got.dtype == ref.dtype == want, name
        gauge_ok(got, truth, ref, want, f"{name} {what}")
    for name, got, ref in zip(("yq", "yk"), ym, yr):
        close_to_reference(got, ref, f"{name} {what}", rounding=dtype)


CASES = [
    # (batch, q_heads, kv_heads, seq, head_dim, cos_batch)
    (2, 4, 2, 16, 128, 1),
    (2, 4, 2, 16, 128, 2),
    (1, 8, 1, 33, 64, 1),
    (3, 2, 2, 5, 256, 3),
    (1, 3, 1, 7, 32, 1),
    (2, 1, 1, 1, 16, 2),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=str)
def test_qk_norm_rope(case, dtype):
    _check(*case, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=str)
def test_qk_norm_rope_fp32_tables(case, dtype):
    """16-bit q/k and weights with fp32 tables: fp32 outputs (and cotangents), 16-bit gradients."""
    _check(*case, dtype, table_dtype=torch.float32)


@pytest.mark.parametrize("table_dtype", [None, torch.float32], ids=str)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=str)
def test_qk_norm_rope_fp32_weights(case, dtype, table_dtype):
    """16-bit q/k with fp32 weights (autocast's norm parameters): fp32 outputs, fp32 weight gradients."""
    _check(*case, dtype, table_dtype=table_dtype, weight_dtype=torch.float32)


@pytest.mark.parametrize("case", [(2, 4, 2, 16, 128, 1), (1, 3, 1, 9, 8, 1), (2, 2, 1, 40, 64, 2)], ids=str)
def test_qk_norm_rope_fp32(case):
    _check(*case, torch.float32)


def test_qk_norm_rope_eps_and_unequal_table_halves():
    _check(2, 4, 2, 24, 128, 2, torch.bfloat16, eps=1e-5, seed=3, duplicated=False)


def test_qk_norm_rope_strided_views_match_contiguous():
    """[b, s, h, d] projections viewed as [b, h, s, d] give the contiguous result bit for bit, gradients too."""
    b, s, hq, hkv, d = 2, 50, 8, 2, 128
    qkv = seeded((b, s, hq + 2 * hkv, d), 21, torch.bfloat16).to(DEV)
    q, k = qkv[:, :, :hq].transpose(1, 2), qkv[:, :, hq:hq + hkv].transpose(1, 2)
    qw, kw = seeded((d,), 22, torch.bfloat16).to(DEV), seeded((d,), 23, torch.bfloat16).to(DEV)
    cos, sin = (t.to(torch.bfloat16).to(DEV) for t in tables(1, s, d, 24))
    gq = seeded((b, hq, s, d), 25, torch.bfloat16).to(DEV)
    gk = seeded((b, hkv, s, d), 26, torch.bfloat16).to(DEV)
    results = []
    for qq, kk in ((q, k), (q.contiguous(), k.contiguous())):
        leaves = [t.detach().clone().requires_grad_() if t.is_contiguous() else t.detach().requires_grad_()
                  for t in (qq, kk, qw, kw)]
        ys = impls.qk_norm_rope(*leaves, cos, sin)
        results.append((*ys, *torch.autograd.grad(ys, leaves, (gq, gk))))
    for a, c in zip(*results):
        assert torch.equal(a, c)


def test_qk_norm_rope_is_deterministic():
    """dw comes from per-block partial rows summed in a fixed order: two runs agree bit for bit."""
    b, hq, hkv, s, d = 2, 16, 4, 300, 128
    q = seeded((b, hq, s, d), 31, torch.bfloat16).to(DEV)
    k = seeded((b, hkv, s, d), 32, torch.bfloat16).to(DEV)
    qw, kw = seeded((d,), 33, torch.bfloat16).to(DEV), seeded((d,), 34, torch.bfloat16).to(DEV)
    cos, sin = (t.to(torch.bfloat16).to(DEV) for t in tables(1, s, d, 35))
    gq, gk = seeded((b, hq, s, d), 36, torch.bfloat16).to(DEV), seeded((b, hkv, s, d), 37, torch.bfloat16).to(DEV)
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_() for t in (q, k, qw, kw)]
        runs.append(torch.autograd.grad(impls.qk_norm_rope(*leaves, cos, sin), leaves, (gq, gk)))
    for a, c in zip(*runs):
        assert torch.equal(a, c)


def test_qk_norm_rope_unsupported_head_dim_raises_and_is_declined():
    q = torch.zeros(1, 2, 4, 96, dtype=torch.bfloat16, device=DEV)  # 6 packs per half: not a power of two
    w = torch.ones(96, dtype=torch.bfloat16, device=DEV)
    cs = torch.ones(1, 4, 96, dtype=torch.bfloat16, device=DEV)
    assert not backend.qk_norm_rope_supported(q, q, w, w, cs, cs, 1e-6)
    with pytest.raises(Exception, match="head_dim"):
        impls.qk_norm_rope(q, q, w, w, cs, cs)


def test_qk_norm_rope_notebook_shape_against_fp32_torch():
    """q [4, 32, 4096, 128], k [4, 8, 4096, 128] bf16 (the notebook's benchmark shape), forward and backward."""
    b, hq, hkv, s, d = 4, 32, 8, 4096, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(b, hq, s, d, generator=gen, device=DEV).to(torch.bfloat16).requires_grad_()
    k = torch.randn(b, hkv, s, d, generator=gen, device=DEV).to(torch.bfloat16).requires_grad_()
    qw = torch.randn(d, generator=gen, device=DEV).to(torch.bfloat16).requires_grad_()
    kw = torch.randn(d, generator=gen, device=DEV).to(torch.bfloat16).requires_grad_()
    half = torch.randn(1, s, d // 2, generator=gen, device=DEV).to(torch.bfloat16)
    cos, sin = torch.cos(half).repeat(1, 1, 2), torch.sin(half).repeat(1, 1, 2)
    gq = torch.randn(b, hq, s, d, generator=gen, device=DEV).to(torch.bfloat16)
    gk = torch.randn(b, hkv, s, d, generator=gen, device=DEV).to(torch.bfloat16)
    yq, yk = impls.qk_norm_rope(q, k, qw, kw, cos, sin)
    dq, dk, dqw, dkw = torch.autograd.grad((yq, yk), (q, k, qw, kw), (gq, gk))
    # fp32 torch on the device, one (q or k) side at a time
    for x, w, y, g, dx, dw in ((q, qw, yq, gq, dq, dqw), (k, kw, yk, gk, dk, dkw)):
        xf = x.detach().float().requires_grad_()
        wf = w.detach().float().requires_grad_()
        n = torch.nn.functional.rms_norm(xf, (d,), wf, 1e-6)
        want = n * cos.float()[:, None] + R.rotate_half(n) * sin.float()[:, None]
        gx, gw = torch.autograd.grad(want, (xf, wf), g.float())
        for name, got, ref in (("y", y, want), ("dx", dx, gx), ("dw", dw, gw)):
            err = (got.float() - ref).abs().max().item()
            scale = max(1.0, ref.abs().max().item())
            tol = 2e-2 if name != "dw" else 1e-2  # dw sums 524288 rows in fp32 and rounds once
            assert err <= tol * scale, f"{name}: {err:.3e} vs scale {scale:.2f}"


def test_qk_norm_rope_contiguous_views_at_odd_offsets():
    """q, k and the weights starting 2 bytes into their buffers give the aligned result bit for bit."""
    b, hq, hkv, s, d = 1, 4, 2, 40, 128
    flat = seeded((b * (hq + hkv) * s * d + 2 * d + 5,), 41, torch.bfloat16).to(DEV)
    n_q, n_k = b * hq * s * d, b * hkv * s * d
    q = flat[1:1 + n_q].view(b, hq, s, d)
    k = flat[1 + n_q:1 + n_q + n_k].view(b, hkv, s, d)
    qw = flat[1 + n_q + n_k:1 + n_q + n_k + d]
    kw = flat[1 + n_q + n_k + d:1 + n_q + n_k + 2 * d]
    assert q.data_ptr() % 16 != 0 and qw.data_ptr() % 16 != 0
    cos, sin = (t.to(torch.bfloat16).to(DEV) for t in tables(1, s, d, 42))
    with torch.no_grad():
        got = impls.qk_norm_rope(q, k, qw, kw, cos, sin)
        want = impls.qk_norm_rope(q.clone(), k.clone(), qw.clone(), kw.clone(), cos, sin)
    for a, c in zip(got, want):
        assert torch.equal(a, c)
