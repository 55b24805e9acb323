"""Pins the float64 CPU oracle (oracle/reference.py) against facts it does not restate.

Each oracle function is checked against at least one independent route to the
same numbers (a library routine, a different formulation, finite differences
or a closed-form special case), chosen so that a plausible slip in the oracle
-- a dropped eps, a transposed operand, a sign error, a wrong GQA head map, an
off-by-one in the causal mask -- fails at least one test. The last test plants
such slips in copies of the oracle and shows the checks catch them.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.special
import torch
import torch.nn.functional as F

from oracle import reference as O


def rng(seed=0):
    return np.random.default_rng(seed)


# --------------------------------------------------------------------------- rms_norm


def test_rms_norm_matches_torch_functional():
    r = rng(1)
    x = r.standard_normal((5, 3, 48))
    w = 1 + 0.1 * r.standard_normal(48)
    for eps in (1e-6, 1e-5, 0.3):
        want = F.rms_norm(torch.from_numpy(x), (48,), torch.from_numpy(w), eps=eps).numpy()
        np.testing.assert_allclose(O.rms_norm(x, w, None, eps), want, rtol=1e-13, atol=1e-13)


def test_rms_norm_bias_is_added_after_scaling():
    r = rng(2)
    x, w, b = r.standard_normal((4, 16)), r.standard_normal(16), r.standard_normal(16)
    np.testing.assert_allclose(O.rms_norm(x, w, b) - O.rms_norm(x, w), np.broadcast_to(b, x.shape), atol=1e-14)


def test_rms_norm_output_rms_closed_form():
    """With w = 1: rms(y) = sqrt(ms / (ms + eps)) where ms = mean(x^2)."""
    r = rng(3)
    x = r.standard_normal((7, 33)) * np.arange(1, 8)[:, None]
    eps = 0.05
    y = O.rms_norm(x, np.ones(33), None, eps)
    ms = np.mean(x * x, axis=-1)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), np.sqrt(ms / (ms + eps)), rtol=1e-13)


def test_rms_norm_scale_invariance_and_zero_row():
    r = rng(4)
    x, w = r.standard_normal((3, 64)), r.standard_normal(64)
    np.testing.assert_allclose(O.rms_norm(7.5 * x, w, None, 0.0), O.rms_norm(x, w, None, 0.0), rtol=1e-12)
    z = O.rms_norm(np.zeros((2, 64)), w, None, 1e-6)
    assert np.all(z == 0)


def _finite_diff(f, x, h=1e-6):
    g = np.zeros_like(x)
    flat, gf = x.reshape(-1), g.reshape(-1)
    for i in range(flat.size):
        old = flat[i]
        flat[i] = old + h
        up = f()
        flat[i] = old - h
        down = f()
        flat[i] = old
        gf[i] = (up - down) / (2 * h)
    return g


def test_rms_norm_bwd_finite_differences():
    r = rng(5)
    x, w, b = r.standard_normal((3, 8)), 1 + 0.2 * r.standard_normal(8), r.standard_normal(8)
    dy = r.standard_normal((3, 8))
    eps = 1e-2
    loss = lambda: float(np.sum(O.rms_norm(x, w, b, eps) * dy))  # noqa: E731
    dx, dw, db = O.rms_norm_bwd(x, w, dy, eps)
    np.testing.assert_allclose(dx, _finite_diff(loss, x), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dw, _finite_diff(loss, w), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(db, _finite_diff(loss, b), rtol=1e-6, atol=1e-8)


def test_rms_norm_bwd_matches_torch_autograd():
    r = rng(6)
    x, w, dy = r.standard_normal((2, 5, 32)), r.standard_normal(32), r.standard_normal((2, 5, 32))
    xt, wt = torch.from_numpy(x).requires_grad_(), torch.from_numpy(w).requires_grad_()
    y = F.rms_norm(xt, (32,), wt, eps=1e-6)
    gx, gw = torch.autograd.grad(y, (xt, wt), torch.from_numpy(dy))
    dx, dw, _ = O.rms_norm_bwd(x, w, dy, 1e-6)
    np.testing.assert_allclose(dx, gx.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(dw, gw.numpy(), rtol=1e-11, atol=1e-12)


def test_rms_norm_bwd_orthogonal_to_x():
    """With w = 1 and eps = 0, y is invariant to scaling x, so <dx, x> = 0 per row."""
    r = rng(7)
    x, dy = r.standard_normal((4, 40)), r.standard_normal((4, 40))
    dx, _, _ = O.rms_norm_bwd(x, np.ones(40), dy, 0.0)
    np.testing.assert_allclose(np.sum(dx * x, axis=-1), 0.0, atol=1e-12)


# --------------------------------------------------------------------------- add_rms_norm


def test_add_rms_norm_matches_torch_functional():
    r = rng(41)
    x, res = r.standard_normal((3, 5, 40)), r.standard_normal((3, 5, 40))
    w = 1 + 0.1 * r.standard_normal(40)
    for eps, offset in ((1e-6, 0.0), (1e-5, 1.0), (0.2, -0.5)):
        y, s = O.add_rms_norm(x, res, w, eps, offset)
        st = torch.from_numpy(x) + torch.from_numpy(res)
        want = F.rms_norm(st, (40,), torch.from_numpy(w) + offset, eps=eps).numpy()
        np.testing.assert_allclose(y, want, rtol=1e-13, atol=1e-13)
        np.testing.assert_array_equal(s, x + res)


def test_add_rms_norm_reduces_to_rms_norm():
    r = rng(42)
    x, w = r.standard_normal((6, 24)), r.standard_normal(24)
    y, s = O.add_rms_norm(x, np.zeros_like(x), w, 1e-6, 0.0)
    np.testing.assert_array_equal(y, O.rms_norm(x, w, None, 1e-6))
    np.testing.assert_array_equal(s, x)


def test_add_rms_norm_bwd_matches_torch_autograd_through_both_outputs():
    r = rng(43)
    x, res, dy, ds = (r.standard_normal((4, 2, 32)) for _ in range(4))
    w = 1 + 0.1 * r.standard_normal(32)
    for offset, with_ds in ((0.0, True), (1.0, True), (1.0, False)):
        xt, rt, wt = (torch.from_numpy(a).requires_grad_() for a in (x, res, w))
        st = xt + rt
        yt = F.rms_norm(st, (32,), wt + offset, eps=1e-5)
        loss = (yt * torch.from_numpy(dy)).sum() + ((st * torch.from_numpy(ds)).sum() if with_ds else 0.0)
        gx, gr, gw = torch.autograd.grad(loss, (xt, rt, wt))
        dx, dres, dw = O.add_rms_norm_bwd(x, res, w, dy, ds if with_ds else None, 1e-5, offset)
        np.testing.assert_allclose(dx, gx.numpy(), rtol=1e-11, atol=1e-12)
        np.testing.assert_allclose(dres, gr.numpy(), rtol=1e-11, atol=1e-12)
        np.testing.assert_allclose(dw, gw.numpy(), rtol=1e-11, atol=1e-12)


def test_add_rms_norm_bwd_finite_differences():
    r = rng(44)
    x, res, dy, ds = (r.standard_normal((2, 7)) for _ in range(4))
    w = r.standard_normal(7)
    eps, offset, h = 1e-3, 0.75, 1e-6

    def loss(xv, rv, wv):
        y, s = O.add_rms_norm(xv, rv, wv, eps, offset)
        return float(np.sum(y * dy) + np.sum(s * ds))

    dx, dres, dw = O.add_rms_norm_bwd(x, res, w, dy, ds, eps, offset)
    for grad, which in ((dx, 0), (dres, 1), (dw, 2)):
        args = [x, res, w]
        base = args[which]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            plus, minus = base.copy(), base.copy()
            plus[idx] += h
            minus[idx] -= h
            a_p, a_m = list(args), list(args)
            a_p[which], a_m[which] = plus, minus
            num[idx] = (loss(*a_p) - loss(*a_m)) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-7)


# --------------------------------------------------------------------------- swiglu


def test_swiglu_matches_expit():
    a = np.linspace(-80, 80, 2001)
    b = rng(8).standard_normal(a.shape)
    np.testing.assert_allclose(O.swiglu(a, b), a * scipy.special.expit(a) * b, rtol=1e-14, atol=1e-300)


def test_swiglu_special_values():
    b = np.ones(4)
    y = O.swiglu(np.array([0.0, 50.0, -50.0, 1.0]), b)
    assert y[0] == 0.0
    assert abs(y[1] - 50.0) < 1e-15 * 50
    assert abs(y[2]) < 1e-19
    assert abs(y[3] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-15


def test_swiglu_bwd_finite_differences_and_autograd():
    r = rng(9)
    a, b, g = r.standard_normal((3, 7)) * 3, r.standard_normal((3, 7)), r.standard_normal((3, 7))
    loss = lambda: float(np.sum(O.swiglu(a, b) * g))  # noqa: E731
    da, db = O.swiglu_bwd(g, a, b)
    np.testing.assert_allclose(da, _finite_diff(loss, a), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(db, _finite_diff(loss, b), rtol=1e-6, atol=1e-8)
    at, bt = torch.from_numpy(a).requires_grad_(), torch.from_numpy(b).requires_grad_()
    gat, gbt = torch.autograd.grad(F.silu(at) * bt, (at, bt), torch.from_numpy(g))
    np.testing.assert_allclose(da, gat.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(db, gbt.numpy(), rtol=1e-12, atol=1e-14)


# --------------------------------------------------------------------------- rotary


def _tables(seq, half, theta=10000.0):
    pos = np.arange(seq)[:, None]
    ang = pos * theta ** (-np.arange(half) / half)
    return np.cos(ang), np.sin(ang)


def test_rotary_neox_is_complex_multiplication():
    r = rng(10)
    x = r.standard_normal((2, 6, 3, 16))
    c, s = r.standard_normal((6, 8)), r.standard_normal((6, 8))
    z = (x[..., :8] + 1j * x[..., 8:]) * (c + 1j * s)[None, :, None, :]
    want = np.concatenate([z.real, z.imag], axis=-1)
    np.testing.assert_allclose(O.rotary_embedding(x, c, s), want, rtol=1e-13, atol=1e-13)


def test_rotary_interleaved_is_complex_multiplication_of_pairs():
    r = rng(11)
    x = r.standard_normal((1, 5, 2, 12))
    c, s = r.standard_normal((5, 6)), r.standard_normal((5, 6))
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * (c + 1j * s)[None, :, None, :]
    want = np.stack([z.real, z.imag], axis=-1).reshape(x.shape)
    np.testing.assert_allclose(O.rotary_embedding(x, c, s, interleaved=True), want, rtol=1e-13, atol=1e-13)


def test_rotary_identity_tables_and_partial_passthrough():
    r = rng(12)
    x = r.standard_normal((2, 4, 3, 20))
    c, s = np.ones((4, 6)), np.zeros((4, 6))
    np.testing.assert_array_equal(O.rotary_embedding(x, c, s), x)
    c2, s2 = _tables(4, 6)
    y = O.rotary_embedding(x, c2, s2)
    np.testing.assert_array_equal(y[..., 12:], x[..., 12:])
    assert not np.allclose(y[..., :12], x[..., :12])


def test_rotary_unit_tables_preserve_pair_norms_and_conjugate_inverts():
    r = rng(13)
    x = r.standard_normal((2, 9, 4, 32))
    c, s = _tables(9, 16, 500000.0)
    for il in (False, True):
        y = O.rotary_embedding(x, c, s, il)
        if il:
            nx, ny = x[..., 0::2] ** 2 + x[..., 1::2] ** 2, y[..., 0::2] ** 2 + y[..., 1::2] ** 2
        else:
            nx, ny = x[..., :16] ** 2 + x[..., 16:] ** 2, y[..., :16] ** 2 + y[..., 16:] ** 2
        np.testing.assert_allclose(ny, nx, rtol=1e-12)
        np.testing.assert_allclose(O.rotary_embedding_bwd(y, c, s, il), x, rtol=1e-12, atol=1e-12)


def test_rotary_bwd_is_transpose_by_finite_differences():
    r = rng(14)
    x = r.standard_normal((1, 3, 2, 8))
    c, s, g = r.standard_normal((3, 4)), r.standard_normal((3, 4)), r.standard_normal((1, 3, 2, 8))
    for il in (False, True):
        loss = lambda: float(np.sum(O.rotary_embedding(x, c, s, il) * g))  # noqa: E731
        np.testing.assert_allclose(O.rotary_embedding_bwd(g, c, s, il), _finite_diff(loss, x), rtol=1e-6, atol=1e-8)


def _dup(t):
    """[..., half] -> [..., 2*half] with the row repeated (Popcorn's rope table convention)."""
    return np.concatenate([t, t], axis=-1)


def test_rope_with_duplicated_tables_is_neox_rotary_of_q_and_k():
    r = rng(15)
    b, hq, hkv, seq, d = 2, 4, 2, 7, 16
    q, k = r.standard_normal((b, hq, seq, d)), r.standard_normal((b, hkv, seq, d))
    c, s = r.standard_normal((seq, d // 2)), r.standard_normal((seq, d // 2))
    yq, yk = O.rope(q, k, _dup(c)[None], _dup(s)[None])
    for x, y in ((q, yq), (k, yk)):
        want = O.rotary_embedding(x.transpose(0, 2, 1, 3), c, s).transpose(0, 2, 1, 3)
        np.testing.assert_allclose(y, want, rtol=1e-13, atol=1e-13)
    # cos_batch = batch: each batch row uses its own table
    cb, sb = r.standard_normal((b, seq, d // 2)), r.standard_normal((b, seq, d // 2))
    yq, yk = O.rope(q, k, _dup(cb), _dup(sb))
    for i in range(b):
        want = O.rotary_embedding(q[i : i + 1].transpose(0, 2, 1, 3), cb[i], sb[i]).transpose(0, 2, 1, 3)
        np.testing.assert_allclose(yq[i : i + 1], want, rtol=1e-13, atol=1e-13)


def test_rope_identity_and_rotate_half_tables():
    r = rng(16)
    q, k = r.standard_normal((1, 3, 5, 8)), r.standard_normal((1, 1, 5, 8))
    one, zero = np.ones((1, 5, 8)), np.zeros((1, 5, 8))
    for x, y in zip((q, k), O.rope(q, k, one, zero)):
        np.testing.assert_array_equal(y, x)
    for x, y in zip((q, k), O.rope(q, k, zero, one)):
        np.testing.assert_array_equal(y[..., :4], -x[..., 4:])
        np.testing.assert_array_equal(y[..., 4:], x[..., :4])


def test_rope_unequal_halves_by_explicit_loops():
    r = rng(17)
    b, h, seq, d = 2, 2, 3, 6
    q, k = r.standard_normal((b, h, seq, d)), r.standard_normal((b, 1, seq, d))
    c, s = r.standard_normal((b, seq, d)), r.standard_normal((b, seq, d))
    yq, _ = O.rope(q, k, c, s)
    half = d // 2
    for i in range(b):
        for hh in range(h):
            for t in range(seq):
                for j in range(d):
                    partner = -q[i, hh, t, j + half] if j < half else q[i, hh, t, j - half]
                    want = q[i, hh, t, j] * c[i, t, j] + partner * s[i, t, j]
                    assert abs(yq[i, hh, t, j] - want) < 1e-14


def test_rope_bwd_is_the_adjoint():
    r = rng(18)
    q, k = r.standard_normal((1, 2, 3, 8)), r.standard_normal((1, 1, 3, 8))
    c, s = r.standard_normal((1, 3, 8)), r.standard_normal((1, 3, 8))
    gq, gk = r.standard_normal(q.shape), r.standard_normal(k.shape)
    dq, dk = O.rope_bwd(gq, gk, c, s)
    loss = lambda: float(sum(np.sum(y * g) for y, g in zip(O.rope(q, k, c, s), (gq, gk))))  # noqa: E731
    np.testing.assert_allclose(dq, _finite_diff(loss, q), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dk, _finite_diff(loss, k), rtol=1e-6, atol=1e-8)
    # unit duplicated tables: a rotation, so the adjoint inverts it
    cu, su = _tables(3, 4)
    cu, su = _dup(cu)[None], _dup(su)[None]
    back = O.rope_bwd(*O.rope(q, k, cu, su), cu, su)
    np.testing.assert_allclose(back[0], q, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(back[1], k, rtol=1e-12, atol=1e-12)


def _qknr_torch64(q, k, qw, kw, c, s, eps):
    """float64 torch: F.rms_norm over head rows, then y = n*cos + rotate_half(n)*sin."""
    out = []
    for x, w in ((q, qw), (k, kw)):
        n = torch.nn.functional.rms_norm(torch.from_numpy(x), (x.shape[-1],), torch.from_numpy(w), eps)
        h = x.shape[-1] // 2
        rot = torch.cat((-n[..., h:], n[..., :h]), -1)
        out.append(n * torch.from_numpy(c)[:, None] + rot * torch.from_numpy(s)[:, None])
    return out


def test_qk_norm_rope_matches_float64_torch_and_its_invariants():
    r = rng(19)
    b, hq, hkv, seq, d = 2, 4, 2, 5, 16
    q, k = r.standard_normal((b, hq, seq, d)), r.standard_normal((b, hkv, seq, d))
    qw, kw = r.standard_normal(d), r.standard_normal(d)
    for cb in (1, b):
        c, s = r.standard_normal((cb, seq, d)), r.standard_normal((cb, seq, d))
        for got, want in zip(O.qk_norm_rope(q, k, qw, kw, c, s, 1e-5), _qknr_torch64(q, k, qw, kw, c, s, 1e-5)):
            np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)
    # eps = 0: each head row may be scaled by any positive factor
    c, s = r.standard_normal((1, seq, d)), r.standard_normal((1, seq, d))
    scale = np.exp(r.standard_normal((b, hq, seq, 1)))
    a1 = O.qk_norm_rope(q, k, qw, kw, c, s, 0.0)[0]
    a2 = O.qk_norm_rope(q * scale, k, qw, kw, c, s, 0.0)[0]
    np.testing.assert_allclose(a1, a2, rtol=1e-12, atol=1e-12)
    # unit weights, rotation tables: row RMS is sqrt(ms / (ms + eps))
    cu, su = _tables(seq, d // 2)
    cu, su = _dup(cu)[None], _dup(su)[None]
    eps = 0.3
    y = O.qk_norm_rope(q, k, np.ones(d), np.ones(d), cu, su, eps)[0]
    ms = np.mean(q * q, axis=-1)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), np.sqrt(ms / (ms + eps)), rtol=1e-12)


def test_qk_norm_rope_bwd_by_finite_differences_and_autograd():
    r = rng(20)
    b, hq, hkv, seq, d = 1, 2, 1, 3, 8
    q, k = r.standard_normal((b, hq, seq, d)), r.standard_normal((b, hkv, seq, d))
    qw, kw = r.standard_normal(d), r.standard_normal(d)
    c, s = r.standard_normal((1, seq, d)), r.standard_normal((1, seq, d))
    gq, gk = r.standard_normal(q.shape), r.standard_normal(k.shape)
    eps = 1e-3
    dq, dk, dqw, dkw = O.qk_norm_rope_bwd(q, k, qw, kw, c, s, gq, gk, eps)

    def loss():
        yq, yk = O.qk_norm_rope(q, k, qw, kw, c, s, eps)
        return float(np.sum(yq * gq) + np.sum(yk * gk))

    for got, x in ((dq, q), (dk, k), (dqw, qw), (dkw, kw)):
        np.testing.assert_allclose(got, _finite_diff(loss, x), rtol=1e-6, atol=1e-7)
    leaves = [torch.from_numpy(t.copy()).requires_grad_() for t in (q, k, qw, kw)]
    tq, tk, tqw, tkw = leaves
    outs = []
    for x, w in ((tq, tqw), (tk, tkw)):
        n = torch.nn.functional.rms_norm(x, (d,), w, eps)
        rot = torch.cat((-n[..., d // 2:], n[..., : d // 2]), -1)
        outs.append(n * torch.from_numpy(c)[:, None] + rot * torch.from_numpy(s)[:, None])
    grads = torch.autograd.grad(outs, leaves, [torch.from_numpy(gq), torch.from_numpy(gk)])
    for got, want in zip((dq, dk, dqw, dkw), grads):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------------------- attention


def _sdpa64(q, k, v, causal, scale):
    """float64 torch SDPA on [B, H, S, D] with kv heads repeated per group."""
    group = q.shape[2] // k.shape[2]
    qt = torch.from_numpy(q).transpose(1, 2)
    kt = torch.from_numpy(k).repeat_interleave(group, dim=2).transpose(1, 2)
    vt = torch.from_numpy(v).repeat_interleave(group, dim=2).transpose(1, 2)
    return F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, scale=scale).transpose(1, 2).numpy()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [None, 0.25])
def test_attention_matches_float64_sdpa(causal, scale):
    r = rng(15)
    q, k, v = r.standard_normal((2, 11, 6, 8)), r.standard_normal((2, 11, 2, 8)), r.standard_normal((2, 11, 2, 8))
    o, lse = O.attention(q, k, v, causal, scale)
    np.testing.assert_allclose(o, _sdpa64(q, k, v, causal, scale), rtol=1e-12, atol=1e-12)
    # lse against scipy's logsumexp of explicitly masked scores
    sc = 8**-0.5 if scale is None else scale
    for b, h in [(0, 0), (1, 5)]:
        s = q[b, :, h] @ k[b, :, h // 3].T * sc
        if causal:
            s = np.where(np.triu(np.ones((11, 11), bool), 1), -np.inf, s)
        np.testing.assert_allclose(lse[b, h], scipy.special.logsumexp(s, axis=-1), rtol=1e-13)


def test_attention_rows_agree_with_full():
    r = rng(16)
    q, k, v = r.standard_normal((1, 13, 4, 8)), r.standard_normal((1, 13, 1, 8)), r.standard_normal((1, 13, 1, 8))
    o, lse = O.attention(q, k, v, True)
    rows = np.array([0, 5, 12])
    oo, ll = O.attention_rows(q[0, :, 3], k[0, :, 0], v[0, :, 0], rows, True)
    np.testing.assert_allclose(oo, o[0, rows, 3], rtol=1e-13)
    np.testing.assert_allclose(ll, lse[0, 3, rows], rtol=1e-13)


def test_attention_special_cases():
    r = rng(17)
    s, d = 9, 4
    v = r.standard_normal((1, s, 1, d))
    k = r.standard_normal((1, s, 1, d))
    o, lse = O.attention(np.zeros((1, s, 2, d)), k, v, True)
    prefix = np.cumsum(v[0, :, 0], axis=0) / np.arange(1, s + 1)[:, None]
    np.testing.assert_allclose(o[0, :, 1], prefix, rtol=1e-13)
    np.testing.assert_allclose(lse[0, 0], np.log(np.arange(1, s + 1)), rtol=1e-13)
    # the first query sees only key 0 under the causal mask
    q = r.standard_normal((1, s, 2, d))
    o, _ = O.attention(q, k, v, True)
    np.testing.assert_allclose(o[0, 0, 0], v[0, 0, 0], rtol=1e-13)
    # a single position: o = v
    o1, l1 = O.attention(q[:, :1], k[:, :1], v[:, :1], False)
    np.testing.assert_allclose(o1[0, 0, 1], v[0, 0, 0], rtol=1e-13)


def test_attention_gqa_head_map():
    """q head h reads kv head h // group, not h % kv_heads."""
    r = rng(18)
    q = r.standard_normal((1, 5, 4, 8))
    k, v = r.standard_normal((1, 5, 2, 8)), r.standard_normal((1, 5, 2, 8))
    o, _ = O.attention(q, k, v, False)
    o1, _ = O.attention(q[:, :, 1:2], k[:, :, 0:1], v[:, :, 0:1], False)
    np.testing.assert_allclose(o[:, :, 1:2], o1, rtol=1e-13)


# --------------------------------------------------------------------------- attention_varlen


def test_attention_varlen_single_segment_is_dense_attention():
    r = rng(51)
    q, k, v = r.standard_normal((13, 4, 8)), r.standard_normal((13, 2, 8)), r.standard_normal((13, 2, 8))
    for causal in (False, True):
        o, lse = O.attention_varlen(q, k, v, [0, 13], causal, 0.4)
        od, ld = O.attention(q[None], k[None], v[None], causal, 0.4)
        np.testing.assert_array_equal(o, od[0])
        np.testing.assert_array_equal(lse, ld[0])


def test_attention_varlen_segments_are_independent():
    r = rng(52)
    q, k, v = r.standard_normal((20, 4, 8)), r.standard_normal((20, 1, 8)), r.standard_normal((20, 1, 8))
    cu = [0, 7, 8, 20]
    o, lse = O.attention_varlen(q, k, v, cu, True)
    k2, v2 = k.copy(), v.copy()
    k2[8:] += 5.0
    v2[8:] -= 3.0
    o2, lse2 = O.attention_varlen(q, k2, v2, cu, True)
    np.testing.assert_array_equal(o[:8], o2[:8])  # the first two segments never see the third
    np.testing.assert_array_equal(lse[:, :8], lse2[:, :8])
    assert not np.allclose(o[8:], o2[8:])
    np.testing.assert_allclose(o[7], np.repeat(v[7], 4, axis=0), rtol=1e-15)  # length-1 segment: o = v
    # matches float64 SDPA run per segment
    for lo, hi in zip(cu, cu[1:]):
        qt = torch.from_numpy(q[lo:hi]).transpose(0, 1)
        kt = torch.from_numpy(k[lo:hi]).repeat_interleave(4, 1).transpose(0, 1)
        vt = torch.from_numpy(v[lo:hi]).repeat_interleave(4, 1).transpose(0, 1)
        want = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True).transpose(0, 1).numpy()
        np.testing.assert_allclose(o[lo:hi], want, rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------------------- attention backward


def test_attention_bwd_matches_torch_autograd():
    r = rng(61)
    q, do = r.standard_normal((2, 9, 4, 8)), r.standard_normal((2, 9, 4, 8))
    k, v = r.standard_normal((2, 9, 2, 8)), r.standard_normal((2, 9, 2, 8))
    # (torch's SDPA gives NaN for a negative scale under its causal mask, so that sign is checked unmasked)
    for causal, scale in ((False, None), (True, 0.3), (False, -0.5)):
        qt, kt, vt = (torch.from_numpy(t).requires_grad_() for t in (q, k, v))
        out = F.scaled_dot_product_attention(qt.transpose(1, 2), kt.repeat_interleave(2, 2).transpose(1, 2),
                                             vt.repeat_interleave(2, 2).transpose(1, 2), is_causal=causal,
                                             scale=scale).transpose(1, 2)
        gq, gk, gv = torch.autograd.grad(out, (qt, kt, vt), torch.from_numpy(do))
        dq, dk, dv = O.attention_bwd(q, k, v, do, causal, scale)
        np.testing.assert_allclose(dq, gq.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(dk, gk.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(dv, gv.numpy(), rtol=1e-10, atol=1e-12)


def test_attention_bwd_finite_differences():
    r = rng(62)
    q, do = r.standard_normal((1, 4, 2, 3)), r.standard_normal((1, 4, 2, 3))
    k, v = r.standard_normal((1, 4, 1, 3)), r.standard_normal((1, 4, 1, 3))
    h = 1e-6
    dq, dk, dv = O.attention_bwd(q, k, v, do, True, 0.7)

    def loss(qq, kk, vv):
        return float(np.sum(O.attention(qq, kk, vv, True, 0.7)[0] * do))

    for grad, which in ((dq, 0), (dk, 1), (dv, 2)):
        args = [q, k, v]
        base = args[which]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            plus, minus = base.copy(), base.copy()
            plus[idx] += h
            minus[idx] -= h
            ap, am = list(args), list(args)
            ap[which], am[which] = plus, minus
            num[idx] = (loss(*ap) - loss(*am)) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


def test_attention_bwd_zero_scale_and_varlen():
    r = rng(63)
    q, do = r.standard_normal((1, 6, 2, 4)), r.standard_normal((1, 6, 2, 4))
    k, v = r.standard_normal((1, 6, 2, 4)), r.standard_normal((1, 6, 2, 4))
    dq, dk, dv = O.attention_bwd(q, k, v, do, False, 0.0)  # uniform attention: no dependence on q or k
    assert np.abs(dq).max() == 0 and np.abs(dk).max() == 0
    np.testing.assert_allclose(dv[0, :, 0], np.broadcast_to(do[0, :, 0].mean(0), (6, 4)), rtol=1e-12)
    # varlen: two segments equal the dense backward of each segment
    cu = [0, 2, 6]
    vq, vk, vv, vdo = q[0], k[0], v[0], do[0]
    dqv, dkv, dvv = O.attention_varlen_bwd(vq, vk, vv, vdo, cu, True, 0.5)
    for lo, hi in zip(cu, cu[1:]):
        a, b_, c = O.attention_bwd(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], do[:, lo:hi], True, 0.5)
        np.testing.assert_array_equal(dqv[lo:hi], a[0])
        np.testing.assert_array_equal(dkv[lo:hi], b_[0])
        np.testing.assert_array_equal(dvv[lo:hi], c[0])


# --------------------------------------------------------------------------- planted mistakes


def test_planted_mistakes_are_caught(monkeypatch):
    """Copies of the oracle with a typical slip each fail one of the checks above."""
    r = rng(19)
    x, w = r.standard_normal((3, 16)), 1 + 0.1 * r.standard_normal(16)

    # rms_norm without eps
    bad = lambda x, w, b=None, eps=1e-6: x / np.sqrt(np.mean(x * x, -1, keepdims=True)) * w  # noqa: E731
    want = F.rms_norm(torch.from_numpy(x), (16,), torch.from_numpy(w), eps=0.3).numpy()
    assert not np.allclose(bad(x, w, None, 0.3), want, rtol=1e-6)

    # rotary with the sign of sin flipped
    xr = r.standard_normal((1, 3, 2, 8))
    c, s = r.standard_normal((3, 4)), r.standard_normal((3, 4))
    flipped = O.rotary_embedding(xr, c, -s)
    z = (xr[..., :4] + 1j * xr[..., 4:]) * (c + 1j * s)[None, :, None, :]
    assert not np.allclose(flipped, np.concatenate([z.real, z.imag], -1))

    # attention with kv head h % kv_heads instead of h // group
    q = r.standard_normal((1, 5, 4, 8))
    k, v = r.standard_normal((1, 5, 2, 8)), r.standard_normal((1, 5, 2, 8))
    k_mod = k[:, :, [0, 1, 0, 1]]
    v_mod = v[:, :, [0, 1, 0, 1]]
    o_bad, _ = O.attention(q, k_mod, v_mod, False)
    assert not np.allclose(o_bad, _sdpa64(q, k, v, False, None))

    # causal mask shifted by one (diagonal excluded)
    o_good, _ = O.attention(q, k, v, True)
    qt = torch.from_numpy(q).transpose(1, 2)
    kt = torch.from_numpy(k).repeat_interleave(2, 2).transpose(1, 2)
    vt = torch.from_numpy(v).repeat_interleave(2, 2).transpose(1, 2)
    strict = torch.ones(5, 5, dtype=torch.bool).tril(-1)
    strict[0, 0] = True  # keep row 0 defined
    o_shift = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=strict).transpose(1, 2).numpy()
    assert not np.allclose(o_good, o_shift)

    # swiglu backward missing the a*(1-s) term
    a, b, g = r.standard_normal(10) * 2, r.standard_normal(10), r.standard_normal(10)
    sg = scipy.special.expit(a)
    da_bad = g * b * sg
    da, _ = O.swiglu_bwd(g, a, b)
    assert not np.allclose(da, da_bad)

    # add_rms_norm backward that forgets the offset, or drops the gradient reaching s directly
    xa, ra, dya, dsa = (r.standard_normal((2, 12)) for _ in range(4))
    wa = 1 + 0.1 * r.standard_normal(12)
    xt, rt, wt = (torch.from_numpy(v).requires_grad_() for v in (xa, ra, wa))
    st = xt + rt
    loss = (F.rms_norm(st, (12,), wt + 1.0, eps=1e-6) * torch.from_numpy(dya)).sum() + (st * torch.from_numpy(dsa)).sum()
    gx, _, _ = torch.autograd.grad(loss, (xt, rt, wt))
    no_offset, _, _ = O.add_rms_norm_bwd(xa, ra, wa, dya, dsa, 1e-6, 0.0)
    no_ds, _, _ = O.add_rms_norm_bwd(xa, ra, wa, dya, None, 1e-6, 1.0)
    assert not np.allclose(no_offset, gx.numpy())
    assert not np.allclose(no_ds, gx.numpy())
