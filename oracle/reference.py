"""CPU oracle: float64 numpy restatement of Popcorn's transformer-block references.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import this module, and only as the
checker / the CPU figure. The product path (`popcorn_amd`) never calls it.

Every function restates the arithmetic of one Popcorn reference (cited
file:line under tilde-research/popcorn) in float64, with no rounding between
steps: this is the "truth" of Popcorn's comparison rule (bench/compare.py:205,
the reference evaluated on float64 clones), which removes every intermediate
cast. The forward formulas are Popcorn's; the backward formulas are the
closed-form derivatives of those forwards (Popcorn takes them from torch
autograd, bench/compare.py:243-278).

Pinning (tests/test_oracle.py): every function is checked against at least one
independent fact that a plausible slip would break:
  rms_norm          torch.nn.functional.rms_norm (float64); output RMS closed form;
                    scale invariance; zero row -> 0
  rms_norm_bwd      float64 autograd of F.rms_norm; central finite differences;
                    <dx, x> = 0 when w = 1, eps = 0; dw = sum dy*n
  add_rms_norm      float64 F.rms_norm of x + residual with weight + offset;
                    residual = 0, offset = 0 reduces to rms_norm
  add_rms_norm_bwd  float64 autograd through both outputs (y and s); central
                    finite differences; d(x) = d(residual)
  swiglu            scipy.special.expit formulation; silu(0) = 0; silu(x) -> x
  swiglu_bwd        central finite differences; float64 autograd of F.silu
  rotary_embedding  complex multiplication (x1 + i x2)(c + i s); identity tables;
                    norm preservation for unit tables; conjugate inverts forward
  rope              duplicated tables equal the NeoX rotary_embedding of q and k;
                    cos = 1, sin = 0 is the identity; cos = 0, sin = 1 is rotate_half;
                    explicit per-channel loops with unequal halves
  rope_bwd          central finite differences; <rope(x), g> = <x, rope_bwd(g)>;
                    duplicated unit tables: rope_bwd inverts rope
  qk_norm_rope      float64 torch F.rms_norm per head row then the complex rotation;
                    eps = 0: invariant under scaling each row; unit tables and unit
                    weights: every output row has RMS sqrt(ms / (ms + eps))
  qk_norm_rope_bwd  central finite differences for dq, dk and both weights; float64
                    torch autograd of F.rms_norm + rotate_half rope
  attention         explicit per-query loops; float64 SDPA with repeat_interleave;
                    q = 0 gives prefix means of v and lse = log(t + 1); S = 1 gives v
  attention_bwd     float64 torch autograd of SDPA (repeat_interleave grouping);
                    central finite differences; a scale of 0 gives dq = dk = 0
  attention_varlen_bwd  segments are independent; one segment equals attention_bwd
  attention_varlen  one segment equals `attention`; segments are independent
                    (changing one leaves the others' rows bit-identical);
                    length-1 segments give v
No function here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "rms_norm",
    "rms_norm_bwd",
    "add_rms_norm",
    "add_rms_norm_bwd",
    "swiglu",
    "swiglu_bwd",
    "rotary_embedding",
    "rotary_embedding_bwd",
    "attention",
    "attention_rows",
    "attention_varlen",
    "attention_bwd",
    "attention_varlen_bwd",
    "rope",
    "rope_bwd",
    "qk_norm_rope",
    "qk_norm_rope_bwd",
]


def _f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


def rms_norm(x, weight, bias=None, eps: float = 1e-6) -> np.ndarray:
    """y = x * rsqrt(mean(x^2, -1) + eps) * weight (+ bias).

    Follows kernels/rms_norm.py:29-30 and `rms` kernels/_utils.py:14-16
    (mean over the last axis, eps inside the square root).
    """
    x, w = _f64(x), _f64(weight)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * r * w
    return y if bias is None else y + _f64(bias)


def rms_norm_bwd(x, weight, dy, eps: float = 1e-6):
    """Gradients of `rms_norm` for cotangent dy: (dx, dweight, dbias).

    With r = (mean(x^2) + eps)^-1/2, n = x r, u = dy w:
      dx = r (u - n mean(u n)),  dweight = sum_rows dy n,  dbias = sum_rows dy.
    """
    x, w, g = _f64(x), _f64(weight), _f64(dy)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    n = x * r
    u = g * w
    dx = r * (u - n * np.mean(u * n, axis=-1, keepdims=True))
    lead = tuple(range(x.ndim - 1))
    return dx, np.sum(g * n, axis=lead), np.sum(g, axis=lead)


def add_rms_norm(x, residual, weight, eps: float = 1e-6, offset: float = 0.0):
    """(y, s) with s = x + residual and y = s * rsqrt(mean(s^2, -1) + eps) * (weight + offset).

    Follows kernels/add_rms_norm.py:25-26 (`s = x + residual`,
    `rms(s, eps) * (weight + offset)`, returning (y, s)).
    """
    s = _f64(x) + _f64(residual)
    return rms_norm(s, _f64(weight) + offset, None, eps), s


def add_rms_norm_bwd(x, residual, weight, dy, ds=None, eps: float = 1e-6, offset: float = 0.0):
    """Gradients of `add_rms_norm` for cotangents dy (of y) and ds (of s, or None):
    (dx, dresidual, dweight).

    The sum s feeds both outputs, so its gradient is the RMSNorm input gradient
    (with weight + offset) plus ds, and x and residual each receive it.
    """
    s = _f64(x) + _f64(residual)
    dsum, dw, _ = rms_norm_bwd(s, _f64(weight) + offset, dy, eps)
    if ds is not None:
        dsum = dsum + _f64(ds)
    return dsum, dsum.copy(), dw


def _sigmoid(a: np.ndarray) -> np.ndarray:
    # split by sign so exp never overflows
    out = np.empty_like(a)
    pos = a >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-a[pos]))
    e = np.exp(a[~pos])
    out[~pos] = e / (1.0 + e)
    return out


def swiglu(a, b) -> np.ndarray:
    """y = silu(a) * b, silu(a) = a * sigmoid(a). kernels/swiglu.py:18."""
    a, b = _f64(a), _f64(b)
    return a * _sigmoid(a) * b


def swiglu_bwd(dy, a, b):
    """(da, db) of `swiglu`: s = sigmoid(a); da = dy b s (1 + a (1 - s)); db = dy a s.

    The same closed form as impls/swiglu.cu:60-61.
    """
    g, a, b = _f64(dy), _f64(a), _f64(b)
    s = _sigmoid(a)
    return g * b * s * (1.0 + a * (1.0 - s)), g * a * s


def rotary_embedding(x, cos, sin, interleaved: bool = False) -> np.ndarray:
    """Rotate channel pairs of x [batch, seq, heads, head_dim] by cos/sin [seq, half].

    kernels/rotary_embedding.py:35-46: NeoX pairs (j, j + half) or GPT-J
    pairs (2j, 2j + 1); y1 = x1 c - x2 s, y2 = x1 s + x2 c; channels from
    2*half on are copied unchanged.
    """
    x = _f64(x)
    c = _f64(cos)[None, :, None, :]
    s = _f64(sin)[None, :, None, :]
    half = c.shape[-1]
    y = x.copy()
    if interleaved:
        x1, x2 = x[..., 0 : 2 * half : 2], x[..., 1 : 2 * half : 2]
        y[..., 0 : 2 * half : 2] = x1 * c - x2 * s
        y[..., 1 : 2 * half : 2] = x1 * s + x2 * c
    else:
        x1, x2 = x[..., :half], x[..., half : 2 * half]
        y[..., :half] = x1 * c - x2 * s
        y[..., half : 2 * half] = x1 * s + x2 * c
    return y


def rotary_embedding_bwd(dy, cos, sin, interleaved: bool = False) -> np.ndarray:
    """dx of `rotary_embedding`: the transpose of the rotation, i.e. rotation by -sin."""
    return rotary_embedding(dy, cos, -_f64(sin), interleaved)


def rope(q, k, cos, sin):
    """Paired rotary embedding (kernels/rope.py:23-36): x*cos + rotate_half(x)*sin for x in (q, k).

    q [B, Hq, S, D], k [B, Hkv, S, D], cos/sin [cos_batch, S, D] broadcast over
    heads (cos_batch 1 or B); rotate_half(x) = (-x[h:], x[:h]) with h = D/2
    (kernels/rope.py:8-10). The two halves of a table row may differ.
    """
    c, s = _f64(cos)[:, None], _f64(sin)[:, None]
    return tuple(x * c + _rotate_half(x) * s for x in (_f64(q), _f64(k)))


def rope_bwd(dq, dk, cos, sin):
    """(dq_in, dk_in) of `rope`: the transpose g*cos + rotate_half^T(g*sin), rotate_half^T = -rotate_half."""
    c, s = _f64(cos)[:, None], _f64(sin)[:, None]
    return tuple(g * c - _rotate_half(g * s) for g in (_f64(dq), _f64(dk)))


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps: float = 1e-6):
    """RMSNorm of every q and k head row (weights over head_dim) then `rope`.

    The kernel-writing notebook's reference (examples/03_write_a_kernel.ipynb,
    cell 3): `rms(q, eps) * q_weight`, `rms(k, eps) * k_weight` (`rms`,
    kernels/_utils.py:14-16), then kernels/rope.py:35-36.
    """
    return rope(rms_norm(q, q_weight, None, eps), rms_norm(k, k_weight, None, eps), cos, sin)


def qk_norm_rope_bwd(q, k, q_weight, k_weight, cos, sin, dyq, dyk, eps: float = 1e-6):
    """(dq, dk, dq_weight, dk_weight) of `qk_norm_rope`: rope's transpose, then the RMSNorm backward per side."""
    gq, gk = rope_bwd(dyq, dyk, cos, sin)
    dq, dqw, _ = rms_norm_bwd(q, q_weight, gq, eps)
    dk, dkw, _ = rms_norm_bwd(k, k_weight, gk, eps)
    return dq, dk, dqw, dkw


def _rotate_half(x: np.ndarray) -> np.ndarray:
    h = x.shape[-1] // 2
    return np.concatenate((-x[..., h:], x[..., :h]), axis=-1)


def attention_rows(q, k, v, rows, causal: bool, scale: float | None = None):
    """o and lse for selected query rows of one (batch, head): q [S, D], k, v [S, D].

    softmax(q k^T scale + M) v as in kernels/attn.py:30-37 (SDPA, top-left
    causal mask: key j visible to query i iff j <= i). lse = log sum exp of the
    masked scaled scores (natural log). Returns (o [len(rows), D], lse [len(rows)]).
    """
    q, k, v = _f64(q), _f64(k), _f64(v)
    d = q.shape[-1]
    scale = d**-0.5 if scale is None else scale
    rows = np.asarray(rows)
    out = np.empty((rows.size, v.shape[-1]))
    lse = np.empty(rows.size)
    for n, i in enumerate(rows):
        keys = k[: i + 1] if causal else k
        vals = v[: i + 1] if causal else v
        s = keys @ q[i] * scale
        m = s.max()
        p = np.exp(s - m)
        total = p.sum()
        out[n] = p @ vals / total
        lse[n] = m + np.log(total)
    return out, lse


def attention(q, k, v, causal: bool = False, scale: float | None = None):
    """Grouped-query attention over q [B, S, Hq, D], k, v [B, S, Hkv, D].

    q head h reads kv head h // (Hq / Hkv) (SDPA's enable_gqa grouping,
    kernels/attn.py:30-37). Returns (o [B, S, Hq, D], lse [B, Hq, S]).
    """
    q, k, v = _f64(q), _f64(k), _f64(v)
    batch, seq, hq, d = q.shape
    hkv = k.shape[2]
    if hq % hkv:
        raise ValueError("q heads must be a multiple of kv heads")
    group = hq // hkv
    scale = d**-0.5 if scale is None else scale
    o = np.empty_like(q)
    lse = np.empty((batch, hq, seq))
    mask = np.triu(np.ones((seq, seq), dtype=bool), 1) if causal else None
    for b in range(batch):
        for h in range(hq):
            kh, vh = k[b, :, h // group], v[b, :, h // group]
            s = q[b, :, h] @ kh.T * scale
            if mask is not None:
                s = np.where(mask, -np.inf, s)
            m = s.max(axis=-1, keepdims=True)
            p = np.exp(s - m)
            total = p.sum(axis=-1, keepdims=True)
            o[b, :, h] = p @ vh / total
            lse[b, h] = (m + np.log(total))[:, 0]
    return o, lse


def attention_varlen(q, k, v, cu_seqlens, causal: bool = False, scale: float | None = None):
    """Packed-sequence attention: q [total, Hq, D], k, v [total, Hkv, D], segments
    [cu[i], cu[i+1]) attended independently (kernels/attn_varlen.py:41-54).

    Returns (o [total, Hq, D], lse [Hq, total]).
    """
    q, k, v = _f64(q), _f64(k), _f64(v)
    bounds = [int(c) for c in np.asarray(cu_seqlens).tolist()]
    o = np.empty_like(q)
    lse = np.empty((q.shape[1], q.shape[0]))
    for lo, hi in zip(bounds, bounds[1:]):
        if hi == lo:
            continue
        oo, ll = attention(q[None, lo:hi], k[None, lo:hi], v[None, lo:hi], causal, scale)
        o[lo:hi] = oo[0]
        lse[:, lo:hi] = ll[0]
    return o, lse


def attention_bwd(q, k, v, do, causal: bool = False, scale: float | None = None):
    """Gradients of `attention` for cotangent do: (dq, dk, dv), shapes of q, k, v.

    Per (batch, q head) with z = scale q k^T (+ mask), P = softmax(z), o = P v:
      dv += P^T do,  dP = do v^T,  dz = P (dP - rowsum(do * o)),
      dq = scale dz k,  dk += scale dz^T q,
    where dk and dv of a kv head sum over the q heads that read it (h // group).
    """
    q, k, v, g = _f64(q), _f64(k), _f64(v), _f64(do)
    batch, seq, hq, d = q.shape
    hkv = k.shape[2]
    group = hq // hkv
    scale = d**-0.5 if scale is None else scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    mask = np.triu(np.ones((seq, seq), dtype=bool), 1) if causal else None
    for b in range(batch):
        for h in range(hq):
            kh, vh = k[b, :, h // group], v[b, :, h // group]
            z = q[b, :, h] @ kh.T * scale
            if mask is not None:
                z = np.where(mask, -np.inf, z)
            z = z - z.max(axis=-1, keepdims=True)
            p = np.exp(z)
            p /= p.sum(axis=-1, keepdims=True)
            o = p @ vh
            gh = g[b, :, h]
            dv[b, :, h // group] += p.T @ gh
            dp = gh @ vh.T
            dz = p * (dp - np.sum(gh * o, axis=-1, keepdims=True))
            dq[b, :, h] = scale * dz @ kh
            dk[b, :, h // group] += scale * dz.T @ q[b, :, h]
    return dq, dk, dv


def attention_varlen_bwd(q, k, v, do, cu_seqlens, causal: bool = False, scale: float | None = None):
    """Gradients of `attention_varlen` (dq, dk, dv), segment by segment."""
    q, k, v, g = _f64(q), _f64(k), _f64(v), _f64(do)
    bounds = [int(c) for c in np.asarray(cu_seqlens).tolist()]
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for lo, hi in zip(bounds, bounds[1:]):
        if hi == lo:
            continue
        a, b_, c = attention_bwd(q[None, lo:hi], k[None, lo:hi], v[None, lo:hi], g[None, lo:hi], causal, scale)
        dq[lo:hi], dk[lo:hi], dv[lo:hi] = a[0], b_[0], c[0]
    return dq, dk, dv
