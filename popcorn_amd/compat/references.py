"""Popcorn's registered PyTorch references for the four transformer-block ops.

These are the op definitions of Popcorn: each is the `torch` implementation
its dispatcher always holds, and what its harness evaluates on float64 clones
for truth and at native dtype for the error budget. They are restated here in
eager torch with the same sequence of tensor ops, because that sequence fixes
the native-dtype rounding the budget measures:

    rms_norm          kernels/rms_norm.py:16-30 (`rms`, `upcast`: kernels/_utils.py:6-16)
    add_rms_norm      kernels/add_rms_norm.py:8-26
    swiglu            kernels/swiglu.py:9-18
    rotary_embedding  kernels/rotary_embedding.py:12-40
    rope              kernels/rope.py:8-36 (`_rotate_half`, `_table`: kernels/rope.py:8-14)
    qk_norm_rope      examples/03_write_a_kernel.ipynb, cell 3 (`rms`: kernels/_utils.py:14-16)
    attn              kernels/attn.py:10-37
    attn_varlen       kernels/attn_varlen.py:15-54 (`cuts`: kernels/_varlen.py:8-13)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor


def upcast(t: Tensor) -> Tensor:
    """The wider of t's dtype and fp32 (fp64 is kept)."""
    return t.to(torch.promote_types(t.dtype, torch.float32))


def rms(x: Tensor, eps: float) -> Tensor:
    """x / sqrt(mean(x^2) + eps) over the last dimension in >= fp32, rounded to x's dtype."""
    h = upcast(x)
    return (h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True) + eps)).to(x.dtype)


def rms_norm(x: Tensor, weight: Tensor, bias: Tensor | None = None, eps: float = 1e-6) -> Tensor:
    """Normalise in >= fp32, round to x's dtype, then scale (and shift) in that dtype."""
    y = rms(x, eps) * weight
    return y if bias is None else y + bias


def add_rms_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float = 1e-6,
                 offset: float = 0.0) -> tuple[Tensor, Tensor]:
    """s = x + residual at the inputs' dtype; (rms(s) rounded to that dtype) * (weight + offset); returns (y, s)."""
    s = x + residual
    h = upcast(s)
    normed = (h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True) + eps)).to(s.dtype)
    return normed * (weight + offset), s


def swiglu(a: Tensor, b: Tensor) -> Tensor:
    """silu(a) * b: two eager ops, so at 16-bit dtypes silu is rounded before the product."""
    return F.silu(a) * b


def rotary_embedding(x: Tensor, cos: Tensor, sin: Tensor, interleaved: bool = False) -> Tensor:
    """Rotate channel pairs in >= fp32 and round once; channels past 2*half pass through."""
    half = cos.shape[-1]
    c = upcast(cos.detach()).unsqueeze(1)  # [seq, 1, half], broadcast over batch and heads
    s = upcast(sin.detach()).unsqueeze(1)
    if interleaved:
        u, v = upcast(x[..., 0 : 2 * half : 2]), upcast(x[..., 1 : 2 * half : 2])
    else:
        u, v = upcast(x[..., :half]), upcast(x[..., half : 2 * half])
    first, second = u * c - v * s, u * s + v * c
    if interleaved:
        rotated = torch.stack((first, second), dim=-1).flatten(-2)
    else:
        rotated = torch.cat((first, second), dim=-1)
    rotated = rotated.to(x.dtype)
    if 2 * half == x.shape[-1]:
        return rotated
    return torch.cat((rotated, x[..., 2 * half :]), dim=-1)


def rotate_half(x: Tensor) -> Tensor:
    """(x1, x2) -> (-x2, x1) over the last dimension's halves."""
    x1, x2 = x.chunk(2, -1)
    return torch.cat((-x2, x1), -1)


def rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """x*cos + rotate_half(x)*sin for x in (q, k), eager at the inputs' dtype (three roundings per output).

    cos, sin [cos_batch, seq, head_dim] broadcast over heads and get no gradient.
    """
    cos, sin = cos.detach()[:, None], sin.detach()[:, None]
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def qk_norm_rope(q: Tensor, k: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor,
                 eps: float = 1e-6) -> tuple[Tensor, Tensor]:
    """`rms` of every q and k head row times its weight, then `rope`, eager at the inputs' dtype."""
    return rope(rms(q, eps) * q_weight, rms(k, eps) * k_weight, cos, sin)


def rope_table(f):
    """Popcorn's rope test-input transform: f of the draw with its first half repeated over the row."""
    return lambda t: f(t).chunk(2, -1)[0].repeat(1, 1, 2)


def attn(q: Tensor, k: Tensor, v: Tensor, causal: bool = False, softmax_scale: float | None = None) -> Tensor:
    """softmax(q k^T * scale + causal mask) v with grouped kv heads, in [batch, seq, heads, dim].

    On the CPU, and for 16-bit inputs on a HIP device, this is Popcorn's own
    call: SDPA on head-major views with enable_gqa=True (on the device limited
    to the fused flash / memory-efficient kernels). Torch's batched products
    on transposed 16-bit views have faulted MI355X boxes, so no device path
    reaches them: when no fused kernel takes the views, the kv heads are
    repeated per group (SDPA's enable_gqa grouping, q head h reads kv head
    h // group) into contiguous operands first, and fp32 / fp64 inputs take
    an explicit softmax over products of contiguous operands, one
    (batch, kv group) at a time.
    """
    heads_first = [t.transpose(1, 2) for t in (q, k, v)]
    if q.device.type != "cuda":
        out = F.scaled_dot_product_attention(*heads_first, scale=softmax_scale, is_causal=causal, enable_gqa=True)
        return out.transpose(1, 2)
    if q.dtype in (torch.float16, torch.bfloat16):
        from torch.nn.attention import SDPBackend, sdpa_kernel

        # Popcorn's own call, restricted to the fused kernels (on MI355X the flash
        # kernel takes grouped heads directly: 4.6 ms for B=4, S=8192, 32/8 heads,
        # causal, against 5.4 ms with the kv heads repeated first)
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                out = F.scaled_dot_product_attention(*heads_first, scale=softmax_scale, is_causal=causal,
                                                     enable_gqa=True)
            return out.transpose(1, 2)
        except RuntimeError:
            pass  # no fused kernel takes these views: repeat the kv heads below
    group = q.shape[2] // k.shape[2]
    qh = q.transpose(1, 2).contiguous()
    kh = k.repeat_interleave(group, dim=2).transpose(1, 2).contiguous()
    vh = v.repeat_interleave(group, dim=2).transpose(1, 2).contiguous()
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    if q.dtype in (torch.float16, torch.bfloat16):
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out = F.scaled_dot_product_attention(qh, kh, vh, scale=scale, is_causal=causal)
        return out.transpose(1, 2)
    # One (batch, kv group) at a time: the scores of a whole 4 x 32-head call at
    # 8192 tokens in float64 would need 69 GB per intermediate.
    out = torch.empty_like(qh)
    seq_q, seq_k = qh.shape[-2], kh.shape[-2]
    mask = torch.ones(seq_q, seq_k, dtype=torch.bool, device=q.device).triu(1) if causal else None
    for b in range(qh.shape[0]):
        for h0 in range(0, qh.shape[1], group):
            rows = slice(h0, h0 + group)
            scores = torch.matmul(qh[b, rows], kh[b, rows].transpose(-2, -1).contiguous()) * scale
            if mask is not None:
                scores = scores.masked_fill(mask, float("-inf"))
            out[b, rows] = torch.matmul(torch.softmax(scores, dim=-1), vh[b, rows])
    return out.transpose(1, 2)


def attn_varlen(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, causal: bool = False,
                softmax_scale: float | None = None) -> Tensor:
    """`attn` on each packed segment [cu[i], cu[i+1]) of [total, heads, dim] tensors, concatenated."""
    bounds = cu_seqlens.tolist()
    return torch.cat([
        attn(q[lo:hi][None], k[lo:hi][None], v[lo:hi][None], causal, softmax_scale)[0]
        for lo, hi in zip(bounds, bounds[1:])
    ])


def cuts(t: Tensor, dims, generator: torch.Generator) -> Tensor:
    """Random cu_seqlens for `total` tokens: len(t) - 1 non-empty segments, offsets from 0 to total.

    Popcorn's test-input transform for packed sequences (kernels/_varlen.py:8-13):
    the inner offsets are the first segments - 1 entries of a seeded random
    permutation of 1 .. total - 1, sorted.
    """
    total, segments = dims["total"], t.shape[-1] - 1
    if total < segments:
        raise ValueError(f"total={total} cannot hold {segments} non-empty segments")
    inner = (torch.randperm(total - 1, generator=generator)[: segments - 1] + 1).sort().values
    return torch.cat([torch.zeros(1, dtype=inner.dtype), inner, torch.full((1,), total, dtype=inner.dtype)]).int()
