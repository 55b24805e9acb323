"""Registers the MI355X kernels as one Popcorn backend.

    import popcorn, popcorn.kernels       # or: from popcorn_amd import compat as popcorn
    from popcorn_amd import backend
    backend.register(popcorn)

This is the whole integration: one `declare_backend` (core/sources.py:40-47)
and one `op.register(name, source=..., predicate=..., forward_only=...)` per
op (core/dispatcher.py:324-345), exactly what a backend module under
`popcorn/kernels/` does. Each registration is source-only: the
`popcorn_amd.impls` functions already carry the reference signatures, so
Popcorn calls them directly (core/dispatcher.py:184-201).

The backend's distribution is `popcorn-amd` at `popcorn_amd.__version__`
(setup.py), pinned as both bounds of the version gate; the gate resolves for
an installed copy, and in a source tree once `python -m popcorn_amd.build` (or
`__graft_entry__.build()`) has written the metadata beside the package.

The predicates only describe what the kernels cover -- tensors on a HIP
device, one floating dtype per call, the shapes the kernels implement.
Anything else is declined, and Popcorn serves it with the next eligible
implementation (the torch reference); inside the kernels an unsupported call
raises instead of falling back.
"""

from __future__ import annotations

from types import ModuleType
from typing import Any

import torch

from popcorn_amd import __version__

BACKEND = "mi355x"
DISTRIBUTION = "popcorn-amd"


def _on_hip(*tensors: Any) -> bool:
    ts = [t for t in tensors if t is not None]
    return (
        torch.version.hip is not None
        and all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in ts)
        and len({t.device for t in ts}) == 1
    )


_FLOATS = (torch.float32, torch.bfloat16, torch.float16)
_HALF = (torch.bfloat16, torch.float16)


def rms_norm_supported(x, weight, bias, eps) -> bool:
    """One float dtype, or a 16-bit x with fp32 weight and bias (the output promotes to fp32)."""
    return (
        _on_hip(x, weight, bias)
        and x.dtype in _FLOATS
        and (weight.dtype == x.dtype or (x.dtype in _HALF and weight.dtype == torch.float32))
        and (bias is None or bias.dtype == weight.dtype)
        and x.shape[-1] > 0
    )


def add_rms_norm_supported(x, residual, weight, eps, offset) -> bool:
    return (
        _on_hip(x, residual, weight)
        and x.dtype == residual.dtype
        and x.dtype in _FLOATS
        and (weight.dtype == x.dtype or (x.dtype in _HALF and weight.dtype == torch.float32))
        and x.shape == residual.shape
        and x.shape[-1] > 0
    )


def swiglu_supported(a, b) -> bool:
    return _on_hip(a, b) and a.dtype == b.dtype and a.dtype in _FLOATS and a.shape == b.shape


def rotary_supported(x, cos, sin, interleaved) -> bool:
    return (
        _on_hip(x, cos, sin)
        and x.dtype in _FLOATS
        and cos.dtype in _FLOATS
        and cos.dtype == sin.dtype
        and x.dim() == 4
        and 2 * cos.shape[-1] <= x.shape[-1]
    )


def rope_supported(q, k, cos, sin) -> bool:
    """q, k one float dtype; cos, sin one float dtype (fp32 tables beside 16-bit q/k promote the outputs)."""
    return (
        _on_hip(q, k, cos, sin)
        and q.dtype in _FLOATS
        and q.dtype == k.dtype
        and cos.dtype in _FLOATS
        and cos.dtype == sin.dtype
        and q.dim() == k.dim() == 4
        and cos.dim() == 3
        and cos.shape == sin.shape
        and q.shape[-1] % 2 == 0
        and k.shape[0] == q.shape[0]
        and k.shape[2:] == q.shape[2:]
        and cos.shape[1:] == q.shape[2:]
        and cos.shape[0] in (1, q.shape[0])
    )


def _norm_rope_head_dim(head_dim: int, dtype: torch.dtype) -> bool:
    """head_dim / 2 = (16-byte pack) * 2^k with at most 64 packs: one row inside one wavefront."""
    pack = 16 // torch.empty((), dtype=dtype).element_size()
    half = head_dim // 2
    if head_dim % 2 or half % pack:
        return False
    packs = half // pack
    return 1 <= packs <= 64 and packs & (packs - 1) == 0


def qk_norm_rope_supported(q, k, q_weight, k_weight, cos, sin, eps) -> bool:
    return (
        _on_hip(q, k, q_weight, k_weight, cos, sin)
        and q.dtype in _FLOATS
        and q.dtype == k.dtype
        and q_weight.dtype == k_weight.dtype
        and (q_weight.dtype == q.dtype or (q.dtype in _HALF and q_weight.dtype == torch.float32))
        and cos.dtype in _FLOATS
        and cos.dtype == sin.dtype
        and q.dim() == k.dim() == 4
        and cos.dim() == 3
        and cos.shape == sin.shape
        and k.shape[0] == q.shape[0]
        and k.shape[2:] == q.shape[2:]
        and q_weight.shape == k_weight.shape == q.shape[-1:]
        and cos.shape[1:] == q.shape[2:]
        and cos.shape[0] in (1, q.shape[0])
        and _norm_rope_head_dim(q.shape[-1], q.dtype)
    )


def _attn_head_dim(head_dim: int) -> bool:
    """head_dim a multiple of 8 up to 256, in every dtype, forward and backward alike (so whether autograd
    records the call does not matter)."""
    return head_dim % 8 == 0 and 8 <= head_dim <= 256


def attn_supported(q, k, v, causal, softmax_scale) -> bool:
    return (
        _on_hip(q, k, v)
        and q.dtype in _FLOATS
        and q.dtype == k.dtype == v.dtype
        and _attn_head_dim(q.shape[-1])
        and k.shape[2] > 0
        and q.shape[2] % k.shape[2] == 0
    )


def attn_varlen_supported(q, k, v, cu_seqlens, causal, softmax_scale) -> bool:
    return (
        _on_hip(q, k, v)
        and isinstance(cu_seqlens, torch.Tensor)
        and not cu_seqlens.is_floating_point()
        and cu_seqlens.dim() == 1
        and q.dtype in _FLOATS
        and q.dtype == k.dtype == v.dtype
        and q.dim() == 3
        and _attn_head_dim(q.shape[-1])
        and k.shape[1] > 0
        and q.shape[1] % k.shape[1] == 0
    )


# (op, source, predicate, forward_only): every op has its backward kernels.
REGISTRATIONS = (
    ("rms_norm", "popcorn_amd.impls.rms_norm", rms_norm_supported, False),
    ("add_rms_norm", "popcorn_amd.impls.add_rms_norm", add_rms_norm_supported, False),
    ("swiglu", "popcorn_amd.impls.swiglu", swiglu_supported, False),
    ("rotary_embedding", "popcorn_amd.impls.rotary_embedding", rotary_supported, False),
    ("rope", "popcorn_amd.impls.rope", rope_supported, False),
    ("qk_norm_rope", "popcorn_amd.impls.qk_norm_rope", qk_norm_rope_supported, False),
    ("attn", "popcorn_amd.impls.attn", attn_supported, False),
    ("attn_varlen", "popcorn_amd.impls.attn_varlen", attn_varlen_supported, False),
)


def _popcorn() -> ModuleType:
    try:
        import popcorn
        import popcorn.kernels  # noqa: F401  registers Popcorn's ops

        return popcorn
    except ImportError:
        from popcorn_amd import compat

        return compat


def register(popcorn: ModuleType | None = None) -> ModuleType:
    """Declare the backend and register its ops on `popcorn` (default: the real package, else compat)."""
    pc = popcorn if popcorn is not None else _popcorn()
    pc.declare_backend(BACKEND, package=DISTRIBUTION, min_version=__version__, max_version=__version__)
    for op_name, source, predicate, forward_only in REGISTRATIONS:
        op = pc.KERNELS.get(op_name)
        if op is None:  # qk_norm_rope exists once defined (Popcorn's notebook does; compat ships it)
            continue
        if BACKEND not in op.available_backends():  # registering twice is a no-op, not an error
            op.register(BACKEND, source=source, predicate=predicate, forward_only=forward_only)
    return pc
