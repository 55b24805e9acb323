"""MI355X implementations of Popcorn's transformer-block ops.

Each public function has exactly the reference's signature, so Popcorn can
register it as a bare `source=` (its leading parameters must equal the
reference's names, core/dispatcher.py:184-201), and returns new tensors of the
reference's output structure. Arithmetic happens in the HIP kernels of
`libpopcorn_amd.so`, launched on torch's current stream; there is no
host-side or torch fallback: an input the kernels do not cover raises.

    rms_norm(x, weight, bias=None, eps=1e-6)        kernels/rms_norm.py:16-30
    add_rms_norm(x, residual, weight, eps=1e-6, offset=0.0)  kernels/add_rms_norm.py:8-26
    swiglu(a, b)                                    kernels/swiglu.py:9-18
    rotary_embedding(x, cos, sin, interleaved=False) kernels/rotary_embedding.py:12-40
    rope(q, k, cos, sin)                            kernels/rope.py:19-36
    qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps=1e-6)
                                                    examples/03_write_a_kernel.ipynb, cell 3
    attn(q, k, v, causal=False, softmax_scale=None) kernels/attn.py:10-37
    attn_varlen(q, k, v, cu_seqlens, causal=False, softmax_scale=None)
                                                    kernels/attn_varlen.py:15-54
"""

from __future__ import annotations

import torch
from torch import Tensor

from popcorn_amd import _lib

__all__ = ["rms_norm", "add_rms_norm", "swiglu", "rotary_embedding", "attn", "attn_with_lse", "attn_varlen",
           "attn_varlen_with_lse", "rotary_embedding_", "rope",
           "qk_norm_rope"]


def _require_cuda(*tensors: Tensor | None) -> torch.device:
    devices = {t.device for t in tensors if t is not None}
    if len(devices) != 1:
        raise ValueError(f"popcorn_amd: tensors on several devices {sorted(map(str, devices))}")
    device = devices.pop()
    if device.type != "cuda":
        raise ValueError(f"popcorn_amd: tensors must be on a HIP device, got {device}")
    return device


def _same_dtype(name: str, *tensors: Tensor | None) -> torch.dtype:
    dtypes = {t.dtype for t in tensors if t is not None}
    if len(dtypes) != 1:
        raise TypeError(f"popcorn_amd.{name}: mixed dtypes {sorted(map(str, dtypes))}")
    dtype = dtypes.pop()
    _lib.dtype_code(dtype)
    return dtype


_HALF = (torch.bfloat16, torch.float16)


def _tracks_grad(*tensors: Tensor | None) -> bool:
    """Whether autograd must record the call: grad mode on and some input requiring grad.

    Calls that need no graph skip the autograd node (one launch, nothing saved).
    """
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def _norm_dtypes(name: str, x: Tensor, weight: Tensor, bias: Tensor | None) -> tuple[torch.dtype, torch.dtype]:
    """(x dtype, weight dtype): one dtype, or a 16-bit x with fp32 weight (and bias), whose product promotes to fp32."""
    if bias is not None and bias.dtype != weight.dtype:
        raise TypeError(f"popcorn_amd.{name}: bias dtype {bias.dtype} differs from weight dtype {weight.dtype}")
    if x.dtype != weight.dtype and not (x.dtype in _HALF and weight.dtype == torch.float32):
        raise TypeError(f"popcorn_amd.{name}: x {x.dtype} with weight {weight.dtype} is not supported "
                        "(one dtype, or a 16-bit x with an fp32 weight)")
    _lib.dtype_code(x.dtype)
    _lib.dtype_code(weight.dtype)
    return x.dtype, weight.dtype


def _table_dtype(name: str, cos: Tensor, sin: Tensor) -> torch.dtype:
    if cos.dtype != sin.dtype:
        raise TypeError(f"popcorn_amd.{name}: cos {cos.dtype} and sin {sin.dtype} differ")
    _lib.dtype_code(cos.dtype)
    return cos.dtype


# --------------------------------------------------------------------------- rms_norm


def _rms_norm_fwd(x: Tensor, weight: Tensor, bias: Tensor | None, eps: float, want_rstd: bool):
    """One pk_rmsnorm_fwd launch: (y in x's shape, x as [rows, cols], weight, rstd or None)."""
    device = _require_cuda(x, weight, bias)
    dtype, wdtype = _norm_dtypes("rms_norm", x, weight, bias)
    cols = x.shape[-1]
    if weight.shape != (cols,) or (bias is not None and bias.shape != (cols,)):
        raise ValueError(f"popcorn_amd.rms_norm: weight/bias must be [{cols}]")
    x2 = x.reshape(-1, cols)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    b = None if bias is None else bias.contiguous()
    rows = x2.shape[0]
    y = torch.empty(x.shape, dtype=wdtype, device=device)
    rstd = torch.empty(rows, dtype=torch.float32, device=device) if want_rstd else None
    lib = _lib.load()
    with _lib.on_device(device):
        _lib.check(
            lib.pk_rmsnorm_fwd(
                x2.data_ptr(),
                w.data_ptr(),
                None if b is None else b.data_ptr(),
                y.data_ptr(),
                None if rstd is None else rstd.data_ptr(),
                rows,
                cols,
                float(eps),
                _lib.DTYPE_CODES[dtype],
                _lib.DTYPE_CODES[wdtype],
                _lib.stream_handle(device),
            ),
            lib,
        )
    return y, x2, w, rstd


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Tensor | None, eps: float) -> Tensor:
        y, x2, w, rstd = _rms_norm_fwd(x, weight, bias, eps, want_rstd=True)
        ctx.save_for_backward(x2, w, rstd)
        ctx.has_bias = bias is not None
        ctx.shape = x.shape
        return y

    @staticmethod
    def backward(ctx, dy: Tensor):
        x2, w, rstd = ctx.saved_tensors
        rows, cols = x2.shape
        dy2 = dy.reshape(rows, cols).to(w.dtype).contiguous()
        dx = torch.empty_like(x2)
        dw = torch.empty_like(w)
        db = torch.empty_like(w) if ctx.has_bias else None
        if rows == 0:
            dw.zero_()
            if db is not None:
                db.zero_()
        else:
            lib = _lib.load()
            code = _lib.dtype_code(x2.dtype)
            nbytes = lib.pk_rmsnorm_bwd_workspace(rows, cols, code)
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=x2.device)
            with _lib.on_device(x2.device):
                _lib.check(
                    lib.pk_rmsnorm_bwd(
                        x2.data_ptr(),
                        w.data_ptr(),
                        rstd.data_ptr(),
                        dy2.data_ptr(),
                        dx.data_ptr(),
                        dw.data_ptr(),
                        db.data_ptr() if db is not None else None,
                        workspace.data_ptr(),
                        nbytes,
                        rows,
                        cols,
                        code,
                        _lib.dtype_code(w.dtype),
                        _lib.stream_handle(x2.device),
                    ),
                    lib,
                )
        return dx.view(ctx.shape), dw, db, None


def rms_norm(x: Tensor, weight: Tensor, bias: Tensor | None = None, eps: float = 1e-6) -> Tensor:
    """y = round(round(x * rsqrt(mean(x^2) + eps)) * weight) [+ bias], fp32 statistics.

    x [..., normalized_shape]; weight, bias [normalized_shape]; one dtype for all
    (fp32, bf16 or fp16), or a 16-bit x with fp32 weight and bias, where the
    normalized x is rounded to x's dtype and the output promotes to fp32
    (kernels/rms_norm.py:29). Backward gives dx (x's dtype), dweight, dbias
    (the weight's). Without a gradient to track, the call is one launch with no
    autograd node and no saved statistics.
    """
    if _tracks_grad(x, weight, bias):
        return _RMSNorm.apply(x, weight, bias, eps)
    return _rms_norm_fwd(x, weight, bias, eps, want_rstd=False)[0]


# --------------------------------------------------------------------------- add_rms_norm


def _add_rms_norm_fwd(x: Tensor, residual: Tensor, weight: Tensor, eps: float, offset: float):
    """One pk_add_rmsnorm_fwd launch: (y, s) as [rows, cols], the weight and rstd."""
    device = _require_cuda(x, residual, weight)
    if residual.dtype != x.dtype:
        raise TypeError(f"popcorn_amd.add_rms_norm: residual {residual.dtype} differs from x {x.dtype}")
    dtype, wdtype = _norm_dtypes("add_rms_norm", x, weight, None)
    cols = x.shape[-1]
    if residual.shape != x.shape:
        raise ValueError(f"popcorn_amd.add_rms_norm: residual {tuple(residual.shape)} != x {tuple(x.shape)}")
    if weight.shape != (cols,):
        raise ValueError(f"popcorn_amd.add_rms_norm: weight must be [{cols}]")
    x2 = x.reshape(-1, cols).contiguous()
    r2 = residual.reshape(-1, cols).contiguous()
    w = weight.contiguous()
    rows = x2.shape[0]
    y = torch.empty((rows, cols), dtype=wdtype, device=device)
    s = torch.empty_like(x2)
    rstd = torch.empty(rows, dtype=torch.float32, device=device)
    lib = _lib.load()
    with _lib.on_device(device):
        _lib.check(
            lib.pk_add_rmsnorm_fwd(
                x2.data_ptr(), r2.data_ptr(), w.data_ptr(), y.data_ptr(), s.data_ptr(), rstd.data_ptr(), rows, cols,
                float(eps), float(offset), _lib.dtype_code(dtype), _lib.dtype_code(wdtype), _lib.stream_handle(device),
            ),
            lib,
        )
    return y, s, w, rstd


class _AddRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, residual: Tensor, weight: Tensor, eps: float, offset: float):
        y, s, w, rstd = _add_rms_norm_fwd(x, residual, weight, eps, offset)
        ctx.save_for_backward(s, w, rstd)
        ctx.offset = float(offset)
        ctx.shape = x.shape
        ctx.set_materialize_grads(False)
        return y.view(x.shape), s.view(x.shape)

    @staticmethod
    def backward(ctx, dy: Tensor | None, ds: Tensor | None):
        s, w, rstd = ctx.saved_tensors
        rows, cols = s.shape
        if dy is None:  # only the residual stream was used downstream
            dsum = ds.reshape(rows, cols).to(s.dtype) if ds is not None else torch.zeros_like(s)
            return dsum.view(ctx.shape), dsum.view(ctx.shape), torch.zeros_like(w), None, None
        dy2 = dy.reshape(rows, cols).to(w.dtype).contiguous()
        ds2 = ds.reshape(rows, cols).to(s.dtype).contiguous() if ds is not None else None
        dsum = torch.empty_like(s)
        dw = torch.empty_like(w)
        if rows == 0:
            dw.zero_()
        else:
            lib = _lib.load()
            code = _lib.dtype_code(s.dtype)
            nbytes = lib.pk_rmsnorm_bwd_workspace(rows, cols, code)
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=s.device)
            with _lib.on_device(s.device):
                _lib.check(
                    lib.pk_add_rmsnorm_bwd(
                        s.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy2.data_ptr(),
                        ds2.data_ptr() if ds2 is not None else None, dsum.data_ptr(), dw.data_ptr(),
                        workspace.data_ptr(), nbytes, rows, cols, ctx.offset, code, _lib.dtype_code(w.dtype),
                        _lib.stream_handle(s.device),
                    ),
                    lib,
                )
        # s = x + residual: both receive the gradient of s (as torch's add backward hands them)
        return dsum.view(ctx.shape), dsum.view(ctx.shape), dw, None, None


def add_rms_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float = 1e-6,
                 offset: float = 0.0) -> tuple[Tensor, Tensor]:
    """(y, s): s = round(x + residual), y = round(round(s * rsqrt(mean(s^2) + eps)) * round(weight + offset)).

    x, residual [..., hidden]; weight [hidden]; one dtype for all, or 16-bit x and
    residual with an fp32 weight, where y promotes to fp32 and s keeps x's dtype
    (kernels/add_rms_norm.py:26). Backward gives d(x) = d(residual) in x's dtype
    and dweight in the weight's.
    """
    if _tracks_grad(x, residual, weight):
        return _AddRMSNorm.apply(x, residual, weight, eps, offset)
    y, s, _, _ = _add_rms_norm_fwd(x, residual, weight, eps, offset)
    return y.view(x.shape), s.view(x.shape)


# --------------------------------------------------------------------------- swiglu


def _swiglu_fwd(a: Tensor, b: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """One pk_swiglu_fwd launch: (y, a and b as the contiguous tensors it read)."""
    device = _require_cuda(a, b)
    dtype = _same_dtype("swiglu", a, b)
    if a.shape != b.shape:
        raise ValueError(f"popcorn_amd.swiglu: shapes differ {tuple(a.shape)} vs {tuple(b.shape)}")
    a_c, b_c = a.contiguous(), b.contiguous()
    y = torch.empty_like(a_c)
    lib = _lib.load()
    with _lib.on_device(device):
        _lib.check(
            lib.pk_swiglu_fwd(
                a_c.data_ptr(), b_c.data_ptr(), y.data_ptr(), a_c.numel(), _lib.dtype_code(dtype),
                _lib.stream_handle(device),
            ),
            lib,
        )
    return y, a_c, b_c


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor) -> Tensor:
        y, a_c, b_c = _swiglu_fwd(a, b)
        ctx.save_for_backward(a_c, b_c)
        return y

    @staticmethod
    def backward(ctx, dy: Tensor):
        a_c, b_c = ctx.saved_tensors
        g = dy.to(a_c.dtype).contiguous()
        da, db = torch.empty_like(a_c), torch.empty_like(b_c)
        lib = _lib.load()
        with _lib.on_device(a_c.device):
            _lib.check(
                lib.pk_swiglu_bwd(
                    g.data_ptr(), a_c.data_ptr(), b_c.data_ptr(), da.data_ptr(), db.data_ptr(), a_c.numel(),
                    _lib.dtype_code(a_c.dtype), _lib.stream_handle(a_c.device),
                ),
                lib,
            )
        return da, db


def swiglu(a: Tensor, b: Tensor) -> Tensor:
    """y = silu(a) * b elementwise (a, b of one shape and dtype); differentiable."""
    if _tracks_grad(a, b):
        return _SwiGLU.apply(a, b)
    return _swiglu_fwd(a, b)[0]


# --------------------------------------------------------------------------- rotary


def _rotate(x: Tensor, cos: Tensor, sin: Tensor, out: Tensor, interleaved: bool, conjugate: bool) -> None:
    device = _require_cuda(x, cos, sin, out)
    if x.dim() != 4:
        raise ValueError(f"popcorn_amd.rotary_embedding: x must be [batch, seq, heads, head_dim], got {tuple(x.shape)}")
    batch, seq, heads, head_dim = x.shape
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[0] != seq:
        raise ValueError(f"popcorn_amd.rotary_embedding: cos/sin must be [{seq}, half], got {tuple(cos.shape)}")
    if cos.dtype != sin.dtype:
        raise TypeError("popcorn_amd.rotary_embedding: cos and sin dtypes differ")
    half = cos.shape[1]
    if 2 * half > head_dim:
        raise ValueError(f"popcorn_amd.rotary_embedding: half={half} > head_dim/2")
    lib = _lib.load()
    strides = (_lib._i64 * 6)(x.stride(0), x.stride(1), x.stride(2), out.stride(0), out.stride(1), out.stride(2))
    with _lib.on_device(device):
        _lib.check(
            lib.pk_rotary(
                x.data_ptr(),
                cos.data_ptr(),
                sin.data_ptr(),
                out.data_ptr(),
                strides,
                batch,
                seq,
                heads,
                head_dim,
                half,
                _lib.dtype_code(x.dtype),
                _lib.dtype_code(cos.dtype),
                int(interleaved),
                int(conjugate),
                _lib.stream_handle(device),
            ),
            lib,
        )


def _last_contiguous(t: Tensor) -> Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _rotary_fwd(x: Tensor, cos: Tensor, sin: Tensor, interleaved: bool) -> tuple[Tensor, Tensor, Tensor]:
    """One pk_rotary launch into a new tensor: (y, cos, sin as the contiguous tables it read)."""
    xs = _last_contiguous(x.detach())
    cos_c, sin_c = cos.detach().contiguous(), sin.detach().contiguous()
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _rotate(xs, cos_c, sin_c, y, interleaved, conjugate=False)
    return y, cos_c, sin_c


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, cos: Tensor, sin: Tensor, interleaved: bool) -> Tensor:
        y, cos_c, sin_c = _rotary_fwd(x, cos, sin, interleaved)
        ctx.save_for_backward(cos_c, sin_c)
        ctx.interleaved = interleaved
        return y

    @staticmethod
    def backward(ctx, dy: Tensor):
        cos_c, sin_c = ctx.saved_tensors
        g = _last_contiguous(dy)
        dx = torch.empty(dy.shape, dtype=dy.dtype, device=dy.device)
        _rotate(g, cos_c, sin_c, dx, ctx.interleaved, conjugate=True)
        return dx, None, None, None


def rotary_embedding(x: Tensor, cos: Tensor, sin: Tensor, interleaved: bool = False) -> Tensor:
    """Rotate x [batch, seq, heads, head_dim] by cos/sin [seq, half] (fp32 math, one rounding).

    NeoX halves by default, GPT-J pairs with interleaved=True; channels past
    2*half are passed through. Returns a new tensor; cos and sin get no gradient.
    """
    if _tracks_grad(x):
        return _Rotary.apply(x, cos, sin, interleaved)
    return _rotary_fwd(x, cos, sin, interleaved)[0]


def rotary_embedding_(x: Tensor, cos: Tensor, sin: Tensor, interleaved: bool = False) -> Tensor:
    """In-place variant of `rotary_embedding` (no autograd): x is overwritten and returned."""
    if torch.is_grad_enabled() and x.requires_grad:
        raise RuntimeError("popcorn_amd.rotary_embedding_: in-place rotation of a tensor that requires grad")
    if x.stride(-1) != 1:
        raise ValueError("popcorn_amd.rotary_embedding_: last dimension must be contiguous")
    _rotate(x, cos.contiguous(), sin.contiguous(), x, interleaved, conjugate=False)
    return x


def _rope(q: Tensor | None, k: Tensor | None, cos: Tensor, sin: Tensor, transpose: bool,
          out_dtype: torch.dtype | None = None):
    """One pk_rope launch over whichever of q, k is given; returns (yq, yk) (None for an absent side).

    The outputs have `out_dtype`, by default q/k's dtype promoted with the tables'.
    """
    sides = [t for t in (q, k) if t is not None]
    device = _require_cuda(*sides, cos, sin)
    dtype = _same_dtype("rope", *sides)
    cs_dtype = _table_dtype("rope", cos, sin)
    out_dtype = torch.promote_types(dtype, cs_dtype) if out_dtype is None else out_dtype
    if any(t.dim() != 4 for t in sides) or cos.dim() != 3 or cos.shape != sin.shape:
        raise ValueError("popcorn_amd.rope: q [b, hq, s, d], k [b, hkv, s, d] and cos, sin [cos_batch, s, d] expected")
    batch, _, seq, head_dim = sides[0].shape
    for t in sides:
        if t.shape[0] != batch or t.shape[2] != seq or t.shape[3] != head_dim:
            raise ValueError(f"popcorn_amd.rope: q/k shapes {[tuple(t.shape) for t in sides]} disagree")
    if cos.shape[1:] != (seq, head_dim) or cos.shape[0] not in (1, batch):
        raise ValueError(f"popcorn_amd.rope: cos/sin {tuple(cos.shape)} must be [1 or {batch}, {seq}, {head_dim}]")
    if head_dim % 2:
        raise ValueError(f"popcorn_amd.rope: head_dim={head_dim} is odd")
    xq, xk = (None if t is None else _last_contiguous(t.detach()) for t in (q, k))
    yq, yk = (None if t is None else torch.empty(t.shape, dtype=out_dtype, device=device) for t in (q, k))
    cs, sn = cos.detach().contiguous(), sin.detach().contiguous()

    def strides(t):
        return (0, 0, 0) if t is None else t.stride()[:3]

    lib = _lib.load()
    st = (_lib._i64 * 12)(*strides(xq), *strides(xk), *strides(yq), *strides(yk))
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    with _lib.on_device(device):
        _lib.check(
            lib.pk_rope(
                ptr(xq), ptr(xk), cs.data_ptr(), sn.data_ptr(), ptr(yq), ptr(yk), st, batch,
                0 if q is None else q.shape[1], 0 if k is None else k.shape[1], seq, head_dim, cos.shape[0],
                _lib.dtype_code(dtype), _lib.dtype_code(out_dtype), _lib.dtype_code(cs_dtype), int(transpose),
                _lib.stream_handle(device),
            ),
            lib,
        )
    return yq, yk


class _Rope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q: Tensor, k: Tensor, cos: Tensor, sin: Tensor):
        yq, yk = _rope(q, k, cos, sin, transpose=False)
        ctx.save_for_backward(cos.detach().contiguous(), sin.detach().contiguous())
        ctx.dtypes = q.dtype, yq.dtype
        return yq, yk

    @staticmethod
    def backward(ctx, gq: Tensor | None, gk: Tensor | None):
        cos, sin = ctx.saved_tensors
        if gq is None and gk is None:
            return None, None, None, None
        x_dtype, y_dtype = ctx.dtypes
        gq, gk = (None if g is None else g.to(y_dtype) for g in (gq, gk))
        dq, dk = _rope(gq, gk, cos, sin, transpose=True, out_dtype=x_dtype)
        return dq, dk, None, None


def rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """Paired rotary embedding: (q*cos + rotate_half(q)*sin, k*cos + rotate_half(k)*sin).

    q [batch, q_heads, seq, head_dim], k [batch, kv_heads, seq, head_dim],
    cos, sin [cos_batch, seq, head_dim] with cos_batch 1 or batch; q, k one
    dtype and cos, sin one dtype, the outputs their promotion (16-bit q/k with
    fp32 tables give fp32, kernels/rope.py:35-36). The two halves of a table
    row may differ. fp32 arithmetic, one rounding per output; one launch for q
    and k. Gradients have q/k's dtype; cos and sin get none.
    """
    if _tracks_grad(q, k):
        return _Rope.apply(q, k, cos, sin)
    return _rope(q, k, cos, sin, transpose=False)


def _qk_norm_rope_shapes(q, k, q_weight, k_weight, cos, sin):
    device = _require_cuda(q, k, q_weight, k_weight, cos, sin)
    dtype = _same_dtype("qk_norm_rope", q, k)
    if q_weight.dtype != k_weight.dtype or not (
            q_weight.dtype == dtype or (dtype in _HALF and q_weight.dtype == torch.float32)):
        raise TypeError(f"popcorn_amd.qk_norm_rope: weights {q_weight.dtype}/{k_weight.dtype} with q/k {dtype} are not "
                        "supported (q/k's dtype, or fp32 beside 16-bit q/k)")
    _table_dtype("qk_norm_rope", cos, sin)
    if q.dim() != 4 or k.dim() != 4 or cos.dim() != 3 or cos.shape != sin.shape:
        raise ValueError("popcorn_amd.qk_norm_rope: q [b, hq, s, d], k [b, hkv, s, d], cos, sin [cb, s, d] expected")
    batch, _, seq, head_dim = q.shape
    if k.shape[0] != batch or k.shape[2:] != q.shape[2:]:
        raise ValueError(f"popcorn_amd.qk_norm_rope: q {tuple(q.shape)} and k {tuple(k.shape)} disagree")
    if q_weight.shape != (head_dim,) or k_weight.shape != (head_dim,):
        raise ValueError(f"popcorn_amd.qk_norm_rope: weights must be [{head_dim}]")
    if cos.shape[1:] != (seq, head_dim) or cos.shape[0] not in (1, batch):
        raise ValueError(
            f"popcorn_amd.qk_norm_rope: cos/sin {tuple(cos.shape)} must be [1 or {batch}, {seq}, {head_dim}]")
    return device, dtype, batch, seq, head_dim


def _dense(t: Tensor) -> Tensor:
    """Contiguous and 16-byte aligned (weights and tables)."""
    c = t.detach().contiguous()
    return c if c.data_ptr() % 16 == 0 else c.clone()


def _qk_norm_rope_fwd(q, k, q_weight, k_weight, cos, sin, eps):
    """One pk_qk_norm_rope_fwd launch: (yq, yk, and what the backward reads: q, k, weights, tables, rstd)."""
    device, dtype, batch, seq, head_dim = _qk_norm_rope_shapes(q, k, q_weight, k_weight, cos, sin)
    q_, k_ = _aligned_rows(q.detach()), _aligned_rows(k.detach())
    qw, kw, cs, sn = (_dense(t) for t in (q_weight, k_weight, cos, sin))
    out_dtype = torch.promote_types(torch.promote_types(dtype, qw.dtype), cs.dtype)
    yq = torch.empty(q.shape, dtype=out_dtype, device=device)
    yk = torch.empty(k.shape, dtype=out_dtype, device=device)
    rq = torch.empty((batch, q.shape[1], seq), dtype=torch.float32, device=device)
    rk = torch.empty((batch, k.shape[1], seq), dtype=torch.float32, device=device)
    lib = _lib.load()
    st = (_lib._i64 * 12)(*(x for t in (q_, k_, yq, yk) for x in t.stride()[:3]))
    code = _lib.dtype_code(dtype)
    with _lib.on_device(device):
        _lib.check(
            lib.pk_qk_norm_rope_fwd(
                q_.data_ptr(), k_.data_ptr(), qw.data_ptr(), kw.data_ptr(), cs.data_ptr(), sn.data_ptr(),
                yq.data_ptr(), yk.data_ptr(), rq.data_ptr(), rk.data_ptr(), st, batch, q.shape[1], k.shape[1], seq,
                head_dim, cos.shape[0], float(eps), code, _lib.dtype_code(out_dtype), _lib.dtype_code(cs.dtype),
                _lib.dtype_code(qw.dtype), _lib.stream_handle(device),
            ),
            lib,
        )
    return yq, yk, (q_, k_, qw, kw, cs, sn, rq, rk)


class _QkNormRope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, cos, sin, eps):
        yq, yk, saved = _qk_norm_rope_fwd(q, k, q_weight, k_weight, cos, sin, eps)
        ctx.out_dtype = yq.dtype
        ctx.save_for_backward(*saved)
        return yq, yk

    @staticmethod
    def backward(ctx, gq, gk):
        q_, k_, qw, kw, cs, sn, rq, rk = ctx.saved_tensors
        batch, _, seq, head_dim = q_.shape
        gdt = ctx.out_dtype
        gq = torch.zeros(q_.shape, dtype=gdt, device=q_.device) if gq is None else _aligned_rows(gq.to(gdt))
        gk = torch.zeros(k_.shape, dtype=gdt, device=k_.device) if gk is None else _aligned_rows(gk.to(gdt))
        dq, dk = torch.empty(q_.shape, dtype=q_.dtype, device=q_.device), torch.empty(k_.shape, dtype=k_.dtype,
                                                                                       device=k_.device)
        dw = torch.empty((2, head_dim), dtype=qw.dtype, device=q_.device)
        lib = _lib.load()
        code = _lib.dtype_code(q_.dtype)
        nbytes = lib.pk_qk_norm_rope_bwd_workspace(batch, q_.shape[1], k_.shape[1], seq, head_dim, code)
        if nbytes < 0:
            raise ValueError(f"popcorn_amd.qk_norm_rope: head_dim={head_dim} is not supported")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q_.device)
        st = (_lib._i64 * 18)(*(x for t in (q_, k_, gq, gk, dq, dk) for x in t.stride()[:3]))
        with _lib.on_device(q_.device):
            _lib.check(
                lib.pk_qk_norm_rope_bwd(
                    q_.data_ptr(), k_.data_ptr(), qw.data_ptr(), kw.data_ptr(), cs.data_ptr(), sn.data_ptr(),
                    rq.data_ptr(), rk.data_ptr(), gq.data_ptr(), gk.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                    dw.data_ptr(), ws.data_ptr(), nbytes, st, batch, q_.shape[1], k_.shape[1], seq, head_dim,
                    cs.shape[0], code, _lib.dtype_code(gdt), _lib.dtype_code(cs.dtype), _lib.dtype_code(qw.dtype),
                    _lib.stream_handle(q_.device),
                ),
                lib,
            )
        return dq, dk, dw[0], dw[1], None, None, None


def qk_norm_rope(q: Tensor, k: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor,
                 eps: float = 1e-6) -> tuple[Tensor, Tensor]:
    """Per-head RMSNorm of q and k (weights over head_dim), then `rope`, fused into one pass.

    q [batch, q_heads, seq, head_dim], k [batch, kv_heads, seq, head_dim],
    q_weight, k_weight [head_dim], cos, sin [cos_batch, seq, head_dim]; q and k
    one dtype, the weights q/k's dtype or fp32 beside 16-bit q/k, cos and sin one
    dtype, the outputs the promotion of all three (16-bit q/k with fp32 tables
    or fp32 weights give fp32); head_dim / 2 a 16-byte pack count (of q's dtype)
    times a power of two up to 64. fp32 arithmetic, one rounding per output.
    Backward gives dq, dk in q's dtype and the two weight gradients in the
    weights'; cos and sin get none.
    """
    if _tracks_grad(q, k, q_weight, k_weight):
        return _QkNormRope.apply(q, k, q_weight, k_weight, cos, sin, eps)
    return _qk_norm_rope_fwd(q, k, q_weight, k_weight, cos, sin, eps)[:2]


# --------------------------------------------------------------------------- attention


def attn_with_lse(
    q: Tensor, k: Tensor, v: Tensor, causal: bool = False, softmax_scale: float | None = None
) -> tuple[Tensor, Tensor]:
    """Forward attention returning (o [batch, seq, q_heads, head_dim], lse [batch, q_heads, seq] fp32); no autograd."""
    return _attn_fwd(q, k, v, causal, softmax_scale, want_lse=True)


def attn(q: Tensor, k: Tensor, v: Tensor, causal: bool = False, softmax_scale: float | None = None) -> Tensor:
    """softmax(q k^T * scale + causal mask) v with grouped kv heads.

    q [batch, seq, q_heads, head_dim], k, v [batch, seq, kv_heads, head_dim];
    bf16, fp16 or fp32 with head_dim a multiple of 8 up to 256; scale
    defaults to head_dim ** -0.5. Backward gives dq, dk, dv.
    """
    if _tracks_grad(q, k, v):
        _grad_supported("attn", q.shape[-1], q.dtype)
        return _Attention.apply(q, k, v, causal, softmax_scale)
    return _attn_fwd(q, k, v, causal, softmax_scale, want_lse=False)[0]


def _grad_supported(op: str, head_dim: int, dtype: torch.dtype) -> None:
    """Refuse, before any work, a call whose backward the kernels do not cover: head_dim above 256, where
    the forward kernels stop too."""
    if head_dim > 256:
        raise ValueError(f"popcorn_amd.{op}: head_dim={head_dim} is past the attention kernels' 256")


def _scale(head_dim: int, softmax_scale: float | None) -> float:
    return head_dim**-0.5 if softmax_scale is None else float(softmax_scale)


def _attn_fwd(q, k, v, causal, softmax_scale, want_lse):
    device = _require_cuda(q, k, v)
    dtype = _same_dtype("attn", q, k, v)
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError("popcorn_amd.attn: q [b, s, hq, d] and k, v [b, s, hkv, d] expected")
    batch, seq, q_heads, head_dim = q.shape
    if k.shape[0] != batch or k.shape[1] != seq or k.shape[3] != head_dim:
        raise ValueError(f"popcorn_amd.attn: k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    kv_heads = k.shape[2]
    q_, k_, v_ = (_aligned_rows(t.detach()) for t in (q, k, v))
    o = torch.empty((batch, seq, q_heads, head_dim), dtype=dtype, device=device)
    lse = torch.empty((batch, q_heads, seq), dtype=torch.float32, device=device) if want_lse else None
    lib = _lib.load()
    strides = (_lib._i64 * 12)(*(s for t in (q_, k_, v_, o) for s in t.stride()[:3]))
    with _lib.on_device(device):
        _lib.check(
            lib.pk_attn_fwd(
                q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr(), lse.data_ptr() if lse is not None else None,
                strides, batch, seq, q_heads, kv_heads, head_dim, _scale(head_dim, softmax_scale), int(bool(causal)),
                _lib.dtype_code(dtype), _lib.stream_handle(device),
            ),
            lib,
        )
    return o, lse


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal, softmax_scale):
        o, lse = _attn_fwd(q, k, v, causal, softmax_scale, want_lse=True)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.causal, ctx.softmax_scale = bool(causal), softmax_scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        batch, seq, q_heads, head_dim = q.shape
        q_, k_, v_, do_ = (_aligned_rows(t) for t in (q, k, v, do.to(q.dtype)))
        dq, dk, dv = torch.empty(q.shape, dtype=q.dtype, device=q.device), torch.empty_like(k_), torch.empty_like(v_)
        dk, dv = dk.contiguous(), dv.contiguous()
        lib = _lib.load()
        # D, lse2 and (for grids too small to fill the device) dk/dv partials of q-head splits
        nbytes = lib.pk_attn_bwd_workspace(batch, seq, q_heads, k.shape[2], head_dim)
        if nbytes < 0:
            raise _lib.KernelError(f"pk_attn_bwd_workspace: invalid shape {tuple(q.shape)} / {tuple(k.shape)}")
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
        strides = (_lib._i64 * 24)(*(s for t in (q_, k_, v_, o, do_, dq, dk, dv) for s in t.stride()[:3]))
        with _lib.on_device(q.device):
            _lib.check(
                lib.pk_attn_bwd(
                    q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr(), do_.data_ptr(), lse.data_ptr(),
                    ws.data_ptr(), ws.numel(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), strides, batch, seq,
                    q_heads, k.shape[2], head_dim, _scale(head_dim, ctx.softmax_scale), int(ctx.causal),
                    _lib.dtype_code(q.dtype), _lib.stream_handle(q.device),
                ),
                lib,
            )
        return dq, dk, dv, None, None


def _aligned_rows(t: Tensor) -> Tensor:
    """A view the kernel can read with 16-byte loads, copying only when it must."""
    unit = 16 // t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % unit == 0 and s >= 0 for s in t.stride()[:-1])
    if ok:
        return t
    c = t.contiguous()
    return c if c.data_ptr() % 16 == 0 else c.clone()  # a contiguous view at an odd offset


def attn_varlen_with_lse(
    q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, causal: bool = False, softmax_scale: float | None = None
) -> tuple[Tensor, Tensor]:
    """Packed-sequence attention returning (o [total, q_heads, head_dim], lse [q_heads, total] fp32); no autograd."""
    cu, num_seqs, longest = _cut_points(cu_seqlens, q.shape[0], q.device)
    return _attn_varlen_fwd(q, k, v, cu, num_seqs, longest, causal, softmax_scale, want_lse=True)


def attn_varlen(
    q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, causal: bool = False, softmax_scale: float | None = None
) -> Tensor:
    """Attention over packed variable-length sequences, each attended independently.

    q [total, q_heads, head_dim], k, v [total, kv_heads, head_dim]; cu_seqlens
    int32 [num_seqs + 1] offsets from 0 to total (the flash-attention varlen
    layout). Causal masks are top-left aligned within each sequence. head_dim
    as for `attn`. Backward gives dq, dk, dv.
    """
    cu, num_seqs, longest = _cut_points(cu_seqlens, q.shape[0], q.device)
    if _tracks_grad(q, k, v):
        _grad_supported("attn_varlen", q.shape[-1], q.dtype)
        return _AttentionVarlen.apply(q, k, v, cu, num_seqs, longest, causal, softmax_scale)
    return _attn_varlen_fwd(q, k, v, cu, num_seqs, longest, causal, softmax_scale, want_lse=False)[0]


def _cut_points(cu_seqlens: Tensor, total: int, device: torch.device) -> tuple[Tensor, int, int]:
    """(cu_seqlens as an int32 device tensor, number of sequences, longest sequence); one host read."""
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2 or cu_seqlens.is_floating_point():
        raise ValueError("popcorn_amd.attn_varlen: cu_seqlens must be a 1-D integer tensor of num_seqs + 1 offsets")
    cuts = cu_seqlens.tolist()
    if cuts[0] != 0 or cuts[-1] != total or any(b < a for a, b in zip(cuts, cuts[1:])):
        raise ValueError(f"popcorn_amd.attn_varlen: cu_seqlens must rise from 0 to total={total}, got {cuts[:8]}...")
    longest = max(b - a for a, b in zip(cuts, cuts[1:]))
    return cu_seqlens.to(device=device, dtype=torch.int32).contiguous(), len(cuts) - 1, longest


def _attn_varlen_fwd(q, k, v, cu, num_seqs, longest, causal, softmax_scale, want_lse):
    device = _require_cuda(q, k, v)
    dtype = _same_dtype("attn_varlen", q, k, v)
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape:
        raise ValueError("popcorn_amd.attn_varlen: q [total, hq, d] and k, v [total, hkv, d] expected")
    total, q_heads, head_dim = q.shape
    if k.shape[0] != total or k.shape[2] != head_dim:
        raise ValueError(f"popcorn_amd.attn_varlen: k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    q_, k_, v_ = (_aligned_rows(t.detach()) for t in (q, k, v))
    o = torch.empty((total, q_heads, head_dim), dtype=dtype, device=device)
    lse = torch.empty((q_heads, total), dtype=torch.float32, device=device) if want_lse else None
    lib = _lib.load()
    strides = (_lib._i64 * 8)(*(s for t in (q_, k_, v_, o) for s in t.stride()[:2]))
    with _lib.on_device(device):
        _lib.check(
            lib.pk_attn_varlen_fwd(
                q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr(), lse.data_ptr() if lse is not None else None,
                cu.data_ptr(), strides, num_seqs, total, longest, q_heads, k.shape[1], head_dim,
                _scale(head_dim, softmax_scale), int(bool(causal)), _lib.dtype_code(dtype), _lib.stream_handle(device),
            ),
            lib,
        )
    return o, lse


class _AttentionVarlen(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu, num_seqs, longest, causal, softmax_scale):
        o, lse = _attn_varlen_fwd(q, k, v, cu, num_seqs, longest, causal, softmax_scale, want_lse=True)
        ctx.save_for_backward(q, k, v, o, lse, cu)
        ctx.meta = (num_seqs, longest, bool(causal), softmax_scale)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, cu = ctx.saved_tensors
        num_seqs, longest, causal, softmax_scale = ctx.meta
        total, q_heads, head_dim = q.shape
        q_, k_, v_, do_ = (_aligned_rows(t) for t in (q, k, v, do.to(q.dtype)))
        dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
        dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        lib = _lib.load()
        nbytes = lib.pk_attn_varlen_bwd_workspace(num_seqs, total, longest, q_heads, k.shape[1], head_dim)
        if nbytes < 0:
            raise _lib.KernelError(f"pk_attn_varlen_bwd_workspace: invalid shape {tuple(q.shape)} / {tuple(k.shape)}")
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
        strides = (_lib._i64 * 16)(*(s for t in (q_, k_, v_, o, do_, dq, dk, dv) for s in t.stride()[:2]))
        with _lib.on_device(q.device):
            _lib.check(
                lib.pk_attn_varlen_bwd(
                    q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr(), do_.data_ptr(), lse.data_ptr(),
                    ws.data_ptr(), ws.numel(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), cu.data_ptr(), strides,
                    num_seqs, total, longest, q_heads, k.shape[1], head_dim, _scale(head_dim, softmax_scale),
                    int(causal), _lib.dtype_code(q.dtype), _lib.stream_handle(q.device),
                ),
                lib,
            )
        return dq, dk, dv, None, None, None, None, None
