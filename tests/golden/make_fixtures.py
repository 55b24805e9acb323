"""Write the golden fixtures of tests/golden/: seeded small inputs and the float64 oracle's outputs.

    python tests/golden/make_fixtures.py

Popcorn's own tests hold no value-level fixtures for these ops, so the vectors
come from `oracle.reference` (float64, pinned in tests/test_oracle.py). Each
`<op>.npz` stores its inputs, scalar arguments and expected outputs; the
inputs are N(0,1) draws rounded to bfloat16 values (exactly representable in
bf16, fp16 up to range, and fp32), so the GPU tests can feed them at any
supported dtype without a rounding step of their own.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import reference as O  # noqa: E402

HERE = Path(__file__).resolve().parent


def to_bf16(x):
    """x rounded to the nearest bfloat16 value, ties to even (kept as float64)."""
    bits = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    bits = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    return bits.astype(np.uint32).view(np.float32).astype(np.float64)


def bf16_values(rng, shape, scale=1.0):
    """N(0,1) * scale rounded to bfloat16 values."""
    return to_bf16(rng.standard_normal(shape) * scale)


def save(name, inputs=(), **arrays):
    """Inputs (bf16 values) are stored as float32, which holds them exactly; outputs as float64."""
    out = {k: np.asarray(v, dtype=np.float32) if k in inputs else np.asarray(v) for k, v in arrays.items()}
    np.savez_compressed(HERE / f"{name}.npz", **out)


def main():
    rng = np.random.default_rng(2024)
    # rms_norm (with and without bias) and its backward
    x, w = bf16_values(rng, (6, 96)), to_bf16(1 + 0.1 * rng.standard_normal(96))
    bias, dy = bf16_values(rng, (96,)), bf16_values(rng, (6, 96))
    dx, dw, db = O.rms_norm_bwd(x, w, dy, 1e-5)
    save("rms_norm", ('x', 'weight', 'bias', 'dy'), x=x, weight=w, bias=bias, dy=dy, eps=1e-5, y=O.rms_norm(x, w, None, 1e-5),
         y_bias=O.rms_norm(x, w, bias, 1e-5), dx=dx, dweight=dw, dbias=db)
    # add_rms_norm
    r, ds = bf16_values(rng, (6, 96)), bf16_values(rng, (6, 96))
    y, s = O.add_rms_norm(x, r, w, 1e-6, 1.0)
    dxa, dra, dwa = O.add_rms_norm_bwd(x, r, w, dy, ds, 1e-6, 1.0)
    save("add_rms_norm", ('x', 'residual', 'weight', 'dy', 'ds'), x=x, residual=r, weight=w, dy=dy, ds=ds, eps=1e-6, offset=1.0, y=y, s=s, dx=dxa,
         dresidual=dra, dweight=dwa)
    # swiglu
    a, b, g = bf16_values(rng, (5, 80), 2.0), bf16_values(rng, (5, 80)), bf16_values(rng, (5, 80))
    da, dbb = O.swiglu_bwd(g, a, b)
    save("swiglu", ('a', 'b', 'dy'), a=a, b=b, dy=g, y=O.swiglu(a, b), da=da, db=dbb)
    # rotary_embedding, NeoX and GPT-J, partial rotary
    xr = bf16_values(rng, (2, 7, 3, 64))
    ang = np.arange(7)[:, None] * 500000.0 ** (-np.arange(24) / 24)
    cos, sin = np.cos(ang), np.sin(ang)
    gr = bf16_values(rng, (2, 7, 3, 64))
    save("rotary_embedding", ('x', 'dy'), x=xr, cos=cos, sin=sin, dy=gr, y=O.rotary_embedding(xr, cos, sin, False),
         y_interleaved=O.rotary_embedding(xr, cos, sin, True), dx=O.rotary_embedding_bwd(gr, cos, sin, False),
         dx_interleaved=O.rotary_embedding_bwd(gr, cos, sin, True))
    # rope and qk_norm_rope, per-batch tables whose halves differ
    q, k = bf16_values(rng, (2, 4, 9, 32)), bf16_values(rng, (2, 2, 9, 32))
    tc, ts = np.cos(bf16_values(rng, (2, 9, 32))), np.sin(bf16_values(rng, (2, 9, 32)))
    gq, gk = bf16_values(rng, (2, 4, 9, 32)), bf16_values(rng, (2, 2, 9, 32))
    yq, yk = O.rope(q, k, tc, ts)
    dq, dk = O.rope_bwd(gq, gk, tc, ts)
    save("rope", ('q', 'k', 'dyq', 'dyk'), q=q, k=k, cos=tc, sin=ts, dyq=gq, dyk=gk, yq=yq, yk=yk, dq=dq, dk=dk)
    qw, kw = bf16_values(rng, (32,)), bf16_values(rng, (32,))
    nq, nk = O.qk_norm_rope(q, k, qw, kw, tc, ts, 1e-6)
    ndq, ndk, ndqw, ndkw = O.qk_norm_rope_bwd(q, k, qw, kw, tc, ts, gq, gk, 1e-6)
    save("qk_norm_rope", ('q', 'k', 'q_weight', 'k_weight', 'dyq', 'dyk'), q=q, k=k, q_weight=qw, k_weight=kw, cos=tc, sin=ts, dyq=gq, dyk=gk, eps=1e-6, yq=nq,
         yk=nk, dq=ndq, dk=ndk, dq_weight=ndqw, dk_weight=ndkw)
    # attention: causal and full GQA, its LSE and its backward
    qa, ka, va = bf16_values(rng, (1, 29, 4, 64)), bf16_values(rng, (1, 29, 2, 64)), bf16_values(rng, (1, 29, 2, 64))
    doa = bf16_values(rng, (1, 29, 4, 64))
    out = {}
    for causal in (False, True):
        o, lse = O.attention(qa, ka, va, causal, None)
        gq_, gk_, gv_ = O.attention_bwd(qa, ka, va, doa, causal, None)
        tag = "causal" if causal else "full"
        out.update({f"o_{tag}": o, f"lse_{tag}": lse, f"dq_{tag}": gq_, f"dk_{tag}": gk_, f"dv_{tag}": gv_})
    save("attn", ('q', 'k', 'v', 'do'), q=qa, k=ka, v=va, do=doa, **out)
    # packed sequences
    cu = np.array([0, 5, 6, 21, 33], dtype=np.int32)
    qv, kv_, vv = bf16_values(rng, (33, 2, 64)), bf16_values(rng, (33, 1, 64)), bf16_values(rng, (33, 1, 64))
    ov, lv = O.attention_varlen(qv, kv_, vv, cu, True, 0.2)
    save("attn_varlen", ('q', 'k', 'v'), q=qv, k=kv_, v=vv, cu_seqlens=cu, softmax_scale=0.2, o=ov, lse=lv)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
