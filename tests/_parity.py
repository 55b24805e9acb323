"""Parity helpers for the GPU tests.

`gauge_ok` is Popcorn's pass rule (bench/compare.py:14,49-54,279-294 and
bench/model.py:61-71): with err = max|mine - truth|, budget = max|ref@native -
truth| and scale = max(1, max|truth|), an output passes iff
err <= max(2*budget, floor*scale); floor is 2e-5 (fp32), 1e-3 (fp16),
2e-2 (bf16). `close_to_reference` is the north star's fixed tolerance
against the registered reference at native dtype.
"""

from __future__ import annotations

import math

import numpy as np
import torch

FLOORS = {torch.float32: 2e-5, torch.float16: 1e-3, torch.bfloat16: 2e-2}
NORTH_STAR = {torch.float32: (1e-5, 1e-5), torch.float16: (2e-2, 2e-2), torch.bfloat16: (2e-2, 2e-2)}


def _as64(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().to("cpu", torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


def max_err(value, truth) -> float:
    a, b = _as64(value), _as64(truth)
    if a.size == 0:
        return 0.0
    same = (a == b) | (np.isnan(a) & np.isnan(b))
    diff = np.where(same, 0.0, np.abs(a - b))
    err = float(diff.max())
    return err if math.isfinite(err) else float("inf")


def gauge_ok(mine, truth, ref_native, dtype: torch.dtype, what: str = "out") -> dict:
    floor = FLOORS[dtype]
    t = _as64(truth)
    err = max_err(mine, t)
    budget = max_err(ref_native, t)
    # a reference that is not finite where the truth is would make any error pass
    assert math.isfinite(budget), f"{what}: the native-dtype reference is not finite against the float64 truth"
    scale = max(1.0, float(np.abs(t).max()) if t.size else 1.0)
    limit = max(2 * budget, floor * scale)
    assert math.isfinite(err) and err <= limit, (
        f"{what}: err {err:.3e} > max(2*{budget:.3e}, {floor:.0e}*{scale:.2f})"
    )
    return {"err": err, "budget": budget, "scale": scale}


def close_to_reference(mine: torch.Tensor, ref: torch.Tensor, what: str = "out",
                       rounding: torch.dtype | None = None) -> None:
    """`rounding`: the dtype whose tolerance applies when an fp32 output carries a 16-bit rounding
    (a 16-bit input promoted by an fp32 operand); by default the output's own dtype."""
    rtol, atol = NORTH_STAR[ref.dtype if rounding is None else rounding]
    torch.testing.assert_close(mine.detach().cpu(), ref.detach().cpu(), rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def seeded(shape, seed: int, dtype: torch.dtype, device="cpu", scale: float = 1.0, offset: float = 0.0):
    """Popcorn's input recipe (bench/grid.py:675-716): N(0,1) drawn in fp32 on a
    seeded CPU generator, then cast, then moved."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(shape, generator=g) * scale + offset
    return t.to(dtype).to(device)
