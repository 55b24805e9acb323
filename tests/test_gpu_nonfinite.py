"""Non-finite inputs: NaN and ±Inf land where Popcorn's torch reference puts them.

Popcorn's pass rule counts NaN against NaN as equal (bench/compare.py:49-54), so an implementation
that turned a reference NaN into a number, or a number into NaN, would fail a check that the
seeded N(0,1) inputs never exercise. Each case plants NaN, ±Inf and overflowing values in a few
rows of otherwise seeded inputs, runs the kernel on the GPU and the reference on the CPU at native
dtype, and requires the same NaN positions, the same ±Inf positions and signs, and the finite
values within the north star's tolerance.
"""

import math

import pytest
import torch

from popcorn_amd import impls
from popcorn_amd.compat import references as R
from tests._parity import NORTH_STAR, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
INF, NAN = math.inf, math.nan


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _same_pattern(mine: torch.Tensor, ref: torch.Tensor, what: str, rounding: torch.dtype | None = None):
    mine, ref = mine.detach().cpu().float(), ref.detach().float()
    assert mine.shape == ref.shape, what
    assert torch.equal(mine.isnan(), ref.isnan()), f"{what}: NaN positions differ"
    assert torch.equal(mine.isposinf(), ref.isposinf()), f"{what}: +Inf positions differ"
    assert torch.equal(mine.isneginf(), ref.isneginf()), f"{what}: -Inf positions differ"
    fin = ref.isfinite()
    rtol, atol = NORTH_STAR[rounding or torch.bfloat16]
    torch.testing.assert_close(mine[fin], ref[fin], rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def _plant(t: torch.Tensor, spots) -> torch.Tensor:
    t = t.clone()
    for index, value in spots:
        t[index] = value
    return t


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
def test_rms_norm_nonfinite_rows(dtype):
    """Row 0 holds +Inf (its rsqrt is 0: Inf * 0 = NaN there, zeros elsewhere), row 1 a NaN (all NaN),
    row 2 a value whose square overflows fp32 (the same zeros), row 3 stays finite."""
    big = 1e30 if dtype == torch.float32 else 6e4 if dtype == torch.float16 else 1e30
    x = _plant(seeded((5, 256), 1, dtype), [((0, 7), INF), ((1, 100), NAN), ((2, 3), big), ((2, 4), -big)])
    w = (1 + 0.1 * seeded((256,), 2, torch.float32)).to(dtype)
    with torch.no_grad():
        ref = R.rms_norm(x, w, None, 1e-6)
        mine = impls.rms_norm(x.to(DEV), w.to(DEV), None, 1e-6)
    _same_pattern(mine, ref, f"rms_norm {dtype}", rounding=dtype)


def test_add_rms_norm_nonfinite_residual():
    x = seeded((4, 512), 3, torch.bfloat16)
    r = _plant(seeded((4, 512), 4, torch.bfloat16), [((0, 9), INF), ((1, 1), NAN), ((2, 0), -INF)])
    w = (1 + 0.1 * seeded((512,), 5, torch.float32))
    with torch.no_grad():
        y_ref, s_ref = R.add_rms_norm(x, r, w, 1e-6, 0.0)
        y, s = impls.add_rms_norm(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6, 0.0)
    _same_pattern(s, s_ref, "add_rms_norm s")
    _same_pattern(y, y_ref, "add_rms_norm y")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_swiglu_nonfinite(dtype):
    """silu(+Inf) * b = Inf, silu(-Inf) = -Inf * 0 = NaN, silu(0) * Inf = NaN, a NaN anywhere gives NaN,
    and silu of a large negative value is a tiny number, not NaN."""
    a = _plant(seeded((3, 1024), 6, dtype), [((0, 0), INF), ((0, 1), -INF), ((0, 2), NAN), ((0, 3), -80.0),
                                            ((0, 4), 0.0), ((1, 5), 80.0)])
    b = _plant(seeded((3, 1024), 7, dtype), [((0, 4), INF), ((1, 5), -INF), ((2, 6), NAN)])
    with torch.no_grad():
        ref = R.swiglu(a, b)
        mine = impls.swiglu(a.to(DEV), b.to(DEV))
    _same_pattern(mine, ref, f"swiglu {dtype}", rounding=dtype)


@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "gptj"])
def test_rotary_nonfinite(interleaved):
    x = _plant(seeded((1, 16, 4, 128), 8, torch.bfloat16),
               [((0, 0, 0, 0), INF), ((0, 1, 1, 70), NAN), ((0, 2, 2, 5), -INF)])
    ang = seeded((16, 64), 9, torch.float32)
    cos, sin = ang.cos(), ang.sin()
    with torch.no_grad():
        ref = R.rotary_embedding(x, cos, sin, interleaved)
        mine = impls.rotary_embedding(x.to(DEV), cos.to(DEV), sin.to(DEV), interleaved)
    _same_pattern(mine, ref, f"rotary interleaved={interleaved}")


def test_rope_nonfinite():
    q = _plant(seeded((1, 4, 8, 64), 10, torch.bfloat16), [((0, 0, 0, 0), INF), ((0, 1, 3, 40), NAN)])
    k = _plant(seeded((1, 2, 8, 64), 11, torch.bfloat16), [((0, 1, 7, 63), -INF)])
    ang = seeded((1, 8, 32), 12, torch.float32).repeat(1, 1, 2)
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    with torch.no_grad():
        rq, rk = R.rope(q, k, cos, sin)
        mq, mk = impls.rope(q.to(DEV), k.to(DEV), cos.to(DEV), sin.to(DEV))
    _same_pattern(mq, rq, "rope q")
    _same_pattern(mk, rk, "rope k")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_nonfinite_key_and_value(causal, dtype):
    """A NaN in key 5 of kv head 0 makes every query of that group that sees key 5 NaN (all of them
    without the mask, rows 5 on with it); an Inf in a value row makes those queries' outputs in that
    dim Inf or NaN exactly as the reference's softmax-weighted sum does; other heads stay finite.
    fp32 runs the fp32 kernel's online softmax, bf16 the fixed-max sweep and its exact resweep."""
    b, s, hq, hkv, d = 1, 64, 4, 2, 64
    q = seeded((b, s, hq, d), 13, dtype)
    k = _plant(seeded((b, s, hkv, d), 14, dtype), [((0, 5, 0, 3), NAN)])
    v = _plant(seeded((b, s, hkv, d), 15, dtype), [((0, 40, 1, 7), INF)])
    with torch.no_grad():
        ref = R.attn(q, k, v, causal)
        mine = impls.attn(q.to(DEV), k.to(DEV), v.to(DEV), causal)
    _same_pattern(mine, ref, f"attn {dtype} causal={causal}")
