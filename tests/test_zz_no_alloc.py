"""pk_rmsnorm_bwd_noalloc against pk_rmsnorm_bwd, both called through the C ABI.

The allocation-free entry point runs the same kernels, grid and summation order
as the workspace entry point, with its partial rows in a fixed device array, so
every output must match bit for bit. Two calls in a row, the second smaller,
show that the array's leftover contents from a larger call do not leak into a
later one. A shape whose partials do not fit the array is refused on the host.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import reference as O
from popcorn_amd import _lib
from tests._parity import seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return _lib.load()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _inputs(rows, cols, dtype, seed, with_bias, wdtype=None):
    """x in `dtype`; weight, bias and the cotangent dy in `wdtype` (default `dtype`)."""
    wdtype = dtype if wdtype is None else wdtype
    x = seeded((rows, cols), seed, dtype).to(DEV)
    w = (1 + 0.1 * seeded((cols,), seed + 1, torch.float32)).to(wdtype).to(DEV)
    dy = seeded((rows, cols), seed + 2, wdtype).to(DEV)
    bias = seeded((cols,), seed + 3, wdtype).to(DEV) if with_bias else None
    return x, w, dy, bias


def _forward_rstd(lib, x, w, bias, rows, cols, code, wcode, stream):
    y = torch.empty(x.shape, dtype=w.dtype, device=DEV)
    rstd = torch.empty(rows, dtype=torch.float32, device=DEV)
    _lib.check(lib.pk_rmsnorm_fwd(_ptr(x), _ptr(w), _ptr(bias), _ptr(y), _ptr(rstd), rows, cols, 1e-6, code, wcode,
                                  stream),
               lib)
    return rstd


def _backward_with_workspace(lib, x, w, rstd, dy, with_bias, rows, cols, code, wcode, stream):
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    db = torch.empty_like(w) if with_bias else None
    nbytes = lib.pk_rmsnorm_bwd_workspace(rows, cols, code)
    work = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    _lib.check(lib.pk_rmsnorm_bwd(_ptr(x), _ptr(w), _ptr(rstd), _ptr(dy), _ptr(dx), _ptr(dw), _ptr(db), _ptr(work),
                                  nbytes, rows, cols, code, wcode, stream), lib)
    return dx, dw, db


def _backward_noalloc(lib, x, w, rstd, dy, with_bias, rows, cols, code, wcode, stream):
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    db = torch.empty_like(w) if with_bias else None
    # poison the outputs so a skipped write cannot pass as a match
    for t in (dx, dw, db):
        if t is not None:
            t.fill_(float("nan"))
    _lib.check(lib.pk_rmsnorm_bwd_noalloc(_ptr(x), _ptr(w), _ptr(rstd), _ptr(dy), _ptr(dx), _ptr(dw), _ptr(db),
                                          rows, cols, code, wcode, stream), lib)
    return dx, dw, db


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _compare(lib, rows, cols, dtype, seed, with_bias, wdtype=None):
    wdtype = dtype if wdtype is None else wdtype
    code, wcode = _lib.dtype_code(dtype), _lib.dtype_code(wdtype)
    stream = _lib.stream_handle(torch.device(DEV))
    print(f"[noalloc] rows={rows} cols={cols} dtype={dtype} weight={wdtype} bias={with_bias}", flush=True)
    x, w, dy, bias = _inputs(rows, cols, dtype, seed, with_bias, wdtype)
    rstd = _forward_rstd(lib, x, w, bias, rows, cols, code, wcode, stream)
    ref = _backward_with_workspace(lib, x, w, rstd, dy, with_bias, rows, cols, code, wcode, stream)
    mine = _backward_noalloc(lib, x, w, rstd, dy, with_bias, rows, cols, code, wcode, stream)
    torch.cuda.synchronize()
    for name, a, b in zip(("dx", "dw", "db"), mine, ref):
        if b is None:
            continue
        assert torch.equal(_bits(a), _bits(b)), f"{name} differs from pk_rmsnorm_bwd at ({rows}, {cols}) {dtype}"
    return x, w, dy, mine


def test_noalloc_matches_workspace_entry_point_on_two_calls(lib):
    for cols in (1024, 4096, 8192, 16384):
        for code in (_lib.F32, _lib.BF16):
            print(f"[noalloc] workspace rows=65536 cols={cols} dtype={code}: "
                  f"{lib.pk_rmsnorm_bwd_workspace(65536, cols, code)} bytes", flush=True)
    # the C4 backward fills most of the array, then a smaller call must not see its leftovers
    _compare(lib, 65536, 8192, torch.bfloat16, 0, False)
    x, w, dy, (dx, dw, _) = _compare(lib, 300, 2048, torch.bfloat16, 7, False)
    # the small call also meets the float64 oracle within the bf16 tolerance
    tdx, tdw, _ = O.rms_norm_bwd(x.double().cpu().numpy(), w.double().cpu().numpy(), dy.double().cpu().numpy(), 1e-6)
    scale = max(1.0, float(np.abs(tdx).max()))
    assert float(np.abs(dx.double().cpu().numpy() - tdx).max()) <= 2e-2 * scale
    scale = max(1.0, float(np.abs(tdw).max()))
    assert float(np.abs(dw.double().cpu().numpy() - tdw).max()) <= 2e-2 * scale


def test_noalloc_other_dtypes_bias_and_row_widths(lib):
    _compare(lib, 4096, 4096, torch.float32, 1, False)
    _compare(lib, 1030, 1000, torch.float16, 2, True)  # unaligned width: the one-block-per-row kernels
    _compare(lib, 9001, 256, torch.bfloat16, 3, True)  # four rows per block
    _compare(lib, 17, 8192, torch.float32, 4, True)
    _compare(lib, 4096, 8192, torch.bfloat16, 5, False, torch.float32)  # 16-bit x, fp32 weight and dy
    _compare(lib, 1030, 1000, torch.float16, 6, True, torch.float32)


def test_noalloc_refuses_a_shape_beyond_the_array(lib):
    # 4096 rows of 2^18 fp32 columns: a partial row is 1 MiB, and the grid holds at least one
    # block per CU (256), so 256 MiB of partials against the 96 MiB array. The host-side layout
    # says so first; the call then passes null pointers, so it can never launch: the entry point
    # checks the size before the pointers, and were that check ever to regress, the null check
    # would refuse the call with PK_ERR_INVALID instead of running out of bounds.
    rows, cols = 4096, 1 << 18
    assert lib.pk_rmsnorm_bwd_workspace(rows, cols, _lib.F32) > 96 << 20
    rc = lib.pk_rmsnorm_bwd_noalloc(None, None, None, None, None, None, None, rows, cols, _lib.F32, _lib.F32,
                                    _lib.stream_handle(torch.device(DEV)))
    assert rc == _lib.ERR_UNSUPPORTED, lib.pk_last_error().decode()
    assert "scratch" in lib.pk_last_error().decode()
    # within the limit, the same null pointers are refused as such (the order of the two checks)
    rc = lib.pk_rmsnorm_bwd_noalloc(None, None, None, None, None, None, None, 64, 1024, _lib.F32, _lib.F32,
                                    _lib.stream_handle(torch.device(DEV)))
    assert rc == _lib.ERR_INVALID and "null pointer" in lib.pk_last_error().decode()
