"""The C ABI library loads and exports every entry point include/popcorn_amd.h declares.

Only argument validation is exercised here: those paths return before any
HIP call, so they run without a GPU. Compute calls are the GPU tests' job.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from popcorn_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "popcorn_amd.h"


def declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(pk_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIBRARY.exists():
        pytest.fail(f"{_lib.LIBRARY} is not built; run __graft_entry__.build()")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_typed(lib):
    names = declared()
    assert names, "no pk_* declarations found"
    assert names == set(_lib.SIGNATURES), "ctypes bindings and the header disagree"
    raw = ctypes.CDLL(str(_lib.LIBRARY))
    for name in names:
        assert hasattr(raw, name), f"{name} is declared but not exported"


def test_version_and_status_codes(lib):
    assert lib.pk_version() == _lib.ABI_VERSION
    text = HEADER.read_text()
    for name, value in (("PK_OK", _lib.OK), ("PK_ERR_INVALID", _lib.ERR_INVALID),
                        ("PK_ERR_UNSUPPORTED", _lib.ERR_UNSUPPORTED), ("PK_ERR_HIP", _lib.ERR_HIP),
                        ("PK_F32", _lib.F32), ("PK_BF16", _lib.BF16), ("PK_F16", _lib.F16)):
        assert re.search(rf"#define {name} {value}\b", text), name


def test_attention_backward_workspace_queries(lib):
    """Host logic only: two fp32 row vectors (D and log2-scaled lse) per (row, q head), padded to 256 bytes,
    plus fp32 dK and dV partials per q-head split when a grid of 128-key blocks cannot fill a 256-CU device
    twice over (this container has no device, so the library assumes MI355X's 256 CUs)."""
    mib = 1 << 20
    # B=8, S=1024, 32/8 heads: 8 key blocks x 8 x 8 = 512 blocks = two per CU, so no split
    assert lib.pk_attn_bwd_workspace(8, 1024, 32, 8, 128) == 2 * 8 * 32 * 1024 * 4 == 2 * mib
    # B=1: 64 blocks; no divisor of the group of 4 reaches 512, so one q head per block (4 splits)
    assert lib.pk_attn_bwd_workspace(1, 1024, 32, 8, 128) == 2 * 32 * 1024 * 4 + 4 * 2 * 1024 * 8 * 128 * 4
    # B=4, S=1024: 256 blocks, two splits give 512
    assert lib.pk_attn_bwd_workspace(4, 1024, 32, 8, 64) == 2 * 4 * 32 * 1024 * 4 + 2 * 2 * 4 * 1024 * 8 * 64 * 4
    assert lib.pk_attn_bwd_workspace(1, 3, 1, 1, 64) == 256  # 6 floats, padded; a group of one never splits
    assert lib.pk_attn_bwd_workspace(0, 1024, 32, 8, 128) == 0
    for bad in ((-1, 8, 4, 4, 64), (1, 8, 6, 4, 64), (1, 8, 4, 0, 64), (1, -8, 4, 4, 64)):
        assert lib.pk_attn_bwd_workspace(*bad) == -1, bad
    # packed sequences: rows = total tokens, blocks counted at the longest sequence
    assert lib.pk_attn_varlen_bwd_workspace(64, 64 * 1024, 1024, 32, 8, 128) == 2 * 32 * 64 * 1024 * 4
    assert lib.pk_attn_varlen_bwd_workspace(2, 1500, 1024, 8, 2, 128) == (
        (2 * 8 * 1500 * 4 + 255) // 256 * 256 + 4 * 2 * 1500 * 2 * 128 * 4)
    assert lib.pk_attn_varlen_bwd_workspace(2, 1500, 1024, 8, 3, 128) == -1


def test_invalid_arguments_are_rejected_before_any_launch(lib):
    assert lib.pk_swiglu_fwd(None, None, None, -1, _lib.BF16, None) == _lib.ERR_INVALID
    assert "negative size" in lib.pk_last_error().decode()
    assert lib.pk_swiglu_fwd(None, None, None, 0, _lib.BF16, None) == _lib.OK  # empty: nothing to do
    assert lib.pk_swiglu_fwd(None, None, None, 8, 7, None) in (_lib.ERR_INVALID, _lib.ERR_UNSUPPORTED)
    assert lib.pk_rmsnorm_fwd(None, None, None, None, None, -1, 8, 1e-6, _lib.F32, _lib.F32, None) == _lib.ERR_INVALID
    assert lib.pk_rmsnorm_bwd_workspace(0, 8, _lib.BF16) == 0
    assert lib.pk_rmsnorm_bwd_workspace(4096, 8192, _lib.BF16) > 0
    strides = (ctypes.c_int64 * 12)(*([8] * 12))
    rc = lib.pk_attn_fwd(None, None, None, None, None, strides, 1, 16, 4, 3, 64, 0.125, 1, _lib.BF16, None)
    assert rc == _lib.ERR_INVALID  # null pointers
    rot = (ctypes.c_int64 * 6)(*([128] * 6))
    rc = lib.pk_rotary(None, None, None, None, rot, 1, 4, 2, 128, 80, _lib.BF16, _lib.F32, 0, 0, None)
    assert rc == _lib.ERR_INVALID and "half" in lib.pk_last_error().decode()
    rc = lib.pk_add_rmsnorm_fwd(None, None, None, None, None, None, 4, 64, 1e-6, 0.0, _lib.BF16, _lib.BF16, None)
    assert rc == _lib.ERR_INVALID and "null pointer" in lib.pk_last_error().decode()
    assert lib.pk_add_rmsnorm_fwd(None, None, None, None, None, None, 0, 64, 1e-6, 0.0, _lib.BF16, _lib.BF16,
                                  None) == _lib.OK
    rc = lib.pk_add_rmsnorm_bwd(None, None, None, None, None, None, None, None, 0, 4, 64, 1.0, _lib.BF16, _lib.BF16,
                                None)
    assert rc == _lib.ERR_INVALID and "null pointer" in lib.pk_last_error().decode()
    rc = lib.pk_add_rmsnorm_fwd(None, None, None, None, None, None, 4, 64, 1e-6, 0.0, 9, 9, None)
    assert rc == _lib.ERR_UNSUPPORTED and "dtype" in lib.pk_last_error().decode()
    rs = (ctypes.c_int64 * 12)(*([64] * 12))
    rc = lib.pk_rope(None, None, None, None, None, None, rs, 2, 4, 2, 8, 63, 1, _lib.BF16, _lib.BF16, _lib.BF16, 0, None)
    assert rc == _lib.ERR_INVALID and "odd" in lib.pk_last_error().decode()
    rc = lib.pk_rope(None, None, None, None, None, None, rs, 2, 4, 2, 8, 64, 3, _lib.BF16, _lib.BF16, _lib.BF16, 0, None)
    assert rc == _lib.ERR_INVALID and "cos_batch" in lib.pk_last_error().decode()
    rc = lib.pk_rope(None, None, None, None, None, None, rs, 2, 4, 2, 8, 64, 2, _lib.BF16, _lib.BF16, _lib.BF16, 0, None)
    assert rc == _lib.ERR_INVALID and "null pointer" in lib.pk_last_error().decode()
    assert lib.pk_rope(None, None, None, None, None, None, rs, 2, 0, 0, 8, 64, 1, _lib.BF16, _lib.BF16, _lib.BF16, 0, None) == 0
    # dtype pairs: one dtype, or a 16-bit side beside fp32 (rope); x's, or fp32 from 16 bits (qk_norm_rope)
    fake = ctypes.c_void_p(16)
    rc = lib.pk_rope(fake, fake, fake, fake, fake, fake, rs, 2, 4, 2, 8, 64, 1, _lib.BF16, _lib.F16, _lib.F32, 0, None)
    assert rc == _lib.ERR_UNSUPPORTED and "dtype" in lib.pk_last_error().decode()
    rc = lib.pk_qk_norm_rope_fwd(None, None, None, None, None, None, None, None, None, None, rs, 2, 4, 2, 8, 64, 1,
                                 1e-6, _lib.F32, _lib.BF16, _lib.F32, _lib.F32, None)
    assert rc == _lib.ERR_UNSUPPORTED and "dtype" in lib.pk_last_error().decode()
    # fp32 weights beside 16-bit q/k need fp32 outputs
    rc = lib.pk_qk_norm_rope_fwd(None, None, None, None, None, None, None, None, None, None, rs, 2, 4, 2, 8, 64, 1,
                                 1e-6, _lib.BF16, _lib.BF16, _lib.BF16, _lib.F32, None)
    assert rc == _lib.ERR_UNSUPPORTED and "dtype" in lib.pk_last_error().decode()
    rc = lib.pk_rmsnorm_fwd(fake, fake, None, fake, None, 4, 64, 1e-6, _lib.F32, _lib.BF16, None)
    assert rc == _lib.ERR_UNSUPPORTED and "weight dtype" in lib.pk_last_error().decode()


def test_missing_library_raises(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(tmp_path / "absent.so")
