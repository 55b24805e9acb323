"""The backend through Popcorn's register -> validate -> record -> select path, on an MI355X.

`op.benchmark(..., backend="mi355x")` runs the harness (float64 truth,
native-dtype budget, timings) and writes a schema-3 row to the user cache;
a plain `op(...)` afterwards must route to the backend exactly when its
recorded time beats torch's by more than the 3% indifference margin
(core/policy.py:30, 164-172). The first tests do that at small shapes for
every op; the `test_baseline_*` tests do it at the five BASELINE configs and
require the backend to be the one chosen. Reference-side attention is
evaluated through fused SDPA kernels or explicit contiguous products
(compat.references.attn).
"""

from __future__ import annotations

import json

import pytest
import torch

from popcorn_amd import backend, compat, impls
from popcorn_amd.compat import store

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAME = backend.BACKEND


@pytest.fixture(scope="module", autouse=True)
def _registered():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    backend.register(compat)


@pytest.fixture(autouse=True)
def _fresh_selection(tmp_path, monkeypatch):
    monkeypatch.setattr(store, "BUNDLED_REPORTS", tmp_path / "bundled")
    for op in compat.KERNELS.values():
        op.tuner.forget()
    yield
    for op in compat.KERNELS.values():
        op.tuner.forget()


def _randn(*shape, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(DEV)


def _selected(op):
    choice = op.tuner.last_choice()
    assert choice is not None, "no selection was made"
    return choice


def _check_record_and_route(op, record, call):
    r = record.result
    assert record.impl == NAME and r.status == "pass", (r.status, r.reason)
    assert r.benchmarked and r.bench["fwd_ms"] > 0 and r.bench["ref_fwd_ms"] > 0, r.bench_error
    ours = r.bench["fwd_ms"] + r.bench.get("bwd_ms", 0.0)
    theirs = r.bench["ref_fwd_ms"] + r.bench.get("ref_bwd_ms", 0.0)
    print(f"{op.name}: {NAME} {ours:.4f} ms vs torch {theirs:.4f} ms ({theirs / ours:.1f}x)", flush=True)
    op.tuner.forget()
    call()
    expect = NAME if ours * 1.03 < theirs else "torch"
    assert _selected(op) == expect
    rows = [json.loads(line) for line in (store.user_reports() / f"{op.name}.jsonl").read_text().splitlines()]
    assert any(row["impl"] == NAME and row["status"] == "pass" for row in rows)


def test_rms_norm_records_and_routes_with_grad():
    op = compat.KERNELS["rms_norm"]
    x = _randn(4096, 4096).requires_grad_()
    w = (1 + 0.1 * _randn(4096, dtype=torch.float32, seed=1)).bfloat16().requires_grad_()
    [record] = op.benchmark(x, w, backend=NAME)
    assert record.result.grad and "x" in record.result.bwd and "weight" in record.result.bwd
    _check_record_and_route(op, record, lambda: op(x, w))


def test_add_rms_norm_records_and_routes_with_grad():
    """Two outputs (y, s), both graded with their own cotangents, and offset 1.0 from the test pool."""
    op = compat.KERNELS["add_rms_norm"]
    x, res = _randn(4096, 4096).requires_grad_(), _randn(4096, 4096, seed=2).requires_grad_()
    w = (1 + 0.1 * _randn(4096, dtype=torch.float32, seed=1)).bfloat16().requires_grad_()
    [record] = op.benchmark(x, res, w, 1e-6, 1.0, backend=NAME)
    assert record.result.grad and {"x", "residual", "weight"} <= set(record.result.bwd)
    _check_record_and_route(op, record, lambda: op(x, res, w, 1e-6, 1.0))


def test_swiglu_records_and_routes_with_grad():
    op = compat.KERNELS["swiglu"]
    a, b = _randn(4096, 8192).requires_grad_(), _randn(4096, 8192, seed=1).requires_grad_()
    [record] = op.benchmark(a, b, backend=NAME)
    _check_record_and_route(op, record, lambda: op(a, b))


def test_rotary_records_and_routes():
    op = compat.KERNELS["rotary_embedding"]
    x = _randn(4, 1024, 16, 128).requires_grad_()
    cos, sin = _randn(1024, 64, seed=1), _randn(1024, 64, seed=2)  # the harness's all-bf16 randn tables
    [record] = op.benchmark(x, cos, sin, backend=NAME)
    _check_record_and_route(op, record, lambda: op(x, cos, sin))


def test_rope_records_and_routes_with_grad():
    op = compat.KERNELS["rope"]
    q, k = _randn(4, 32, 1024, 128).requires_grad_(), _randn(4, 8, 1024, 128, seed=1).requires_grad_()
    ang = _randn(1, 1024, 64, dtype=torch.float32, seed=2)
    cos, sin = (f(ang).repeat(1, 1, 2).bfloat16() for f in (torch.cos, torch.sin))
    [record] = op.benchmark(q, k, cos, sin, backend=NAME)
    assert record.result.grad and {"q", "k"} <= set(record.result.bwd)
    _check_record_and_route(op, record, lambda: op(q, k, cos, sin))


def test_qk_norm_rope_records_and_routes_with_grad():
    op = compat.KERNELS["qk_norm_rope"]
    q, k = _randn(4, 32, 1024, 128).requires_grad_(), _randn(4, 8, 1024, 128, seed=1).requires_grad_()
    qw, kw = _randn(128, seed=3).requires_grad_(), _randn(128, seed=4).requires_grad_()
    ang = _randn(1, 1024, 64, dtype=torch.float32, seed=2)
    cos, sin = (f(ang).repeat(1, 1, 2).bfloat16() for f in (torch.cos, torch.sin))
    [record] = op.benchmark(q, k, qw, kw, cos, sin, 1e-6, backend=NAME)
    assert record.result.grad and {"q", "k", "q_weight", "k_weight"} <= set(record.result.bwd)
    _check_record_and_route(op, record, lambda: op(q, k, qw, kw, cos, sin, 1e-6))


def test_recorded_rows_publish_to_popcorns_parquet_layout(tmp_path):
    """Rows this device records load back from `<op>.parquet` unchanged, ready to merge into Popcorn's reports."""
    op = compat.KERNELS["swiglu"]
    a, b = _randn(2048, 4096).requires_grad_(), _randn(2048, 4096, seed=1).requires_grad_()
    [record] = op.benchmark(a, b, backend=NAME)
    assert store.publish(tmp_path, ops=["swiglu"]) >= 1
    back = store.read_file(tmp_path / "swiglu.parquet")
    assert any(r.to_dict() == record.to_dict() for r in back)
    assert {r.environment.device for r in back} == {torch.cuda.get_device_name()}


def test_attn_records_and_routes_with_grad():
    op = compat.KERNELS["attn"]
    q, k, v = _randn(1, 1024, 8, 128), _randn(1, 1024, 2, 128, seed=1), _randn(1, 1024, 2, 128, seed=2)
    with torch.no_grad():
        [record] = op.benchmark(q, k, v, True, backend=NAME)
        assert not record.result.grad
        _check_record_and_route(op, record, lambda: op(q, k, v, True))
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    op.tuner.forget()
    [record] = op.benchmark(qg, kg, vg, True, backend=NAME)
    assert record.result.grad and {"q", "k", "v"} <= set(record.result.bwd)
    _check_record_and_route(op, record, lambda: op(qg, kg, vg, True))


def test_attn_varlen_records_and_routes_with_grad():
    op = compat.KERNELS["attn_varlen"]
    total = 3000
    q, k, v = _randn(total, 8, 128), _randn(total, 2, 128, seed=1), _randn(total, 2, 128, seed=2)
    cu = torch.tensor([0, 1000, 1001, 2500, total], dtype=torch.int32, device=DEV)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    [record] = op.benchmark(qg, kg, vg, cu, True, backend=NAME)
    assert record.result.grad
    _check_record_and_route(op, record, lambda: op(qg, kg, vg, cu, True))


def test_mixed_dtype_rotary_is_served_in_registration_order():
    """bf16 x with fp32 tables has no single dtype, so no record applies (core/config.py:95-99)."""
    op = compat.KERNELS["rotary_embedding"]
    x = _randn(2, 64, 4, 128)
    pos = torch.arange(64, dtype=torch.float64, device=DEV)[:, None]
    ang = pos * 500000.0 ** (-torch.arange(64, dtype=torch.float64, device=DEV) / 64)
    cos, sin = ang.cos().float(), ang.sin().float()
    y = op(x, cos, sin)
    assert _selected(op) == NAME
    assert torch.equal(y, impls.rotary_embedding(x, cos, sin))


def test_mixed_dtype_norms_and_rope_are_served_by_the_backend():
    """16-bit activations with fp32 weights or tables (the autocast model's calls) reach the kernels."""
    x = _randn(64, 1024)
    w = 1 + 0.1 * torch.randn(1024, device=DEV)
    op = compat.KERNELS["rms_norm"]
    y = op(x, w)
    assert _selected(op) == NAME and y.dtype == torch.float32
    assert torch.equal(y, impls.rms_norm(x, w))
    op = compat.KERNELS["add_rms_norm"]
    r = _randn(64, 1024, seed=2)
    y, s = op(x, r, w)
    assert _selected(op) == NAME and y.dtype == torch.float32 and s.dtype == x.dtype
    want = impls.add_rms_norm(x, r, w)
    assert torch.equal(y, want[0]) and torch.equal(s, want[1])
    q, k = _randn(1, 4, 32, 128), _randn(1, 2, 32, 128, seed=1)
    ang = torch.randn(1, 32, 64, device=DEV)
    cos, sin = ang.cos().repeat(1, 1, 2), ang.sin().repeat(1, 1, 2)
    op = compat.KERNELS["rope"]
    yq, yk = op(q, k, cos, sin)
    assert _selected(op) == NAME and yq.dtype == yk.dtype == torch.float32
    want = impls.rope(q, k, cos, sin)
    assert torch.equal(yq, want[0]) and torch.equal(yk, want[1])
    qw, kw = 1 + 0.1 * torch.randn(128, device=DEV), 1 + 0.1 * torch.randn(128, device=DEV)
    op = compat.KERNELS["qk_norm_rope"]
    yq, yk = op(q, k, qw, kw, cos.bfloat16(), sin.bfloat16())
    assert _selected(op) == NAME and yq.dtype == yk.dtype == torch.float32
    want = impls.qk_norm_rope(q, k, qw, kw, cos.bfloat16(), sin.bfloat16())
    assert torch.equal(yq, want[0]) and torch.equal(yk, want[1])


def test_bench_mode_measures_lazily(monkeypatch):
    op = compat.KERNELS["swiglu"]
    monkeypatch.setenv("POPCORN_BENCH", "1")
    a, b = _randn(512, 4096), _randn(512, 4096, seed=1)
    op(a, b)
    rows = [json.loads(line) for line in (store.user_reports() / "swiglu.jsonl").read_text().splitlines()]
    assert [(r["impl"], r["status"], r["benchmarked"]) for r in rows] == [(NAME, "pass", True)]
    op(a, b)  # already measured: no new row
    assert len((store.user_reports() / "swiglu.jsonl").read_text().splitlines()) == 1


# --------------------------------------------------------------------------- the five BASELINE configs


def _auto_selected(op, record, call):
    """The recorded row passes and beats torch by more than the indifference margin, and a plain call picks it."""
    r = record.result
    assert record.impl == NAME and r.status == "pass", (r.status, r.reason)
    assert r.benchmarked, r.bench_error
    ours = r.bench["fwd_ms"] + r.bench.get("bwd_ms", 0.0)
    theirs = r.bench["ref_fwd_ms"] + r.bench.get("ref_bwd_ms", 0.0)
    print(f"[selected] {op.name} {record.case}: {NAME} {ours:.4f} ms, torch on the GPU {theirs:.4f} ms "
          f"({theirs / ours:.2f}x)", flush=True)
    op.tuner.forget()
    out = call()
    assert _selected(op) == NAME, f"torch was chosen: {ours:.4f} ms against torch's {theirs:.4f} ms"
    return out


def test_baseline_c1_rms_norm_fp32_forward_is_auto_selected():
    op = compat.KERNELS["rms_norm"]
    x = _randn(4096, 4096, dtype=torch.float32)
    w = 1 + 0.1 * _randn(4096, dtype=torch.float32, seed=1)
    with torch.no_grad():
        [record] = op.benchmark(x, w, None, 1e-6, backend=NAME)
        y = _auto_selected(op, record, lambda: op(x, w, None, 1e-6))
    assert torch.equal(y, impls.rms_norm(x, w, None, 1e-6))


def test_baseline_c2_swiglu_full_size_is_auto_selected():
    op = compat.KERNELS["swiglu"]
    a, b = _randn(16384, 14336), _randn(16384, 14336, seed=1)
    with torch.no_grad():
        [record] = op.benchmark(a, b, backend=NAME)
        _auto_selected(op, record, lambda: op(a, b))


def test_baseline_c3_rotary_q_and_k_with_bf16_tables_are_auto_selected():
    """C3's two calls with the harness's all-bf16 tables (its fp32-table form has no single dtype, so no
    record applies and registration order serves it: test_mixed_dtype_rotary_is_served_in_registration_order)."""
    op = compat.KERNELS["rotary_embedding"]
    pos = torch.arange(4096, dtype=torch.float64, device=DEV)[:, None]
    ang = pos * 500000.0 ** (-torch.arange(64, dtype=torch.float64, device=DEV) / 64)
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    with torch.no_grad():
        for heads, seed in ((32, 0), (8, 1)):
            x = _randn(8, 4096, heads, 128, seed=seed)
            [record] = op.benchmark(x, cos, sin, backend=NAME)
            _auto_selected(op, record, lambda: op(x, cos, sin))


def test_baseline_c4_rms_norm_bf16_with_grad_is_auto_selected():
    op = compat.KERNELS["rms_norm"]
    x = _randn(65536, 8192).requires_grad_()
    w = (1 + 0.1 * _randn(8192, dtype=torch.float32, seed=1)).bfloat16().requires_grad_()
    [record] = op.benchmark(x, w, backend=NAME)
    assert record.result.grad and {"x", "weight"} <= set(record.result.bwd)
    _auto_selected(op, record, lambda: op(x, w))


def test_baseline_c5_causal_gqa_attention_forward_is_auto_selected():
    op = compat.KERNELS["attn"]
    q, k, v = _randn(4, 8192, 32, 128), _randn(4, 8192, 8, 128, seed=1), _randn(4, 8192, 8, 128, seed=2)
    with torch.no_grad():
        [record] = op.benchmark(q, k, v, True, backend=NAME)
        assert not record.result.grad
        _auto_selected(op, record, lambda: op(q, k, v, True))
