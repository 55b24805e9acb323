"""Dispatch, selection and recording behaviour of popcorn_amd.compat on the CPU.

These restate, as tests of this package, the behaviours Popcorn's own CPU
suite pins for its dispatcher (tests/core/test_core.py TestDispatch :167-383,
TestRegistration :384-580, TestTuning :643-1087, TestForwardOnly :1089-1116,
TestKernelAmbient :1149-1202, TestVersionGate :1204-1295): a toy op `x + 1`
with lambda backends and synthetic report rows in a temporary store.
"""

from __future__ import annotations

import json
import logging
import threading
from typing import Literal

import pytest
import torch
from torch import Tensor

from popcorn_amd.compat import (  # noqa: I001
    BackendUnavailableError,
    BackendVersionError,
    DispatchError,
    Dispatcher,
    Float,
    Range,
    Record,
    declare_backend,
    harness,
    kernel,
    report,
    store,
)
from popcorn_amd.compat.records import call_config, config_id, device_name
from popcorn_amd.compat.sources import installed_version


def make_op(**kwargs):
    def op(x: Float[Tensor, "... D"], weight: Float[Tensor, "D"] | None = None, flag: bool = False):
        return x + 1

    return Dispatcher(op, **kwargs)


@pytest.fixture
def reports(tmp_path, monkeypatch):
    bundled = tmp_path / "bundled"
    bundled.mkdir()
    monkeypatch.setattr(store, "BUNDLED_REPORTS", bundled)
    monkeypatch.setenv("POPCORN_CACHE_DIR", str(tmp_path / "cache"))
    return bundled


def row(op, x, *, backend="alt", status="pass", reason="", ts="2026-01-01T00:00:00+00:00", bench=None, **kwargs):
    bound = op._signature.bind(x, **kwargs)
    bound.apply_defaults()
    arguments = dict(bound.arguments)
    call = call_config(op, op._values(arguments), arguments)
    return {
        "schema": 3, "op": op.name, "impl": backend, "device": call.device_name, "case": "exact",
        "case_id": config_id(call.config), "status": status, "reason": reason, "grad": call.grad,
        "torch": torch.__version__, "backend_version": installed_version(backend), "ref_hash": op.fingerprint,
        "impl_hash": op[backend].fingerprint, "ts": ts, "config": call.config, "fwd": {}, "bwd": {},
        "bench": bench or {}, "benchmarked": bench is not None, "bench_error": "", "reps": 1,
    }


def dims_row(op, backend, dims, ms, ref_ms, batch=(1,), status="pass", bench=True):
    return {
        "schema": 3, "op": op.name, "impl": backend, "device": device_name("cpu"), "case": "",
        "case_id": f"{backend}-{dims}-{batch}", "status": status, "reason": "", "grad": False,
        "torch": torch.__version__, "backend_version": None, "ref_hash": op.fingerprint,
        "impl_hash": op[backend].fingerprint, "ts": "2026-01-01T00:00:00+00:00",
        "config": {"dims": dims, "batch": list(batch), "dtype": "float32", "args": {"flag": False}, "present": []},
        "bench": {"fwd_ms": ms, "ref_fwd_ms": ref_ms} if bench else {}, "benchmarked": bench, "bench_error": "",
        "fwd": {}, "bwd": {}, "reps": 1,
    }


def put(directory, *rows):
    store.write([Record.from_dict(r) for r in rows], directory)


# --------------------------------------------------------------------------- dispatch


def test_reference_is_fallback():
    op = make_op()
    assert op.available_backends() == ("torch",)
    assert torch.equal(op(torch.zeros(3, 4)), torch.ones(3, 4))


def test_registration_order_and_getitem():
    op = make_op()
    op.register("first")(lambda x, weight, flag: x + 10)
    op.register("second")(lambda x, weight, flag: x + 20)
    assert op.available_backends() == ("first", "second", "torch")
    assert torch.equal(op(torch.zeros(2)), torch.full((2,), 10.0))
    assert torch.equal(op["second"](torch.zeros(2)), torch.full((2,), 20.0))
    with pytest.raises(DispatchError, match="unknown backend"):
        op["nope"]


def test_region_gates_resolution(reports):
    op = make_op()
    op.register("fast")(lambda x, weight, flag: x - 1)
    rows = []
    for n in (2, 3, 4, 5, 8):
        r = dims_row(op, "fast", {"D": n}, 1.0, 1.0, batch=(), bench=False,
                     status="pass" if n & (n - 1) == 0 else "fail")
        rows.append(r)
    put(reports, *rows)
    # passes at 2, 4, 8 and fails at 3, 5 fit the region [2, 8] % 2
    assert torch.equal(op(torch.zeros(4)), -torch.ones(4))
    assert torch.equal(op(torch.zeros(6)), -torch.ones(6))  # never measured, inside the region
    assert torch.equal(op(torch.zeros(5)), torch.ones(5))  # recorded failure: torch serves
    assert torch.equal(op(torch.zeros(7)), torch.ones(7))  # odd: outside the modulus
    with pytest.raises(DispatchError, match="outside its validity region"):
        op(torch.zeros(10), backend="fast")


def test_annotation_gates(reports):
    op = make_op()

    @op.register("fast")
    def fast(x, weight, flag: Literal[False]):
        return x - 1

    x = torch.zeros(2, 4)
    put(reports, row(op, x, backend="fast"))
    assert torch.equal(op(x), -torch.ones_like(x))
    assert torch.equal(op(x, flag=True), torch.ones_like(x))
    with pytest.raises(DispatchError, match="does not satisfy"):
        op(x, flag=True, backend="fast")


def test_scope_is_nested_and_thread_local():
    op = make_op()
    op.register("a")(lambda x, weight, flag: x + 10)
    op.register("b")(lambda x, weight, flag: x + 20)

    def probe():
        return op(torch.zeros(2))[0].item()

    assert probe() == 10
    with op["b"] as scoped:
        assert scoped is op and probe() == 20
        with op["a"]:
            assert probe() == 10
        assert probe() == 20
    assert probe() == 10

    seen = {}

    def worker():
        seen["thread"] = probe()

    with op["b"]:
        t = threading.Thread(target=worker)
        t.start()
        t.join()
    assert seen["thread"] == 10  # a scope entered in one thread does not leak into another


def test_dim_consistency_and_predicate():
    op = make_op()
    with pytest.raises(DispatchError, match="dim 'D'"):
        op(torch.zeros(3, 4), weight=torch.zeros(5))
    op.register("alt", predicate=lambda x, weight, flag: x.ndim == 1)(lambda x, weight, flag: x - 1)
    assert torch.equal(op(torch.zeros(2)), -torch.ones(2))
    assert torch.equal(op(torch.zeros(2, 2)), torch.ones(2, 2))


def test_selection_cache_respects_current_eligibility():
    op = make_op()
    op.register("alt", predicate=lambda x, weight, flag: bool(x.sum() > 0))(lambda x, weight, flag: x - 1)
    assert torch.equal(op(torch.ones(2)), torch.zeros(2))
    assert torch.equal(op(-torch.ones(2)), torch.zeros(2))


def test_backward_flows_through_source_adapter():
    def square(x: Float[Tensor, "... D"]):
        return x * x

    op = Dispatcher(square)

    @op.register("alt", source="torch.mul")
    def alt(x):
        return kernel(x, x)

    ref_x = torch.randn(4, requires_grad=True)
    alt_x = ref_x.detach().clone().requires_grad_()
    op(ref_x, backend="torch").sum().backward()
    op(alt_x, backend="alt").sum().backward()
    assert torch.allclose(alt_x.grad, ref_x.grad)


def test_kernel_proxy_outside_dispatch():
    with pytest.raises(RuntimeError, match="only valid inside"):
        kernel(1)
    assert not hasattr(kernel, "anything")


# --------------------------------------------------------------------------- registration


def test_registration_conventions():
    op = make_op()
    with pytest.raises(TypeError, match="parameters must be exactly"):
        op.register("bad")(lambda x, weight: x)
    with pytest.raises(TypeError, match="must not declare defaults"):
        op.register("bad2")(lambda x, weight, flag=False: x)
    with pytest.raises(TypeError, match="does not narrow"):

        @op.register("bad3")
        def widened(x, weight, flag: int):
            return x

    assert op.available_backends() == ("torch",)  # failed attachments are removed
    op.register("ok")(lambda x, weight, flag: x)
    with pytest.raises(ValueError, match="already registered"):
        op.register("ok")
    with pytest.raises(ValueError, match="invalid backend name"):
        op.register("Bad Name")
    with pytest.raises(TypeError, match="not scalar arguments"):
        make_op(test_args={"x": [1]})


def test_source_only_registration_conformance():
    def ref(x: Float[Tensor, "... D"], y: Float[Tensor, "... D"]):
        return x + y

    op = Dispatcher(ref)
    op.register("add", source="torch.add")
    assert torch.equal(op(torch.ones(2), torch.ones(2), backend="add"), torch.full((2,), 2.0))

    op2 = Dispatcher(ref, name="ref2")
    op2.register("mine", source="popcorn_amd.compat.references.swiglu")  # params (a, b) != (x, y)
    with pytest.raises(TypeError, match="register an adapter"):
        op2(torch.ones(2), torch.ones(2), backend="mine")


def test_arg_pools_are_derived():
    op = make_op(test_args={})
    assert op.arg_pools == {"flag": [False, True]}
    eps_op = Dispatcher(lambda x, eps=1e-6: x, test_args={"eps": [1e-5, 1e-6]})
    assert eps_op.arg_pools["eps"] == [1e-6, 1e-5]  # the default comes first


# --------------------------------------------------------------------------- tuning


def test_picks_winner_of_closest_configuration(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    put(reports, dims_row(op, "alt", {"D": 8}, 1.0, 2.0), dims_row(op, "alt", {"D": 1024}, 3.0, 1.0))
    assert torch.equal(op(torch.zeros(3, 16)), -torch.ones(3, 16))  # near D=8: alt faster
    assert torch.equal(op(torch.zeros(3, 2048)), torch.ones(3, 2048))  # near D=1024: torch faster
    assert len(op.tuner._selected) == 2
    op(torch.zeros(3, 16))
    assert len(op.tuner._selected) == 2


def test_indifference_hands_close_calls_to_torch(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    put(reports, dims_row(op, "alt", {"D": 8}, 0.99, 1.0))  # 1% faster: inside the 3% indifference
    assert torch.equal(op(torch.zeros(1, 8)), torch.ones(1, 8))


def test_speed_args_do_not_share_timings_but_neutral_args_do(reports):
    def ref(x: Float[Tensor, "... D"], causal: bool = False, eps: float = 1e-6):
        return x + 1

    op = Dispatcher(ref)
    op.register("alt")(lambda x, causal, eps: x - 1)
    x = torch.zeros(2, 8)
    put(reports, row(op, x, causal=False, bench={"fwd_ms": 0.1, "ref_fwd_ms": 1.0}),
        row(op, x, causal=True, bench={"fwd_ms": 3.0, "ref_fwd_ms": 1.0}),
        row(op, x, causal=False, eps=1e-4))
    assert torch.equal(op(x, causal=False), -torch.ones_like(x))
    assert torch.equal(op(x, causal=True), torch.ones_like(x))
    assert torch.equal(op(x, causal=False, eps=5e-5), -torch.ones_like(x))  # inside the eps band


def test_each_backend_is_compared(reports):
    op = make_op()
    op.register("fast")(lambda x, weight, flag: x - 1)
    op.register("slow")(lambda x, weight, flag: x - 2)
    put(reports, dims_row(op, "fast", {"D": 4}, 0.1, 1.0), dims_row(op, "slow", {"D": 4}, 0.5, 1.0))
    assert torch.equal(op(torch.zeros(1, 4)), -torch.ones(1, 4))


def test_batch_shape_distance(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    put(reports, dims_row(op, "alt", {"D": 4}, 0.1, 1.0, batch=()), dims_row(op, "alt", {"D": 4}, 3.0, 1.0,
                                                                               batch=(2, 3)))
    assert torch.equal(op(torch.zeros(2, 3, 4)), torch.ones(2, 3, 4))


def test_unmapped_backend_serves_in_registration_order(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    assert torch.equal(op(torch.zeros(2, 4)), -torch.ones(2, 4))


def test_mapped_backend_blocked_outside_region_and_unsafe(reports):
    op = make_op()
    op.register("a")(lambda x, weight, flag: x - 1)
    op.register("b")(lambda x, weight, flag: x - 2)
    op.register("c")(lambda x, weight, flag: x - 3)
    put(reports, dims_row(op, "a", {"D": 8}, 0.5, 1.0), dims_row(op, "a", {"D": 16}, 0.5, 1.0),
        dims_row(op, "b", {"D": 8}, 0.2, 1.0), dims_row(op, "b", {"D": 16}, 0.2, 1.0),
        dims_row(op, "c", {"D": 8}, 0.05, 1.0))
    assert torch.equal(op(torch.zeros(1, 32)), torch.ones(1, 32))  # outside every region: torch
    assert torch.equal(op(torch.zeros(1, 32), unsafe=True), torch.zeros(1, 32) - 2)  # nearest proven: b
    with pytest.raises(DispatchError, match="outside its validity region"):
        op(torch.zeros(1, 32), backend="a")
    assert torch.equal(op(torch.zeros(1, 32), backend="a", unsafe=True), torch.zeros(1, 32) - 1)


def test_exact_failure_blocks_and_forcing_raises(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    x = torch.zeros(2, 4)
    put(reports, row(op, x, status="fail", reason="numeric mismatch"))
    assert torch.equal(op(x), torch.ones_like(x))
    for force in (lambda: op(x, backend="alt"), lambda: op["alt"](x)):
        with pytest.raises(DispatchError, match="numeric mismatch"):
            force()
    with op["alt"]:
        with pytest.raises(DispatchError, match="numeric mismatch"):
            op(x)
    # a failure binds only its exact config
    assert torch.equal(op(torch.zeros(3, 4), backend="alt"), -torch.ones(3, 4))
    assert torch.equal(op(x, flag=True, backend="alt"), -torch.ones_like(x))
    assert op(x.double(), backend="alt").dtype == torch.float64


def test_crash_blocks_but_harness_error_does_not(reports):
    x = torch.zeros(2, 4)
    crashed = make_op(name="crashed")
    crashed.register("alt")(lambda x, weight, flag: x - 1)
    put(reports, row(crashed, x, status="crash", reason="kernel crashed"))
    with pytest.raises(DispatchError, match="kernel crashed"):
        crashed(x, backend="alt")
    errored = make_op(name="errored")
    errored.register("alt")(lambda x, weight, flag: x - 1)
    put(reports, row(errored, x, status="error", reason="worker failed"))
    assert torch.equal(errored(x, backend="alt"), -torch.ones_like(x))


@pytest.mark.parametrize(("field", "value"), [("device", "other"), ("torch", "0.0.0"), ("ref_hash", "dead"),
                                              ("impl_hash", "dead")])
def test_rows_from_another_environment_or_stale_code_do_not_apply(reports, field, value):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    r = row(op, torch.zeros(2, 4), status="fail", reason="elsewhere")
    r[field] = value
    put(reports, r)
    assert torch.equal(op(torch.zeros(2, 4), backend="alt"), -torch.ones(2, 4))


@pytest.mark.parametrize(("bundled_ts", "user_ts", "fails"), [("2026-01-01T00:00:00+00:00", "2026-01-02T00:00:00+00:00",
                                                               False),
                                                              ("2026-01-02T00:00:00+00:00", "2026-01-01T00:00:00+00:00",
                                                               True)])
def test_newest_row_wins_across_bundled_and_user(reports, bundled_ts, user_ts, fails):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    x = torch.zeros(2, 4)
    put(reports, row(op, x, status="fail", reason="bundled", ts=bundled_ts))
    put(store.user_reports(), row(op, x, status="pass", reason="user", ts=user_ts))
    if fails:
        with pytest.raises(DispatchError, match="bundled"):
            op(x, backend="alt")
    else:
        assert torch.equal(op(x, backend="alt"), -torch.ones_like(x))


def test_newer_harness_error_cannot_erase_known_failure(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    x = torch.zeros(2, 4)
    put(reports, row(op, x, status="fail", reason="known failure", ts="2026-01-01T00:00:00+00:00"))
    put(store.user_reports(), row(op, x, status="error", reason="worker failed", ts="2026-01-02T00:00:00+00:00"))
    with pytest.raises(DispatchError, match="known failure"):
        op(x, backend="alt")


def test_validate_records_and_invalidates_selection(reports, caplog):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    x = torch.zeros(2, 4)
    op(x)
    assert op.tuner._selected
    with caplog.at_level(logging.INFO, logger="popcorn.bench"):
        [record] = op.validate(x, backend="alt")
    assert record.impl == "alt" and record.result.status == "fail"
    assert any("op:alt [fail]" in m for m in caplog.messages)
    assert not op.tuner._selected
    assert torch.equal(op(x), torch.ones_like(x))  # the recorded failure now blocks alt


def test_benchmark_records_correctness_and_timings(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x + 1)
    [record] = op.benchmark(torch.zeros(2, 4), backend="alt")
    assert record.result.status == "pass" and record.result.benchmarked
    assert record.result.bench["fwd_ms"] > 0 and record.result.bench["ref_fwd_ms"] > 0
    assert report(record).startswith("alt")
    rows = [json.loads(line) for line in (store.user_reports() / "op.jsonl").read_text().splitlines()]
    assert rows[0]["schema"] == 3 and rows[0]["impl"] == "alt"


def test_bench_mode_measures_once_and_routes(reports, monkeypatch):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    monkeypatch.setenv("POPCORN_BENCH", "1")
    assert torch.equal(op(torch.zeros(2, 4)), torch.ones(2, 4))  # alt measured, fails, torch serves
    rows = [json.loads(line) for line in (store.user_reports() / "op.jsonl").read_text().splitlines()]
    assert [r["status"] for r in rows] == ["fail"]


def test_bench_error_does_not_block_dispatch(reports, monkeypatch):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x + 1)

    def boom(*args, **kwargs):
        raise RuntimeError("timer failed")

    monkeypatch.setattr(harness, "_benchmark", boom)
    monkeypatch.setenv("POPCORN_BENCH", "1")
    assert torch.equal(op(torch.zeros(2, 4), backend="alt"), torch.ones(2, 4))
    [r] = [json.loads(line) for line in (store.user_reports() / "op.jsonl").read_text().splitlines()]
    assert r["status"] == "pass" and r["bench_error"] == "RuntimeError: timer failed"


def test_best_across_range(reports):
    op = make_op()
    op.register("alt")(lambda x, weight, flag: x - 1)
    put(reports, dims_row(op, "alt", {"D": 8}, 1.0, 2.0), dims_row(op, "alt", {"D": 16}, 1.0, 2.0),
        dims_row(op, "alt", {"D": 1024}, 3.0, 1.0))
    assert op.tuner.best(device="cpu", grad=False, D=Range(2, 32)).name == "alt"
    assert op.tuner.best(device="cpu", grad=False, D={1024}).name == "torch"
    with op.tuner.best(device="cpu", grad=False, D=Range(2, 32)):
        assert torch.equal(op(torch.zeros(2, 8)), -torch.ones(2, 8))
    with pytest.raises(TypeError, match="unknown filter keys"):
        op.tuner.best(nope=Range(1, 2))
    with pytest.raises(LookupError):
        op.tuner.best(device="cpu", D={7})


def test_forward_only_declines_grad_calls(reports):
    op = make_op()
    op.register("fwd", forward_only=True)(lambda x, weight, flag: x - 1)
    x = torch.zeros(2, requires_grad=True)
    assert torch.equal(op(x), torch.ones(2))
    assert torch.equal(op(torch.zeros(2)), -torch.ones(2))
    with torch.no_grad():
        assert torch.equal(op(x), -torch.ones(2))
    with pytest.raises(DispatchError, match="no backward"):
        op(x, backend="fwd")
    assert "fwd-only" in repr(op)


def test_unhashable_arguments_are_cached():
    op = Dispatcher(lambda x, sections: x, test_args={"sections": [[1, 2]]})
    op.register("alt")(lambda x, sections: x + sum(sections))
    assert torch.equal(op(torch.zeros(1), [1, 2]), torch.tensor([3.0]))
    assert len(op.tuner._selected) == 1


# --------------------------------------------------------------------------- version gate


def test_missing_distribution_is_skipped_not_fatal():
    declare_backend("ghost", package="popcorn-definitely-not-installed")
    op = make_op(name="ghosted")
    op.register("ghost")(lambda x, weight, flag: x - 1)
    assert torch.equal(op(torch.zeros(2)), torch.ones(2))  # ineligible: torch serves
    with pytest.raises(BackendUnavailableError):
        op(torch.zeros(2), backend="ghost")


def test_version_out_of_range_and_undeclared():
    declare_backend("old", package="torch", min_version="0.0.1", max_version="0.0.2")
    op = make_op(name="versioned")
    op.register("old")(lambda x, weight, flag: x - 1)
    op.register("free")(lambda x, weight, flag: x - 2)  # never declared: no gate
    with pytest.raises(BackendVersionError):
        op(torch.zeros(2), backend="old")
    assert torch.equal(op(torch.zeros(2)), torch.zeros(2) - 2)
