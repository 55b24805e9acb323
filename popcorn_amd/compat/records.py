"""Call configurations and report rows (schema 3).

A call is summarised as a canonical config -- dims, batch extent, dtype,
scalar args and which optional tensors are present -- and a stable 12-hex
`config_id` (core/config.py:38-114). One validation / benchmark outcome is a
`Record` whose dictionary form is Popcorn's report-row schema 3
(bench/model.py:105-163). The id scheme and the row keys are kept identical to
Popcorn's so rows written here and rows Popcorn writes name the same cases.
"""

from __future__ import annotations

import hashlib
import json
import math
import platform
from collections.abc import Iterable, Mapping
from dataclasses import asdict, dataclass, field
from typing import TYPE_CHECKING, Any

import torch

from popcorn_amd.compat.shapes import batch_shape

if TYPE_CHECKING:
    from popcorn_amd.compat.dispatcher import Dispatcher

SCHEMA = 3


def dtype_name(dtype: torch.dtype | str | None) -> str | None:
    return None if dtype is None else str(dtype).removeprefix("torch.")


def _plain(value: Any) -> Any:
    """A JSON-stable form of a scalar argument."""
    if isinstance(value, dict):
        return {str(k): _plain(v) for k, v in sorted(value.items(), key=lambda kv: str(kv[0]))}
    if isinstance(value, (list, tuple)):
        return [_plain(v) for v in value]
    if isinstance(value, (set, frozenset)):
        return sorted((_plain(v) for v in value), key=repr)
    if value is None or isinstance(value, (bool, int, float, str)):
        return value
    return str(value)


def make_config(
    dims: Mapping[str, int], batch: Iterable[int], dtype: torch.dtype | str | None, args: Mapping[str, Any],
    present: Iterable[str],
) -> dict[str, Any]:
    return {
        "dims": dict(sorted(dims.items())),
        "batch": list(batch),
        "dtype": dtype_name(dtype),
        "args": {name: _plain(value) for name, value in sorted(args.items())},
        "present": sorted(present),
    }


def config_id(config: Mapping[str, Any]) -> str:
    """sha1 of [dims items, batch, 'torch.<dtype>', args items, present], first 12 hex digits."""
    dtype = str(config["dtype"])
    if not dtype.startswith("torch."):
        dtype = "torch." + dtype
    payload = [
        sorted(config["dims"].items()),
        list(config["batch"]),
        dtype,
        sorted(config["args"].items()),
        sorted(config["present"]),
    ]
    return hashlib.sha1(json.dumps(payload, default=str).encode()).hexdigest()[:12]


def device_name(device: torch.device | str | int | None = None) -> str:
    try:
        target = None if device is None else torch.device(device)
    except (TypeError, RuntimeError, ValueError):
        return str(device)
    if torch.cuda.is_available() and (target is None or target.type == "cuda"):
        return torch.cuda.get_device_name(target)
    return platform.processor() or "cpu"


@dataclass(frozen=True)
class Call:
    """One dispatchable call: its config, whether it needs gradients, its device."""

    config: dict
    grad: bool
    device: torch.device
    device_name: str


def call_config(op: Dispatcher, values: Mapping[str, Any], arguments: Mapping[str, Any]) -> Call | None:
    """The call's canonical config, or None when it has no single one (mixed float
    dtypes or devices, inconsistent batch extents)."""
    dims = {name: values[name] for name in op._dims if name in values}
    if set(dims) != set(op._dims):
        return None
    if any(... in spec.tokens for spec in op.specs):
        batch = batch_shape(op.specs, arguments)
        if batch is None:
            return None
    else:
        batch = ()
    dtype = dtype_name(values.get("dtype"))
    if dtype is None:
        if any("float" in d for spec in op.specs for d in spec.dtypes):
            return None
        dtype = "float32"
    devices = {v.device for v in arguments.values() if isinstance(v, torch.Tensor)}
    if len(devices) > 1:
        return None
    device = next(iter(devices), torch.device("cpu"))
    present = (spec.param for spec in op.specs if spec.optional and arguments[spec.param] is not None)
    config = make_config(dims, batch, dtype, {name: arguments[name] for name in op.arg_pools}, present)
    grad = torch.is_grad_enabled() and any(isinstance(v, torch.Tensor) and v.requires_grad for v in arguments.values())
    return Call(config, grad, device, device_name(device))


@dataclass(frozen=True)
class Case:
    """One grid point: dims, batch extent, dtype, scalar args, present optionals."""

    dims: tuple[tuple[str, int], ...]
    batch: tuple[int, ...]
    dtype: torch.dtype
    args: tuple[tuple[str, Any], ...]
    present: frozenset[str] = frozenset()

    def __str__(self) -> str:
        text = [f"{n}={v}" for n, v in self.dims] + [f"batch={self.batch}", dtype_name(self.dtype) or ""]
        text += [f"{n}={v}" for n, v in self.args] + [f"+{n}" for n in sorted(self.present)]
        return ",".join(text)

    def config(self) -> dict[str, Any]:
        return make_config(dict(self.dims), self.batch, self.dtype, dict(self.args), self.present)

    @property
    def case_id(self) -> str:
        return config_id(self.config())

    @classmethod
    def from_config(cls, config: Mapping[str, Any]) -> Case:
        return cls(
            tuple(config["dims"].items()),
            tuple(config["batch"]),
            getattr(torch, config["dtype"]),
            tuple(config["args"].items()),
            frozenset(config["present"]),
        )


@dataclass
class Gauge:
    """Worst error of one output or gradient, the reference's own error (budget) and the truth's scale."""

    err: float = 0.0
    budget: float = 0.0
    scale: float = 1.0

    def note(self, err: float, budget: float, truth: torch.Tensor) -> None:
        self.err = max(self.err, err)
        self.budget = max(self.budget, budget)
        peak = truth.detach().abs().max().item() if truth.numel() else 1.0
        self.scale = max(self.scale, peak)

    def verdict(self, floor: float) -> str | None:
        """None when err <= max(2 * budget, floor * scale) (bench/model.py:66-71), else the reason."""
        if not math.isfinite(self.err):
            return "err is non-finite"
        if self.err <= max(2 * self.budget, floor * self.scale):
            return None
        return f"err {self.err:.3e} > max(2*{self.budget:.3e}, {floor:.0e}*{self.scale:.1f})"


@dataclass
class Result:
    status: str = "pass"  # pass | fail | crash | oom | error | skip
    reason: str = ""
    grad: bool = False
    fwd: dict[str, Gauge] = field(default_factory=dict)
    bwd: dict[str, Gauge] = field(default_factory=dict)
    bench: dict[str, float] = field(default_factory=dict)
    benchmarked: bool = False
    bench_error: str = ""
    reps: int = 0

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


@dataclass(frozen=True)
class Environment:
    device: str
    torch: str
    backend_version: str | None
    ts: str
    ref_hash: str | None = None
    impl_hash: str | None = None


@dataclass
class Record:
    op: str
    impl: str
    case: str
    case_id: str
    config: dict
    environment: Environment
    result: Result

    def to_dict(self) -> dict[str, Any]:
        env = self.environment
        return {
            "schema": SCHEMA,
            "op": self.op,
            "impl": self.impl,
            "case": self.case,
            "case_id": self.case_id,
            "config": self.config,
            "device": env.device,
            "torch": env.torch,
            "backend_version": env.backend_version,
            "ts": env.ts,
            "ref_hash": env.ref_hash,
            "impl_hash": env.impl_hash,
            **self.result.to_dict(),
        }

    @classmethod
    def from_dict(cls, row: Mapping[str, Any]) -> Record:
        if row.get("schema") != SCHEMA:
            raise ValueError(f"unsupported report schema {row.get('schema')!r}; expected {SCHEMA}")
        result = Result(
            status=row["status"],
            reason=row.get("reason", ""),
            grad=row["grad"],
            fwd={k: Gauge(**v) for k, v in (row.get("fwd") or {}).items()},
            bwd={k: Gauge(**v) for k, v in (row.get("bwd") or {}).items()},
            bench=dict(row.get("bench") or {}),
            benchmarked=row.get("benchmarked", bool(row.get("bench"))),
            bench_error=row.get("bench_error", "") or "",
            reps=row.get("reps", 0) or 0,
        )
        env = Environment(row["device"], row["torch"], row.get("backend_version"), row["ts"], row.get("ref_hash"),
                          row.get("impl_hash"))
        return cls(row["op"], row["impl"], row.get("case", ""), row["case_id"], row["config"], env, result)

    @property
    def key(self) -> tuple[Any, ...]:
        """Identity of a row in a store: newer rows with the same key replace older ones."""
        env = self.environment
        return (self.op, self.impl, env.device, self.case_id, self.result.grad, env.torch, env.backend_version)
