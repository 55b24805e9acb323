"""Case configurations and report rows (schema 3).

A case is summarised as a canonical config -- dims, batch extent, dtype,
scalar args and which optional tensors are present -- with a stable 12-hex
`config_id` (core/config.py:38-64). One validation / benchmark outcome is a
`Record` whose dictionary form is Popcorn's report-row schema 3
(bench/model.py:105-163). The config layout, the id's hash payload and the row
keys are a format shared with Popcorn: rows written here and rows Popcorn
writes name the same cases and load into each other's report files. Popcorn's
selector still drops every row whose `ref_hash` / `impl_hash` differ from the
fingerprints it computes itself (core/tuning.py:93-94, 127-128;
core/fingerprint.py:163-202), and those of rows recorded here are this
package's own, so such rows cannot steer upstream selection: rows meant for
Popcorn's selector must be recorded by Popcorn itself.
"""

from __future__ import annotations

import hashlib
import json
import math
import platform
from collections.abc import Iterable, Mapping
from dataclasses import asdict, dataclass, field
from typing import Any

import torch

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

    def allowance(self, floor: float) -> float:
        """The largest error that passes: twice the reference's own error, or the dtype floor at the truth's scale."""
        return max(2 * self.budget, floor * self.scale)

    def verdict(self, floor: float) -> str | None:
        """None when the worst error is within `allowance(floor)` (bench/model.py:66-71), else why not."""
        if math.isnan(self.err) or math.isinf(self.err):
            return "error is not finite"
        limit = self.allowance(floor)
        if self.err > limit:
            return (f"error {self.err:.3e} above {limit:.3e} (2 x budget {self.budget:.3e}, "
                    f"floor {floor:.0e} x scale {self.scale:.1f})")
        return None


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
        """Rebuild a record from its row; rows of any other schema are refused."""
        schema = row.get("schema")
        if schema != SCHEMA:
            raise ValueError(f"report row has schema {schema!r}; this reader takes schema {SCHEMA} only")
        gauges = {side: {name: Gauge(**fields) for name, fields in (row.get(side) or {}).items()}
                  for side in ("fwd", "bwd")}
        bench = dict(row.get("bench") or {})
        result = Result(
            status=row["status"],
            reason=row.get("reason") or "",
            grad=bool(row["grad"]),
            fwd=gauges["fwd"],
            bwd=gauges["bwd"],
            bench=bench,
            # rows written before the flag existed count as benchmarked when they carry timings
            benchmarked=bool(row["benchmarked"]) if row.get("benchmarked") is not None else bool(bench),
            bench_error=row.get("bench_error") or "",
            reps=int(row.get("reps") or 0),
        )
        environment = Environment(
            device=row["device"], torch=row["torch"], backend_version=row.get("backend_version"), ts=row["ts"],
            ref_hash=row.get("ref_hash"), impl_hash=row.get("impl_hash"),
        )
        return cls(row["op"], row["impl"], row.get("case") or "", row["case_id"], row["config"], environment, result)

    @property
    def key(self) -> tuple[Any, ...]:
        """Identity of a row in a store: newer rows with the same key replace older ones."""
        env = self.environment
        return (self.op, self.impl, env.device, self.case_id, self.result.grad, env.torch, env.backend_version)
