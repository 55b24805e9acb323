"""Ops, registered implementations and call-time selection.

Behaviour follows core/dispatcher.py:55-481:
  * an op (`Dispatcher`) wraps its torch reference and is called like it;
    the keyword-only controls `backend=`, `bench=`, `validate=`, `unsafe=`
    are added to its signature;
  * `op.register(name, source=None, predicate=None, forward_only=False)`
    returns a decorator taking an optional adapter; implementations are kept
    in registration order with the torch reference last; a duplicate or a
    malformed name raises;
  * an adapter must declare exactly the reference's parameters, in order and
    without defaults; annotations that narrow the reference's become gates;
    a bare `source=` must itself start with the reference's parameter names;
  * a call is forced by `backend=`, by calling `op["name"]`, or inside
    `with op["name"]:` (a per-context scope); otherwise every implementation
    that does not reject the call (backend unavailable, gradients needed by
    a forward-only implementation, a failed gate, a predicate veto) is a
    candidate and the tuner picks one from recorded evidence;
  * an exception raised by the chosen implementation propagates: there is no
    fallback to another implementation.
"""

from __future__ import annotations

import inspect
import re
import typing
from collections.abc import Callable, Mapping
from contextvars import ContextVar, Token
from functools import cached_property
from typing import Any

import torch

from popcorn_amd.compat import shapes
from popcorn_amd.compat.errors import DispatchError
from popcorn_amd.compat.fingerprint import fingerprint
from popcorn_amd.compat.harness import BenchmarkService, validation_mode
from popcorn_amd.compat.records import Record, call_config
from popcorn_amd.compat.selection import Tuner
from popcorn_amd.compat.sources import bound_kernel, ensure_available, resolve, unavailable_reason

KERNELS: dict[str, Dispatcher] = {}

_NAME = re.compile(r"^[a-z0-9][a-z0-9_-]*(:[a-z0-9][a-z0-9_-]*)?$")


def _contextual(transform: Callable[..., Any]) -> bool:
    """Does a test-input transform take (tensor, dims, generator) rather than (tensor)?"""
    try:
        sig = inspect.signature(transform)
    except (TypeError, ValueError):
        return False
    try:
        sig.bind(None)
        return False
    except TypeError:
        try:
            sig.bind(None, {}, None)
            return True
        except TypeError:
            raise TypeError(f"test input transform {transform!r} must accept one or three positional arguments") from None


def _signature(fn: Callable[..., Any]) -> inspect.Signature:
    """The signature with string annotations (postponed evaluation) resolved."""
    try:
        return inspect.signature(fn, eval_str=True)
    except (NameError, TypeError, SyntaxError):
        return inspect.signature(fn)


class Implementation:
    """One implementation of an op: a lazily resolved `source`, an adapter, or both."""

    def __init__(self, op: Dispatcher, name: str, adapter: Callable[..., Any] | None = None,
                 source: str | None = None, predicate: Callable[..., bool] | None = None,
                 forward_only: bool = False) -> None:
        if not _NAME.match(name):
            raise ValueError(f"invalid backend name {name!r}")
        self.op, self.name, self.adapter, self.source = op, name, adapter, source
        self.predicate, self.forward_only = predicate, forward_only
        self.gates: dict[str, Any] = {}
        self.source_fn: Callable[..., Any] | None = None
        self._ready = False

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        return self.op(*args, backend=self.name, **kwargs)

    def __enter__(self) -> Dispatcher:
        stack = self.op._scope_stack
        stack.set((*stack.get(), self.op._scoped.set(self.name)))
        return self.op

    def __exit__(self, *exc: object) -> None:
        *rest, token = self.op._scope_stack.get()
        self.op._scoped.reset(token)
        self.op._scope_stack.set(tuple(rest))

    def __str__(self) -> str:
        return f"{self.op.name}:{self.name}"

    def __repr__(self) -> str:
        return f"<{self}" + "".join(f" {n}" for n in self.notes()) + ">"

    def notes(self) -> list[str]:
        return (["fwd-only"] if self.forward_only else []) + ([f"gates={self.gates}"] if self.gates else [])

    @cached_property
    def fingerprint(self) -> str | None:
        parts = [p for p in (self.adapter, self.predicate) if p is not None]
        return fingerprint(*parts, source=self.source)

    def rejects(self, values: Mapping[str, Any], arguments: Mapping[str, Any]) -> str | None:
        if reason := unavailable_reason(self.name):
            return reason
        if self.forward_only and self.op._needs_grad(arguments):
            return "no backward implementation"
        for name, annotation in self.gates.items():
            if not shapes.matches(arguments[name], annotation):
                return f"{name}={shapes.fmt_value(arguments[name])} does not satisfy {annotation}"
        if self.predicate is not None and not self.predicate(**arguments):
            return f"rejected by {getattr(self.predicate, '__name__', 'predicate')}"
        return None

    def attach(self, adapter: Callable[..., Any]) -> None:
        params = list(_signature(adapter).parameters.values())
        names = tuple(p.name for p in params)
        if names != self.op._params:
            raise TypeError(f"{self}: parameters must be exactly {list(self.op._params)}, got {list(names)}")
        if defaulted := [p.name for p in params if p.default is not inspect.Parameter.empty]:
            raise TypeError(f"{self}: parameters must not declare defaults (the reference owns them): {defaulted}")
        gates = {}
        for p in params:
            ref = self.op._signature.parameters[p.name].annotation
            if p.annotation is inspect.Parameter.empty or p.annotation == ref:
                continue
            if not shapes.narrows(p.annotation, ref):
                raise TypeError(f"{self}: {p.name}: {p.annotation} does not narrow {ref}")
            gates[p.name] = p.annotation
        self.gates, self.adapter = gates, adapter

    def invoke(self, arguments: Mapping[str, Any]) -> Any:
        self._prepare()
        args = tuple(arguments[p] for p in self.op._params)
        if self.adapter is None:
            return self.source_fn(*args)
        if self.source_fn is not None:
            with bound_kernel(self.source_fn):
                return self.adapter(*args)
        return self.adapter(*args)

    def _prepare(self) -> None:
        if self._ready:
            return
        if self.adapter is None and self.source is None:
            raise DispatchError(f"{self}: registration has neither adapter nor source")
        ensure_available(self.name)
        if self.source is not None:
            self.source_fn = resolve(self.source)
            if self.adapter is None:
                self._conform(self.source_fn)
        self._ready = True

    def _conform(self, fn: Callable[..., Any]) -> None:
        try:
            params = list(inspect.signature(fn).parameters.values())
        except (TypeError, ValueError):
            return
        if {p.kind for p in params} & {inspect.Parameter.VAR_POSITIONAL, inspect.Parameter.VAR_KEYWORD}:
            return
        head = tuple(p.name for p in params[: len(self.op._params)])
        extra = params[len(self.op._params):]
        if head != self.op._params or any(p.default is inspect.Parameter.empty for p in extra):
            raise TypeError(f"{self}: source signature {list(head)} does not match reference "
                            f"{list(self.op._params)}; register an adapter")


class Dispatcher:
    """An op: its torch reference plus registered implementations, called like the reference."""

    def __init__(self, reference: Callable[..., Any], test_args: Mapping[str, Any] | None = None,
                 test_inputs: Mapping[str, Callable[..., Any]] | None = None, name: str | None = None,
                 tags: Any = None) -> None:
        self.reference = reference
        self.name = name or reference.__name__
        self.__name__ = self.name
        self.__doc__ = reference.__doc__
        self._signature = _signature(reference)
        self._params = tuple(self._signature.parameters)
        controls = [inspect.Parameter(n, inspect.Parameter.KEYWORD_ONLY, default=None, annotation=a)
                    for n, a in (("backend", str), ("bench", bool), ("validate", bool), ("unsafe", bool))]
        self.__signature__ = self._signature.replace(parameters=[*self._signature.parameters.values(), *controls])
        self.specs = shapes.plans(self._signature)
        self._dims = shapes.dim_names(self.specs)
        self.arg_pools = self._pools(dict(test_args or {}))
        self.test_inputs = dict(test_inputs or {})
        tensor_params = {s.param for s in self.specs}
        if unknown := set(self.test_inputs) - tensor_params:
            raise TypeError(f"{self.name}: unknown test_inputs keys {sorted(unknown)}; allowed: {sorted(tensor_params)}")
        if bad := [n for n, f in self.test_inputs.items() if not callable(f)]:
            raise TypeError(f"{self.name}: test_inputs values must be callable: {bad}")
        self._contextual_inputs = frozenset(n for n, f in self.test_inputs.items() if _contextual(f))
        self.tags = frozenset(tags or ())
        self._impls: list[Implementation] = [Implementation(self, "torch", adapter=reference)]
        self.bench = BenchmarkService(self)
        self.tuner = Tuner(self, self.bench.store)
        self._scoped: ContextVar[str | None] = ContextVar(f"popcorn_amd.{self.name}", default=None)
        self._scope_stack: ContextVar[tuple[Token, ...]] = ContextVar(f"popcorn_amd.{self.name}.stack", default=())

    @cached_property
    def fingerprint(self) -> str | None:
        return fingerprint(self.reference)

    def __call__(self, *args: Any, backend: str | None = None, bench: bool | None = None,
                 validate: bool | None = None, unsafe: bool | None = None, **kwargs: Any) -> Any:
        arguments = self._bind(*args, **kwargs)
        values = self._values(arguments)
        forced = backend or self._scoped.get()
        candidates = self._eligible(values, arguments, forced)
        call = call_config(self, values, arguments)
        if validation_mode(bench, validate) == "bench":
            if call is None:
                raise DispatchError(f"{self.name}: this call cannot be represented as a validation case")
            names = [c.name for c in candidates if c.name != "torch"]
            if self.bench.ensure(call, arguments, names, benchmark=True):
                self.tuner.forget()
        policy = self.tuner.policy.bind(unsafe)
        chosen = self.tuner.select(call, candidates, forced, self._signature_key(arguments), policy)
        return chosen.invoke(arguments)

    def validate(self, *args: Any, backend: str | None = None, **kwargs: Any) -> list[Record]:
        return self._assess(args, kwargs, backend, benchmark=False)

    def benchmark(self, *args: Any, backend: str | None = None, **kwargs: Any) -> list[Record]:
        return self._assess(args, kwargs, backend, benchmark=True)

    def __getitem__(self, name: str) -> Implementation:
        for impl in self._impls:
            if impl.name == name:
                ensure_available(name)
                return impl
        raise DispatchError(f"{self.name}: unknown backend {name!r}; available: {', '.join(self.available_backends())}")

    def register(self, name: str, source: str | None = None, predicate: Callable[..., bool] | None = None,
                 forward_only: bool = False) -> Callable[[Callable[..., Any]], Callable[..., Any]]:
        if any(i.name == name for i in self._impls):
            raise ValueError(f"{self.name}: backend {name!r} already registered")
        impl = Implementation(self, name, source=source, predicate=predicate, forward_only=forward_only)
        self._impls.insert(len(self._impls) - 1, impl)
        self.tuner.forget()

        def attach(fn: Callable[..., Any]) -> Callable[..., Any]:
            try:
                impl.attach(fn)
            except Exception:
                self._impls.remove(impl)
                raise
            return fn

        return attach

    def available_backends(self) -> tuple[str, ...]:
        return tuple(i.name for i in self._impls)

    def __repr__(self) -> str:
        lines = [f"{self.name}{self._signature}"]
        lines += [f"  {i.name}" + "".join(f"  {n}" for n in i.notes()) for i in self._impls]
        return "\n".join(lines)

    def _pools(self, test_args: dict[str, Any]) -> dict[str, list[Any] | None]:
        tensors = {s.param for s in self.specs}
        if unknown := set(test_args) - (set(self._params) - tensors):
            raise TypeError(f"{self.name}: test_args keys {sorted(unknown)} are not scalar arguments")
        pools: dict[str, list[Any] | None] = {}
        for name, param in self._signature.parameters.items():
            if name in tensors:
                continue
            if name in test_args:
                pool = list(test_args[name])
                for value in pool:
                    if not shapes.matches(value, param.annotation):
                        raise TypeError(f"{self.name}: test_args[{name!r}] value {value!r} does not satisfy "
                                        f"{param.annotation}")
            elif typing.get_origin(param.annotation) is typing.Literal:
                pool = list(typing.get_args(param.annotation))
            elif param.annotation is bool or isinstance(param.default, bool):
                pool = [False, True]
            elif param.default is not inspect.Parameter.empty:
                pool = [param.default]
            else:
                pools[name] = None
                continue
            if param.default in pool:
                pool.remove(param.default)
                pool.insert(0, param.default)
            pools[name] = pool
        return pools

    def _values(self, arguments: Mapping[str, Any]) -> dict[str, Any]:
        values: dict[str, Any] = shapes.extract(self.specs, arguments)
        floating = {v.dtype for v in arguments.values() if isinstance(v, torch.Tensor) and v.is_floating_point()}
        if len(floating) == 1:
            values["dtype"] = floating.pop()
        return values

    def _bind(self, *args: Any, **kwargs: Any) -> dict[str, Any]:
        bound = self._signature.bind(*args, **kwargs)
        bound.apply_defaults()
        return dict(bound.arguments)

    def _eligible(self, values: Mapping[str, Any], arguments: Mapping[str, Any],
                  forced: str | None = None) -> list[Implementation]:
        if forced is not None:
            impl = self[forced]
            if why := impl.rejects(values, arguments):
                raise DispatchError(f"{self.name}: backend {forced!r} rejected call: {why}")
            return [impl]
        return [i for i in self._impls if i.rejects(values, arguments) is None]

    def _assess(self, args: tuple[Any, ...], kwargs: dict[str, Any], backend: str | None, *,
                benchmark: bool) -> list[Record]:
        arguments = self._bind(*args, **kwargs)
        values = self._values(arguments)
        candidates = self._eligible(values, arguments, backend)
        call = call_config(self, values, arguments)
        if call is None:
            raise DispatchError(f"{self.name}: this call cannot be represented as a validation case")
        records = self.bench.force(call, arguments, [c.name for c in candidates], benchmark=benchmark)
        self.tuner.forget()
        return records

    @staticmethod
    def _signature_key(arguments: Mapping[str, Any]) -> tuple[Any, ...]:
        def key(v: Any) -> Any:
            if isinstance(v, torch.Tensor):
                return (tuple(v.shape), str(v.dtype), str(v.device), v.requires_grad)
            return v

        return torch.is_grad_enabled(), tuple((n, key(v)) for n, v in arguments.items())

    @staticmethod
    def _needs_grad(arguments: Mapping[str, Any]) -> bool:
        return torch.is_grad_enabled() and any(isinstance(v, torch.Tensor) and v.requires_grad
                                               for v in arguments.values())


def register_kernel(fn: Callable[..., Any] | None = None, *, test_args: Mapping[str, Any] | None = None,
                    test_inputs: Mapping[str, Callable[..., Any]] | None = None, name: str | None = None,
                    tags: Any = None) -> Any:
    """Make a reference an op and enter it in KERNELS (usable bare or with keywords)."""

    def wrap(reference: Callable[..., Any]) -> Dispatcher:
        op = Dispatcher(reference, test_args=test_args, test_inputs=test_inputs, name=name, tags=tags)
        if op.name in KERNELS:
            raise ValueError(f"kernel {op.name!r} already registered")
        KERNELS[op.name] = op
        return op

    return wrap(fn) if fn is not None else wrap
