"""Backend declarations, version gates and lazy source resolution.

Behaviour follows core/sources.py:40-163:
  * `declare_backend(name, package, min_version, max_version, extra)` records
    which installed distribution a backend needs. An implementation named
    `backend` or `backend:variant` is usable only when
    `importlib.metadata.version(package)` resolves inside [min, max]; an
    undeclared backend is always usable.
  * `resolve("pkg.mod.attr")` imports lazily, preferring attributes over
    same-named submodules and importing submodules not yet loaded.
  * `kernel` is the source bound for the duration of one adapter call:
    calling it calls the source, attribute access reaches into it.
"""

from __future__ import annotations

import importlib
import importlib.metadata
import warnings
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
from types import ModuleType
from typing import Any

from packaging.version import Version

from popcorn_amd.compat.errors import BackendUnavailableError, BackendVersionError


@dataclass
class _Declared:
    package: str
    min_version: str | None
    max_version: str | None
    extra: str | None
    probed: bool = False
    version: str | None = None
    warned: bool = False


_DECLARED: dict[str, _Declared] = {}


def declare_backend(
    name: str, package: str, min_version: str | None = None, max_version: str | None = None, extra: str | None = None
) -> None:
    _DECLARED[name] = _Declared(package, min_version, max_version, extra)


def _lookup(impl: str) -> _Declared | None:
    declared = _DECLARED.get(impl.split(":")[0])
    if declared is not None and not declared.probed:
        try:
            declared.version = importlib.metadata.version(declared.package)
        except importlib.metadata.PackageNotFoundError:
            declared.version = None
        declared.probed = True
    return declared


def _problem(impl: str) -> Exception | None:
    declared = _lookup(impl)
    if declared is None:
        return None
    if declared.version is None:
        hint = f"popcorn[{declared.extra}]" if declared.extra else declared.package
        return BackendUnavailableError(f"implementation {impl!r} needs {declared.package!r}; install {hint}")
    lo, hi = declared.min_version, declared.max_version
    have = Version(declared.version)
    if (lo is not None and have < Version(lo)) or (hi is not None and have > Version(hi)):
        return BackendVersionError(
            f"{declared.package} {declared.version} is outside the supported range [{lo or '*'}, {hi or '*'}] "
            f"required by implementation {impl!r}"
        )
    return None


def unavailable_reason(impl: str) -> str | None:
    problem = _problem(impl)
    return None if problem is None else str(problem)


def available(impl: str) -> bool:
    return _problem(impl) is None


def installed_version(impl: str) -> str | None:
    declared = _lookup(impl)
    return None if declared is None else declared.version


def ensure_available(impl: str) -> None:
    problem = _problem(impl)
    if problem is not None:
        raise problem
    declared = _lookup(impl)
    if declared is not None and declared.min_version is None and declared.max_version is None and not declared.warned:
        declared.warned = True
        warnings.warn(f"implementation {impl!r}: no supported version range declared for {declared.package}")


def resolve(path: str) -> Any:
    parts = path.split(".")
    found: Any = importlib.import_module(parts[0])
    dotted = parts[0]
    for part in parts[1:]:
        dotted += "." + part
        try:
            found = getattr(found, part)
        except (AttributeError, RecursionError):
            if not isinstance(found, ModuleType):
                raise
            found = importlib.import_module(dotted)
    return found


_bound: ContextVar[Callable[..., Any]] = ContextVar("popcorn_amd_kernel")


class _KernelProxy:
    """The source of the implementation currently running (see module docstring)."""

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        try:
            source = _bound.get()
        except LookupError:
            raise RuntimeError("kernel() is only valid inside an implementation registered with source=") from None
        return source(*args, **kwargs)

    def __getattr__(self, name: str) -> Any:
        try:
            source = _bound.get()
        except LookupError:
            raise AttributeError(f"kernel.{name} is only valid inside an implementation registered with source=") from None
        return getattr(source, name)


kernel = _KernelProxy()


@contextmanager
def bound_kernel(source: Callable[..., Any]) -> Iterator[None]:
    token = _bound.set(source)
    try:
        yield
    finally:
        _bound.reset(token)
