"""Backend declarations, the version gate, and the `kernel` seen by adapters.

An implementation is named after the backend that provides it, optionally
with a variant after a colon (`mi355x`, `fla:chunk`); everything here takes an
implementation name and looks up the backend part. A backend declared with
`declare_backend` is tied to one installed distribution and an optional
version range (Popcorn's gate, core/sources.py:40-104): while that
distribution is missing or outside the range, the backend's implementations
are ineligible for automatic dispatch and raise when forced. A backend that
was never declared has no gate.

The installed version is read from the distribution metadata once per
declaration and kept, since dispatch asks on every call.

`resolve` turns a `source=` dotted path into the object it names, and
`kernel` is the stand-in an adapter calls: while an implementation with a
source runs, `kernel(...)` calls that source and `kernel.name` reaches its
attributes (core/sources.py:106-163 describe the same contract).
"""

from __future__ import annotations

import importlib
import importlib.metadata
import warnings
from collections.abc import Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
from types import ModuleType
from typing import Any

from packaging.version import Version

from popcorn_amd.compat.errors import BackendUnavailableError, BackendVersionError, PopcornError

_UNPROBED = object()


@dataclass
class Declaration:
    """One declared backend: the distribution serving it and the versions it supports."""

    distribution: str
    lowest: str | None = None
    highest: str | None = None
    extra: str | None = None
    probed: Any = _UNPROBED  # installed version string, None when not installed
    warned_unpinned: bool = False

    def version(self) -> str | None:
        if self.probed is _UNPROBED:
            try:
                self.probed = importlib.metadata.version(self.distribution)
            except importlib.metadata.PackageNotFoundError:
                self.probed = None
        return self.probed

    def problem(self, impl: str) -> PopcornError | None:
        """The error a forced call of `impl` raises, or None when the backend is usable."""
        installed = self.version()
        if installed is None:
            hint = f"popcorn[{self.extra}]" if self.extra else self.distribution
            return BackendUnavailableError(
                f"implementation {impl!r} is served by distribution {self.distribution!r}, which is not "
                f"installed (install {hint})"
            )
        too_old = self.lowest is not None and Version(installed) < Version(self.lowest)
        too_new = self.highest is not None and Version(installed) > Version(self.highest)
        if too_old or too_new:
            return BackendVersionError(
                f"implementation {impl!r} supports {self.distribution} in [{self.lowest or '*'}, "
                f"{self.highest or '*'}], but {installed} is installed"
            )
        return None


_DECLARED: dict[str, Declaration] = {}


def _declaration(impl: str) -> Declaration | None:
    return _DECLARED.get(impl.partition(":")[0])


def declare_backend(
    name: str,
    package: str,
    min_version: str | None = None,
    max_version: str | None = None,
    extra: str | None = None,
) -> None:
    """Tie backend `name` to distribution `package` within [min_version, max_version]."""
    _DECLARED[name] = Declaration(package, min_version, max_version, extra)


def unavailable_reason(impl: str) -> str | None:
    """Why `impl` cannot run here, or None when its backend is usable (or undeclared)."""
    declared = _declaration(impl)
    problem = declared.problem(impl) if declared else None
    return None if problem is None else str(problem)


def installed_version(impl: str) -> str | None:
    """Installed version of the distribution behind `impl`'s backend (None when undeclared or absent)."""
    declared = _declaration(impl)
    return declared.version() if declared else None


def ensure_available(impl: str) -> None:
    """Raise the gate's error for `impl`; warn once for a backend declared without a version range."""
    declared = _declaration(impl)
    if declared is None:
        return
    problem = declared.problem(impl)
    if problem is not None:
        raise problem
    if declared.lowest is None and declared.highest is None and not declared.warned_unpinned:
        declared.warned_unpinned = True
        warnings.warn(f"implementation {impl!r}: {declared.distribution} is declared without a supported version range")


def resolve(path: str) -> Any:
    """The object a dotted path names.

    Each segment is taken as an attribute of what the segments before it named;
    only a segment the object lacks is imported as a submodule. So a package
    that re-exports a function under the name of one of its submodules yields
    the function, and `pkg.mod.Class.method` reaches the method.
    """
    parts = path.split(".")
    found: Any = importlib.import_module(parts[0])
    for depth in range(1, len(parts)):
        name = parts[depth]
        try:
            found = getattr(found, name)
            continue
        except AttributeError:
            if not isinstance(found, ModuleType):
                raise
        # a submodule that is not imported yet; an import error inside it propagates
        found = importlib.import_module(".".join(parts[: depth + 1]))
    return found


_SERVING: ContextVar[Any] = ContextVar("popcorn_amd.compat.kernel")


class _KernelProxy:
    """The resolved source of the implementation now running.

    Outside such a call, calling it is a RuntimeError and attribute access an
    AttributeError, so `hasattr(kernel, ...)` probes read as a plain miss.
    """

    @staticmethod
    def _source(what: str, error: type[Exception]) -> Any:
        try:
            return _SERVING.get()
        except LookupError:
            raise error(f"{what} is only valid inside an implementation registered with source=") from None

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        return self._source("kernel(...)", RuntimeError)(*args, **kwargs)

    def __getattr__(self, name: str) -> Any:
        if name.startswith("__") and name.endswith("__"):
            raise AttributeError(name)
        return getattr(self._source(f"kernel.{name}", AttributeError), name)


kernel = _KernelProxy()


@contextmanager
def serving(source: Any) -> Iterator[None]:
    """Bind `kernel` to `source` for the duration of the block (per context, so per thread)."""
    token = _SERVING.set(source)
    try:
        yield
    finally:
        _SERVING.reset(token)
