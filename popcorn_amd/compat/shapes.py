"""Tensor annotations, the shape grammar read from them, and annotation gates.

Popcorn annotates each reference parameter with a jaxtyping type such as
`Float[Tensor, "... hidden"]` (core/annotations.py:89-218) and uses plain
typing (`Literal`, unions, `None`) for adapter gates (core/typecheck.py:22-64).
jaxtyping is not part of this environment, so this module carries a small
annotation vocabulary of its own with the same spelling -- `Float`, `Float16`,
`BFloat16`, `Float32`, `Float64`, each subscripted as `[Tensor, "dims"]` --
and the three operations dispatch needs from it:

  * `plans(signature)`: the tensor parameters, their dim tokens, dtypes and
    whether they are optional;
  * `extract(specs, arguments)`: bind every dim name to one size across all
    tensors (a mismatch is a DispatchError naming the dim);
  * `satisfies(value, annotation)` / `narrower(sub, sup)`: the gate checks,
    over annotations flattened into their alternatives.

Dim tokens are names, integer literals or `...` (the batch extent). Derived
dims (`seq+1`) are not needed by the four transformer-block ops and are not
supported.
"""

from __future__ import annotations

import inspect
import types
import typing
from collections.abc import Mapping
from dataclasses import dataclass
from typing import Any

import torch

from popcorn_amd.compat.errors import DispatchError

_UNIONS = (typing.Union, types.UnionType)


@dataclass(frozen=True)
class TensorType:
    """A tensor annotation: accepted dtypes (names without `torch.`) and a dim string."""

    family: str
    dtypes: tuple[str, ...]
    dim_str: str

    def __repr__(self) -> str:
        return f'{self.family}[Tensor, "{self.dim_str}"]'

    def __instancecheck__(self, value: Any) -> bool:  # isinstance(t, Float[Tensor, "..."])
        return isinstance(value, torch.Tensor) and str(value.dtype).removeprefix("torch.") in self.dtypes

    # typing.Union accepts only types and callables as members
    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        raise TypeError(f"{self!r} is an annotation, not a constructor")

    def __or__(self, other: Any) -> Any:
        return typing.Union[self, other]

    def __ror__(self, other: Any) -> Any:
        return typing.Union[other, self]


class _Family:
    def __init__(self, name: str, dtypes: tuple[str, ...]) -> None:
        self.name, self.dtypes = name, dtypes

    def __getitem__(self, item: tuple[Any, str]) -> TensorType:
        kind, dims = item
        if kind is not torch.Tensor:
            raise TypeError(f"{self.name}[...] annotates torch.Tensor, got {kind!r}")
        return TensorType(self.name, self.dtypes, " ".join(dims.split()))


Float = _Family("Float", ("bfloat16", "float16", "float32", "float64"))
Float16 = _Family("Float16", ("float16",))
BFloat16 = _Family("BFloat16", ("bfloat16",))
Float32 = _Family("Float32", ("float32",))
Float64 = _Family("Float64", ("float64",))
Int32 = _Family("Int32", ("int32",))

Token = typing.Union[str, int, "types.EllipsisType"]


@dataclass(frozen=True)
class TensorSpec:
    """One tensor parameter of a reference: dim tokens, dtypes, optionality."""

    param: str
    tokens: tuple[Any, ...]
    dtypes: tuple[str, ...]
    optional: bool


def _split_optional(annotation: Any) -> tuple[Any, bool]:
    if typing.get_origin(annotation) in _UNIONS:
        members = [m for m in typing.get_args(annotation) if m is not type(None)]
        if len(members) == 1 and len(typing.get_args(annotation)) == 2:
            return members[0], True
    return annotation, False


def _tokens(dim_str: str, param: str) -> tuple[Any, ...]:
    out: list[Any] = []
    for text in dim_str.split():
        if text == "...":
            out.append(...)
        elif text.isdigit():
            out.append(int(text))
        elif text.isidentifier():
            out.append(text)
        else:
            raise TypeError(f"{param}: unsupported dim token {text!r}")
    if out.count(...) > 1:
        raise TypeError(f"{param}: more than one '...'")
    return tuple(out)


def plans(signature: inspect.Signature) -> tuple[TensorSpec, ...]:
    specs = []
    for name, param in signature.parameters.items():
        annotation, optional = _split_optional(param.annotation)
        if isinstance(annotation, TensorType):
            specs.append(TensorSpec(name, _tokens(annotation.dim_str, name), annotation.dtypes, optional))
    return tuple(specs)


def dim_names(specs: tuple[TensorSpec, ...]) -> frozenset[str]:
    return frozenset(t for spec in specs for t in spec.tokens if isinstance(t, str))


def _axes(spec: TensorSpec, shape: tuple[int, ...]) -> tuple[dict[str, int], tuple[int, ...]] | None:
    """(named sizes, batch extent) of one tensor, or None when its rank cannot fit."""
    fixed = [t for t in spec.tokens if t is not ...]
    if ... in spec.tokens:
        if len(shape) < len(fixed):
            return None
        cut = spec.tokens.index(...)
        tail = len(spec.tokens) - cut - 1
        head, batch, rest = shape[:cut], shape[cut : len(shape) - tail], shape[len(shape) - tail :]
        sizes = list(head) + list(rest)
    else:
        if len(shape) != len(fixed):
            return None
        batch, sizes = (), list(shape)
    named: dict[str, int] = {}
    for token, size in zip(fixed, sizes):
        if isinstance(token, int):
            if token != size:
                return None
        else:
            named[token] = size
    return named, tuple(batch)


def extract(specs: tuple[TensorSpec, ...], arguments: Mapping[str, Any]) -> dict[str, int]:
    """Bind every dim name to its size; raise DispatchError on a rank or size conflict."""
    dims: dict[str, int] = {}
    for spec in specs:
        value = arguments.get(spec.param)
        if value is None:
            if spec.optional:
                continue
            raise DispatchError(f"{spec.param}: required tensor is None")
        if not isinstance(value, torch.Tensor):
            raise DispatchError(f"{spec.param}: expected a tensor, got {type(value).__name__}")
        bound = _axes(spec, tuple(value.shape))
        if bound is None:
            raise DispatchError(f"{spec.param}: shape {tuple(value.shape)} does not fit '{' '.join(map(str, spec.tokens))}'")
        for name, size in bound[0].items():
            if dims.setdefault(name, size) != size:
                raise DispatchError(f"dim '{name}': {spec.param} has {size}, another argument has {dims[name]}")
    return dims


def batch_shape(specs: tuple[TensorSpec, ...], arguments: Mapping[str, Any]) -> tuple[int, ...] | None:
    """The common `...` extent of every tensor that has one; None when they disagree."""
    seen: set[tuple[int, ...]] = set()
    for spec in specs:
        value = arguments.get(spec.param)
        if ... in spec.tokens and isinstance(value, torch.Tensor):
            bound = _axes(spec, tuple(value.shape))
            if bound is None:
                return None
            seen.add(bound[1])
    if len(seen) > 1:
        return None
    return next(iter(seen), ())


@dataclass(frozen=True)
class _Exactly:
    """One value of a `Literal[...]` annotation."""

    value: Any


def _alternatives(annotation: Any) -> tuple[Any, ...]:
    """An annotation flattened into the alternatives a value may satisfy.

    Unions (and `X | None`) contribute each member, `Literal[a, b]` one
    `_Exactly` per value, `None` the class of None, and an absent annotation or
    `Any` the single alternative `Any`. Anything else stands for itself.
    """
    if annotation is None:
        return (type(None),)
    if annotation is inspect.Parameter.empty or annotation is typing.Any:
        return (typing.Any,)
    origin = typing.get_origin(annotation)
    if origin in _UNIONS:
        return tuple(alt for member in typing.get_args(annotation) for alt in _alternatives(member))
    if origin is typing.Literal:
        return tuple(_Exactly(value) for value in typing.get_args(annotation))
    return (annotation,)


def _admits(alternative: Any, value: Any) -> bool:
    if alternative is typing.Any:
        return True
    if isinstance(alternative, _Exactly):
        # True == 1 but a bool literal admits only bools: compare the type as well
        return value is alternative.value or (type(value) is type(alternative.value) and value == alternative.value)
    if isinstance(alternative, TensorType):
        return isinstance(value, torch.Tensor) and str(value.dtype).removeprefix("torch.") in alternative.dtypes
    if isinstance(alternative, type):
        try:
            return isinstance(value, alternative)
        except TypeError:  # parametrised generics: not modelled, so no constraint
            return True
    return True  # an annotation this vocabulary does not model constrains nothing


def satisfies(value: Any, annotation: Any) -> bool:
    """Does `value` meet `annotation` (a Literal, union, None, class or tensor type)?"""
    return any(_admits(alternative, value) for alternative in _alternatives(annotation))


def _inside(alternative: Any, wider: tuple[Any, ...]) -> bool:
    """Is every value `alternative` admits also admitted by one of `wider`?"""
    if typing.Any in wider:
        return True
    if isinstance(alternative, _Exactly):
        return any(_admits(w, alternative.value) for w in wider)
    if isinstance(alternative, TensorType):
        return any(isinstance(w, TensorType) and w.dim_str == alternative.dim_str
                   and set(alternative.dtypes) <= set(w.dtypes) for w in wider)
    if isinstance(alternative, type):
        for w in wider:
            if isinstance(w, type):
                try:
                    if issubclass(alternative, w):
                        return True
                except TypeError:
                    pass
        return False
    return alternative in wider


def narrower(sub: Any, sup: Any) -> bool:
    """Does annotation `sub` admit only values that `sup` admits?

    An adapter may narrow a reference annotation (`Literal[True]` for `bool`,
    `BFloat16[...]` for `Float[...]`); the narrowed form becomes a dispatch
    gate. Tensor types narrow when their dims agree and their dtypes are a
    subset.
    """
    if sub == sup:
        return True
    wider = _alternatives(sup)
    return all(_inside(alternative, wider) for alternative in _alternatives(sub))


def fmt_value(value: Any) -> str:
    if isinstance(value, torch.Tensor):
        return f"Tensor[{tuple(value.shape)}, {str(value.dtype).removeprefix('torch.')}]"
    return repr(value)
