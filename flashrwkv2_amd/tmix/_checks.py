"""Declarative argument checks shared by the public ``tmix`` wrappers.

A wrapper describes its arguments as rows ``(name, value, rules)``; each rule
is a predicate with the exception class and message it raises.  ``verify``
walks the rows in order and stops at the first rule that fails, so the order
of the rows is the order in which callers see errors.  The messages are the
operator contract (callers and tests match on them), so they are passed in
verbatim by each wrapper; the ``{name}`` field is filled with the row name.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from numbers import Real
from typing import Any, Callable, Iterable, Sequence

import torch


@dataclass(frozen=True)
class Rule:
    ok: Callable[[Any], bool]
    error: type
    message: str


Row = tuple[str, Any, Sequence[Rule]]


def verify(rows: Iterable[Row]) -> None:
    """Raise the first failing rule's error, rows and rules in order."""
    for name, value, rules in rows:
        for rule in rules:
            if not rule.ok(value):
                raise rule.error(rule.message.format(name=name))


def each(names: Sequence[str], values: Sequence[Any], rules: Sequence[Rule]) -> list[Row]:
    """The same rules for several named values."""
    return [(n, v, rules) for n, v in zip(names, values)]


# ---- rules -----------------------------------------------------------------

def is_tensor(message: str = "{name} must be a torch.Tensor") -> Rule:
    return Rule(lambda t: isinstance(t, torch.Tensor), TypeError, message)


def dtype_in(dtypes: Iterable[torch.dtype], message: str, error: type = TypeError) -> Rule:
    allowed = frozenset(dtypes)
    return Rule(lambda t: t.dtype in allowed, error, message)


def cuda_contiguous(message: str = "{name} must be contiguous CUDA",
                    error: type = ValueError) -> Rule:
    return Rule(lambda t: t.is_cuda and t.is_contiguous(), error, message)


def cuda_contiguous_of(dtype: torch.dtype, message: str, error: type = ValueError) -> Rule:
    """dtype, device kind and layout in one rule (one message for all three)."""
    return Rule(lambda t: t.dtype == dtype and t.is_cuda and t.is_contiguous(), error, message)


def matches(ref: torch.Tensor, message: str, *, shape: bool = True, device: bool = True,
            error: type = ValueError) -> Rule:
    def ok(t: torch.Tensor) -> bool:
        return (not shape or t.shape == ref.shape) and (not device or t.device == ref.device)

    return Rule(ok, error, message)


def on_device_of(ref: torch.Tensor, message: str, error: type = ValueError) -> Rule:
    return matches(ref, message, shape=False, error=error)


def shape_is(shapes: Iterable[tuple[int, ...]], message: str, error: type = ValueError) -> Rule:
    allowed = {tuple(s) for s in shapes}
    return Rule(lambda t: tuple(t.shape) in allowed, error, message)


def holds(predicate: Callable[[Any], bool], message: str, error: type = ValueError) -> Rule:
    return Rule(predicate, error, message)


def optional(rules: Sequence[Rule]) -> list[Rule]:
    """Rules that apply only when the value is not None."""
    return [Rule(lambda t, r=r: t is None or r.ok(t), r.error, r.message) for r in rules]


# ---- scalar helpers ----------------------------------------------------------

def is_int(value: Any) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def positive_int(value: Any) -> bool:
    return is_int(value) and value > 0


def finite(value: Any) -> bool:
    try:
        return math.isfinite(float(value))
    except (TypeError, ValueError):
        return False


def real_number(value: Any) -> bool:
    return isinstance(value, Real) and not isinstance(value, bool)


__all__ = [
    "Rule", "verify", "each", "is_tensor", "dtype_in", "cuda_contiguous", "cuda_contiguous_of",
    "matches", "on_device_of", "shape_is", "holds", "optional", "is_int", "positive_int",
    "finite", "real_number",
]
