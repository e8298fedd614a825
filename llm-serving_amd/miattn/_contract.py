"""Declarative argument checks shared by the drop-in modules.

Each public entry point states its contract as an ordered tuple of :class:`Rule` rows: a
predicate that is true when the arguments break the rule, the exception class the caller
should see, and a message built from the same arguments. :func:`enforce` walks the rows
and raises at the first broken one, so the order of a table is the order in which a
caller learns about mistakes (shape before dtype before device, as the reference's
callers expect).

The exception split follows the reference's convention for this path: a caller bug
(shape, dtype, offsets, indices) is ``ValueError`` / ``IndexError``; a missing capability
(no HIP library, no device, tensors on the wrong kind of device) is ``RuntimeError``.
Messages keep the keywords the reference's tests match on (``"int32"``, ``"capacity"``,
``"head_dim"``, ``"CUDA tensors"``, ``"must start at 0"``, ``"strictly increasing"``,
``"max_seqlen"``, ``"does not match the validated layout"``, ...).
"""

from __future__ import annotations

import operator
from typing import Any, Callable, Iterable, NamedTuple

import torch

__all__ = ["Rule", "enforce", "as_index", "is_pow2", "same_device", "positive_int"]


class Rule(NamedTuple):
    """One contract row: ``broken(args) -> bool``, the exception type, ``message(args)``."""

    broken: Callable[[Any], bool]
    error: type
    message: Callable[[Any], str]


def enforce(rules: Iterable[Rule], args: Any) -> None:
    """Raise the first broken rule's exception; ``args`` is whatever the predicates read."""
    for rule in rules:
        if rule.broken(args):
            raise rule.error(rule.message(args))


def as_index(value, what: str) -> int:
    """An integer-like scalar (int, numpy integer, 0-dim integer tensor) as ``int``."""
    try:
        return operator.index(value)
    except TypeError:
        raise ValueError(f"{what} must be an int, got {type(value).__name__} ({value!r})") from None


def is_pow2(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def same_device(a: torch.device, b: torch.device) -> bool:
    """Device handles that name one device: ``cuda`` (the current one) matches ``cuda:N``."""
    if a.type != b.type:
        return False
    return a.index is None or b.index is None or a.index == b.index


def positive_int(name: str, value) -> int:
    """A plain positive ``int`` (bools rejected), else ``ValueError``."""
    if isinstance(value, bool) or not isinstance(value, int) or value < 1:
        raise ValueError(f"{name} must be a positive int, got {value!r}")
    return value
