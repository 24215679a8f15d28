"""Tunables: the one object a kernel gives the compiler to optimize over.

    @tilejax_amd.tunable
    class MatmulTiles:
        tm: int = tilejax_amd.choice(128, 256, 512, 1024, 2048, default=512)

Same surface as the reference (src/autokernel/tunable.py:31-73): `choice` lists a field's candidate values
(neighbours are one step apart), `tunable` makes a frozen dataclass whose fields are all choices, and
`neighbours` moves one field one step. There is no JAX pytree registration here (no JAX): the spec runs
over the package's own array stand-in, which needs none.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Dict, Iterator, Tuple

__all__ = ["choice", "choices", "is_tunable", "neighbours", "tunable"]

_CHOICES = "tilejax_amd.choices"


def choice(*values: Any, default: Any = None) -> Any:
    """A tunable field's candidate values, in order; its default is `default`, else the first value."""
    if not values:
        raise ValueError("a tunable field needs at least one value to choose from")
    default = values[0] if default is None else default
    if default not in values:
        raise ValueError(f"the default {default!r} isn't one of the choices {values}")
    return dataclasses.field(default=default, metadata={_CHOICES: tuple(values)})


def tunable(cls: type) -> type:
    """Make `cls` a tunable: a frozen dataclass whose fields are all declared with `choice(...)`."""
    cls = dataclasses.dataclass(frozen=True)(cls)
    for f in dataclasses.fields(cls):
        if _CHOICES not in f.metadata:
            raise TypeError(f"{cls.__name__}.{f.name}: declare tunable fields with tilejax_amd.choice(...)")
    cls.__tilejax_tunable__ = True  # type: ignore[attr-defined]
    return cls


def is_tunable(value: Any) -> bool:
    """Is `value` an instance of a `@tunable` class?"""
    return bool(getattr(type(value), "__tilejax_tunable__", False))


def choices(value: Any) -> Dict[str, Tuple[Any, ...]]:
    """Each field of a tunable and the values it may take."""
    return {f.name: f.metadata[_CHOICES] for f in dataclasses.fields(value)}


def neighbours(value: Any) -> Iterator[Any]:
    """The tunables one step away from `value`: one field moved to the next or previous of its choices."""
    for name, options in choices(value).items():
        current = getattr(value, name)
        at = options.index(current) if current in options else None
        for step in (1, -1):
            if at is not None and 0 <= at + step < len(options):
                yield dataclasses.replace(value, **{name: options[at + step]})
