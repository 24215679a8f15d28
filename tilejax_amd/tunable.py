"""Tunables: the one object a kernel hands the compiler to optimize over.

    @tilejax_amd.tunable
    class MatmulTiles:
        tm: int = tilejax_amd.choice(128, 256, 512, 1024, 2048, default=512)

The surface is the reference's (src/autokernel/tunable.py:31-73): `choice` lists a field's candidate values
in order, `tunable` makes a frozen dataclass whose every field is a choice, `neighbours` moves one field
one place along its list. Here a class's choices live in a table on the class (`__tilejax_choices__`), the
fields themselves being plain dataclass fields with their defaults. There is no pytree registration: specs
run over the package's own array stand-in, which needs none.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Dict, Iterator, Tuple

__all__ = ["choice", "choices", "is_tunable", "neighbours", "tunable"]

_TABLE = "__tilejax_choices__"


class _Choice:
    """What `choice(...)` returns: a field's candidate values and its default, until `@tunable` reads it."""

    __slots__ = ("values", "default")

    def __init__(self, values: Tuple[Any, ...], default: Any) -> None:
        self.values, self.default = values, default

    def __repr__(self) -> str:
        return f"choice{self.values} (default {self.default!r})"


def choice(*values: Any, default: Any = None) -> Any:
    """A tunable field's candidate values, in the order neighbours walk them; its default is `default`,
    else the first value."""
    if len(values) == 0:
        raise ValueError("a tunable field needs at least one value to choose from")
    picked = values[0] if default is None else default
    if picked not in values:
        raise ValueError(f"the default {picked!r} isn't one of the choices {values}")
    return _Choice(tuple(values), picked)


def tunable(cls: type) -> type:
    """Make `cls` a tunable: a frozen dataclass whose annotated fields are all declared with
    `choice(...)`."""
    table: Dict[str, Tuple[Any, ...]] = {}
    for name in cls.__dict__.get("__annotations__", {}):
        declared = cls.__dict__.get(name, dataclasses.MISSING)
        if not isinstance(declared, _Choice):
            raise TypeError(f"{cls.__name__}.{name}: declare tunable fields with tilejax_amd.choice(...)")
        table[name] = declared.values
        setattr(cls, name, declared.default)
    stray = [k for k, v in cls.__dict__.items() if isinstance(v, _Choice)]
    if stray:
        raise TypeError(f"{cls.__name__}.{stray[0]}: a choice needs a type annotation, `{stray[0]}: int = choice(...)`")
    setattr(cls, _TABLE, table)
    return dataclasses.dataclass(frozen=True)(cls)


def is_tunable(value: Any) -> bool:
    """Is `value` an instance of a `@tunable` class?"""
    return isinstance(getattr(type(value), _TABLE, None), dict) and dataclasses.is_dataclass(value)


def choices(value: Any) -> Dict[str, Tuple[Any, ...]]:
    """Each field of a tunable and the values it may take, in field order."""
    return dict(getattr(type(value), _TABLE))


def neighbours(value: Any) -> Iterator[Any]:
    """The tunables one move away from `value`, field by field: the field's next value, then its previous
    one (a field whose current value isn't among its choices doesn't move)."""
    for name, values in choices(value).items():
        here = getattr(value, name)
        if here not in values:
            continue
        at = values.index(here)
        for there in (at + 1, at - 1):
            if there in range(len(values)):
                yield dataclasses.replace(value, **{name: values[there]})
