"""The one exception the compiler raises for code it can't compile or run as asked.

Mirrors the reference's `KernelError` (src/autokernel/errors.py:11-24): when the error is about a line of
the user's kernel function, the message starts with `file:line:` and quotes that line.
"""

from __future__ import annotations

import ast
import linecache
from typing import Optional

__all__ = ["KernelError"]


class KernelError(Exception):
    """A kernel function that can't be compiled for gfx950, or can't run as asked."""

    def __init__(self, message: str, *, filename: Optional[str] = None, node: Optional[ast.AST] = None) -> None:
        lineno = getattr(node, "lineno", None)
        if filename and lineno:
            message = f"{filename}:{lineno}: {message}"
            line = linecache.getline(filename, lineno).strip()
            if line:
                message += f"\n    {line}"
        super().__init__(message)
