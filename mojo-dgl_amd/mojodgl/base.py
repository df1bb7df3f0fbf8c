"""Shared names of the API (the reference's python/mojodgl/base.py:1-38)."""

from __future__ import annotations

__all__ = ["ALL", "EID", "ETYPE", "NID", "NTYPE", "DGLError", "is_all"]


class DGLError(RuntimeError):
    """Raised for invalid arguments, under the name DGL callers catch."""


class _All:
    """The "every node / every edge" sentinel; a singleton that is falsy."""

    _one = None

    def __new__(cls):
        if cls._one is None:
            cls._one = super().__new__(cls)
        return cls._one

    def __repr__(self) -> str:
        return "ALL"

    def __bool__(self) -> bool:
        return False


ALL = _All()
EID = ALL
ETYPE = ALL
NID = ALL
NTYPE = ALL


def is_all(x) -> bool:
    return isinstance(x, _All)
