"""Builtin-function base types (reference python/mojodgl/function/base.py:8-32)."""

from __future__ import annotations

__all__ = ["BuiltinFunction", "TargetCode"]


class TargetCode(object):
    """Which endpoint (or the edge) a builtin reads: the C ABI's target codes."""

    SRC = 0
    DST = 1
    EDGE = 2

    CODE2STR = {0: "u", 1: "v", 2: "e"}


class BuiltinFunction(object):
    """Base of the message and reduce builtins."""

    @property
    def name(self):
        raise NotImplementedError
