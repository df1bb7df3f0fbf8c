"""Builtin reduce functions sum / max / min / mean (reference function/reducer.py)."""

from __future__ import annotations

import sys

from .base import BuiltinFunction

__all__ = []


class ReduceFunction(BuiltinFunction):
    """Base of the builtin reduce functions."""

    @property
    def name(self):
        raise NotImplementedError


class SimpleReduceFunction(ReduceFunction):
    """Reduce message field `msg_field` over in-edges into node field `out_field`."""

    def __init__(self, name, msg_field, out_field):
        self._name = name
        self.msg_field = msg_field
        self.out_field = out_field

    @property
    def name(self):
        return self._name


def _make_reducer(name):
    def reducer(msg, out):
        return SimpleReduceFunction(name, msg, out)

    reducer.__name__ = name
    reducer.__qualname__ = name
    reducer.__doc__ = (
        "Builtin reduce function: {0} of message field `msg` over each node's in-edges, "
        "written to node field `out` (nodes without in-edges get 0).\n\n"
        "    >>> reduce_func = mojodgl.function.{0}('m', 'h')\n").format(name)
    return reducer


for _name in ("max", "min", "sum", "mean"):
    setattr(sys.modules[__name__], _name, _make_reducer(_name))
    __all__.append(_name)
