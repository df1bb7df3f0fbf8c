"""Builtin message functions (reference python/mojodgl/function/message.py).

`copy_u`, `copy_e` and the 30 binary builtins `{u,v,e}_{add,sub,mul,div,dot}_
{u,v,e}` (operand targets distinct) are descriptors: `update_all` reads their
fields and dispatches them to the gspmm / gsddmm kernels.
"""

from __future__ import annotations

import sys
from itertools import permutations

from .base import BuiltinFunction, TargetCode

__all__ = ["copy_u", "copy_e", "BinaryMessageFunction", "CopyMessageFunction"]

_CODE = {"u": TargetCode.SRC, "v": TargetCode.DST, "e": TargetCode.EDGE}


class MessageFunction(BuiltinFunction):
    """Base of the builtin message functions."""

    @property
    def name(self):
        raise NotImplementedError


class BinaryMessageFunction(MessageFunction):
    """Message `lhs_field` (at target `lhs`) op `rhs_field` (at target `rhs`)."""

    def __init__(self, binary_op, lhs, rhs, lhs_field, rhs_field, out_field):
        self.binary_op = binary_op
        self.lhs = lhs
        self.rhs = rhs
        self.lhs_field = lhs_field
        self.rhs_field = rhs_field
        self.out_field = out_field

    @property
    def name(self):
        return "{}_{}_{}".format(TargetCode.CODE2STR[self.lhs], self.binary_op,
                                 TargetCode.CODE2STR[self.rhs])


class CopyMessageFunction(MessageFunction):
    """Message = the feature `in_field` of the source node or of the edge."""

    def __init__(self, target, in_field, out_field):
        self.target = target
        self.in_field = in_field
        self.out_field = out_field

    @property
    def name(self):
        return "copy_{}".format(TargetCode.CODE2STR[self.target])


def copy_u(u, out):
    """Builtin message: the source node feature `u`, written to message field `out`.

    Equivalent UDF: ``lambda edges: {out: edges.src[u]}``.
    """
    return CopyMessageFunction(TargetCode.SRC, u, out)


def copy_e(e, out):
    """Builtin message: the edge feature `e`, written to message field `out`.

    Equivalent UDF: ``lambda edges: {out: edges.data[e]}``.
    """
    return CopyMessageFunction(TargetCode.EDGE, e, out)


def _make_binary(lhs, rhs, op):
    name = "{}_{}_{}".format(lhs, op, rhs)
    where = {"u": "source node", "v": "destination node", "e": "edge"}

    def builtin(lhs_field, rhs_field, out):
        return BinaryMessageFunction(op, _CODE[lhs], _CODE[rhs], lhs_field, rhs_field, out)

    builtin.__name__ = name
    builtin.__qualname__ = name
    builtin.__doc__ = (
        "Builtin message function: {op} of the {l} feature `lhs_field` and the {r} feature "
        "`rhs_field`{how}, written to message field `out`. Operands of different feature "
        "shapes broadcast with NumPy's rules.\n\n"
        "    >>> message_func = mojodgl.function.{name}('a', 'b', 'm')\n").format(
            op=op, l=where[lhs], r=where[rhs], name=name,
            how=" (contracting the last axis)" if op == "dot" else " elementwise")
    return builtin


def _register():
    module = sys.modules[__name__]
    for lhs, rhs in permutations("uve", 2):
        for op in ("add", "sub", "mul", "div", "dot"):
            fn = _make_binary(lhs, rhs, op)
            setattr(module, fn.__name__, fn)
            __all__.append(fn.__name__)


_register()
