"""gsddmm and its generated variants (reference python/mojodgl/ops/sddmm.py).

Same entry points, argument meaning and errors as the reference, with two
differences: operands broadcast with NumPy's rules (the reference accepts
1-D and 2-D features only, widening a width-1 operand by copying it,
sddmm.py:50-68), and the result keeps the operands' float32/float64 dtype.
"""

from __future__ import annotations

import math
import sys
from itertools import product

import numpy as np
import torch

from .. import _lib
from .._lib import BINARY_OPS, OP_COPY_LHS, OP_COPY_RHS, TARGETS
from ..base import DGLError
from . import _autograd

__all__ = ["gsddmm", "copy_u", "copy_v", "copy_e"]


def _shape(a):
    if isinstance(a, (np.ndarray, torch.Tensor, _lib.Feat)):
        return tuple(a.shape)
    return tuple(np.shape(a))


def reshape_lhs_rhs(lhs_data, rhs_data):
    r"""Expand dims so that there will be no broadcasting issues with different
    number of dimensions. For example, given two shapes (N, 3, 1), (E, 5, 3, 4)
    that are valid broadcastable shapes, change them to (N, 1, 3, 1) and
    (E, 5, 3, 4).

    The padding goes right after the first (node / edge) axis
    (reference sddmm.py:24-47); numpy arrays and tensors are reshaped as views.
    """
    lhs_shape, rhs_shape = _shape(lhs_data), _shape(rhs_data)
    if len(lhs_shape) != len(rhs_shape):
        nd = max(len(lhs_shape), len(rhs_shape))
        new_l = (lhs_shape[0],) + (1,) * (nd - len(lhs_shape)) + lhs_shape[1:]
        new_r = (rhs_shape[0],) + (1,) * (nd - len(rhs_shape)) + rhs_shape[1:]
        lhs_data = _reshape(lhs_data, new_l)
        rhs_data = _reshape(rhs_data, new_r)
    return lhs_data, rhs_data


def _reshape(a, shape):
    if isinstance(a, _lib.Feat):
        return _lib.Feat(a.data.reshape(shape), a.is_torch, a.device)
    if isinstance(a, (np.ndarray, torch.Tensor)):
        return a.reshape(shape)
    return np.reshape(a, shape)


def feat_shape(shape):
    """Feature shape of an operand; a 1-D operand is read as (n, 1)."""
    shape = tuple(shape)
    return shape[1:] if len(shape) > 1 else (1,)


def width(shape) -> int:
    w = 1
    for x in feat_shape(shape):
        w *= int(x)
    return w


def out_feat_shape(lshape, rshape, dot=False):
    """Broadcast feature shape of two padded operands (dot: last axis contracted)."""
    lf, rf = feat_shape(lshape), feat_shape(rshape)
    if dot:
        if lf[-1] != rf[-1]:
            raise DGLError("dot needs matching feature widths, {} vs {}".format(lf[-1], rf[-1]))
        lf, rf = lf[:-1], rf[:-1]
    if lf == rf:
        return lf + ((1,) if dot else ())
    try:
        out = tuple(np.broadcast_shapes(lf, rf))
    except ValueError:
        raise DGLError("operands are not broadcastable: {} and {}".format(lshape, rshape))
    return out + ((1,) if dot else ())


_SHAPE_ARGS = {}


def shape_ptrs(lshape, rshape):
    """(nd, lhs feature shape, rhs feature shape, their addresses, key) for
    the C ABI: int64 host arrays, kept per shape pair (they are only read),
    their data pointers, which the caller passes while it holds the arrays,
    and the pair of feature-shape tuples they hold."""
    key = (feat_shape(lshape), feat_shape(rshape))
    got = _SHAPE_ARGS.get(key)
    if got is None:
        lf = np.ascontiguousarray(key[0], dtype=np.int64)
        rf = np.ascontiguousarray(key[1], dtype=np.int64)
        assert lf.size == rf.size
        lf.flags.writeable = False
        rf.flags.writeable = False
        got = (int(lf.size), lf, rf, lf.ctypes.data, rf.ctypes.data, key)
        if len(_SHAPE_ARGS) < 4096:
            _SHAPE_ARGS[key] = got
    return got


def _check_rows(a, want: int, what: str) -> None:
    """Reject an operand whose row count is not the one its target implies
    (reference sddmm.py:71-80; the kernels index without bounds checks)."""
    if a.shape[0] != want:
        raise DGLError("{} data must have {} rows, got {}".format(what, want, a.shape[0]))


def gsddmm(g, op, lhs_data, rhs_data, lhs_target="u", rhs_target="v"):
    r"""Generalized Sampled-Dense-Dense Matrix Multiplication interface.
    It computes edge features by :attr:`op` lhs features and rhs features.

    .. math::

        x_{e} = \phi(x_{lhs}, x_{rhs}), \forall (u,e,v)\in \mathcal{G}

    Parameters
    ----------
    g : DGLGraph
        The input graph.
    op : str
        ``add``, ``sub``, ``mul``, ``div``, ``dot``, ``copy_lhs`` or ``copy_rhs``.
    lhs_data, rhs_data : numpy array, torch tensor or None
        The operands (None when the op does not read it).
    lhs_target, rhs_target : str
        ``u`` (source), ``v`` (destination) or ``e`` (edge).

    Returns
    -------
    Edge features of shape ``(E,) + broadcast feature shape`` (``(E, ..., 1)``
    for dot), a numpy array or, when an operand is a tensor, a tensor (which
    takes part in autograd when an operand requires grad).
    """
    num_edges = g.number_of_edges()
    num_nodes = g.number_of_nodes()
    if lhs_target not in TARGETS or rhs_target not in TARGETS:
        raise DGLError("lhs_target/rhs_target must be one of 'u', 'v', 'e'")
    if _autograd.needs_grad(lhs_data, rhs_data):
        return _autograd.GSDDMM.apply(g, op, lhs_data, rhs_data, lhs_target, rhs_target)
    L = R = None
    if op == "copy_lhs":
        L = _lib.feature(lhs_data)
        fshape = feat_shape(L.shape)
        code = OP_COPY_LHS
    elif op == "copy_rhs":
        R = _lib.feature(rhs_data)
        fshape = feat_shape(R.shape)
        code = OP_COPY_RHS
    else:
        if op not in BINARY_OPS:
            raise DGLError("op {} not recognized".format(op))
        L, R = reshape_lhs_rhs(_lib.feature(lhs_data), _lib.feature(rhs_data))
        fshape = out_feat_shape(L.shape, R.shape, dot=(op == "dot"))
        code = BINARY_OPS[op]
    if L is not None:
        _check_rows(L, num_edges if lhs_target == "e" else num_nodes,
                    "edge" if lhs_target == "e" else "node")
    if R is not None:
        _check_rows(R, num_edges if rhs_target == "e" else num_nodes,
                    "edge" if rhs_target == "e" else "node")
    dtype = _lib.common_dtype(L, R)
    as_torch = _lib.wants_torch(L, R)
    dev = _lib.out_device(L, R)
    dout = int(math.prod(fshape[:-1] if op == "dot" else fshape))
    if num_edges == 0 or dout == 0:
        empty = np.zeros((num_edges,) + tuple(fshape), dtype=dtype)
        return torch.from_numpy(empty).to(dev) if as_torch else empty
    lt = L if L is not None else R
    rt = R if R is not None else L
    dl, dr = width(lt.shape), width(rt.shape)
    if code in (OP_COPY_LHS, OP_COPY_RHS):
        nd, lsp, rsp = 0, None, None
    else:
        # the arrays stay referenced (here and in the cache) through the call
        nd, _lsa, _rsa, lsp, rsp, _ = shape_ptrs(L.shape, R.shape)
    lhs = _lib.on_device(L, dtype) if L is not None else None
    rhs = _lib.on_device(R, dtype) if R is not None else None
    uids, vids = g._device_coo()
    # allocated in its final shape: the same row-major bytes as (E, dout)
    out = torch.empty((num_edges,) + tuple(fshape), dtype=_lib.torch_dtype(dtype),
                      device=_lib.device())
    rc = _lib.lib().mdgl_gsddmm(
        _lib.ptr(uids), _lib.ptr(vids), _lib.ptr(lhs), _lib.ptr(rhs), out.data_ptr(), num_edges,
        TARGETS[lhs_target], TARGETS[rhs_target], code, dl, dr, dout, nd, lsp, rsp,
        _lib.dtype_code(dtype), _lib.stream())
    _lib.check(rc, "gsddmm")
    return _lib.give_back(out, as_torch, dev)


def _gen_sddmm_func(lhs_target, rhs_target, binary_op):
    name = "{}_{}_{}".format(lhs_target, binary_op, rhs_target)
    where = {"u": "source node", "e": "edge", "v": "destination node"}

    def func(g, x, y):
        return gsddmm(g, binary_op, x, y, lhs_target=lhs_target, rhs_target=rhs_target)

    func.__name__ = name
    func.__qualname__ = name
    func.__doc__ = (
        "Generalized SDDMM function: edge features by {op} of the {l} features `x` and the "
        "{r} features `y`. Feature shapes broadcast with NumPy's rules.\n\n"
        "Parameters\n----------\ng : DGLGraph\nx : {l} features\ny : {r} features\n\n"
        "Returns\n-------\nThe edge features.\n").format(
            op=binary_op, l=where[lhs_target], r=where[rhs_target])
    return func


def _register_sddmm_func():
    for lhs, rhs in product("uve", "uve"):
        if lhs != rhs:
            for binary_op in ("add", "sub", "mul", "div", "dot"):
                func = _gen_sddmm_func(lhs, rhs, binary_op)
                setattr(sys.modules[__name__], func.__name__, func)
                __all__.append(func.__name__)


def copy_u(g, x):
    """Source node features copied to every edge: ``out[e] = x[u[e]]``."""
    return gsddmm(g, "copy_lhs", x, None)


def copy_v(g, x):
    """Destination node features copied to every edge: ``out[e] = x[v[e]]``."""
    return gsddmm(g, "copy_rhs", None, x)


def copy_e(g, x):
    """Edge features as edge features: returns `x` itself (as the reference)."""
    return x


_register_sddmm_func()
