"""Graph construction (reference python/mojodgl/convert.py)."""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .base import DGLError
from .heterograph import DGLGraph

__all__ = ["graph"]


def _ids(a):
    """GPU tensors stay where they are; anything else becomes numpy."""
    if isinstance(a, torch.Tensor):
        if a.device.type == "cuda":
            return a
        a = a.detach().cpu().numpy()
    return np.asarray(a)


def _integral(a):
    if isinstance(a, torch.Tensor):
        return not (a.is_floating_point() or a.is_complex())
    return np.issubdtype(a.dtype, np.integer)


def graph(data, *, num_nodes=None, idtype=None, device=None, row_sorted=False, col_sorted=False):
    """Create a graph from a ``(u, v)`` pair of node-id arrays or a scipy sparse matrix.

    Parameters
    ----------
    data : tuple of two integer arrays (numpy, list or tensor), or a scipy
        sparse matrix whose nonzero entries are the edges
    num_nodes : int, optional
        Inferred (largest id + 1, or the matrix size) when omitted.
    idtype : int32 or int64 (default), the dtype of the ids the graph's
        queries return.
    device, row_sorted, col_sorted :
        Accepted for signature compatibility. Edges keep the order given.
        Ids given as GPU tensors stay on the GPU; others are copied there
        when the graph is first used.

    Examples
    --------
    >>> g = mojodgl.graph(([0, 1, 2, 3], [1, 2, 3, 4]))
    >>> g.num_nodes()
    5
    """
    if hasattr(data, "tocoo"):
        coo = data.tocoo()
        u, v = coo.row, coo.col
        if num_nodes is None:
            num_nodes = max(data.shape)
    elif isinstance(data, tuple) and len(data) == 2:
        u, v = _ids(data[0]), _ids(data[1])
        if not _integral(u) or not _integral(v):
            raise DGLError("node ids must be integers")
        if isinstance(u, torch.Tensor) != isinstance(v, torch.Tensor):
            u, v = _lib.i64(u), _lib.i64(v)
    else:
        raise DGLError("expect data to be a tuple of two node-id arrays or a scipy sparse matrix")
    return DGLGraph(u, v, num_nodes=num_nodes, idtype=idtype)
