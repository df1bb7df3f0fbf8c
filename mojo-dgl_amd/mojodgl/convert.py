"""Graph construction (reference python/mojodgl/convert.py)."""

from __future__ import annotations

import numpy as np
import torch

from .base import DGLError
from .heterograph import DGLGraph

__all__ = ["graph"]


def _ids(a):
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.asarray(a)


def graph(data, *, num_nodes=None, idtype=None, device=None, row_sorted=False, col_sorted=False):
    """Create a graph from a ``(u, v)`` pair of node-id arrays or a scipy sparse matrix.

    Parameters
    ----------
    data : tuple of two integer arrays (numpy, list or tensor), or a scipy
        sparse matrix whose nonzero entries are the edges
    num_nodes : int, optional
        Inferred (largest id + 1, or the matrix size) when omitted.
    idtype, device, row_sorted, col_sorted :
        Accepted for signature compatibility. Edges keep the order given;
        the graph's GPU copy is made on the current device when first used.

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
        if not np.issubdtype(u.dtype, np.integer) or not np.issubdtype(v.dtype, np.integer):
            raise DGLError("node ids must be integers")
    else:
        raise DGLError("expect data to be a tuple of two node-id arrays or a scipy sparse matrix")
    return DGLGraph(u, v, num_nodes=num_nodes, idtype=idtype or np.int64)
