"""edge_softmax (reference python/mojodgl/ops/edge_softmax.py).

Same arguments, shapes and errors as the reference, including its positional
`eids` rule (edge_softmax.py:119-158): with a subset `eids`, the positions of
`eids` are grouped by endpoint (groups in ascending endpoint id, positions in
the order they appear), position i reads `logits[i]`, and the result is as
long as `logits` with rows past len(eids) zero. The grouping is one stable
radix grouping on the GPU (mdgl_build_csr) instead of a Python loop; logits
keep float32/float64.
"""

from __future__ import annotations

import numpy as np
import torch

from .. import _lib, heterograph
from ..base import ALL, DGLError, is_all
from . import _autograd, _plan

__all__ = ["edge_softmax"]


def edge_softmax(graph, logits, eids=ALL, norm_by="dst"):
    r"""Compute softmax over weights of incoming edges for every node.

    For a node :math:`i`, edge softmax is an operation that computes

    .. math::
      a_{ij} = \frac{\exp(z_{ij})}{\sum_{j\in\mathcal{N}(i)}\exp(z_{ij})}

    where :math:`z_{ij}` is the signal (logit) of edge :math:`j\rightarrow i`.
    ``norm_by='dst'`` normalizes over each node's incoming edges (GAT,
    Transformer); ``norm_by='src'`` over its outgoing edges.

    Parameters
    ----------
    graph : DGLGraph
    logits : array or tensor of shape ``(E,)``, ``(E, 1)`` or ``(E, *, 1)``;
        every trailing column is an independent softmax.
    eids : array of edge ids or ALL
    norm_by : 'src' or 'dst'

    Returns
    -------
    Softmax values, of the same shape as ``logits``. With a torch tensor that
    requires grad the result takes part in autograd (with a subset ``eids``
    the rows past len(eids) are constant zero and get no gradient).

    Examples
    --------
    >>> g = mojodgl.graph(([0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]))
    >>> edge_softmax(g, np.ones((6, 1)))
    array([[1.        ],
           [0.5       ],
           [0.33333333],
           [0.5       ],
           [0.33333333],
           [0.33333333]])
    """
    if _autograd.needs_grad(logits):
        if norm_by not in ("dst", "src"):
            raise DGLError("norm_by must be 'src' or 'dst'")
        return _autograd.EdgeSoftmax.apply(graph, logits, norm_by,
                                           None if is_all(eids) else eids)
    return _edge_softmax(graph, logits, eids, norm_by)


def _edge_softmax(graph, logits, eids, norm_by, keep=None):
    """edge_softmax without autograd (`eids` None or ALL means every edge).
    With a subset and a dict `keep`, the grouping of the selected positions
    is left in it for the backward: `endpoint` (int32 node of each position),
    `indptr` / `eid` (positions grouped by node, in order of appearance)."""
    if eids is None:
        eids = ALL
    num_edges = graph.number_of_edges()
    X = _lib.feature(logits)
    shape = X.shape
    if len(shape) == 1:
        d = 1
    elif len(shape) >= 2 and shape[-1] == 1:
        d = int(np.prod(shape[1:], dtype=np.int64))
    else:
        raise DGLError("logits must be (E,), (E, 1) or (E, *, 1); got shape {}".format(shape))
    if norm_by not in ("dst", "src"):
        raise DGLError("norm_by must be 'src' or 'dst'")
    num_nodes = graph.number_of_nodes()
    if is_all(eids):
        order = None
    else:
        # GPU ids are checked on the GPU (one small read back), host ids on
        # the host before any GPU work
        on_gpu = isinstance(eids, torch.Tensor) and eids.device.type == "cuda"
        order = _lib.i64_device(eids).reshape(-1) if on_gpu else _lib.i64(eids).reshape(-1)
        if order.shape[0]:
            if on_gpu:
                lo, hi = torch.stack((order.min(), order.max())).tolist()
            else:
                lo, hi = int(order.min()), int(order.max())
            if lo < 0 or hi >= num_edges:
                raise DGLError("edge ids must be in [0, {}), got [{}, {})".format(
                    num_edges, lo, hi + 1))
    out_len = shape[0]
    if order is None and out_len != num_edges:
        raise DGLError("logits has {} rows but the graph has {} edges".format(out_len, num_edges))
    if order is not None and order.shape[0] > out_len:
        raise DGLError("{} edge ids selected but logits has only {} rows".format(
            order.shape[0], out_len))

    dtype = X.dtype
    gdev = _lib.device()
    # on the ALL path every edge is in exactly one CSR row, so every output
    # row is written; a subset leaves the rows past len(eids) at zero
    alloc = torch.empty if order is None else torch.zeros
    out = alloc((out_len, d), dtype=_lib.torch_dtype(dtype), device=gdev)
    if out_len and d:
        lg = _lib.on_device(X, dtype).reshape(out_len, d)
        if order is not None:
            lg = lg[: order.shape[0]].contiguous()
        slots, chunk_len = _plan.geometry(d, dtype, lg, out)
        if order is None:
            csr = graph._device_csr("in" if norm_by == "dst" else "out")
            indptr, eid, rows = csr.indptr, csr.eid, num_nodes
            plan = csr.softmax_plan(slots, chunk_len)
        else:
            # positions grouped by (endpoint, appearance): the stable grouping
            # of the selected edges' endpoints, on the GPU; rows are all nodes
            # (the ones no selected edge reaches are empty and skipped)
            uids, vids = graph._device_coo()
            idx = order if isinstance(order, torch.Tensor) else torch.from_numpy(order).to(gdev)
            endpoint = (vids if norm_by == "dst" else uids)[idx]
            indptr, _, eid = heterograph.build_device_csr(endpoint, None, num_nodes)
            if keep is not None:
                keep.update(endpoint=endpoint, indptr=indptr, eid=eid)
            rows = num_nodes if idx.shape[0] else 0
            plan = _plan.SoftmaxPlan.from_device(indptr, slots, chunk_len, ordered=True,
                                                 eid=eid)
        if rows:
            n_edges = lg.shape[0]
            # the second, edge-parallel pass writes the output in edge-id
            # order from the (max, sum) table slot of each edge's row
            row_of = plan.slot_of_edge
            ws, nbytes = _plan.workspace(plan, d, dtype, plan.table_rows)
            rc = _lib.lib().mdgl_edge_softmax_(
                indptr.data_ptr(), None, eid.data_ptr(), None, lg.data_ptr(), out.data_ptr(), None,
                rows, 1, d, _lib.ptr(plan.order), plan.bounds_ptr(), plan.nbins,
                _lib.ptr(plan.packed), _lib.ptr(plan.chunk_row), _lib.ptr(plan.chunk_start), _lib.ptr(plan.chunk_first),
                plan.num_chunks, plan.slots, _lib.ptr(row_of), n_edges, _lib.ptr(ws), nbytes,
                _lib.dtype_code(dtype), _lib.stream())
            _lib.check(rc, "edge_softmax")
    return _lib.give_back(out.reshape(shape), X.is_torch, X.device)
