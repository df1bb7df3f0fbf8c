"""edge_softmax (reference python/mojodgl/ops/edge_softmax.py).

Same arguments, shapes and errors as the reference, including its positional
`eids` rule (edge_softmax.py:119-158): with a subset `eids`, the positions of
`eids` are grouped by endpoint (groups in ascending endpoint id, positions in
the order they appear), position i reads `logits[i]`, and the result is as
long as `logits` with rows past len(eids) zero. The grouping (a stable radix
grouping), the softmax plan and the softmax run in one library call on the
GPU (mdgl_edge_softmax_positional) instead of a Python loop; logits keep
float32/float64.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .. import _lib
from ..base import ALL, DGLError, is_all
from . import _autograd, _plan

# edge_softmax(ALL) writes rows whose size is a multiple of this many bytes
# from its row pass, others through the (max, sum) table and a second pass
TWO_PASS_ROW_BYTES = 64

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
        d = int(math.prod(shape[1:]))
    else:
        raise DGLError("logits must be (E,), (E, 1) or (E, *, 1); got shape {}".format(shape))
    if norm_by not in ("dst", "src"):
        raise DGLError("norm_by must be 'src' or 'dst'")
    num_nodes = graph.number_of_nodes()
    on_gpu = False
    if is_all(eids):
        order = None
    else:
        # host ids are checked on the host before any GPU work; GPU ids by
        # the library, whose id range is read back as soon as it is known
        on_gpu = isinstance(eids, torch.Tensor) and eids.device.type == "cuda"
        order = _lib.i64_device(eids).reshape(-1) if on_gpu else _lib.i64(eids).reshape(-1)
        if order.shape[0] and not on_gpu:
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
    if out_len and d and order is not None:
        m = order.shape[0]
        if m:
            if on_gpu and num_edges == 0:
                raise DGLError("edge ids must be in [0, 0), got {} ids".format(m))
            lg = _lib.on_device(X, dtype).reshape(out_len, d)
            _positional(graph, lg, out, order, m, norm_by, on_gpu, keep)
    elif out_len and d:
        lg = _lib.on_device(X, dtype).reshape(out_len, d)
        slots, chunk_len = _plan.geometry(d, dtype, lg, out)
        csr = graph._device_csr("in" if norm_by == "dst" else "out")
        plan = csr.softmax_plan(slots, chunk_len)
        if num_nodes:
            # rows of less than 64 bytes, or not whole 64-byte pieces: the
            # row pass writes each row's (max, sum) to a table and a second,
            # edge-parallel pass writes the output in edge-id order from it
            # (a scattered store of such a row costs a read of its lines);
            # rows of whole 64-byte pieces are written by the row pass
            # itself (4-5 % faster on the power-law graph for 64- and
            # 128-byte rows, 35-50 % slower for 16- and 32-byte ones)
            two_pass = (d * np.dtype(dtype).itemsize) % TWO_PASS_ROW_BYTES != 0
            ws, nbytes = _plan.workspace(plan, d, dtype, plan.table_rows if two_pass else 0)
            rc = _lib.lib().mdgl_edge_softmax_(
                csr.indptr.data_ptr(), None, csr.eid.data_ptr(), None, lg.data_ptr(),
                out.data_ptr(), None, num_nodes, 1, d, _lib.ptr(plan.order), plan.bounds_ptr(),
                plan.nbins, _lib.ptr(plan.packed), _lib.ptr(plan.chunk_row),
                _lib.ptr(plan.chunk_start), _lib.ptr(plan.chunk_first), plan.num_chunks,
                plan.slots, _lib.ptr(plan.slot_of_edge) if two_pass else None, lg.shape[0],
                _lib.ptr(ws), nbytes,
                _lib.dtype_code(dtype), _lib.stream())
            _lib.check(rc, "edge_softmax")
    return _lib.give_back(out.reshape(shape), X.is_torch, X.device)


def _positional(graph, lg, out, order, m, norm_by, on_gpu, keep):
    """The positional rule in one library call (mdgl_edge_softmax_positional):
    positions grouped by the endpoint of their edge on the GPU, the softmax
    plan built there too, no host read in between. GPU ids are checked from
    the id range the call writes first, copied back while the rest runs."""
    gdev = lg.device
    num_nodes = graph.number_of_nodes()
    d = lg.shape[1]
    code = _lib.dtype_code(np.float32 if lg.dtype == torch.float32 else np.float64)
    uids, vids = graph._device_coo()
    ends = vids if norm_by == "dst" else uids
    idx = order if isinstance(order, torch.Tensor) else torch.from_numpy(order).to(gdev)
    endpoint = torch.empty(m, dtype=torch.int32, device=gdev)
    group_ptr = torch.empty(num_nodes + 1, dtype=torch.int32, device=gdev)
    group_pos = torch.empty(m, dtype=torch.int32, device=gdev)
    id_range = torch.empty(2, dtype=torch.int64, device=gdev)
    L = _lib.lib()
    nbytes = L.mdgl_edge_softmax_positional_workspace_bytes(m, num_nodes, d, lg.data_ptr(),
                                                            out.data_ptr(), code)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=gdev)
    ranged = None
    if on_gpu:
        ranged = torch.cuda.Event()
        ranged.record()  # creates the event; the call records it again once the range is known
    rc = L.mdgl_edge_softmax_positional(
        ends.data_ptr(), ends.shape[0], idx.data_ptr(), m, num_nodes, lg.data_ptr(),
        out.data_ptr(), d, endpoint.data_ptr(), group_ptr.data_ptr(), group_pos.data_ptr(),
        id_range.data_ptr(), ranged.cuda_event if ranged is not None else None, ws.data_ptr(),
        nbytes, code, _lib.stream())
    _lib.check(rc, "edge_softmax")
    if ranged is not None:
        lo, hi = _lib.Readback(id_range, "eids_range", after=ranged).values()
        if lo < 0 or hi >= ends.shape[0]:
            raise DGLError("edge ids must be in [0, {}), got [{}, {})".format(
                ends.shape[0], lo, hi + 1))
    if keep is not None:
        keep.update(endpoint=endpoint, indptr=group_ptr, eid=group_pos)
