"""gspmm and its generated variants (reference python/mojodgl/ops/spmm.py).

Same entry points, argument meaning and errors as the reference; operands
broadcast with NumPy's rules and keep their float32/float64 dtype. `_gspmm`
additionally returns the arg indices of max/min, which the reference does
not produce (its kernel writes values only, src/ported.mojo:352-423).
"""

from __future__ import annotations

import ctypes
import sys

import numpy as np
import torch

from .. import _lib
from .._lib import BINARY_OPS, OP_COPY_LHS, OP_COPY_RHS, REDUCERS
from . import _autograd
from ..base import DGLError
from .sddmm import _check_rows, feat_shape, out_feat_shape, reshape_lhs_rhs, shape_ptrs, width

__all__ = ["gspmm"]


# a scalar edge operand of this many edges or more is put in CSR slot order
# before a one-slab whole-wavefront gspmm (below that the extra launch costs
# more than it saves)
CSR_ORDER_MIN_EDGES = 1 << 20


_OPS = frozenset(BINARY_OPS) | {"copy_lhs", "copy_rhs"}

_LANES = {}


def _lanes(code, dl, dr, dout, sp, lhs, rhs, flags, dtype):
    """(packed, slabs) of the lane layout mdgl_gspmm picks for these operands
    and flags (mdgl_gspmm_lanes): whether several rows share a wavefront
    (slabs of 32 lanes or fewer) and how many column slabs a row is cut
    into. `sp` is shape_ptrs' entry for the operands' feature shapes (None
    for the copy ops). The answer depends only on the sizes, shapes, flags,
    dtype and the operands' alignment (within 128 bytes), so it is kept per
    such key: the query costs more host time than a small gspmm's kernel."""
    key = (code, dl, dr, dout, None if sp is None else sp[5],
           lhs.data_ptr() % 128 if lhs is not None else -1,
           rhs.data_ptr() % 128 if rhs is not None else -1, flags, dtype.str)
    got = _LANES.get(key)
    if got is None:
        if len(_LANES) >= 4096:  # many distinct shapes: start over rather than grow
            _LANES.clear()
        got = _LANES[key] = _lanes_query(code, dl, dr, dout, sp, lhs, rhs, flags, dtype)
    return got


def _lanes_query(code, dl, dr, dout, sp, lhs, rhs, flags, dtype):
    vec, group = ctypes.c_int64(), ctypes.c_int64()
    nd, lsp, rsp = (0, None, None) if sp is None else (sp[0], sp[3], sp[4])
    _lib.check(_lib.lib().mdgl_gspmm_lanes(
        code, dl, dr, dout, nd, lsp, rsp, _lib.ptr(lhs), _lib.ptr(rhs), flags,
        _lib.dtype_code(dtype), ctypes.byref(vec), ctypes.byref(group)), "gspmm_lanes")
    lanes = -(-dout // vec.value)
    return group.value <= 32, -(-lanes // group.value)


def _line_rows_pay(rows, dl, num_edges, dtype):
    """Whether copying lhs to line-aligned rows can pay (_line_rows): rows
    of 512 bytes or more whose size is no multiple of 128 bytes, gathered at
    least 8 times each."""
    row_bytes = dl * np.dtype(dtype).itemsize
    return not (row_bytes % 128 == 0 or row_bytes < 512 or rows == 0 or num_edges < 8 * rows)


def _line_rows(lhs, rows, dl, num_edges, dtype):
    """lhs copied to rows that each start on a 128-byte line (the layout of
    mdgl_gspmm's MDGL_LHS_LINE_ROWS), or None when that does not pay: rows of
    a size that is no multiple of 128 bytes start mid-line, so every column
    slab of them touches one line more than it needs; the copy reads and
    writes the table once, worth it for rows of a slab or more that the
    edges gather at least 8 times each."""
    if not _line_rows_pay(rows, dl, num_edges, dtype):
        return None
    es = np.dtype(dtype).itemsize
    row_bytes = dl * es
    stride = -(-row_bytes // 128) * 128 // es
    free, _ = torch.cuda.mem_get_info(lhs.device)
    if rows * stride * es > free // 4:  # the copy must not crowd out the caller's memory
        return None
    padded = torch.empty((rows, stride), dtype=lhs.dtype, device=lhs.device)
    padded[:, :dl].copy_(lhs.reshape(rows, dl))
    return padded


_FLOATS = (torch.float32, torch.float64)
# positions of the per-call values in mdgl_gspmm's argument list
_A_LHS, _A_RHS, _A_OUT, _A_ARG_U, _A_ARG_E, _A_WS, _A_STREAM = 3, 4, 5, 16, 17, 25, 29
_LAUNCHES_MAX = 256  # call shapes kept per graph


class _Launch:
    """A gspmm call shape seen before on a graph, replayed without the full
    path's validation and choices: the argument list mdgl_gspmm got for
    operands of these shapes, dtypes and alignments, the per-call values
    (operand, result and workspace addresses, the stream) filled in at each
    call. Taken only for GPU tensors that the full path would use in place
    (contiguous, on the current GPU, one float dtype) and calls whose
    choices depend on shapes alone (no line-row copy, no CSR-order edge
    operand). It holds the CSR it was made for and is dropped when the graph
    holds another one (a new chunk length)."""

    __slots__ = ("csr", "args", "shape", "tdt", "gdev", "arg", "arg_dtype", "nbytes", "local",
                 "dev", "sp")

    def run(self, lhs, rhs):
        gdev = self.gdev
        out = torch.empty(self.shape, dtype=self.tdt, device=gdev)
        args = list(self.args)
        args[_A_LHS] = None if lhs is None else lhs.data_ptr()
        args[_A_RHS] = None if rhs is None else rhs.data_ptr()
        args[_A_OUT] = out.data_ptr()
        arg_u = arg_e = None
        if self.arg:
            arg_u = torch.empty(self.shape, dtype=torch.int32, device=gdev)
            arg_e = torch.empty(self.shape, dtype=torch.int32, device=gdev)
            args[_A_ARG_U] = arg_u.data_ptr()
            args[_A_ARG_E] = arg_e.data_ptr()
        ws = None
        if self.nbytes:
            ws = torch.empty(self.nbytes, dtype=torch.uint8, device=gdev)
            args[_A_WS] = ws.data_ptr()
        args[_A_STREAM] = _lib.stream()
        _lib.check(_lib.lib().mdgl_gspmm(*args), "gspmm")
        if self.arg:
            arg_u = arg_u.to(self.arg_dtype)
            arg_e = arg_e.to(self.arg_dtype)
        return out, arg_u, arg_e, True, self.dev


def _operand_key(t):
    """(shape, dtype, address mod 128, device index) of a contiguous float
    GPU tensor, else None (without touching the GPU)."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype not in _FLOATS \
            or not t.is_contiguous():
        return None
    return t.shape, t.dtype, t.data_ptr() % 128, t.get_device()


def _launch_key(op, reduce_op, lhs, rhs, replace_inf, want_arg, arg_dtype, kind, narrow_split):
    """Key of a call shape for _Launch, or None when the call must take the
    full path (operands it would convert or copy: host arrays, another GPU,
    non-contiguous tensors, two dtypes)."""
    lk = rk = None
    if op != "copy_rhs":
        lk = _operand_key(lhs)
        if lk is None:
            return None
    if op != "copy_lhs":
        rk = _operand_key(rhs)
        if rk is None:
            return None
    if lk is not None and rk is not None and lk[1] != rk[1]:
        return None
    dev = _lib.current_device()  # operands on the GPU: its state is up
    if (lk is not None and lk[3] != dev) or (rk is not None and rk[3] != dev):
        return None
    return (kind, op, reduce_op, replace_inf, want_arg, arg_dtype, narrow_split, lk, rk, dev,
            CSR_ORDER_MIN_EDGES, _lanes)


def _run(g, op, reduce_op, lhs_data, rhs_data, replace_inf=False, want_arg=False,
         arg_dtype=torch.int64, kind="in", narrow_split=None, rows=None):
    """Validate, launch, and return device tensors (out, arg_u, arg_e) plus
    the caller-container info. `kind` "out" reduces over the out-CSR instead
    (the reversed graph: rows are sources, the node operand is read at the
    destinations), which the backward passes use. `narrow_split`: when
    several rows share a wavefront, split rows longer than this (instead of
    the graph's chunk length) so a wavefront's rows have bounded lengths --
    their sums then fold in chunks, within the tolerance rule rather than
    bit for bit (the backward passes' reductions use it). `rows` (an int32
    GPU tensor of distinct node ids): reduce those rows only, each whole
    (mdgl_gspmm_rows), the other rows of the result zero. A call shape seen
    before on `g` replays its launch (_Launch)."""
    key = None if rows is not None else _launch_key(
        op, reduce_op, lhs_data, rhs_data, replace_inf, want_arg, arg_dtype, kind, narrow_split)
    if key is not None:
        launch = g._launches.get(key)
        if launch is not None and launch.csr is g._current_csr(kind) \
                and (launch.local is None or g._local() is launch.local):
            # the copy ops read one operand; the other is passed as null
            return launch.run(None if op == "copy_rhs" else lhs_data,
                              None if op == "copy_lhs" else rhs_data)
    if reduce_op not in REDUCERS:
        raise DGLError("reduce_op {} not recognized".format(reduce_op))
    if op not in _OPS:
        raise DGLError("op {} not recognized".format(op))
    if op == "dot":
        raise DGLError("dot is not a gspmm operator; use gsddmm")
    num_dst = g.number_of_nodes()
    num_edges = g.number_of_edges()
    L = R = None
    if op == "copy_lhs":
        L = _lib.feature(lhs_data)
        fshape = feat_shape(L.shape)
        code = OP_COPY_LHS
        _check_rows(L, num_dst, "node")
    elif op == "copy_rhs":
        R = _lib.feature(rhs_data)
        fshape = feat_shape(R.shape)
        code = OP_COPY_RHS
        _check_rows(R, num_edges, "edge")
    else:
        L, R = reshape_lhs_rhs(_lib.feature(lhs_data), _lib.feature(rhs_data))
        fshape = out_feat_shape(L.shape, R.shape)
        code = BINARY_OPS[op]
        _check_rows(L, num_dst, "node")
        _check_rows(R, num_edges, "edge")
    dtype = _lib.common_dtype(L, R)
    as_torch = _lib.wants_torch(L, R)
    dev = _lib.out_device(L, R)
    dout = 1
    for s_ in fshape:
        dout *= int(s_)
    # results allocated in their final shapes: the same row-major bytes as
    # (num_dst, dout)
    shape = (num_dst,) + tuple(fshape)
    tdt = _lib.torch_dtype(dtype)
    dcode = _lib.dtype_code(dtype)
    gdev = _lib.device()
    arg = want_arg and reduce_op in ("max", "min")
    if rows is None:
        out = torch.empty(shape, dtype=tdt, device=gdev)
        arg_u = torch.empty(shape, dtype=torch.int32, device=gdev) if arg else None
        arg_e = torch.empty(shape, dtype=torch.int32, device=gdev) if arg else None
    else:  # the rows that are not listed stay zero (no message: arg -1)
        out = torch.zeros(shape, dtype=tdt, device=gdev)
        arg_u = torch.full(shape, -1, dtype=torch.int32, device=gdev) if arg else None
        arg_e = torch.full(shape, -1, dtype=torch.int32, device=gdev) if arg else None
    if num_dst and dout:
        lt = L if L is not None else R
        rt = R if R is not None else L
        dl, dr = width(lt.shape), width(rt.shape)
        # the shape arrays stay referenced (in `sp` and the cache) through the call
        sp = None if code in (OP_COPY_LHS, OP_COPY_RHS) else shape_ptrs(L.shape, R.shape)
        nd, lsp, rsp = (0, None, None) if sp is None else (sp[0], sp[3], sp[4])
        lhs = _lib.on_device(L, dtype) if L is not None else None
        rhs = _lib.on_device(R, dtype) if R is not None else None
        csr = g._device_csr(kind)
        flags = _lib.REPLACE_INF if replace_inf else 0
        replay = key is not None
        if rows is not None:
            # the layout choices below pay over whole graphs, not a few rows
            return _run_rows(csr, rows, code, reduce_op, lhs, rhs, out, arg_u, arg_e, dl, dr,
                             dout, nd, lsp, rsp, flags, dcode, arg, arg_dtype, as_torch, dev)
        if lhs is not None and code != OP_COPY_RHS:
            replay = replay and not _line_rows_pay(lt.shape[0], dl, num_edges, dtype)
            lined = _line_rows(lhs, lt.shape[0], dl, num_edges, dtype)
            if lined is not None:
                lhs = lined
                flags |= _lib.LHS_LINE_ROWS
        packed, slabs = _lanes(code, dl, dr, dout, sp, lhs, rhs, flags, dtype)
        local = None
        if slabs > 1:
            local = g._local()
        if local:
            # wide rows on a graph whose sources lie near their destinations
            flags |= _lib.NARROW_SLABS
            packed, slabs = _lanes(code, dl, dr, dout, sp, lhs, rhs, flags, dtype)
        sched = csr.chunks
        if narrow_split and packed and narrow_split < sched.chunk_len:
            sched = csr.chunks_for(narrow_split)
        if rhs is not None and code not in (OP_COPY_LHS, OP_COPY_RHS) and dr == 1 \
                and num_edges and (slabs > 1 or (not packed and num_edges >= CSR_ORDER_MIN_EDGES)):
            # a scalar edge operand read by several column slabs: put it in
            # CSR slot order once, so every slab streams it; also for rows of
            # one whole-wavefront slab, whose walk would otherwise wait on a
            # gather by edge id every 64 slots (256 columns: 3-7 % faster;
            # packed rows, several to a wavefront, do better without it)
            perm = torch.empty(num_edges, dtype=tdt, device=gdev)
            _lib.check(_lib.lib().mdgl_gather_rows(rhs.data_ptr(), csr.eid.data_ptr(),
                                                   perm.data_ptr(), num_edges, 1, dcode,
                                                   _lib.stream()),
                       "gather_rows")
            rhs = perm
            flags |= _lib.RHS_CSR_ORDER
            replay = False
        ws = None
        nbytes = 0
        if sched.num_chunks:
            nbytes = _lib.lib().mdgl_gspmm_workspace_bytes(sched.num_chunks, dout,
                                                             REDUCERS[reduce_op], dcode)
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=gdev)
        args = [
            csr.indptr.data_ptr(), csr.indices.data_ptr(), csr.eid.data_ptr(), _lib.ptr(lhs),
            _lib.ptr(rhs), out.data_ptr(), num_dst, code, dl, dr, dout, REDUCERS[reduce_op], None,
            nd, lsp, rsp, _lib.ptr(arg_u), _lib.ptr(arg_e), _lib.ptr(sched.chunk_row),
            _lib.ptr(sched.chunk_start), sched.num_chunks, sched.chunk_len,
            _lib.ptr(sched.heavy_rows), _lib.ptr(sched.heavy_ptr), sched.num_heavy, _lib.ptr(ws),
            nbytes, flags, dcode, _lib.stream()]
        if num_edges == 0:
            _edge_buffers_non_null(args, (1, 2, 4))
            replay = False
        _lib.check(_lib.lib().mdgl_gspmm(*args), "gspmm")
        if replay:
            launch = _Launch()
            launch.csr, launch.sp, launch.local = csr, sp, local
            launch.shape, launch.tdt, launch.gdev, launch.dev = shape, tdt, gdev, dev
            launch.arg, launch.arg_dtype, launch.nbytes = arg, arg_dtype, nbytes
            for i in (_A_LHS, _A_RHS, _A_OUT, _A_ARG_U, _A_ARG_E, _A_WS, _A_STREAM):
                args[i] = None
            launch.args = tuple(args)
            if len(g._launches) >= _LAUNCHES_MAX:
                g._launches.clear()
            g._launches[key] = launch
    if arg:
        arg_u = arg_u.to(arg_dtype)
        arg_e = arg_e.to(arg_dtype)
    return out, arg_u, arg_e, as_torch, dev


def _edge_buffers_non_null(args, positions):
    """On a graph without edges no row has a slot, so the kernels read no
    edge data; the ABI still takes the edge buffers (empty GPU tensors, whose
    address is 0) as non-null pointers: the CSR's indptr stands in."""
    for i in positions:
        if not args[i]:
            args[i] = args[0]


def _run_rows(csr, rows, code, reduce_op, lhs, rhs, out, arg_u, arg_e, dl, dr, dout, nd, lsp,
              rsp, flags, dcode, arg, arg_dtype, as_torch, dev):
    """The listed rows of a gspmm over `csr` (mdgl_gspmm_rows), into the
    zero-filled results."""
    args = [csr.indptr.data_ptr(), csr.indices.data_ptr(), csr.eid.data_ptr(), _lib.ptr(lhs),
            _lib.ptr(rhs), out.data_ptr(), out.shape[0], code, dl, dr, dout,
            REDUCERS[reduce_op], None, nd, lsp, rsp, _lib.ptr(arg_u), _lib.ptr(arg_e),
            rows.data_ptr(), rows.shape[0], flags, dcode, _lib.stream()]
    if csr.eid.shape[0] == 0:
        _edge_buffers_non_null(args, (1, 2, 4))
    _lib.check(_lib.lib().mdgl_gspmm_rows(*args), "gspmm_rows")
    if arg:
        arg_u = arg_u.to(arg_dtype)
        arg_e = arg_e.to(arg_dtype)
    return out, arg_u, arg_e, as_torch, dev


def _mul_sum_dot(g, grad, y, x, kind="out"):
    """Both gradients of a u_mul_e_sum whose edge operand `y` is constant
    over trailing groups of the node operand `x`, in one pass over the `kind`
    CSR (mdgl_gspmm_mul_sum_dot): returns (dx, dy) as GPU tensors shaped like
    x and y, or None when the shapes do not fit the fused kernel (the caller
    then runs gspmm and gsddmm)."""
    G = grad.contiguous()
    X = x.contiguous()
    # y as (E, *x's leading feature axes, 1): the same rank as the node rows
    Y = y.contiguous().reshape((y.shape[0],) + tuple(x.shape[1:-1]) + (1,))
    if not (G.dtype == X.dtype == Y.dtype and G.dtype in (torch.float32, torch.float64)
            and G.is_cuda and X.is_cuda and Y.is_cuda):
        return None
    dtype = np.float32 if G.dtype == torch.float32 else np.float64
    nd, _lsa, _rsa, lsp, rsp, _ = shape_ptrs(G.shape, Y.shape)
    dout = width(G.shape)
    dr = width(Y.shape)
    num_rows = g.number_of_nodes()
    E = g.number_of_edges()
    if X.shape != G.shape or Y.shape[0] != E or G.shape[0] != num_rows or dr == 0:
        return None
    if E == 0:  # no messages: both gradients are zero
        return torch.zeros_like(x), torch.zeros_like(y)
    csr = g._device_csr(kind)
    sched = csr.chunks
    gdev = _lib.device()
    dx = torch.empty((num_rows, dout), dtype=G.dtype, device=gdev)
    dot = torch.empty((E, dr), dtype=G.dtype, device=gdev)
    nbytes = _lib.lib().mdgl_gspmm_workspace_bytes(sched.num_chunks, dout, REDUCERS["sum"],
                                                     _lib.dtype_code(dtype))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gdev) if nbytes else None
    rc = _lib.lib().mdgl_gspmm_mul_sum_dot(
        csr.indptr.data_ptr(), csr.indices.data_ptr(), csr.eid.data_ptr(), G.data_ptr(),
        Y.data_ptr(), X.data_ptr(), dx.data_ptr(), dot.data_ptr(), num_rows, dout, dr, dout, nd,
        lsp, rsp, _lib.ptr(sched.chunk_row), _lib.ptr(sched.chunk_start),
        sched.num_chunks, sched.chunk_len, _lib.ptr(sched.heavy_rows), _lib.ptr(sched.heavy_ptr),
        sched.num_heavy, _lib.ptr(ws), nbytes, _lib.dtype_code(dtype), _lib.stream())
    if rc == _lib.ENOTSUP:
        return None
    _lib.check(rc, "gspmm_mul_sum_dot")
    # the edge gradient came out in CSR slot order: gather it to edge-id order
    dy = torch.empty((E, dr), dtype=G.dtype, device=gdev)
    if E:
        _lib.check(_lib.lib().mdgl_gather_rows(dot.data_ptr(), csr.slot_of_eid().data_ptr(),
                                               dy.data_ptr(), E, dr, _lib.dtype_code(dtype),
                                               _lib.stream()), "gather_rows")
    return dx.reshape(x.shape), dy.reshape(y.shape)


def gspmm(g, op, reduce_op, lhs_data, rhs_data):
    r"""Generalized Sparse Matrix Multiplication interface.
    It fuses two steps into one kernel.

    1. Computes messages by :attr:`op` source node and edge features.
    2. Aggregate the messages by :attr:`reduce_op` as the features on destination nodes.

    .. math::
        x_v = \psi_{(u, v, e) \in \mathcal{G}}(\rho(x_u, x_e))

    Parameters
    ----------
    g : DGLGraph
    op : str
        ``add``, ``sub``, ``mul``, ``div``, ``copy_lhs`` or ``copy_rhs``.
    reduce_op : str
        ``sum``, ``max``, ``min`` or ``mean``.
    lhs_data, rhs_data : numpy array, torch tensor or None
        Source-node and edge operands (None when the op does not read it).

    Returns
    -------
    Node features of shape ``(N,) + broadcast feature shape``. A node with no
    in-edges gets 0 (sum, mean), -inf (max) or +inf (min). With torch tensors
    that require grad the result takes part in autograd.
    """
    if _autograd.needs_grad(lhs_data, rhs_data):
        return _autograd.GSpMM.apply(g, op, reduce_op, lhs_data, rhs_data, False)
    out, _, _, as_torch, dev = _run(g, op, reduce_op, lhs_data, rhs_data)
    return _lib.give_back(out, as_torch, dev)


def _gspmm(g, op, reduce_op, lhs_data, rhs_data):
    """gspmm that also returns ``(arg_u, arg_e)`` for max/min (else ``(None, None)``).

    arg_u / arg_e hold, per output element, the source node and the edge id
    of the message selected by max/min: the first in CSR order (smallest edge
    id) among equal values; -1 where no message was selected (a node with no
    in-edges, or only messages that never beat the identity).
    """
    out, au, ae, as_torch, dev = _run(g, op, reduce_op, lhs_data, rhs_data, want_arg=True)
    res = _lib.give_back(out, as_torch, dev)
    if au is None:
        return res, (None, None)
    return res, (_lib.give_back(au, as_torch, dev), _lib.give_back(ae, as_torch, dev))


def _gen_spmm_func(binary_op, reduce_op):
    name = "u_{}_e_{}".format(binary_op, reduce_op)

    def func(g, x, y):
        return gspmm(g, binary_op, reduce_op, x, y)

    func.__name__ = name
    func.__qualname__ = name
    func.__doc__ = (
        "Generalized SpMM function: messages {op} of source node features `x` and edge "
        "features `y`, aggregated by {red} on destination nodes. Feature shapes broadcast "
        "with NumPy's rules.{zero}\n").format(op=binary_op, red=reduce_op, zero=_zero_note(
            reduce_op))
    return func


def _gen_copy_reduce_func(binary_op, reduce_op):
    name = "{}_{}".format(binary_op, reduce_op)

    def func(g, x):
        if binary_op == "copy_u":
            return gspmm(g, "copy_lhs", reduce_op, x, None)
        return gspmm(g, "copy_rhs", reduce_op, None, x)

    what = "source node" if binary_op == "copy_u" else "edge"
    func.__name__ = name
    func.__qualname__ = name
    func.__doc__ = ("Generalized SpMM function: {w} features `x` as messages, aggregated by "
                    "{red} on destination nodes.{zero}\n").format(w=what, red=reduce_op,
                                                                  zero=_zero_note(reduce_op))
    return func


def _zero_note(reduce_op):
    if reduce_op in ("max", "min"):
        return (" A node with no in-edges gets {}inf here; update_all replaces it with "
                "zero.".format("-" if reduce_op == "max" else "+"))
    return " A node with no in-edges gets zero."


def _register_spmm_func():
    for binary_op in ("add", "sub", "mul", "div", "copy_u", "copy_e"):
        for reduce_op in ("sum", "max", "min", "mean"):
            if binary_op.startswith("copy"):
                func = _gen_copy_reduce_func(binary_op, reduce_op)
            else:
                func = _gen_spmm_func(binary_op, reduce_op)
            setattr(sys.modules[__name__], func.__name__, func)
            __all__.append(func.__name__)


_register_spmm_func()
