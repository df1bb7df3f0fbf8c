"""Backward passes of gspmm, gsddmm and edge_softmax for torch autograd.

The reference has no backward pass (its README.md:110-114 leaves autograd out);
these follow the calculus of the forward ops and run on the same kernels:

* gspmm(op, reduce) with node operand X, edge operand Y, output gradient G:
  - sum / mean: the gradient reaching edge e = (u, v) is G[v] (divided by
    max(deg v, 1) for mean: ``mdgl_rows_by_degree`` on G first); for mul
    with an edge operand constant over x's last axis (attention weights),
    dX and dY come from one pass over the out-CSR
    (``mdgl_gspmm_mul_sum_dot``: G[v] gathered once per edge, dY in CSR slot
    order, then gathered to edge order);
    dX[u] = sum over u's out-edges of that gradient times d msg / dX, a
    gspmm over the out-CSR (copy for copy_lhs / add / sub, mul / div by Y for
    mul / div); dY[e] = gradient times d msg / dY, a gsddmm (copy of G[v],
    its negation for sub, X[u] * G[v] for mul -- a per-head dot when Y
    broadcasts over X's trailing axes --, -X[u] G[v] / Y[e]^2 for div);
  - max / min: only the arg edge of an output element receives its
    gradient: ``mdgl_gspmm_edge_grad`` writes the masked per-edge gradient M,
    then dX is a gspmm over the out-CSR of M (times d msg / dX) and dY is M
    times d msg / dY, per edge;
* gsddmm(op, X at target tx, Y at target ty): the per-edge gradient times
  d op / dX (dY) is reduced over the edges of each node of the operand's
  target by a gspmm copy_rhs sum (in-CSR for v, out-CSR for u; nothing for e);
* edge_softmax: dX = a * (G - s[row]) with s[row] = sum over the row of G * a:
  gsddmm e_mul_e, gspmm copy_rhs sum over the CSR of norm_by, then
  ``mdgl_edge_softmax_grad`` (the subtraction and product in one pass); over a
  subset of eids the rows are the forward's groups of positions (their sums by
  ``segment_reduce`` after the products are put in group order), and the rows
  past the selection, constant zero, get zero;
* segment_mm / gather_mm (out[i] = a[i] @ b[g(i)]): da = grad @ b[g]^T on the
  grouped GEMM with the blocks taken transposed, db[g] = sum over g's rows of
  a^T grad per chunk of rows on the matrix cores, chunks added in order
  (``mdgl_segment_mm_grad`` / ``mdgl_gather_mm_grad``);
* segment_reduce / segment_softmax: the segments are CSR rows over the value
  rows themselves (``mdgl_segment_ids`` maps rows to segments): sum / mean /
  max / min as gspmm copy_rhs (max / min through the arg row of
  ``mdgl_segment_reduce_arg``), softmax as edge_softmax.

The backward passes run on the library's kernels, outside torch's graph, so
they are differentiable once: a second derivative through them raises.

Gradients come back in the operand's shape: an operand broadcast along its
trailing feature axes gets its gradient summed over them (a segmented sum,
``segment_reduce``); other broadcast layouts raise DGLError in backward.
Only torch tensors take part (numpy operands have no autograd).
"""

from __future__ import annotations

import math

import numpy as np
import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from ..base import DGLError

__all__ = ["needs_grad", "GSpMM", "GSDDMM", "EdgeSoftmax", "SegmentReduce", "SegmentSoftmax",
           "SegmentMM", "GatherMM"]


def needs_grad(*xs) -> bool:
    return torch.is_grad_enabled() and any(
        isinstance(x, torch.Tensor) and x.requires_grad for x in xs)


def _gpu(t):
    """A saved operand or an incoming gradient on the library's GPU (host
    tensors copied): the backward kernels read device memory only."""
    return None if t is None else t.to(_lib.device())


def _code(t):
    return 0 if t.dtype == torch.float32 else 1


def _scale(t, alpha):
    t = t.contiguous()
    out = torch.empty_like(t)
    _lib.check(_lib.lib().mdgl_scale(t.data_ptr(), out.data_ptr(), t.numel(), float(alpha),
                                     _code(t), _lib.stream()), "scale")
    return out


def _rows_by_degree(csr, x):
    x = x.contiguous()
    out = torch.empty_like(x)
    rows = x.shape[0]
    d = x.numel() // max(rows, 1)
    _lib.check(_lib.lib().mdgl_rows_by_degree(csr.indptr.data_ptr(), x.data_ptr(),
                                              out.data_ptr(), rows, d, _code(x), _lib.stream()),
               "rows_by_degree")
    return out


def _edge_grad(g, grad, arg_e, mean, alpha):
    """Per-edge gradient of a max / min / mean gspmm (see the module doc)."""
    grad = grad.contiguous()
    E = g.number_of_edges()
    d = grad.numel() // max(grad.shape[0], 1)
    out = torch.empty((E,) + tuple(grad.shape[1:]), dtype=grad.dtype, device=grad.device)
    _, vids = g._device_coo()
    csr = g._device_csr("in")
    ae = None if arg_e is None else arg_e.to(torch.int32).contiguous()
    _lib.check(_lib.lib().mdgl_gspmm_edge_grad(
        vids.data_ptr(), csr.indptr.data_ptr(), grad.data_ptr(), _lib.ptr(ae), out.data_ptr(), E,
        d, 1 if mean else 0, float(alpha), _code(grad), _lib.stream()), "gspmm_edge_grad")
    return out


# Rows longer than this are split in the backward passes' reductions when
# several rows share a wavefront (narrow features): on skewed degrees a
# wavefront otherwise waits on its longest row (GAT backward on the power-law
# graph: 24.4 -> 23.3 ms).
NARROW_SPLIT = 64


def _gspmm(g, op, red, x, y, kind="in"):
    from .spmm import _run

    out, _, _, _, _ = _run(g, op, red, x, y, kind=kind, narrow_split=NARROW_SPLIT)
    return out


def _gsddmm(g, op, x, y, tx, ty):
    from .sddmm import gsddmm

    return gsddmm(g, op, x, y, lhs_target=tx, rhs_target=ty)


def _node_reduce(g, p, target):
    """Sum a per-edge tensor over the edges of each node of `target`."""
    if target == "e":
        return p
    return _gspmm(g, "copy_rhs", "sum", None, p, kind="in" if target == "v" else "out")


def _reduce_to(t, shape):
    """Sum `t` (rows, *full) down to `shape` (rows, *part): `part` must equal
    `full` up to trailing axes of size one (after left padding with ones)."""
    shape = tuple(shape)
    if tuple(t.shape) == shape:
        return t
    rows = t.shape[0]
    full = tuple(t.shape[1:])
    part = shape[1:] if len(shape) > 1 else (1,)
    pad = (1,) * (len(full) - len(part)) + tuple(part)
    keep = len(pad)
    while keep > 0 and pad[keep - 1] == 1 and full[keep - 1] != 1:
        keep -= 1
    if pad[:keep] != full[:keep] or any(p != 1 for p in pad[keep:]):
        raise DGLError("backward of an operand broadcast along {} -> {} is not supported "
                       "(only trailing broadcast axes)".format(part, full))
    inner = int(math.prod(full[keep:]))
    from .segment import segment_reduce

    flat = t.contiguous().reshape(-1, 1)
    seg = torch.full((flat.shape[0] // inner,), inner, dtype=torch.int64, device=t.device)
    out = segment_reduce(seg, flat, "sum")
    return out.reshape((rows,) + tuple(shape[1:]))


def _fix_shape(grad, like):
    return grad.reshape(like.shape)


class GSpMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, op, red, x, y, replace_inf):
        from .spmm import _run

        out, _, arg_e, _, dev = _run(g, op, red, x, y, replace_inf=replace_inf,
                                     want_arg=red in ("max", "min"), arg_dtype=torch.int32)
        ctx.g, ctx.op, ctx.red = g, op, red
        ctx.save_for_backward(x if isinstance(x, torch.Tensor) else None,
                              y if isinstance(y, torch.Tensor) else None, arg_e)
        ctx.out_shape = out.shape
        return _lib.give_back(out, True, dev)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        g, op, red = ctx.g, ctx.op, ctx.red
        x0, y0, arg_e = ctx.saved_tensors
        x, y = _gpu(x0), _gpu(y0)
        G = _gpu(grad_out).contiguous()
        need_x = ctx.needs_input_grad[3] and x is not None
        need_y = ctx.needs_input_grad[4] and y is not None
        dx = dy = None
        if red in ("sum", "mean"):
            if red == "mean":
                G = _rows_by_degree(g._device_csr("in"), G)
            if op == "mul" and need_x and need_y:
                # both gradients in one pass over the out-CSR when the edge
                # operand is constant over trailing groups of x (attention)
                from .spmm import _mul_sum_dot

                fused = _mul_sum_dot(g, G, y, x) if _trailing_groups(x, y) else None
                if fused is not None:
                    return None, None, None, _back(fused[0], x0), _back(fused[1], y0), None
            if need_x:
                if op in ("copy_lhs", "add", "sub"):
                    dx = _gspmm(g, "copy_lhs", "sum", G, None, kind="out")
                else:
                    dx = _gspmm(g, op, "sum", G, y, kind="out")
                dx = _reduce_to(dx, _padded(x.shape, dx.shape))
            if need_y:
                if op in ("copy_rhs", "add"):
                    dy = _gsddmm(g, "copy_lhs", G, None, "v", "v")
                elif op == "sub":
                    dy = _scale(_gsddmm(g, "copy_lhs", G, None, "v", "v"), -1.0)
                elif op == "mul":
                    dy = _mul_grad(g, x, G, y.shape)
                else:  # div: -x[u] g[v] / y^2
                    t = _gsddmm(g, "mul", x, G, "u", "v")
                    t = _gsddmm(g, "div", t, y, "e", "e")
                    dy = _scale(_gsddmm(g, "div", t, y, "e", "e"), -1.0)
                dy = _reduce_to(dy, _padded(y.shape, dy.shape))
        else:
            # only the selected edge of each output element receives its
            # gradient (none where nothing was selected or update_all replaced
            # an infinite value: the kernel's arg is -1 there); the terms of
            # the other edges are exactly zero, not 0 times their operand
            M = _edge_grad(g, G, arg_e, False, 1.0)
            if need_x:
                if op in ("copy_lhs", "add", "sub"):
                    p = M
                else:
                    p = _keep_where(M, _gsddmm(g, op, M, y, "e", "e"))
                dx = _reduce_to(_node_reduce(g, p, "u"), _padded(x.shape, M.shape))
            if need_y:
                if op in ("copy_rhs", "add"):
                    dy = M
                elif op == "sub":
                    dy = _scale(M, -1.0)
                elif op == "mul":
                    dy = _keep_where(M, _gsddmm(g, "mul", x, M, "u", "e"))
                else:
                    t = _gsddmm(g, "mul", x, M, "u", "e")
                    t = _gsddmm(g, "div", t, y, "e", "e")
                    dy = _keep_where(M, _scale(_gsddmm(g, "div", t, y, "e", "e"), -1.0))
                dy = _reduce_to(dy, _padded(y.shape, dy.shape))
        if dx is not None:
            dx = dx.reshape(x.shape)
        if dy is not None:
            dy = dy.reshape(y.shape)
        return None, None, None, _back(dx, x0), _back(dy, y0), None


def _keep_where(mask, t):
    """t where mask is non-zero, else exactly 0 (same shape and dtype;
    mdgl_keep_where)."""
    mask, t = mask.contiguous(), t.contiguous()
    out = torch.empty_like(t)
    _lib.check(_lib.lib().mdgl_keep_where(mask.data_ptr(), t.data_ptr(), out.data_ptr(),
                                          t.numel(), _code(t), _lib.stream()), "keep_where")
    return out


def _trailing_groups(x, y):
    """y (E, ...) is x's feature shape with its trailing axes collapsed to
    one (y = (E, *lead, 1) against x = (N, *lead, D))."""
    xs = tuple(x.shape[1:])
    ys = tuple(y.shape[1:]) if y.dim() > 1 else (1,)
    if len(ys) != len(xs) or not xs or ys[-1] != 1 or xs[-1] == 1:
        return False
    return ys[:-1] == xs[:-1]


def _padded(shape, full):
    """`shape` with ones inserted after the first axis to the rank of `full`."""
    shape = tuple(shape)
    if len(shape) == 1:
        shape = shape + (1,)
    nd = len(full)
    if len(shape) < nd:
        shape = (shape[0],) + (1,) * (nd - len(shape)) + shape[1:]
    return shape


def _mul_grad(g, x, G, yshape):
    """dY of a u_mul_e gspmm: x[u] * G[v] per edge, summed over the axes where
    Y broadcasts; when those are X's trailing axes, a per-edge dot."""
    full = G.shape[1:]
    ypad = _padded(yshape, G.shape)[1:]
    keep = len(ypad)
    while keep > 0 and ypad[keep - 1] == 1 and full[keep - 1] != 1:
        keep -= 1
    if keep < len(ypad) and tuple(ypad[:keep]) == tuple(full[:keep]) \
            and tuple(x.shape[1:]) == tuple(full):
        inner = int(math.prod(full[keep:]))
        lead = tuple(full[:keep])
        xs = x.reshape((x.shape[0],) + lead + (inner,))
        gs = G.reshape((G.shape[0],) + lead + (inner,))
        return _gsddmm(g, "dot", xs, gs, "u", "v")
    return _gsddmm(g, "mul", x, G, "u", "v")


class GSDDMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, op, x, y, tx, ty):
        from .sddmm import gsddmm

        out = gsddmm(g, op, x, y, lhs_target=tx, rhs_target=ty)
        ctx.g, ctx.op, ctx.tx, ctx.ty = g, op, tx, ty
        ctx.save_for_backward(x if isinstance(x, torch.Tensor) else None,
                              y if isinstance(y, torch.Tensor) else None)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        g, op, tx, ty = ctx.g, ctx.op, ctx.tx, ctx.ty
        x0, y0 = ctx.saved_tensors
        x, y = _gpu(x0), _gpu(y0)
        G = _gpu(grad_out).contiguous()
        need_x = ctx.needs_input_grad[2] and x is not None
        need_y = ctx.needs_input_grad[3] and y is not None
        dx = dy = None
        if need_x:
            if op in ("copy_lhs", "add", "sub"):
                p = G
            elif op in ("mul", "dot"):
                p = _gsddmm(g, "mul", G, y, "e", ty)
            else:
                p = _gsddmm(g, "div", G, y, "e", ty)
            p = _node_reduce(g, p, tx)
            dx = _reduce_to(p, _padded(x.shape, p.shape)).reshape(x.shape)
        if need_y:
            if op in ("copy_rhs", "add"):
                p = G
            elif op == "sub":
                p = _scale(G, -1.0)
            elif op in ("mul", "dot"):
                p = _gsddmm(g, "mul", G, x, "e", tx)
            else:  # div: -G x / y^2
                t = _gsddmm(g, "mul", G, x, "e", tx)
                t = _gsddmm(g, "div", t, y, "e", ty)
                p = _scale(_gsddmm(g, "div", t, y, "e", ty), -1.0)
            p = _node_reduce(g, p, ty)
            dy = _reduce_to(p, _padded(y.shape, p.shape)).reshape(y.shape)
        return None, None, _back(dx, x0), _back(dy, y0), None, None


def _group_softmax_grad(y, g, row_of, offsets, num_groups, order=None, out=None):
    """dx = y * (g - s[row_of]) for a softmax over groups of rows (y its
    output, g the output gradient, both (k, d) contiguous on the GPU): s[r] is
    the sum of g * y over group r, whose rows are order[offsets[r] ..
    offsets[r + 1]) (int32 positions; None: the rows themselves, groups
    contiguous), folded in that order. Written into `out` when given."""
    k, d = y.shape
    code, st, lib = _code(y), _lib.stream(), _lib.lib()
    p = torch.empty_like(y)
    _lib.check(lib.mdgl_gsddmm(None, None, g.data_ptr(), y.data_ptr(), p.data_ptr(), k,
                               _lib.TARGETS["e"], _lib.TARGETS["e"], _lib.BINARY_OPS["mul"], d,
                               d, d, 0, None, None, code, st), "gsddmm")
    if order is not None:
        pg = torch.empty_like(p)
        _lib.check(lib.mdgl_gather_rows(p.data_ptr(), order.data_ptr(), pg.data_ptr(), k, d, code,
                                        st), "gather_rows")
        p = pg
    s = torch.empty((num_groups, d), dtype=y.dtype, device=y.device)
    _lib.check(lib.mdgl_segment_reduce(offsets.data_ptr(), p.data_ptr(), s.data_ptr(), num_groups,
                                       d, _lib.REDUCERS["sum"], k, 0, code, st), "segment_reduce")
    dx = torch.empty_like(y) if out is None else out
    _lib.check(lib.mdgl_edge_softmax_grad(row_of.data_ptr(), y.data_ptr(), g.data_ptr(),
                                          s.data_ptr(), dx.data_ptr(), k, d, code, st),
               "edge_softmax_grad")
    return dx


def _subset_softmax_grad(grouping, a, grad_out):
    """Gradient of edge_softmax over a subset of eids: position i < k (the
    selection's length) belongs to the group of its endpoint, so
    dx[i] = a[i] * (G[i] - s[endpoint i]) with s the per-group sums of G * a
    (folded in the group's order of appearance); rows past k are zero."""
    L = a.shape[0]
    d = math.prod(a.shape[1:])
    a2 = a.reshape(L, d)
    dx = torch.zeros_like(a2)
    endpoint = grouping.get("endpoint")
    if endpoint is None or endpoint.numel() == 0 or d == 0:
        return dx.reshape(a.shape)
    k = endpoint.numel()
    indptr = grouping["indptr"]
    gk = grad_out.contiguous().reshape(L, d)[:k]
    _group_softmax_grad(a2[:k], gk, endpoint, indptr, indptr.numel() - 1,
                        order=grouping["eid"], out=dx[:k])
    return dx.reshape(a.shape)


def _segment_ids(seg, n):
    """int32 segment of each of the n rows of validated segments `seg`."""
    off = seg.device()
    ids = torch.empty(n, dtype=torch.int32, device=off.device)
    _lib.check(_lib.lib().mdgl_segment_ids(off.data_ptr(), seg.num, n, ids.data_ptr(),
                                           _lib.stream()), "segment_ids")
    return ids


def _flat(shape):
    return 1 if len(shape) < 2 else int(math.prod(shape[1:]))


class SegmentReduce(torch.autograd.Function):
    """segment_reduce with a gradient: row i of segment s receives dout[s]
    (sum), dout[s] / max(len s, 1) (mean), or dout[s][k] when it is the row
    max / min selected for column k (``mdgl_segment_reduce_arg``), through
    ``mdgl_gspmm_edge_grad`` with the segments as CSR rows."""

    @staticmethod
    def forward(ctx, seglen, value, reducer):
        from .segment import _segment_reduce

        out, seg, arg = _segment_reduce(seglen, value, reducer, want_arg=True)
        ctx.seg, ctx.arg, ctx.reducer = seg, arg, reducer
        ctx.vshape, ctx.vdev = tuple(value.shape), value.device
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        seg, vshape = ctx.seg, ctx.vshape
        n = vshape[0] if len(vshape) else 0
        d = _flat(vshape)
        gdev = _lib.device()
        dv = torch.zeros((n, d), dtype=grad_out.dtype, device=gdev)
        if n and d and seg.num:
            G = grad_out.to(gdev).contiguous().reshape(seg.num, d)
            ids = _segment_ids(seg, n)
            _lib.check(_lib.lib().mdgl_gspmm_edge_grad(
                ids.data_ptr(), seg.device().data_ptr(), G.data_ptr(), _lib.ptr(ctx.arg),
                dv.data_ptr(), n, d, 1 if ctx.reducer == "mean" else 0, 1.0, _code(G),
                _lib.stream()), "gspmm_edge_grad")
        return None, dv.reshape(vshape).to(ctx.vdev), None


class SegmentSoftmax(torch.autograd.Function):
    """segment_softmax with a gradient: dx = y * (g - s[segment]) with s the
    per-segment sums of g * y (rows in order)."""

    @staticmethod
    def forward(ctx, seglen, value):
        from .segment import _segment_softmax

        out, seg = _segment_softmax(seglen, value)
        ctx.seg, ctx.vdev = seg, value.device
        ctx.save_for_backward(out)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        (y,) = ctx.saved_tensors
        seg, shape = ctx.seg, tuple(y.shape)
        n = shape[0] if len(shape) else 0
        d = _flat(shape)
        gdev = _lib.device()
        dx = torch.zeros((n, d), dtype=y.dtype, device=gdev)
        if n and d and seg.num:
            Y = y.to(gdev).contiguous().reshape(n, d)
            G = grad_out.to(gdev).contiguous().reshape(n, d)
            dx = _group_softmax_grad(Y, G, _segment_ids(seg, n), seg.device(), seg.num)
        return None, dx.reshape(shape).to(ctx.vdev)


class EdgeSoftmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, logits, norm_by, eids=None):
        from .edge_softmax import _edge_softmax

        keep = None if eids is None else {}
        out = _edge_softmax(g, logits, eids, norm_by, keep)
        ctx.g, ctx.norm_by, ctx.grouping = g, norm_by, keep
        ctx.like = torch.empty(0, dtype=logits.dtype, device=logits.device)
        ctx.save_for_backward(out)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        g, norm_by = ctx.g, ctx.norm_by
        (a0,) = ctx.saved_tensors
        a, grad_out = _gpu(a0), _gpu(grad_out)
        if ctx.grouping is not None:
            dx = _subset_softmax_grad(ctx.grouping, a, grad_out)
            return None, _back(dx, ctx.like), None, None
        E, d = a.shape[0], math.prod(a.shape[1:])
        if E == 0 or d == 0:  # no logits: the gradient is as empty as they are
            return None, _back(torch.zeros_like(a), ctx.like), None, None
        a2 = a.reshape(E, d)
        G = grad_out.contiguous().reshape(E, d)
        p = _gsddmm(g, "mul", G, a2, "e", "e")
        row = "v" if norm_by == "dst" else "u"
        s = _node_reduce(g, p, row).contiguous()
        # dx = a * (G - s[row]) in one pass
        uids, vids = g._device_coo()
        a2 = a2.contiguous()
        dx = torch.empty_like(a2)
        _lib.check(_lib.lib().mdgl_edge_softmax_grad(
            (vids if row == "v" else uids).data_ptr(), a2.data_ptr(), G.data_ptr(), s.data_ptr(),
            dx.data_ptr(), E, a2.shape[1], _code(a2), _lib.stream()), "edge_softmax_grad")
        return None, _back(dx.reshape(a.shape), ctx.like), None, None


def _grouped_grad(a, b, grad_out, seglen, idx, covered, need_a, need_b):
    """(da, db) of out[i] = a[i] @ b[g(i)] (segment_mm with `seglen`, gather_mm
    with `idx`): rows of a past `covered` (in no segment) get zero."""
    from .gather_mm import GATHER_MAX_BLOCKS, group_rows, move_rows

    A, B = _lib.feature(a), _lib.feature(b)
    dtype = _lib.common_dtype(A, B)
    tdt, code, gdev = _lib.torch_dtype(dtype), _lib.dtype_code(dtype), _lib.device()
    Ad, Bd = _lib.on_device(A, dtype), _lib.on_device(B, dtype)
    n, d1 = Ad.shape
    r, _, d2 = Bd.shape
    if covered == 0 or d1 == 0 or d2 == 0 or not (need_a or need_b):
        zeros = (lambda *shape: torch.zeros(shape, dtype=tdt, device=gdev))
        return (zeros(n, d1) if need_a else None), (zeros(r, d1, d2) if need_b else None)
    # the kernels write every row of a group and every element of db
    da = torch.empty((n, d1), dtype=tdt, device=gdev) if need_a else None
    if da is not None and covered < n:
        da[covered:].zero_()
    db = torch.empty((r, d1, d2), dtype=tdt, device=gdev) if need_b else None
    G = grad_out.to(device=gdev, dtype=tdt).contiguous()
    L = _lib.lib()
    if idx is not None and r > GATHER_MAX_BLOCKS:
        # too many blocks to bucket: rows grouped by block (stably), then the
        # segment form, as the forward's sorted route
        perm, sl = group_rows(idx, r)
        da_s, db = _grouped_grad(move_rows(Ad, perm), Bd, move_rows(G, perm), sl, None, n,
                                 need_a, need_b)
        return (move_rows(da_s, perm, scatter=True) if need_a else None), db
    if idx is not None:
        nbytes = L.mdgl_gather_mm_grad_workspace_bytes(n, d1, d2, r, code)
    else:
        nbytes = L.mdgl_segment_mm_grad_workspace_bytes(n, d1, d2, r, code)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=gdev)
    if idx is not None:
        rc = L.mdgl_gather_mm_grad(Ad.data_ptr(), Bd.data_ptr(), idx.data_ptr(), G.data_ptr(),
                                   _lib.ptr(da), _lib.ptr(db), n, d1, d2, r, ws.data_ptr(), nbytes,
                                   code, _lib.stream())
        _lib.check(rc, "gather_mm_grad")
    else:
        sl = torch.as_tensor(seglen, dtype=torch.int64).to(gdev).contiguous()
        rc = L.mdgl_segment_mm_grad(Ad.data_ptr(), Bd.data_ptr(), G.data_ptr(), sl.data_ptr(),
                                    _lib.ptr(da), _lib.ptr(db), n, d1, r, d2, ws.data_ptr(),
                                    nbytes, code, _lib.stream())
        _lib.check(rc, "segment_mm_grad")
    return da, db


def _back(g, like):
    """A gradient in the operand's dtype and on its device (None for numpy)."""
    if g is None or not isinstance(like, torch.Tensor):
        return None
    return g.to(device=like.device, dtype=like.dtype)


def _save_operands(ctx, a, b):
    """Tensors through save_for_backward; a numpy operand (no gradient) kept as is."""
    ta, tb = (x if isinstance(x, torch.Tensor) else None for x in (a, b))
    ctx.save_for_backward(ta, tb)
    ctx.host = (None if ta is not None else a, None if tb is not None else b)


def _saved_operands(ctx):
    ta, tb = ctx.saved_tensors
    return (ta if ta is not None else ctx.host[0]), (tb if tb is not None else ctx.host[1])


class SegmentMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, seglen):
        from .segment import _segment_mm

        out, sl, covered = _segment_mm(a, b, seglen)
        ctx.sl, ctx.covered = sl, covered
        _save_operands(ctx, a, b)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        a, b = _saved_operands(ctx)
        da, db = _grouped_grad(a, b, grad_out, ctx.sl, None, ctx.covered,
                               ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return _back(da, a), _back(db, b), None


class GatherMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, idx_b):
        from .gather_mm import _gather_mm

        out, idx = _gather_mm(a, b, idx_b)
        ctx.idx = idx
        _save_operands(ctx, a, b)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        a, b = _saved_operands(ctx)
        da, db = _grouped_grad(a, b, grad_out, None, ctx.idx, a.shape[0],
                               ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return _back(da, a), _back(db, b), None
