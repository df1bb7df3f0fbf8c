"""gather_mm (reference python/mojodgl/ops/gather_mm.py).

Same arguments and validation. Both of the reference's routes are kept and
give the same numbers: above `_SEGMENT_BLOCK` (D1 * D2) the rows are grouped
by `idx_b` (stably, as the reference's argsort: libmdgl's radix grouping,
mdgl_build_csr), gathered in that order, multiplied with segment_mm and put
back (mdgl_gather_rows / mdgl_scatter_rows), as the reference does;
otherwise one mdgl_gather_mm call buckets the rows on the GPU and multiplies
them block by block on the matrix cores.
"""

from __future__ import annotations

import os

import torch

from .. import _lib
from ..base import DGLError
from . import _autograd
from .segment import _grouped_mm

__all__ = ["gather_mm"]

# D1 * D2 above which the sorted segment_mm route is taken (the reference's
# switch, overridable by the same environment variable).
_SEGMENT_BLOCK = int(os.environ.get("MOJODGL_GATHER_MM_SEGMENT_BLOCK", 16384))
# b blocks the bucketed route takes (mdgl_gather_mm keeps 5 ints per block in
# LDS); more go the sorted route
GATHER_MAX_BLOCKS = 2048


def group_rows(idx: torch.Tensor, num_groups: int):
    """(perm, seglen) of the rows grouped by `idx` (a GPU int64 tensor with
    values in [0, num_groups)): perm (int32) lists the rows of group 0, then
    of group 1, ..., each group in row order -- numpy's stable argsort of idx
    -- and seglen (int64) the group sizes; by libmdgl's stable radix
    grouping (mdgl_build_csr with idx as the key)."""
    from ..heterograph import build_device_csr

    indptr, _, perm = build_device_csr(idx.to(torch.int32), None, num_groups)
    return perm, (indptr[1:] - indptr[:-1]).to(torch.int64)


def move_rows(x: torch.Tensor, perm: torch.Tensor, scatter: bool = False) -> torch.Tensor:
    """Rows of the 2-D GPU tensor x taken in `perm`'s order (out[i] = x[perm[i]],
    mdgl_gather_rows) or put back (out[perm[i]] = x[i], mdgl_scatter_rows)."""
    x = x.contiguous()
    out = torch.empty_like(x)
    n, width = x.shape
    code = _lib.FLOAT32 if x.dtype == torch.float32 else _lib.FLOAT64
    L = _lib.lib()
    fn = L.mdgl_scatter_rows if scatter else L.mdgl_gather_rows
    _lib.check(fn(x.data_ptr(), perm.data_ptr(), out.data_ptr(), n, width, code, _lib.stream()),
               "scatter_rows" if scatter else "gather_rows")
    return out


def gather_mm(a, b, *, idx_b):
    r"""Gather data according to the given indices and perform matrix multiplication.

    Let the result tensor be ``c``, the operator conducts the following computation:

      c[i] = a[i] @ b[idx_b[i]]
      , where len(c) == len(idx_b)

    Parameters
    ----------
    a : (N, D1) array or tensor
    b : (R, D1, D2) array or tensor
    idx_b : (N,) integer indices into the first axis of b

    Returns
    -------
    The (N, D2) product. With torch tensors that require grad the result
    takes part in autograd.
    """
    if _autograd.needs_grad(a, b):
        return _autograd.GatherMM.apply(a, b, idx_b)
    return _gather_mm(a, b, idx_b)[0]


def _gather_mm(a, b, idx_b):
    """gather_mm returning (result, idx_b as a GPU int64 tensor)."""
    A = _lib.feature(a)
    B = _lib.feature(b)
    if A.ndim != 2 or B.ndim != 3:
        raise DGLError("gather_mm wants a 2-D and a 3-D operand")
    N, D1 = A.shape
    R, b_d1, D2 = B.shape
    if b_d1 != D1:
        raise DGLError("inner dimensions do not match: a is {} wide, b blocks are {}".format(
            D1, b_d1))
    # GPU indices are checked on the GPU (their minimum and maximum read
    # back); host indices on the host, before any GPU work
    on_gpu = isinstance(idx_b, torch.Tensor) and idx_b.device.type == "cuda"
    idx = _lib.i64_device(idx_b) if on_gpu else _lib.i64(idx_b)
    if idx.ndim != 1 or idx.shape[0] != N:
        raise DGLError("idx_b must be 1-D with one index per row of a: got shape {} for "
                       "N={}".format(tuple(idx.shape), N))
    sorted_route = D1 * D2 > _SEGMENT_BLOCK or R > GATHER_MAX_BLOCKS
    pending = None
    if N:
        if on_gpu:
            pending = _lib.Readback(torch.stack(torch.aminmax(idx)), "gather_mm_range")
            if sorted_route:  # the grouping needs valid keys: check first
                _check_range(pending.values(), R)
                pending = None
        else:
            _check_range((int(idx.min()), int(idx.max())), R)
    if not on_gpu:
        idx = torch.from_numpy(idx).to(_lib.device())
    as_torch, dev = _lib.wants_torch(A, B), _lib.out_device(A, B)
    if sorted_route:
        # the rows grouped by block in a stable order: the reference's stable
        # host argsort (gather_mm.py:79-87), on the GPU
        perm, seglen = group_rows(idx, R)
        a_sorted = move_rows(_lib.on_device(A, _lib.common_dtype(A, B)), perm)
        out_sorted = _grouped_mm(_lib.Feat(a_sorted, True, _lib.device()), B, None, seglen,
                                 gather=False, covered=N)
        out = move_rows(out_sorted, perm, scatter=True)
    else:
        # the bucketing counts and places only indices in [0, R), so the
        # kernels may run before the range comes back
        out = _grouped_mm(A, B, idx, None, gather=True, covered=N)
        if pending is not None:
            _check_range(pending.values(), R)
    return _lib.give_back(out, as_torch, dev), idx


def _check_range(lo_hi, R):
    lo, hi = lo_hi
    if lo < 0 or hi >= R:
        raise DGLError("idx_b must be in [0, {}), got [{}, {})".format(R, lo, hi + 1))
