"""Segment operators (reference python/mojodgl/ops/segment.py).

segment_reduce, segment_softmax and segment_mm with the reference's
arguments, validation and empty-segment conventions; values keep their
float32/float64 dtype. The offsets ([0] + cumsum(seglen)) are formed where
the lengths live: host lengths are validated and summed on the host and
uploaded as int32; GPU lengths stay on the GPU and are validated there with
one small read back.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .. import _lib
from .._lib import REDUCERS
from ..base import DGLError
from . import _autograd, _plan

__all__ = ["segment_reduce", "segment_softmax", "segment_mm"]


def _offsets(seglen: np.ndarray) -> np.ndarray:
    out = np.zeros(seglen.size + 1, dtype=np.int64)
    np.cumsum(seglen, out=out[1:])
    return out


def _check_lengths(seglen: np.ndarray, n: int) -> None:
    """Each length in [0, n]: with that, the int64 offsets cannot wrap
    around, so a sum that lands on n is the true sum."""
    if seglen.size and (int(seglen.min()) < 0 or int(seglen.max()) > n):
        raise DGLError(
            "segment lengths must be non-negative and sum to {}, got lengths in [{}, {}]".format(
                n, int(seglen.min()), int(seglen.max())))


def _check_offsets(offsets, n):
    if offsets.size and (int(offsets[-1]) != n or bool(np.any(np.diff(offsets) < 0))):
        raise DGLError(
            "segment lengths must be non-negative and sum to {}, got offsets ending at {} for "
            "{} rows".format(n, int(offsets[-1]) if offsets.size else 0, n))


class _Segments:
    """Validated segments: `off` is the int32 GPU offsets tensor, `host` the
    int64 host offsets when the lengths came from the host (None when they
    were a GPU tensor, whose offsets are formed and checked on the GPU with
    one small read back), `heavy` the number of chunks of `chunk_len` rows
    the segments longer than `chunk_len` split into (GPU lengths only),
    `longest` the largest length.

    With `defer` the checks of GPU lengths come back later: the caller may
    queue kernels that read the offsets (they clamp every offset into the
    rows, so invalid lengths cannot send them out of bounds) and must call
    verify() before it returns anything; until then `longest` is None. The
    figures are then copied on a side stream behind the offsets kernel, so
    the caller's kernels do not queue behind the copy."""

    def __init__(self, seglen, n, chunk_len=None, defer=False):
        self._pending = None
        self._stats = None
        if isinstance(seglen, torch.Tensor) and seglen.device.type == "cuda":
            sl = _lib.i64_device(seglen).reshape(-1)
            self.num = sl.numel()
            self.host = None
            self.heavy = 0
            if n >= 2 ** 31:
                raise DGLError("segment operators take fewer than 2**31 rows, got {}".format(n))
            # offsets and the checks' figures in one pass (mdgl_segment_offsets),
            # then one small read back
            dev = sl.device
            off = torch.empty(self.num + 1, dtype=torch.int32, device=dev)
            stats = torch.empty(4, dtype=torch.int64, device=dev)
            L = _lib.lib()
            nbytes = L.mdgl_segment_offsets_workspace_bytes(self.num)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes > 0 else None
            _lib.check(L.mdgl_segment_offsets(sl.data_ptr(), self.num, chunk_len or 0,
                                              off.data_ptr(), stats.data_ptr(), _lib.ptr(ws),
                                              max(nbytes, 0), _lib.stream()),
                       "segment_offsets")
            self.off = off
            self.longest = None
            self._n, self._chunked = n, chunk_len is not None
            if defer:
                self._ready = torch.cuda.Event()
                self._ready.record()
                self._stats = stats
            else:
                self._check(stats.tolist())
        else:
            sl = _lib.i64(seglen)
            self.num = sl.size
            _check_lengths(sl, n)
            self.longest = int(sl.max()) if sl.size else 0
            self.host = _offsets(sl)
            _check_offsets(self.host, n)
            self.off = None

    def _check(self, figures):
        low, total, heavy, high = figures
        n = self._n
        # every length in [0, n] first: then the total cannot have wrapped
        if low < 0 or high > n or total != n:
            raise DGLError(
                "segment lengths must be non-negative and sum to {}, got lengths in "
                "[{}, {}] summing to {}".format(n, low, high, total))
        if self._chunked:
            self.heavy = heavy
        self.longest = high

    def start_check(self):
        """Start the read back of a deferred check (after the caller queued
        its kernels; a no-op otherwise)."""
        if self._stats is not None:
            stats, self._stats = self._stats, None
            self._pending = _lib.Readback(stats, "segment_offsets", after=self._ready)

    def verify(self):
        """Finish a deferred check (a no-op otherwise)."""
        self.start_check()
        if self._pending is not None:
            pending, self._pending = self._pending, None
            self._check(pending.values())

    def device(self):
        if self.off is None:
            self.off = _lib.i32_device(self.host)
        return self.off


def _flat_width(shape):
    return 1 if len(shape) < 2 else int(math.prod(shape[1:]))


def segment_reduce(seglen, value, reducer="sum"):
    """Segment reduction operator.

    It aggregates the value tensor along the first dimension by segments.
    The first argument ``seglen`` stores the length of each segment. Its
    summation must be equal to the first dimension of the ``value`` tensor.
    Zero-length segments are allowed.

    Parameters
    ----------
    seglen : array or tensor of segment lengths
    value : array or tensor to aggregate
    reducer : 'sum', 'max', 'min' or 'mean'

    Returns
    -------
    Aggregated values of shape ``(len(seglen), value.shape[1:])`` (a 1-D value
    gives ``(len(seglen), 1)``). Empty segments give 0 for every reducer.
    With a torch tensor that requires grad the result takes part in autograd
    (max / min pass the gradient to the selected row).

    Examples
    --------
    >>> val = np.ones((10, 3))
    >>> seg = np.array([1, 0, 5, 4])
    >>> segment_reduce(seg, val)
    array([[1., 1., 1.],
           [0., 0., 0.],
           [5., 5., 5.],
           [4., 4., 4.]])
    """
    if reducer not in ("sum", "max", "min", "mean"):
        raise DGLError("reducer {} not recognized.".format(reducer))
    if _autograd.needs_grad(value):
        return _autograd.SegmentReduce.apply(seglen, value, reducer)
    return _segment_reduce(seglen, value, reducer)[0]


def _segment_reduce(seglen, value, reducer, want_arg=False):
    """segment_reduce returning (result, validated segments, arg): arg is the
    (num_seg, d) int32 row of each max / min with `want_arg`, else None."""
    V = _lib.feature(value)
    n = V.shape[0] if V.ndim else 0
    d = _flat_width(V.shape)
    fshape = tuple(V.shape[1:]) if V.ndim > 1 else (1,)
    dtype = V.dtype
    on_gpu = isinstance(seglen, torch.Tensor) and seglen.device.type == "cuda"
    if not on_gpu:
        seg = _Segments(seglen, n)  # host lengths: checked before any GPU work
    gdev = _lib.device()
    num_seg = seglen.numel() if on_gpu else seg.num
    # the output and the value block first, so that the offsets kernels of GPU
    # lengths and the reduction are queued back to back
    out = torch.empty((num_seg, d), dtype=_lib.torch_dtype(dtype), device=gdev)
    val = _lib.on_device(V, dtype) if num_seg and d else None
    if on_gpu:
        # their checks come back while the reduction runs
        seg = _Segments(seglen, n, defer=True)
    arg = None
    if num_seg and d:
        off = seg.device()
        L = _lib.lib()
        flags = _lib.REPLACE_INF if reducer in ("max", "min") else 0
        if seg.longest is None:
            # longest length not known yet: segments over the split length
            # are left for a second call, made once the check is back
            flags |= _lib.SEGMENTS_SKIP_LONG
        elif seg.longest <= _lib.SEGMENT_SPLIT_ROWS:
            flags |= _lib.SEGMENTS_SHORT  # no split pass needed
        if want_arg and reducer in ("max", "min"):
            arg = torch.empty((num_seg, d), dtype=torch.int32, device=gdev)

        def run(fl):
            if arg is not None:
                return L.mdgl_segment_reduce_arg(off.data_ptr(), val.data_ptr(), out.data_ptr(),
                                                 arg.data_ptr(), num_seg, d, REDUCERS[reducer], n,
                                                 fl, _lib.dtype_code(dtype), _lib.stream())
            return L.mdgl_segment_reduce(off.data_ptr(), val.data_ptr(), out.data_ptr(), num_seg,
                                         d, REDUCERS[reducer], n, fl, _lib.dtype_code(dtype),
                                         _lib.stream())

        _lib.check(run(flags), "segment_reduce")
        seg.verify()  # raises for invalid GPU lengths before anything is returned
        if flags & _lib.SEGMENTS_SKIP_LONG and seg.longest > _lib.SEGMENT_SPLIT_ROWS:
            _lib.check(run((flags & ~_lib.SEGMENTS_SKIP_LONG) | _lib.SEGMENTS_LONG_ONLY),
                       "segment_reduce")
    seg.verify()
    return _lib.give_back(out.reshape((num_seg,) + fshape), V.is_torch, V.device), seg, arg


def segment_softmax(seglen, value):
    """Softmax over the rows of each segment, per column.

    The first argument ``seglen`` stores the length of each segment. Its
    summation must be equal to the first dimension of the ``value`` tensor.
    Zero-length segments are allowed.

    Returns
    -------
    Result of the same shape as ``value``. With a torch tensor that requires
    grad the result takes part in autograd.
    """
    if _autograd.needs_grad(value):
        return _autograd.SegmentSoftmax.apply(seglen, value)
    return _segment_softmax(seglen, value)[0]


def _segment_softmax(seglen, value):
    """segment_softmax returning (result, validated segments)."""
    V = _lib.feature(value)
    shape = V.shape
    n = shape[0] if len(shape) else 0
    d = _flat_width(shape)
    dtype = V.dtype
    on_gpu = isinstance(seglen, torch.Tensor) and seglen.device.type == "cuda"
    if not on_gpu:
        seg = _Segments(seglen, n)  # host lengths: checked before any GPU work
    gdev = _lib.device()
    # every row lies in one segment, so the kernel writes all of `out`
    out = torch.empty((n, d), dtype=_lib.torch_dtype(dtype), device=gdev)
    val = _lib.on_device(V, dtype).reshape(n, d) if n and d else None
    slots = chunk_len = None
    if val is not None:
        slots, chunk_len = _plan.geometry(d, dtype, val, out)
    if on_gpu:
        seg = _Segments(seglen, n, chunk_len, defer=True)
        if seg.num and n and d:
            # start without the longest length: the staged kernel takes every
            # segment of at most chunk_len rows; a longer one (known once the
            # check is back) sends the call through the chunk plan below,
            # which rewrites every row
            rc = _lib.lib().mdgl_segment_softmax_short(
                seg.off.data_ptr(), val.data_ptr(), out.data_ptr(), seg.num, d, n,
                _lib.dtype_code(dtype), _lib.stream())
            seg.verify()
            if rc != _lib.ENOTSUP:
                _lib.check(rc, "segment_softmax")
                if seg.heavy == 0:
                    return _lib.give_back(out.reshape(shape), V.is_torch, V.device), seg
        seg.verify()
    num_seg = seg.num
    if num_seg and n and d:
        off = seg.device()
        # segments in their own order, one wavefront each (a degree-sorted
        # plan costs more to build per call than it saves here)
        if seg.host is not None:
            plan = _plan.SoftmaxPlan(seg.host, slots, chunk_len, ordered=False)
        else:
            plan = _plan.SoftmaxPlan.from_device(seg.off, slots, chunk_len, ordered=False,
                                                 num_chunks=seg.heavy)
        ws, nbytes = _plan.workspace(plan, d, dtype)
        rc = _lib.lib().mdgl_segment_softmax(
            off.data_ptr(), val.data_ptr(), out.data_ptr(), None, num_seg, d, n,
            _lib.ptr(plan.order), plan.bounds_ptr(), plan.nbins, _lib.ptr(plan.packed),
            _lib.ptr(plan.chunk_row), _lib.ptr(plan.chunk_start), _lib.ptr(plan.chunk_first),
            plan.num_chunks, plan.slots, _lib.ptr(ws), nbytes, _lib.dtype_code(dtype),
            _lib.stream())
        _lib.check(rc, "segment_softmax")
    return _lib.give_back(out.reshape(shape), V.is_torch, V.device), seg


def _grouped_mm(a, b, idx_b, seglen, gather, covered):
    """Launch the grouped GEMM; returns the (n, d2) GPU tensor. The kernel
    writes the first `covered` rows (every row of a group); the rest are
    zeroed here."""
    n, d1 = a.shape
    r, _, d2 = b.shape
    dtype = _lib.common_dtype(a, b)
    gdev = _lib.device()
    tdt = _lib.torch_dtype(dtype)
    out = torch.empty((n, d2), dtype=tdt, device=gdev)
    if covered < n:
        out[covered:].zero_()
    if covered == 0 or d2 == 0:
        return out
    A = _lib.on_device(a, dtype)
    B = _lib.on_device(b, dtype)
    code = _lib.dtype_code(dtype)
    L = _lib.lib()
    if gather:
        nbytes = L.mdgl_gather_mm_workspace_bytes(n, d1, d2, r, code)
    else:
        nbytes = L.mdgl_segment_mm_workspace_bytes(n, d1, d2, r, code)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=gdev)
    if gather:
        idx = idx_b
        rc = L.mdgl_gather_mm(A.data_ptr(), B.data_ptr(), idx.data_ptr(), out.data_ptr(), n, d1,
                              d2, r, ws.data_ptr(), nbytes, code, _lib.stream())
        _lib.check(rc, "gather_mm")
    else:
        sl = torch.as_tensor(seglen, dtype=torch.int64).to(gdev).contiguous()
        rc = L.mdgl_segment_mm(A.data_ptr(), B.data_ptr(), out.data_ptr(), sl.data_ptr(), n, d1, r,
                               d2, ws.data_ptr(), nbytes, code, _lib.stream())
        _lib.check(rc, "segment_mm")
    return out


def segment_mm(a, b, seglen_a):
    r"""Performs matrix multiplication according to segments.

    Suppose ``seglen_a == [10, 5, 0, 3]``, the operator will perform
    four matrix multiplications::

        a[0:10] @ b[0], a[10:15] @ b[1],
        a[15:15] @ b[2], a[15:18] @ b[3]

    Parameters
    ----------
    a : (N, D1) array or tensor
    b : (R, D1, D2) array or tensor
    seglen_a : (R,) integer lengths, non-negative, summing to at most N

    Returns
    -------
    The (N, D2) product; rows past ``sum(seglen_a)`` are zero. With torch
    tensors that require grad the result takes part in autograd.
    """
    if _autograd.needs_grad(a, b):
        return _autograd.SegmentMM.apply(a, b, seglen_a)
    return _segment_mm(a, b, seglen_a)[0]


def _segment_mm(a, b, seglen_a):
    """segment_mm returning (result, seglen as int64 numpy, rows covered)."""
    A = _lib.feature(a)
    B = _lib.feature(b)
    if A.ndim != 2 or B.ndim != 3:
        raise DGLError("segment_mm wants a 2-D left operand and a 3-D right operand")
    n, d1 = A.shape
    r, b_d1, d2 = B.shape
    if b_d1 != d1:
        raise DGLError("inner dimensions do not match: {} vs {}".format(d1, b_d1))
    seglen_a = _lib.i64(seglen_a)
    if seglen_a.size != r:
        raise DGLError("seglen_a must have one entry per b block: {} != {}".format(
            seglen_a.size, r))
    if seglen_a.size:
        lo, hi = int(seglen_a.min()), int(seglen_a.max())
        # each length in [0, n] before the sum: no int64 wrap-around
        total = int(seglen_a.sum()) if hi <= n else n + 1
        if lo < 0 or hi > n or total > n:
            raise DGLError(
                "segment lengths must be non-negative and sum to {}, got a minimum of {} and a "
                "sum of {}".format(n, lo, total))
    covered = total if r else 0
    out = _grouped_mm(A, B, None, seglen_a, gather=False, covered=covered)
    return _lib.give_back(out, _lib.wants_torch(A, B), _lib.out_device(A, B)), seglen_a, covered


def _replace_inf_with_zero(x):
    """+-inf -> 0, elementwise (reference segment.py:55-59), through the GPU kernel."""
    X = _lib.feature(x)
    dtype = X.dtype
    t = _lib.on_device(X, dtype)
    out = torch.empty_like(t)
    rc = _lib.lib().mdgl_replace_inf_with_zero(t.data_ptr(), out.data_ptr(), t.numel(),
                                               _lib.dtype_code(dtype), _lib.stream())
    _lib.check(rc, "replace_inf_with_zero")
    return _lib.give_back(out, X.is_torch, X.device)
