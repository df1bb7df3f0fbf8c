"""CPU oracle for the message-passing kernel layer.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` import this package, and only as what GPU
results are compared against (or as the timed CPU baseline). The product
package `mojodgl` never imports it.

`liboracle.so` (built from `mdgl_oracle.cpp` by `make -C oracle`) restates the
reference's kernels (src/ported.mojo); this module restates the reference's
host-side semantics around them, with numpy:

* graph CSR / CSC construction: python/mojodgl/heterograph.py:69-86
  (bincount, cumsum, stable argsort by endpoint);
* operand reshape: python/mojodgl/ops/sddmm.py:24-47 (`reshape_lhs_rhs`);
* broadcasting: the reference only widens a width-1 operand
  (sddmm.py:62-68); this oracle extends that to NumPy broadcasting through
  offset tables built with `np.broadcast_to` on index arrays;
* gspmm host: python/mojodgl/ops/spmm.py:21-110;
* gsddmm host: python/mojodgl/ops/sddmm.py:83-170;
* edge_softmax host, including the positional `eids` rule:
  python/mojodgl/ops/edge_softmax.py:11-173;
* segment ops host: python/mojodgl/ops/segment.py:12-214 (offsets by cumsum,
  mean divided by clamp(seglen, 1, n) in the value dtype, max/min with
  +-inf replaced by zero);
* gather_mm host: python/mojodgl/ops/gather_mm.py:18-92 (fused kernel only:
  the sorted route gives the same numbers, test_ops.py:405-413).

Parity status per function is in oracle/README.txt.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# MDGL_ORACLE_LIB names another build of mdgl_oracle.cpp (the sanitizer build of the tests)
LIB_PATH = os.environ.get("MDGL_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

SRC, DST, EDGE = 0, 1, 2
OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3, "dot": 4, "copy_lhs": 5, "copy_rhs": 6}
REDUCERS = {"sum": 0, "max": 1, "min": 2, "mean": 3}
TARGETS = {"u": SRC, "v": DST, "e": EDGE}

_P = ctypes.c_void_p
_I = ctypes.c_int64
_C = ctypes.c_int

_SIGS = {
    "oracle_set_workers": ([_C], _C),
    "oracle_workers": ([], _C),
    "oracle_cumsum": ([_P, _P, _I], None),
    "oracle_clamp_i64": ([_P, _P, _I, _I, _I], None),
    "oracle_replace_inf_with_zero": ([_P, _P, _I, _C], None),
    "oracle_gsddmm": ([_P, _P, _P, _P, _P, _I, _C, _C, _C, _I, _I, _I, _P, _P, _I, _C], None),
    "oracle_gspmm": ([_P, _P, _P, _P, _P, _P, _I, _C, _I, _I, _I, _C, _P, _P, _P, _P, _P, _C],
                     None),
    "oracle_segment_reduce": ([_P, _P, _P, _I, _I, _C, _I, _C], None),
    "oracle_segment_softmax": ([_P, _P, _P, _I, _I, _I, _C], None),
    "oracle_segment_mm": ([_P, _P, _P, _P, _I, _I, _I, _I, _C], None),
    "oracle_gather_mm": ([_P, _P, _P, _P, _I, _I, _I, _C], None),
    "oracle_edge_softmax": ([_P, _P, _P, _P, _P, _I, _C, _I, _C], None),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The oracle library, built with `make -C oracle` when it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import subprocess

            subprocess.run(["make", "-C", HERE], check=True, capture_output=True)
        _lib = ctypes.CDLL(LIB_PATH)
        for name, (argtypes, restype) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
    return _lib


def set_workers(n: int) -> int:
    """Worker threads of the static split (the reference uses 32)."""
    return lib().oracle_set_workers(int(n))


def _code(dtype) -> int:
    dtype = np.dtype(dtype)
    if dtype == np.float32:
        return 0
    if dtype == np.float64:
        return 1
    raise TypeError("oracle dtype must be float32 or float64, got {}".format(dtype))


def _p(a):
    return None if a is None else a.ctypes.data


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int64)


def _f(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ graph
def csr(u, v, num_nodes, by="dst"):
    """(indptr, indices, eid) of the CSR grouped by `by` (heterograph.py:69-86).

    Rows are ordered by the grouping endpoint and, inside a row, by edge id,
    because the argsort is stable; that order fixes the fold order and the
    tie order of every CSR kernel.
    """
    u = _i64(u)
    v = _i64(v)
    key, other = (v, u) if by == "dst" else (u, v)
    deg = np.bincount(key, minlength=num_nodes).astype(np.int64)
    indptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.cumsum(deg, out=indptr[1:])
    order = np.argsort(key, kind="stable").astype(np.int64)
    return indptr, _i64(other[order]), order


# ------------------------------------------------------------------ broadcast
def reshape_lhs_rhs(lshape, rshape):
    """Pad the shorter feature shape with ones after the first axis (sddmm.py:24-47)."""
    lshape, rshape = tuple(lshape), tuple(rshape)
    if len(lshape) != len(rshape):
        nd = max(len(lshape), len(rshape))
        lshape = (lshape[0],) + (1,) * (nd - len(lshape)) + lshape[1:]
        rshape = (rshape[0],) + (1,) * (nd - len(rshape)) + rshape[1:]
    return lshape, rshape


def _feat(shape):
    """Feature shape of an operand; a 1-D operand is read as (n, 1) (sddmm.py:50-59)."""
    shape = tuple(shape)
    return shape[1:] if len(shape) > 1 else (1,)


def bcast(lshape, rshape, dot=False):
    """(out_feature_shape, lhs_off, rhs_off, red) for NumPy broadcasting.

    `lhs_off[o]` / `rhs_off[o]` is the index, inside one operand row, of the
    `red`-long vector output column `o` reads; red is 1 except for dot, which
    contracts the last axis. Built by broadcasting arange index arrays, which
    is NumPy's own definition of which element a broadcast position reads.
    """
    lshape, rshape = reshape_lhs_rhs(lshape, rshape)
    lf, rf = _feat(lshape), _feat(rshape)
    red = 1
    if dot:
        if lf[-1] != rf[-1]:
            raise ValueError("dot needs matching last axes")
        red = int(lf[-1])
        lf, rf = lf[:-1], rf[:-1]
    out = np.broadcast_shapes(lf, rf)
    lidx = np.arange(int(np.prod(lf)), dtype=np.int64).reshape(lf)
    ridx = np.arange(int(np.prod(rf)), dtype=np.int64).reshape(rf)
    lhs_off = np.ascontiguousarray(np.broadcast_to(lidx, out).ravel())
    rhs_off = np.ascontiguousarray(np.broadcast_to(ridx, out).ravel())
    out_shape = tuple(out) + ((1,) if dot else ())
    return out_shape, lhs_off, rhs_off, red


def _row_width(shape):
    return int(np.prod(_feat(shape)))


# ------------------------------------------------------------------ ops
def gspmm(u, v, num_nodes, op, reduce_op, lhs, rhs, dtype=np.float64, with_arg=False,
          graph_csr=None):
    """ops.gspmm (spmm.py:21-110) over the in-CSR; returns out (and arg_u, arg_e)."""
    if graph_csr is None:
        graph_csr = csr(u, v, num_nodes, "dst")
    indptr, indices, eid = graph_csr
    num_edges = int(indices.size)
    if op == "copy_lhs":
        lhs = _f(lhs, dtype)
        rhs = lhs
        fshape = _feat(lhs.shape)
        lhs_off = rhs_off = None
        dl = dr = _row_width(lhs.shape)
    elif op == "copy_rhs":
        rhs = _f(rhs, dtype)
        lhs = rhs
        fshape = _feat(rhs.shape)
        lhs_off = rhs_off = None
        dl = dr = _row_width(rhs.shape)
    else:
        lhs = _f(lhs, dtype)
        rhs = _f(rhs, dtype)
        fshape, lhs_off, rhs_off, _ = bcast(lhs.shape, rhs.shape)
        dl, dr = _row_width(lhs.shape), _row_width(rhs.shape)
    dout = int(np.prod(fshape))
    out = np.empty((num_nodes, dout), dtype=dtype)
    deg = np.diff(indptr).astype(np.int64)
    arg_u = np.zeros((num_nodes, dout), dtype=np.int64) if with_arg else None
    arg_e = np.zeros((num_nodes, dout), dtype=np.int64) if with_arg else None
    lib().oracle_gspmm(_p(indptr), _p(indices), _p(eid), _p(lhs), _p(rhs), _p(out), num_nodes,
                       OPS[op], dl, dr, dout, REDUCERS[reduce_op], _p(deg), _p(lhs_off),
                       _p(rhs_off), _p(arg_u), _p(arg_e), _code(dtype))
    del num_edges
    shape = (num_nodes,) + tuple(fshape)
    if with_arg:
        return out.reshape(shape), arg_u.reshape(shape), arg_e.reshape(shape)
    return out.reshape(shape)


def gsddmm(u, v, num_nodes, op, lhs, rhs, lhs_target="u", rhs_target="v", dtype=np.float64):
    """ops.gsddmm (sddmm.py:83-170) in edge-id order."""
    u = _i64(u)
    v = _i64(v)
    num_edges = int(u.size)
    if op == "copy_lhs":
        lhs = _f(lhs, dtype)
        rhs = lhs
        fshape, lhs_off, rhs_off, red = _feat(lhs.shape), None, None, 1
        dl = dr = _row_width(lhs.shape)
    elif op == "copy_rhs":
        rhs = _f(rhs, dtype)
        lhs = rhs
        fshape, lhs_off, rhs_off, red = _feat(rhs.shape), None, None, 1
        dl = dr = _row_width(rhs.shape)
    else:
        lhs = _f(lhs, dtype)
        rhs = _f(rhs, dtype)
        fshape, lhs_off, rhs_off, red = bcast(lhs.shape, rhs.shape, dot=(op == "dot"))
        dl, dr = _row_width(lhs.shape), _row_width(rhs.shape)
    dout = int(np.prod(fshape)) if op != "dot" else int(np.prod(fshape[:-1]))
    out = np.empty((num_edges, dout), dtype=dtype)
    lib().oracle_gsddmm(_p(u), _p(v), _p(lhs), _p(rhs), _p(out), num_edges,
                        TARGETS[lhs_target], TARGETS[rhs_target], OPS[op], dl, dr, dout,
                        _p(lhs_off), _p(rhs_off), red, _code(dtype))
    return out.reshape((num_edges,) + tuple(fshape))


def edge_softmax(u, v, num_nodes, logits, eids=None, norm_by="dst", dtype=np.float64):
    """ops.edge_softmax (edge_softmax.py:11-173), `eids=None` meaning ALL.

    With a subset `eids` the reference's positional rule applies: positions
    of `eids` are grouped by endpoint (groups in ascending endpoint id, and
    positions inside a group in the order they appear), position i reads
    `logits[i]`, and the output is as long as `logits` with rows past
    len(eids) zero.
    """
    u = _i64(u)
    v = _i64(v)
    logits = _f(logits, dtype)
    shape = logits.shape
    d = 1 if len(shape) == 1 else int(np.prod(shape[1:]))
    flat = logits.reshape(shape[0], d)
    if eids is None:
        indptr, _, eid = csr(u, v, num_nodes, norm_by)
        rows = num_nodes
        out = np.empty((flat.shape[0], d), dtype=dtype)
    else:
        order = _i64(eids)
        key = v if norm_by == "dst" else u
        groups = {}
        for i, e in enumerate(order.tolist()):
            groups.setdefault(int(key[e]), []).append(i)
        eid_list, ptr = [], [0]
        for n in sorted(groups):
            eid_list.extend(groups[n])
            ptr.append(ptr[-1] + len(groups[n]))
        eid = np.array(eid_list, dtype=np.int64)
        indptr = np.array(ptr, dtype=np.int64)
        rows = len(groups)
        flat = np.ascontiguousarray(flat[: order.size])
        out = np.zeros((shape[0], d), dtype=dtype)
    mask = np.ones(1, dtype=np.int8)
    if rows:
        lib().oracle_edge_softmax(_p(indptr), _p(eid), _p(mask), _p(flat), _p(out), rows, 1, d,
                                  _code(dtype))
    return out.reshape(shape)


def offsets_of(seglen):
    """[0] + cumsum(seglen) through the restated cumsum (segment.py:12-21)."""
    seglen = _i64(seglen)
    src = np.concatenate([np.zeros(1, dtype=np.int64), seglen])
    dst = np.zeros_like(src)
    lib().oracle_cumsum(_p(src), _p(dst), src.size)
    return dst


def segment_reduce(seglen, value, reducer="sum", dtype=np.float64):
    """ops.segment_reduce (segment.py:62-112)."""
    seglen = _i64(seglen)
    value = _f(value, dtype)
    shape = value.shape
    d = 1 if value.ndim == 1 else int(np.prod(shape[1:]))
    flat = value.reshape(shape[0], d)
    n = flat.shape[0]
    offsets = offsets_of(seglen)
    num_seg = seglen.size
    red = "sum" if reducer == "mean" else reducer
    out = np.empty((num_seg, d), dtype=dtype)
    lib().oracle_segment_reduce(_p(offsets), _p(flat), _p(out), num_seg, d, REDUCERS[red], n,
                                _code(dtype))
    if reducer == "mean":
        z = np.zeros_like(seglen)
        lib().oracle_clamp_i64(_p(seglen), _p(z), seglen.size, 1, n)
        out = out / z.astype(dtype).reshape(-1, 1)
    elif reducer in ("max", "min"):
        res = np.zeros_like(out)
        lib().oracle_replace_inf_with_zero(_p(out), _p(res), out.size, _code(dtype))
        out = res
    return out.reshape((num_seg,) + tuple(shape[1:]))


def segment_softmax(seglen, value, dtype=np.float64):
    """ops.segment_softmax (segment.py:115-154); output pre-zeroed."""
    seglen = _i64(seglen)
    value = _f(value, dtype)
    shape = value.shape
    d = 1 if value.ndim == 1 else int(np.prod(shape[1:]))
    flat = value.reshape(shape[0], d)
    offsets = offsets_of(seglen)
    out = np.zeros_like(flat)
    if seglen.size and flat.shape[0]:
        lib().oracle_segment_softmax(_p(offsets), _p(flat), _p(out), seglen.size, d,
                                     flat.shape[0], _code(dtype))
    return out.reshape(shape)


def segment_mm(a, b, seglen, dtype=np.float64):
    """ops.segment_mm (segment.py:157-214); rows past sum(seglen) stay zero."""
    a = _f(a, dtype)
    b = _f(b, dtype)
    seglen = _i64(seglen)
    n, d1 = a.shape
    r, _, d2 = b.shape
    out = np.zeros((n, d2), dtype=dtype)
    if n:
        lib().oracle_segment_mm(_p(a), _p(b), _p(out), _p(seglen), n, d1, r, d2, _code(dtype))
    return out


def gather_mm(a, b, idx_b, dtype=np.float64):
    """ops.gather_mm fused route (gather_mm.py:88-92 and ported.mojo:1089-1130)."""
    a = _f(a, dtype)
    b = _f(b, dtype)
    idx_b = _i64(idx_b)
    n, d1 = a.shape
    _, _, d2 = b.shape
    out = np.empty((n, d2), dtype=dtype)
    if n:
        lib().oracle_gather_mm(_p(a), _p(b), _p(idx_b), _p(out), n, d1, d2, _code(dtype))
    return out


def replace_inf_with_zero(x, dtype=np.float64):
    x = _f(x, dtype)
    out = np.empty_like(x)
    lib().oracle_replace_inf_with_zero(_p(x), _p(out), x.size, _code(dtype))
    return out


def clamp_i64(x, lo, hi):
    x = _i64(x)
    out = np.empty_like(x)
    lib().oracle_clamp_i64(_p(x), _p(out), x.size, int(lo), int(hi))
    return out


def cumsum(x):
    x = _i64(x)
    out = np.empty_like(x)
    lib().oracle_cumsum(_p(x), _p(out), x.size)
    return out
