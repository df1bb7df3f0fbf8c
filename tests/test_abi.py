"""The C ABI of libmdgl.so without a GPU: it loads, exports every entry point
include/mdgl.h declares, and rejects invalid arguments before launching."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mdgl.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mdgl_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from mojodgl import _lib

    return _lib.lib()


def test_header_declares_the_reference_entry_points():
    names = declared()
    # the 11 symbols of the reference's capi.mojo keep their names
    for ref in ("mdgl_workers", "mdgl_cumsum", "mdgl_replace_inf_with_zero", "mdgl_clamp_i64",
                "mdgl_gsddmm", "mdgl_gspmm", "mdgl_segment_reduce", "mdgl_segment_softmax",
                "mdgl_segment_mm", "mdgl_edge_softmax_", "mdgl_gather_mm"):
        assert ref in names


def test_every_declared_symbol_is_exported(lib):
    for name in declared():
        assert hasattr(lib, name), name


def test_workers_is_parallel(lib):
    assert lib.mdgl_workers() > 1


def err(lib):
    return lib.mdgl_last_error().decode()


def test_gspmm_lane_query(lib):
    """mdgl_gspmm_lanes reports the lane width and lanes per row slab
    mdgl_gspmm launches with (host pointers stand in: the query reads only
    their alignment)."""
    import numpy as np
    from mojodgl import _lib

    buf = np.zeros(4096, dtype=np.float64)
    base = (buf.ctypes.data + 255) // 256 * 256          # 256-byte aligned
    mul, cl = _lib.BINARY_OPS["mul"], _lib.OP_COPY_LHS

    def lanes(op, dl, dr, dout, lshape=None, rshape=None, lhs=base, rhs=base, flags=0, dt=0):
        out, grp = ctypes.c_int64(-1), ctypes.c_int64(-1)
        nd = 0 if lshape is None else len(lshape)
        ls = None if lshape is None else (ctypes.c_int64 * nd)(*lshape)
        rs = None if rshape is None else (ctypes.c_int64 * nd)(*rshape)
        rc = lib.mdgl_gspmm_lanes(op, dl, dr, dout, nd, ls, rs, lhs, rhs, flags, dt,
                                  ctypes.byref(out), ctypes.byref(grp))
        assert rc == 0, err(lib)
        rc = lib.mdgl_gspmm_lanes(op, dl, dr, dout, nd, ls, rs, lhs, rhs, flags, dt,
                                  ctypes.byref(out), None)     # the group is optional
        assert rc == 0, err(lib)
        return out.value, grp.value

    def vec(*args, **kw):
        return lanes(*args, **kw)[0]

    assert vec(cl, 64, 64, 64) == 4                      # 16-byte float32 lanes
    assert vec(cl, 64, 64, 64, dt=1) == 2                # 16-byte float64 lanes
    assert vec(cl, 602, 602, 602) == 2                   # even float32 width: 8-byte lanes
    assert vec(cl, 601, 601, 601) == 1
    assert vec(cl, 602, 602, 602, flags=_lib.LHS_LINE_ROWS) == 4   # rows padded to lines
    assert vec(cl, 64, 64, 64, lhs=base + 4) == 1        # a misaligned node operand
    # GAT heads: 8 heads of 32 columns, one weight per head: 16-byte lanes
    assert vec(mul, 256, 8, 256, (8, 32), (8, 1)) == 4
    # heads of 6 columns: 16-byte lanes would straddle heads, 8-byte ones do not
    assert vec(mul, 48, 8, 48, (8, 6), (8, 1)) == 2
    # heads of 3 columns: one element per lane
    assert vec(mul, 12, 4, 12, (4, 3), (4, 1)) == 1
    # lanes per slab: the power of two covering the row's lanes, at most 64;
    # with NARROW_SLABS 32 for wider rows when that makes at most 5 slabs
    line, narrow = _lib.LHS_LINE_ROWS, _lib.LHS_LINE_ROWS | _lib.NARROW_SLABS
    assert lanes(cl, 64, 64, 64) == (4, 16)
    assert lanes(cl, 602, 602, 602, flags=line) == (4, 64)             # 151 lanes, 3 slabs
    assert lanes(cl, 602, 602, 602, flags=narrow) == (4, 32)           # 5 slabs
    assert lanes(cl, 602, 602, 602, flags=narrow, dt=1) == (2, 64)     # 301 lanes: 10 would be
    assert lanes(cl, 130, 130, 130, flags=_lib.NARROW_SLABS, dt=1) == (2, 32)   # 65 lanes: 3
    # float64 rows of 129-256 columns (a multiple of 4): 32-byte lanes, one slab
    assert lanes(cl, 256, 256, 256, dt=1) == (4, 64)
    assert lanes(cl, 200, 200, 200, dt=1) == (4, 64)
    assert lanes(cl, 258, 258, 258, dt=1) == (2, 64)                            # 2 slabs
    assert lanes(mul, 256, 8, 256, (8, 32), (8, 1), dt=1) == (4, 64)            # GAT heads
    assert lanes(cl, 256, 256, 256, flags=_lib.NARROW_SLABS) == (4, 64)         # one slab
    assert lanes(mul, 256, 8, 256, (8, 32), (8, 1), flags=_lib.NARROW_SLABS) == (4, 64)
    rc = lib.mdgl_gspmm_lanes(_lib.BINARY_OPS["dot"], 4, 4, 4, 0, None, None, base, base, 0, 0,
                              ctypes.byref(ctypes.c_int64()), None)
    assert rc == -1 and "op" in err(lib)
    rc = lib.mdgl_gspmm_lanes(cl, 64, 64, 64, 0, None, None, base + 16, base,
                              _lib.LHS_LINE_ROWS, 0, ctypes.byref(ctypes.c_int64()), None)
    assert rc == -1 and "128-byte" in err(lib)


def test_invalid_arguments_are_rejected_without_launching(lib):
    # bad op / reducer / dtype / target codes: negative status, named in the message
    rc = lib.mdgl_gspmm(None, None, None, None, None, None, 10, 4, 1, 1, 1, 0, None, 0, None,
                        None, None, None, None, None, 0, 0, None, None, 0, None, 0, 0, 0, None)
    assert rc == -1 and "dot" in err(lib)
    rc = lib.mdgl_gspmm(None, None, None, None, None, None, 10, 2, 1, 1, 1, 9, None, 0, None,
                        None, None, None, None, None, 0, 0, None, None, 0, None, 0, 0, 0, None)
    assert rc == -1 and "reduce_op" in err(lib)
    rc = lib.mdgl_gsddmm(None, None, None, None, None, 5, 0, 3, 0, 1, 1, 1, 0, None, None, 0, None)
    assert rc == -1 and "target" in err(lib)
    rc = lib.mdgl_segment_reduce(None, None, None, 4, 2, 0, 8, 0, 7, None)
    assert rc == -1 and "dtype" in err(lib)
    # null buffers for a non-empty problem
    rc = lib.mdgl_gspmm(None, None, None, None, None, None, 10, 2, 4, 4, 4, 0, None, 0, None,
                        None, None, None, None, None, 0, 0, None, None, 0, None, 0, 0, 0, None)
    assert rc == -1 and "null" in err(lib)
    # widths that do not match the broadcast shapes
    import numpy as np

    ls = np.array([8, 32], dtype=np.int64)
    rs = np.array([8, 2], dtype=np.int64)
    rc = lib.mdgl_gspmm(None, None, None, None, None, None, 10, 2, 256, 16, 256, 0, None, 2,
                        ls.ctypes.data, rs.ctypes.data, None, None, None, None, 0, 0, None, None,
                        0, None, 0, 0, 0, None)
    assert rc == -1 and "broadcastable" in err(lib)
    # a chunk schedule without its workspace, or with a misaligned one
    rc = lib.mdgl_gspmm(1, 1, 1, 1, 1, 1, 10, 2, 4, 4, 4, 0, None, 0, None, None, None, None, 1,
                        1, 3, 8, 1, 1, 1, None, 0, 0, 0, None)
    assert rc == -2 and "workspace" in err(lib)
    rc = lib.mdgl_gspmm(1, 1, 1, 1, 1, 1, 10, 2, 4, 4, 4, 0, None, 0, None, None, None, None, 1,
                        1, 3, 8, 1, 1, 1, 4096 + 8, 1 << 20, 0, 0, None)
    assert rc == -1 and "aligned" in err(lib)
    # node rows on 128-byte lines need an lhs on a 128-byte boundary
    rc = lib.mdgl_gspmm(1, 1, 1, 8, 16, 16, 10, 2, 4, 4, 4, 0, None, 0, None, None, None, None,
                        None, None, 0, 0, None, None, 0, None, 0, 8, 0, None)
    assert rc == -1 and "128-byte" in err(lib)
    # segment_reduce pass flags: at most one of SHORT, SKIP_LONG and LONG_ONLY
    rc = lib.mdgl_segment_reduce(None, None, None, 4, 2, 0, 8, 4 | 8, 0, None)
    assert rc == -1 and "at most one" in err(lib)
    rc = lib.mdgl_segment_reduce(None, None, None, 4, 2, 0, 8, 8 | 16, 0, None)
    assert rc == -1 and "at most one" in err(lib)
    rc = lib.mdgl_segment_softmax_short(None, None, None, 4, 2, 8, 7, None)
    assert rc == -1 and "dtype" in err(lib)
    rc = lib.mdgl_segment_softmax_short(None, None, None, 4, 2, 8, 0, None)
    assert rc == -1 and "null" in err(lib)
    # too many b blocks for the GPU bucketing
    rc = lib.mdgl_gather_mm(1, 1, 1, 1, 100, 4, 4, 100000, 1, 1 << 40, 0, None)
    assert rc == -3
    # a row list: its count must not be negative, and a non-empty one needs its rows
    rc = lib.mdgl_gspmm_rows(1, 1, 1, 1, 1, 1, 10, 2, 4, 4, 4, 0, None, 0, None, None, None,
                             None, None, -1, 0, 0, None)
    assert rc == -1 and "negative" in err(lib)
    rc = lib.mdgl_gspmm_rows(1, 1, 1, 1, 1, 1, 10, 2, 4, 4, 4, 0, None, 0, None, None, None,
                             None, None, 3, 0, 0, None)
    assert rc == -1 and "null rows" in err(lib)
    rc = lib.mdgl_gspmm_rows(1, 1, 1, 1, 1, 1, 10, 2, 4, 4, 4, 7, None, 0, None, None, None,
                             None, 1, 3, 0, 0, None)
    assert rc == -1 and "reduce_op" in err(lib)
    # the row-read ceiling: row sizes, counts, buffers and their alignment
    for row_bytes in (0, 8, 24, 1040):
        assert lib.mdgl_read_rows(16, 10, row_bytes, 16, 64, None, 0, 16, None) == -1
        assert "row_bytes" in err(lib)
    assert lib.mdgl_read_rows(16, 10, 64, 16, -1, None, 0, 16, None) == -1
    assert lib.mdgl_read_rows(16, 10, 64, 16, 1 << 31, None, 0, 16, None) == -1
    assert lib.mdgl_read_rows(16, 10, 64, None, 64, None, 0, 16, None) == -1
    assert "null" in err(lib)
    assert lib.mdgl_read_rows(16, 10, 64, 16, 64, None, 5, 16, None) == -1  # rows, no dst
    assert lib.mdgl_read_rows(8, 10, 64, 16, 64, None, 0, 16, None) == -1
    assert "aligned" in err(lib)
    assert lib.mdgl_read_rows_sink_bytes(65) == 32 and lib.mdgl_read_rows_sink_bytes(-1) == -1


def test_empty_problems_are_no_ops(lib):
    assert lib.mdgl_gspmm(None, None, None, None, None, None, 0, 2, 4, 4, 4, 0, None, 0, None,
                          None, None, None, None, None, 0, 0, None, None, 0, None, 0, 0, 0,
                          None) == 0
    assert lib.mdgl_segment_mm(None, None, None, None, 0, 4, 2, 3, None, 0, 0, None) == 0
    # no rows listed: nothing to do, whatever the buffers
    assert lib.mdgl_gspmm_rows(None, None, None, None, None, None, 10, 2, 4, 4, 4, 0, None, 0,
                               None, None, None, None, None, 0, 0, 0, None) == 0
    assert lib.mdgl_cumsum(None, None, 0, None) == 0
    assert lib.mdgl_segment_softmax_short(None, None, None, 0, 4, 0, 0, None) == 0
    assert lib.mdgl_read_rows(None, 0, 64, None, 0, None, 0, None, None) == 0


def test_build_csr_arguments(lib):
    assert lib.mdgl_build_csr(None, None, -1, 4, None, None, None, None, 0, None) == -1
    assert lib.mdgl_build_csr(None, None, 2 ** 31, 4, None, None, None, None, 0, None) == -1
    rc = lib.mdgl_build_csr(None, None, 5, 0, None, None, None, None, 0, None)
    assert rc == -1 and "no rows" in err(lib)
    rc = lib.mdgl_build_csr(None, None, 5, 300, None, None, None, None, 0, None)
    assert rc == -1 and "null" in err(lib)
    rc = lib.mdgl_build_csr(8, 8, 5, 300, 8, 8, 8, None, 0, None)
    assert rc == -2 and "workspace" in err(lib)
    # workspaces must be 256-byte aligned (their arrays are read 16 bytes at a time)
    rc = lib.mdgl_build_csr(8, 8, 5, 300, 8, 8, 8, 4096 + 16, 1 << 20, None)
    assert rc == -1 and "aligned" in err(lib)
    # one row or no edges: no workspace and no sort
    assert lib.mdgl_build_csr_workspace_bytes(1000, 1) == 0
    assert lib.mdgl_build_csr_workspace_bytes(0, 1000) == 0
    assert lib.mdgl_build_csr_workspace_bytes(1000, 300) >= 3 * 1000 * 4
    assert lib.mdgl_build_csr_workspace_bytes(-1, 3) == -1


def test_backward_helper_arguments(lib):
    assert lib.mdgl_gspmm_edge_grad(None, None, None, None, None, 5, 3, 0, 1.0, 9, None) == -1
    assert lib.mdgl_gspmm_edge_grad(None, None, None, None, None, -1, 3, 0, 1.0, 0, None) == -1
    rc = lib.mdgl_gspmm_edge_grad(None, None, None, None, None, 5, 3, 1, 1.0, 0, None)
    assert rc == -1 and "null" in err(lib)
    assert lib.mdgl_gspmm_edge_grad(None, None, None, None, None, 0, 3, 1, 1.0, 0, None) == 0
    assert lib.mdgl_rows_by_degree(None, None, None, 4, 2, 0, None) == -1
    assert lib.mdgl_rows_by_degree(None, None, None, 0, 2, 0, None) == 0
    assert lib.mdgl_scale(None, None, 4, -1.0, 0, None) == -1
    assert lib.mdgl_scale(None, None, 0, -1.0, 0, None) == 0
    assert lib.mdgl_scale(None, None, 4, -1.0, 5, None) == -1
    assert lib.mdgl_edge_softmax_grad(None, None, None, None, None, 5, 2, 7, None) == -1
    rc = lib.mdgl_edge_softmax_grad(None, None, None, None, None, 5, 2, 0, None)
    assert rc == -1 and "null" in err(lib)
    assert lib.mdgl_edge_softmax_grad(None, None, None, None, None, 0, 2, 0, None) == 0
    # segment gradients: the row -> segment map and max / min with their rows
    assert lib.mdgl_segment_ids(None, -1, 4, None, None) == -1
    rc = lib.mdgl_segment_ids(None, 0, 4, None, None)
    assert rc == -1 and "no segments" in err(lib)
    rc = lib.mdgl_segment_ids(None, 2, 4, None, None)
    assert rc == -1 and "null" in err(lib)
    assert lib.mdgl_segment_ids(None, 0, 0, None, None) == 0
    rc = lib.mdgl_segment_reduce_arg(None, None, None, None, 3, 2, 0, 6, 0, 0, None)
    assert rc == -1 and "max or min" in err(lib)
    rc = lib.mdgl_segment_reduce_arg(1, 1, 1, None, 3, 2, 1, 6, 0, 0, None)
    assert rc == -1 and "null" in err(lib)
    assert lib.mdgl_segment_reduce_arg(None, None, None, None, 0, 2, 2, 0, 0, 0, None) == 0
    # grouped GEMM gradients: sizes, outputs, workspace
    assert lib.mdgl_segment_mm_grad_workspace_bytes(-1, 4, 4, 2, 0) == -1
    assert lib.mdgl_gather_mm_grad_workspace_bytes(10, 4, 4, 2, 0) > 0
    rc = lib.mdgl_segment_mm_grad(1, 1, 1, 1, 1, 1, 10, 4, 2, 4, None, 0, 0, None)
    assert rc == -2 and "workspace" in err(lib)
    assert lib.mdgl_segment_mm_grad(1, 1, 1, 1, None, None, 10, 4, 2, 4, None, 0, 0, None) == 0
    rc = lib.mdgl_gather_mm_grad(1, 1, 1, 1, 1, 1, 10, 4, 4, 4096, None, 0, 0, None)
    assert rc == -3 and "blocks" in err(lib)
    rc = lib.mdgl_gather_mm_grad(1, 1, None, 1, 1, 1, 10, 4, 4, 2, None, 0, 0, None)
    assert rc == -1 and "null" in err(lib)
    # the fused u_mul_e backward refuses other ops' shapes before launching
    rc = lib.mdgl_gspmm_mul_sum_dot(1, 1, 1, 1, 1, None, 1, 1, 10, 12, 2, 12, 0, None, None,
                                    None, None, 0, 0, None, None, 0, None, 0, 0, None)
    assert rc in (-1, -3)


def test_workspace_sizes(lib):
    assert lib.mdgl_gspmm_workspace_bytes(0, 64, 0, 0) == 0
    assert lib.mdgl_gspmm_workspace_bytes(10, 64, 0, 0) >= 10 * 64 * 4
    assert lib.mdgl_gspmm_workspace_bytes(10, 64, 1, 1) >= 10 * 64 * (8 + 4 + 4)
    assert lib.mdgl_gather_mm_workspace_bytes(1000, 128, 128, 64, 0) >= 64 * 128 * 128 * 4 + 4000
    assert lib.mdgl_segment_mm_workspace_bytes(1000, 5, 3, 7, 1) > 0
    # gradients: the forward's workspace for da (b's blocks as [D1][D2]), the
    # grouping again for db, and one D1 x D2 partial per chunk of rows (at
    # most n / 4096 + r chunks at 4096 rows; longer chunks keep the partials
    # near 256 MB when D1 x D2 is large)
    for gather in (False, True):
        grad = lib.mdgl_gather_mm_grad_workspace_bytes if gather \
            else lib.mdgl_segment_mm_grad_workspace_bytes
        fwd = lib.mdgl_gather_mm_workspace_bytes if gather \
            else lib.mdgl_segment_mm_workspace_bytes
        n, d1, d2, r = 10 ** 7, 128, 128, 64
        small = grad(n, d1, d2, r, 0)
        assert small >= fwd(n, d2, d1, r, 0) + (n // 4096 + r) * d1 * d2 * 4
        assert grad(2 * n, d1, d2, r, 0) >= small
        wide = grad(n, 2048, 2048, r, 0)
        assert wide - fwd(n, 2048, 2048, r, 0) < (1 << 28) + r * 2048 * 2048 * 4 + (1 << 27)
        assert grad(n, d1, d2, r, 1) > small


@pytest.mark.parametrize("setting,expect", [(None, 0), ("0", 0), ("1", 1)])
def test_trace_ranges_follow_the_environment(setting, expect):
    """MDGL_ROCTX turns the per-entry-point roctx ranges on (the ROCm roctx
    library ships in the image); calls that fail validation still return
    their status with a range open around them."""
    import subprocess
    import sys

    env = dict(os.environ)
    env.pop("MDGL_ROCTX", None)
    if setting is not None:
        env["MDGL_ROCTX"] = setting
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from mojodgl import _lib\n"
        "lib = _lib.lib()\n"
        "print(lib.mdgl_trace_ranges(), lib.mdgl_cumsum(None, None, -1, None),"
        " lib.mdgl_trace_ranges())\n" % os.path.join(ROOT, "mojo-dgl_amd"))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    on, status, again = out.stdout.split()
    assert int(on) == int(again) == expect
    assert int(status) == -1  # MDGL_EINVAL
