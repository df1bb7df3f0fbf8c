"""HIP kernels (through the mojodgl API and libmdgl.so) against the CPU oracle.

Tolerance rule for sums and softmaxes, stated once: with ref the float64
oracle on the same inputs and T the oracle's result on |inputs| (the sum of
absolute terms), |gpu - ref| <= tol * max(|ref|, T), tol = 1e-5 for float32
and 1e-12 for float64. Where the GPU folds in the reference's order (gspmm /
segment_reduce rows that are not split) it is also checked bit for bit
against the oracle run in the same precision. max/min values, their arg
indices and every integer output are bit-exact.
"""

import importlib
import itertools

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.function as fn
import mojodgl.heterograph as hg
import mojodgl.ops as ops
import oracle

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-5, np.float64: 1e-12}


def rand_graph(n, e, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, n, e), rng.integers(0, n, e)


def close(got, ref, bound, dtype, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = np.maximum(np.abs(ref), np.abs(np.asarray(bound, dtype=np.float64)))
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = np.abs(got - ref)
    ok = err <= TOL[dtype] * bound + 1e-300
    if not ok.all():
        i = np.unravel_index(np.argmax(err - TOL[dtype] * bound), err.shape)
        raise AssertionError("{}: {} of {} outside tolerance; worst at {}: got {} ref {} bound "
                             "{}".format(what, int((~ok).sum()), ok.size, i, got[i], ref[i],
                                         bound[i]))


ABS_OP = {"add": "add", "sub": "add", "mul": "mul", "div": "div"}


@pytest.fixture(params=[None, 4], ids=["whole-rows", "split-rows"])
def chunk_len(request, monkeypatch):
    """Run each gspmm test with row splitting off and forced on (chunks of 4)."""
    monkeypatch.setattr(hg, "CHUNK_LEN", request.param if request.param else 2 ** 30)
    return request.param


# ------------------------------------------------------------------ gspmm
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "copy_u", "copy_e"])
@pytest.mark.parametrize("reduce_op", ["sum", "max", "min", "mean"])
def test_gspmm_all_families(dtype, op, reduce_op, chunk_len):
    n, e = 300, 4000
    u, v = rand_graph(n, e, 1)
    u[:300] = 7  # one hub source, plus a hub destination below
    v[:600] = 11
    rng = np.random.default_rng(2)
    d = 13
    x = rng.normal(size=(n, d)).astype(dtype)
    w = (rng.random((e, d)) + 0.25).astype(dtype)
    if op == "copy_u":
        oop, L, R = "copy_lhs", x, None
    elif op == "copy_e":
        oop, L, R = "copy_rhs", None, w
    else:
        oop, L, R = op, x, w
    g = dgl.graph((u, v), num_nodes=n)
    got, (au, ae) = ops.spmm._gspmm(g, oop, reduce_op, L, R)
    assert got.dtype == dtype
    ref64 = oracle.gspmm(u, v, n, oop, reduce_op, L, R, np.float64)
    if reduce_op in ("max", "min"):
        same, ru, re_ = oracle.gspmm(u, v, n, oop, reduce_op, L, R, dtype, with_arg=True)
        np.testing.assert_array_equal(got, same)
        np.testing.assert_array_equal(au, ru)
        np.testing.assert_array_equal(ae, re_)
        return
    if chunk_len is None:
        np.testing.assert_array_equal(got, oracle.gspmm(u, v, n, oop, reduce_op, L, R, dtype))
    absop = "copy_lhs" if oop == "copy_lhs" else "copy_rhs" if oop == "copy_rhs" else ABS_OP[op]
    bound = oracle.gspmm(u, v, n, absop, reduce_op, None if L is None else np.abs(L),
                         None if R is None else np.abs(R), np.float64)
    close(got, ref64, bound, dtype, "{} {}".format(op, reduce_op))


@pytest.mark.parametrize("d", [1, 2, 3, 5, 7, 8, 16, 33, 64, 130, 602])
def test_gspmm_feature_widths(d):
    n, e = 200, 3000
    u, v = rand_graph(n, e, 3)
    rng = np.random.default_rng(4)
    x = rng.normal(size=(n, d)).astype(np.float32)
    w = rng.normal(size=(e, d)).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    for name, oop, L, R in (("u_mul_e_sum", "mul", x, w), ("u_div_e_min", "div", x, w),
                            ("copy_u_max", "copy_lhs", x, None), ("copy_e_mean", "copy_rhs",
                                                                  None, w)):
        got = getattr(ops, name)(g, *[a for a in (L, R) if a is not None])
        red = name.rsplit("_", 1)[1]
        np.testing.assert_array_equal(got, oracle.gspmm(u, v, n, oop, red, L, R, np.float32),
                                      err_msg="{} d={}".format(name, d))


@pytest.mark.parametrize("d,heads", [(132, None), (200, None), (256, None), (256, 8), (260, None)])
def test_gspmm_float64_wide_lanes(d, heads, chunk_len):
    """float64 rows of 129-256 columns (a multiple of 4) take 32-byte lanes, one
    slab per row (260 columns keep 16-byte lanes and two slabs): values and
    args bit-identical to the oracle in float64, whole rows and rows split
    into chunks, a full edge operand and one per head splat over its columns
    (the GAT layout), every reducer."""
    from mojodgl.ops import spmm

    n, e = 300, 6000
    u, v = rand_graph(n, e, 50 + d)
    rng = np.random.default_rng(51 + d)
    g = dgl.graph((u, v), num_nodes=n)
    if heads:
        x = rng.normal(size=(n, heads, d // heads))
        w = rng.random((e, heads, 1))
    else:
        x = rng.normal(size=(n, d))
        w = rng.normal(size=(e, d))
    for oop, red in (("mul", "sum"), ("mul", "mean"), ("add", "max"), ("div", "min"),
                     ("copy_lhs", "max")):
        R = None if oop == "copy_lhs" else w
        got, (au, ae) = spmm._gspmm(g, oop, red, x, R)
        what = "{} {} d={} heads={} chunk={}".format(oop, red, d, heads, chunk_len)
        if red in ("max", "min"):
            want, ru, re_ = oracle.gspmm(u, v, n, oop, red, x, R, np.float64, with_arg=True)
            np.testing.assert_array_equal(au, ru, err_msg=what)
            np.testing.assert_array_equal(ae, re_, err_msg=what)
            np.testing.assert_array_equal(got, want, err_msg=what)
        else:
            want = oracle.gspmm(u, v, n, oop, red, x, R, np.float64)
            if chunk_len is None:
                np.testing.assert_array_equal(got, want, err_msg=what)
            else:
                bound = oracle.gspmm(u, v, n, oop, red, np.abs(x), None if R is None
                                     else np.abs(R), np.float64)
                close(got, want, bound, np.float64, what)


@pytest.mark.parametrize("longest", [600, 640, 641])
def test_gspmm_rows_just_over_a_chunk(longest):
    """With 512-slot chunks, rows of up to 640 slots stay whole when no row is
    longer (sums then fold in CSR order, bit for bit the oracle's float32
    fold); one row of 641 slots splits every row over 512 again."""
    n = 300
    deg = np.full(n, 20)
    deg[[3, 50, 200]] = [513, 580, longest]
    rng = np.random.default_rng(13)
    v = np.repeat(np.arange(n), deg)
    perm = rng.permutation(v.size)
    v = v[perm]
    u = rng.integers(0, n, v.size)
    x = rng.normal(size=(n, 24)).astype(np.float32)
    w = rng.random((v.size, 1)).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    got = ops.u_mul_e_sum(g, x, w)
    split = g._device_csr("in").chunks.num_chunks > 0
    assert split == (longest > 640)
    same = oracle.gspmm(u, v, n, "mul", "sum", x, w, np.float32)
    if split:
        whole = deg <= 512
        np.testing.assert_array_equal(got[whole], same[whole])
        ref64 = oracle.gspmm(u, v, n, "mul", "sum", x, w, np.float64)
        bound = oracle.gspmm(u, v, n, "mul", "sum", np.abs(x), w, np.float64)
        close(got, ref64, bound, np.float32, "split rows")
    else:
        np.testing.assert_array_equal(got, same)
    gmax, (au, ae) = ops.spmm._gspmm(g, "mul", "max", x, w)
    rmax, ru, re_ = oracle.gspmm(u, v, n, "mul", "max", x, w, np.float32, with_arg=True)
    np.testing.assert_array_equal(gmax, rmax)
    np.testing.assert_array_equal(au, ru)
    np.testing.assert_array_equal(ae, re_)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 4, 12, 32, 128, 256])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("csr_order", ["no", "wide", "all"],
                         ids=["edge-order", "csr-order-wide", "csr-order-all"])
def test_gspmm_scalar_edge_operand(dtype, d, op, chunk_len, csr_order, monkeypatch):
    """One value per edge over every column of the node row (the GCN edge
    weight): loaded with the ids and broadcast across the lane group, for rows
    packed several to a wavefront and for whole-wavefront rows alike; with
    `csr_order` "wide" whole-wavefront rows get the weight put in CSR slot
    order first (MDGL_RHS_CSR_ORDER), as large graphs do, with "all" every
    width does (packed rows then read it by slot, as a C caller may ask)."""
    monkeypatch.setattr(ops.spmm, "CSR_ORDER_MIN_EDGES", 1 << 62 if csr_order == "no" else 0)
    if csr_order == "all":
        lanes = ops.spmm._lanes
        monkeypatch.setattr(ops.spmm, "_lanes", lambda *a: (lanes(*a)[0], 2))
    n, e = 400, 6000
    u, v = rand_graph(n, e, 11)
    v[:700] = 5  # a hub destination, split into chunks when chunk_len is set
    rng = np.random.default_rng(12)
    x = rng.normal(size=(n, d)).astype(dtype)
    w = (rng.random((e, 1)) + 0.5).astype(dtype)
    g = dgl.graph((u, v), num_nodes=n)
    for red in ("sum", "max", "min", "mean"):
        got, (au, ae) = ops.spmm._gspmm(g, op, red, x, w)
        what = "{} {} d={}".format(op, red, d)
        assert got.shape == (n, d) and got.dtype == dtype, what
        if red in ("max", "min"):
            same, ru, re_ = oracle.gspmm(u, v, n, op, red, x, w, dtype, with_arg=True)
            np.testing.assert_array_equal(got, same, err_msg=what)
            np.testing.assert_array_equal(au, ru, err_msg=what)
            np.testing.assert_array_equal(ae, re_, err_msg=what)
            continue
        if chunk_len is None:
            np.testing.assert_array_equal(got, oracle.gspmm(u, v, n, op, red, x, w, dtype),
                                          err_msg=what)
        ref64 = oracle.gspmm(u, v, n, op, red, x, w, np.float64)
        bound = oracle.gspmm(u, v, n, ABS_OP[op], red, np.abs(x), np.abs(w), np.float64)
        close(got, ref64, bound, dtype, what)


@pytest.mark.parametrize("lshape,rshape", [((8, 32), (8, 1)), ((602,), (1,)), ((4, 3), (4, 1)),
                                           ((1,), (6,)), ((2, 3, 4), (2, 1, 4)),
                                           ((3, 1), (1, 5))])
def test_gspmm_broadcast(lshape, rshape, chunk_len):
    n, e = 150, 2500
    u, v = rand_graph(n, e, 5)
    rng = np.random.default_rng(6)
    x = rng.normal(size=(n,) + lshape).astype(np.float32)
    w = rng.normal(size=(e,) + rshape).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    got = ops.u_mul_e_sum(g, x, w)
    ref = oracle.gspmm(u, v, n, "mul", "sum", x, w, np.float64)
    assert got.shape == ref.shape
    bound = oracle.gspmm(u, v, n, "mul", "sum", np.abs(x), np.abs(w), np.float64)
    close(got, ref, bound, np.float32, "bcast {} {}".format(lshape, rshape))
    if chunk_len is None:
        np.testing.assert_array_equal(got, oracle.gspmm(u, v, n, "mul", "sum", x, w, np.float32))
    gmax, (au, ae) = ops.spmm._gspmm(g, "mul", "max", x, w)
    rmax, ru, re_ = oracle.gspmm(u, v, n, "mul", "max", x, w, np.float32, with_arg=True)
    np.testing.assert_array_equal(gmax, rmax)
    np.testing.assert_array_equal(au, ru)
    np.testing.assert_array_equal(ae, re_)


@pytest.mark.parametrize("dtype,d", [(np.float32, 602), (np.float32, 130), (np.float64, 602),
                                     (np.float64, 70)])
def test_gspmm_line_aligned_rows(dtype, d):
    """Node rows whose size is no multiple of 128 bytes, gathered many times
    (here 33 per row): gspmm copies them to rows on 128-byte lines
    (MDGL_LHS_LINE_ROWS) and the results stay bit-identical to the oracle,
    values and args, for the C3 shapes (a scalar edge weight, copy_u)."""
    from mojodgl.ops import spmm

    rng = np.random.default_rng(30 + d)
    n, e = 600, 20000
    u, v = rand_graph(n, e, 31)
    x = rng.normal(size=(n, d)).astype(dtype)
    w = rng.random((e, 1)).astype(dtype)
    lined = spmm._line_rows(torch.from_numpy(x).cuda(), n, d, e, dtype)
    assert lined is not None and lined.stride(0) * lined.element_size() % 128 == 0
    g = dgl.graph((u, v), num_nodes=n)
    for oop, red, L, R in (("mul", "sum", x, w), ("mul", "mean", x, w),
                           ("copy_lhs", "max", x, None), ("mul", "min", x, w)):
        got, (au, ae) = spmm._gspmm(g, oop, red, L, R)
        if red in ("max", "min"):
            want, ru, re_ = oracle.gspmm(u, v, n, oop, red, L, R, dtype, with_arg=True)
            np.testing.assert_array_equal(au, ru, err_msg=red)
            np.testing.assert_array_equal(ae, re_, err_msg=red)
        else:
            want = oracle.gspmm(u, v, n, oop, red, L, R, dtype)
        np.testing.assert_array_equal(got, want, err_msg="{} {} d={}".format(oop, red, d))


def _block_graph(n, e, block, inside, seed):
    """Edges mostly inside blocks of `block` consecutive node ids (a fraction
    `inside`), the rest uniform: the community layout of a local graph."""
    rng = np.random.default_rng(seed)
    v = rng.integers(0, n, e)
    local = rng.random(e) < inside
    lo = (v // block) * block
    u = np.where(local, lo + rng.integers(0, block, e), rng.integers(0, n, e))
    return np.minimum(u, n - 1), v


@pytest.mark.parametrize("dtype,d", [(np.float32, 602), (np.float32, 300), (np.float64, 256),
                                     (np.float64, 602)])
def test_gspmm_narrow_slabs_are_bit_identical(dtype, d, monkeypatch):
    """On a local graph, gspmm cuts rows wider than one 64-lane slab into
    32-lane slabs (MDGL_NARROW_SLABS, two rows per wavefront) when that makes
    at most 5 slabs: values and args bit-identical to the 64-lane layout for
    sum / mean / max / min with and without an edge weight, rows split into
    chunks or not; against the oracle bit-exact for whole rows and max/min,
    within the tolerance for split sums (chunk partials fold in chunk
    order)."""
    from mojodgl.ops import spmm

    n, e = 3000, 120000
    u, v = _block_graph(n, e, 300, 0.95, 40 + d)
    rng = np.random.default_rng(41 + d)
    x = rng.normal(size=(n, d)).astype(dtype)
    w = rng.random((e, 1)).astype(dtype)
    results = {}
    for local in (True, False):
        monkeypatch.setattr(hg, "LOCAL_FRACTION", 0.0 if local else 2.0)
        g = dgl.graph((u, v), num_nodes=n)
        assert g._local() is local
        for chunk in (512, 16):
            monkeypatch.setattr(hg, "CHUNK_LEN", chunk)
            for oop, red, L, R in (("mul", "sum", x, w), ("copy_lhs", "mean", x, None),
                                   ("copy_lhs", "max", x, None), ("mul", "min", x, w)):
                got, (au, ae) = spmm._gspmm(g, oop, red, L, R)
                results[(local, chunk, oop, red)] = (got, au, ae)
    for key, (got, au, ae) in results.items():
        local, chunk, oop, red = key
        L, R = x, (w if oop == "mul" else None)
        what = "{} {} local={} chunk={}".format(oop, red, local, chunk)
        wide = results[(False, chunk, oop, red)]
        for a_, b_ in zip((got, au, ae), wide):
            if a_ is not None:
                np.testing.assert_array_equal(a_, b_, err_msg=what + " against 64 lanes")
        if red in ("max", "min"):
            want, ru, re_ = oracle.gspmm(u, v, n, oop, red, L, R, dtype, with_arg=True)
            np.testing.assert_array_equal(au, ru, err_msg=what)
            np.testing.assert_array_equal(ae, re_, err_msg=what)
            np.testing.assert_array_equal(got, want, err_msg=what)
            continue
        want = oracle.gspmm(u, v, n, oop, red, L, R, dtype)
        if chunk == 512:
            np.testing.assert_array_equal(got, want, err_msg=what)
        else:
            absx = np.abs(x)
            bound = oracle.gspmm(u, v, n, oop, red, absx, R, dtype)
            close(got, want, bound, dtype, what)


def test_coo_locality_counts_and_graph_predicate():
    """mdgl_coo_locality: the per-workgroup counts add up to the number of
    edges with |u - v| < window (numpy), for windows 0, 1, 4096 and one past
    every difference, and for no edges; a block graph is local, a uniform one
    is not."""
    from mojodgl import _lib

    L = _lib.lib()
    rng = np.random.default_rng(44)
    n, e = 200000, 1_000_003
    u = rng.integers(0, n, e).astype(np.int32)
    v = np.where(rng.random(e) < 0.3, np.clip(u + rng.integers(-5000, 5000, e), 0, n - 1),
                 rng.integers(0, n, e)).astype(np.int32)
    ut, vt = torch.from_numpy(u).cuda(), torch.from_numpy(v).cuda()
    part = torch.full((_lib.COO_LOCALITY_BLOCKS,), -7, dtype=torch.int64, device="cuda")
    diff = np.abs(u.astype(np.int64) - v.astype(np.int64))
    for window in (0, 1, 4096, n + 1):
        assert L.mdgl_coo_locality(ut.data_ptr(), vt.data_ptr(), e, window, part.data_ptr(),
                                   _lib.stream()) == 0
        assert int(part.cpu().numpy().sum()) == int((diff < window).sum()), window
    assert L.mdgl_coo_locality(None, None, 0, 4096, part.data_ptr(), _lib.stream()) == 0
    assert np.all(part.cpu().numpy() == 0)
    assert L.mdgl_coo_locality(None, None, 0, 4096, None, _lib.stream()) == _lib.EINVAL
    bu, bv = _block_graph(100000, 500000, 4000, 0.95, 45)
    assert dgl.graph((bu, bv), num_nodes=100000)._local()
    ru, rv = rand_graph(100000, 500000, 46)
    assert not dgl.graph((ru, rv), num_nodes=100000)._local()
    none = np.zeros(0, dtype=np.int64)
    assert dgl.graph((none, none), num_nodes=5)._source_locality() == 0.0


def test_gspmm_power_law_hubs_against_oracle():
    """Degrees spanning 0 .. 5000 with the default split threshold."""
    rng = np.random.default_rng(7)
    n = 3000
    z = np.minimum(rng.zipf(2.1, n), 5000)
    deg = rng.multinomial(60000, z / z.sum())
    v = rng.permutation(np.repeat(np.arange(n), deg))
    u = rng.integers(0, n, v.size)
    x = rng.normal(size=(n, 8, 32)).astype(np.float32)
    a = rng.normal(size=(v.size, 8, 1)).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    got = ops.u_mul_e_sum(g, x, a)
    ref = oracle.gspmm(u, v, n, "mul", "sum", x, a, np.float64)
    bound = oracle.gspmm(u, v, n, "mul", "sum", np.abs(x), np.abs(a), np.float64)
    close(got, ref, bound, np.float32, "power law")
    gm, (au, ae) = ops.spmm._gspmm(g, "copy_lhs", "max", x, None)
    rm, ru, re_ = oracle.gspmm(u, v, n, "copy_lhs", "max", x, None, np.float32, with_arg=True)
    np.testing.assert_array_equal(gm, rm)
    np.testing.assert_array_equal(au, ru)
    np.testing.assert_array_equal(ae, re_)


@pytest.mark.parametrize("reduce_op", ["max", "min"])
def test_gspmm_nan_messages_are_never_selected(reduce_op):
    """max / min ignore NaN messages (strict comparison: a NaN never replaces
    the running value, IEEE maxNum / minNum); a row of only NaN messages keeps
    the identity, and update_all turns it into 0. Values and args against the
    oracle bit for bit, in whole rows and in rows split into chunks."""
    rng = np.random.default_rng(19)
    n, e = 200, 5000
    u, v = rand_graph(n, e, 20)
    v[:1500] = 4  # a hub split into chunks
    x = rng.normal(size=(n, 6)).astype(np.float32)
    w = rng.normal(size=(e, 6)).astype(np.float32)
    w[rng.random(e) < 0.2, 2] = np.nan
    w[v == int(v[3000]), 4] = np.nan  # one row: column 4 only NaN messages
    g = dgl.graph((u, v), num_nodes=n)
    got, (au, ae) = ops.spmm._gspmm(g, "mul", reduce_op, x, w)
    ref, ru, re_ = oracle.gspmm(u, v, n, "mul", reduce_op, x, w, np.float32, with_arg=True)
    assert not np.isnan(got).any()
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(au, ru)
    np.testing.assert_array_equal(ae, re_)
    assert got[int(v[3000]), 4] == (-np.inf if reduce_op == "max" else np.inf)
    g.ndata["x"] = x
    g.edata["w"] = w
    g.update_all(fn.u_mul_e("x", "w", "m"), getattr(fn, reduce_op)("m", "z"))
    assert g.ndata["z"][int(v[3000]), 4] == 0


def test_gspmm_zero_degree_and_empty_graph():
    u, v = np.array([0, 1]), np.array([1, 2])
    g = dgl.graph((u, v), num_nodes=5)
    x = np.random.default_rng(8).normal(size=(5, 4))
    e = np.ones((2, 4))
    assert np.all(ops.copy_u_max(g, x)[[0, 3, 4]] == -np.inf)
    assert np.all(ops.copy_e_min(g, e)[[0, 3, 4]] == np.inf)
    assert np.all(ops.u_mul_e_mean(g, x, e)[[0, 3, 4]] == 0)
    empty = dgl.graph((np.array([], dtype=np.int64), np.array([], dtype=np.int64)))
    assert ops.u_mul_e_sum(empty, np.zeros((0, 4)), np.zeros((0, 4))).shape == (0, 4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_graph_with_nodes_and_no_edges(dtype):
    """A graph of nodes without edges (empty GPU edge buffers, whose address
    is 0): gspmm gives every row the reduce identity (args -1), twice in a
    row (the second call a replay), update_all and pull give zeros for every
    builtin, gsddmm and edge_softmax give empty results, and the gradients
    through them are zero or empty."""
    from mojodgl.ops import spmm

    n = 37
    empty = np.zeros(0, dtype=np.int64)
    g = dgl.graph((empty, empty), num_nodes=n)
    dev = torch.device("cuda")
    x = torch.randn(n, 8, 4, dtype=dtype, device=dev)
    w = torch.randn(0, 8, 1, dtype=dtype, device=dev)
    ident = {"sum": 0.0, "mean": 0.0, "max": -np.inf, "min": np.inf}
    for _ in range(2):
        for op, L, R in (("mul", x, w), ("add", x, w), ("copy_lhs", x, None),
                         ("copy_rhs", None, w)):
            for red in ("sum", "mean", "max", "min"):
                out, (au, ae) = spmm._gspmm(g, op, red, L, R)
                assert out.shape == (n, 8, 4 if op != "copy_rhs" else 1)
                assert torch.all(out == ident[red]), (op, red)
                if au is not None:
                    assert torch.all(au == -1) and torch.all(ae == -1)
    g.ndata["x"] = x
    g.edata["w"] = w
    for msg in (fn.u_mul_e("x", "w", "m"), fn.copy_u("x", "m"), fn.copy_e("w", "m"),
                fn.u_add_v("x", "x", "m")):
        for red in ("sum", "mean", "max", "min"):
            g.update_all(msg, getattr(fn, red)("m", "h"))
            assert torch.all(g.ndata["h"] == 0)
            g.pull(np.array([0, 5, 36]), msg, getattr(fn, red)("m", "p"))
            assert torch.all(g.ndata["p"] == 0)
    g.update_all(lambda edges: {"m": edges.src["x"] * 2}, fn.sum("m", "h"))
    assert torch.all(g.ndata["h"] == 0)
    assert ops.u_add_v(g, x, x).shape == (0, 8, 4)
    assert ops.edge_softmax(g, w).shape == (0, 8, 1)
    # gradients: zero for the node operand, empty for the edge operand
    xr = x.clone().requires_grad_()
    el = torch.randn(n, 8, 1, dtype=dtype, device=dev, requires_grad=True)
    a = ops.edge_softmax(g, torch.nn.functional.leaky_relu(ops.u_add_v(g, el, el), 0.2))
    wr = a.detach().clone().requires_grad_()
    out = ops.u_mul_e_sum(g, xr, wr) + ops.u_mul_e_sum(g, xr, a)
    out.backward(torch.ones_like(out))
    assert torch.all(xr.grad == 0) and wr.grad.shape == (0, 8, 1)
    assert el.grad is None or torch.all(el.grad == 0)
    for red in ("max", "min", "mean"):
        xm = x.clone().requires_grad_()
        ops.gspmm(g, "copy_lhs", red, xm, None).sum().backward()
        assert torch.all(xm.grad == 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_gspmm_replayed_launches_match_the_full_path(dtype, monkeypatch):
    """A gspmm call shape seen before on a graph replays its launch: the
    results of the replay equal those of the full path on a fresh graph, bit
    for bit (values and args), for whole and split rows, packed and wide
    rows, broadcast operands, both copy ops (with an operand they do not read
    passed anyway), an operand one element off its allocation's start, and a
    new chunk length (the replay is dropped with the CSR it was made for);
    numpy operands and mixed dtypes always take the full path."""
    from mojodgl.ops import spmm

    n, e = 3000, 40000
    rng = np.random.default_rng(70)
    u = rng.integers(0, n, e)
    v = np.minimum(rng.zipf(1.8, e) - 1, n - 1)  # hub rows, split at chunk length 16
    dev = torch.device("cuda")
    x64 = torch.randn(n, 64, dtype=dtype, device=dev)
    x602 = torch.randn(n, 602, dtype=dtype, device=dev)
    x512 = torch.randn(n, 512, dtype=dtype, device=dev)  # several column slabs
    w512 = torch.rand(e, 512, dtype=dtype, device=dev)
    xh = torch.randn(n, 4, 16, dtype=dtype, device=dev)
    w64 = torch.rand(e, 64, dtype=dtype, device=dev)
    w1 = torch.rand(e, 1, dtype=dtype, device=dev)
    wh = torch.rand(e, 4, 1, dtype=dtype, device=dev)
    base = torch.randn(n * 64 + 1, dtype=dtype, device=dev)
    xoff = base[1:].view(n, 64)  # contiguous, one element into its allocation
    cases = [("mul", "sum", x64, w64), ("add", "max", x64, w64), ("div", "min", x64, w64),
             ("mul", "mean", x602, w1), ("mul", "sum", xh, wh), ("sub", "max", xh, wh),
             ("copy_lhs", "sum", x64, w64), ("copy_rhs", "max", x64, w64),
             ("copy_lhs", "min", x602, None), ("mul", "sum", xoff, w64),
             ("copy_lhs", "sum", x512, None), ("add", "max", x512, w512)]

    def run(g, op, red, L, R):
        out, (au, ae) = spmm._gspmm(g, op, red, L, R)
        return [t.cpu() if t is not None else None for t in (out, au, ae)]

    def same(a, b, what):
        for p, q in zip(a, b):
            assert (p is None) == (q is None), what
            if p is not None:
                assert torch.equal(p, q), what

    for chunk in (2 ** 30, 16):
        monkeypatch.setattr(hg, "CHUNK_LEN", chunk)
        g = dgl.graph((u, v), num_nodes=n)
        for op, red, L, R in cases:
            what = "{} {} {} chunk={}".format(op, red, tuple(L.shape), chunk)
            first = run(g, op, red, L, R)
            count = len(g._launches)
            assert count >= 1, what
            second = run(g, op, red, L, R)
            assert len(g._launches) == count, what  # replayed, not recorded again
            same(second, first, what + " replay")
            same(second, run(dgl.graph((u, v), num_nodes=n), op, red, L, R), what + " fresh")
    # the graph of the last round met another chunk length: its replays are
    # dropped with the CSR they were made for
    monkeypatch.setattr(hg, "CHUNK_LEN", 2 ** 30)
    for i, (op, red, L, R) in enumerate(cases[:3]):
        same(run(g, op, red, L, R), run(dgl.graph((u, v), num_nodes=n), op, red, L, R),
             "{} {} after a new chunk length".format(op, red))
        assert len(g._launches) == i + 1
    # operands the full path converts are never replayed
    g = dgl.graph((u, v), num_nodes=n)
    other = torch.float64 if dtype == torch.float32 else torch.float32
    spmm._gspmm(g, "mul", "sum", x64.cpu().numpy(), w64.cpu().numpy())
    spmm._gspmm(g, "mul", "sum", x64, w64.to(other))
    assert len(g._launches) == 0


# ------------------------------------------------------------------ gsddmm
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("lt,rt", list(itertools.permutations("uve", 2)))
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "dot"])
def test_gsddmm_all_families(dtype, lt, rt, op):
    n, e = 200, 3000
    u, v = rand_graph(n, e, 9)
    rng = np.random.default_rng(10)
    d = 12
    data = {"u": rng.normal(size=(n, d)), "v": rng.normal(size=(n, d)) + 3,
            "e": rng.normal(size=(e, d)) + 3}
    data = {k: a.astype(dtype) for k, a in data.items()}
    g = dgl.graph((u, v), num_nodes=n)
    got = getattr(ops, "{}_{}_{}".format(lt, op, rt))(g, data[lt], data[rt])
    if op != "dot":
        np.testing.assert_array_equal(got, oracle.gsddmm(u, v, n, op, data[lt], data[rt], lt, rt,
                                                         dtype))
    else:
        ref = oracle.gsddmm(u, v, n, op, data[lt], data[rt], lt, rt, np.float64)
        bound = oracle.gsddmm(u, v, n, op, np.abs(data[lt]), np.abs(data[rt]), lt, rt,
                              np.float64)
        close(got, ref, bound, dtype, "dot")


@pytest.mark.parametrize("d", [1, 3, 4, 8, 33, 128])
def test_gsddmm_widths_and_dot(d):
    n, e = 300, 5000
    u, v = rand_graph(n, e, 11)
    rng = np.random.default_rng(12)
    x = rng.normal(size=(n, d)).astype(np.float32)
    y = rng.normal(size=(e, d)).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    np.testing.assert_array_equal(ops.u_mul_v(g, x, x), oracle.gsddmm(u, v, n, "mul", x, x, "u",
                                                                       "v", np.float32))
    np.testing.assert_array_equal(ops.u_add_e(g, x, y), oracle.gsddmm(u, v, n, "add", x, y, "u",
                                                                       "e", np.float32))
    got = ops.u_dot_v(g, x, x)
    ref = oracle.gsddmm(u, v, n, "dot", x, x, "u", "v", np.float64)
    bound = oracle.gsddmm(u, v, n, "dot", np.abs(x), np.abs(x), "u", "v", np.float64)
    close(got, ref, bound, np.float32, "dot d={}".format(d))


def test_gsddmm_broadcast_copy_and_multihead_dot():
    n, e = 100, 1500
    u, v = rand_graph(n, e, 13)
    rng = np.random.default_rng(14)
    el = rng.normal(size=(n, 8, 1)).astype(np.float32)
    er = rng.normal(size=(n, 8, 1)).astype(np.float32)
    h = rng.normal(size=(n, 8, 32)).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    np.testing.assert_array_equal(ops.u_add_v(g, el, er), el[u] + er[v])
    np.testing.assert_array_equal(ops.u_mul_v(g, h, er), h[u] * er[v])
    np.testing.assert_array_equal(ops.copy_u(g, h), h[u])
    np.testing.assert_array_equal(ops.copy_v(g, h), h[v])
    got = ops.u_dot_v(g, h, h)
    assert got.shape == (e, 8, 1)
    ref = oracle.gsddmm(u, v, n, "dot", h, h, "u", "v", np.float64)
    bound = oracle.gsddmm(u, v, n, "dot", np.abs(h), np.abs(h), "u", "v", np.float64)
    close(got, ref, bound, np.float32, "multi-head dot")


# ------------------------------------------------------------------ edge_softmax
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("norm_by", ["dst", "src"])
@pytest.mark.parametrize("shape", [(), (1,), (3, 1), (8, 1), (2, 4, 1), (40, 1)])
def test_edge_softmax(dtype, norm_by, shape):
    # degrees 0 .. ~520: every row class (packed bins, wavefront rows, chunked hubs)
    n, e = 400, 6000
    u, v = rand_graph(n, e, 15)
    v[:500] = 3  # a hub above the workgroup threshold
    u[:300] = 5
    rng = np.random.default_rng(16)
    logits = (rng.normal(size=(e,) + shape) * 3).astype(dtype)
    g = dgl.graph((u, v), num_nodes=n)
    got = ops.edge_softmax(g, logits, norm_by=norm_by)
    assert got.shape == logits.shape and got.dtype == dtype
    ref = oracle.edge_softmax(u, v, n, logits, norm_by=norm_by, dtype=np.float64)
    close(got, ref, ref, dtype, "edge_softmax")
    key = v if norm_by == "dst" else u
    flat = np.asarray(got, dtype=np.float64).reshape(e, -1)
    sums = np.zeros((n, flat.shape[1]))
    np.add.at(sums, key, flat)
    np.testing.assert_allclose(sums[np.bincount(key, minlength=n) > 0], 1.0,
                               atol=1e-4 if dtype == np.float32 else 1e-12)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_edge_softmax_special_values(dtype):
    """-inf logits (masked attention) give 0 where a row has finite ones; a
    row of only -inf, or one holding NaN or +inf, gives NaN for the whole row
    and column, as the reference's max / exp / sum / divide; the same rows in
    every row class (packed, wavefront, chunked hub)."""
    n, e = 300, 4000
    u, v = rand_graph(n, e, 17)
    v[:700] = 7  # a chunked hub
    rng = np.random.default_rng(18)
    logits = rng.normal(size=(e, 2, 1)).astype(dtype)
    rows = {"part_ninf": 7, "all_ninf": int(v[800]), "nan": int(v[900]), "pinf": int(v[1000])}
    pick = lambda r: np.nonzero(v == r)[0]
    logits[pick(rows["part_ninf"])[::3], 0] = -np.inf
    logits[pick(rows["all_ninf"]), 1] = -np.inf
    logits[pick(rows["nan"])[0], 0] = np.nan
    logits[pick(rows["pinf"])[-1], 1] = np.inf
    g = dgl.graph((u, v), num_nodes=n)
    got = np.asarray(ops.edge_softmax(g, logits), dtype=np.float64)
    ref = oracle.edge_softmax(u, v, n, logits, dtype=np.float64)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    close(got[fin], ref[fin], ref[fin], dtype, "edge_softmax special values")
    assert np.isnan(got[pick(rows["all_ninf"]), 1]).all()
    assert np.isnan(got[pick(rows["nan"]), 0]).all()
    assert np.isnan(got[pick(rows["pinf"]), 1]).all()
    hub = pick(rows["part_ninf"])
    assert (got[hub[::3], 0] == 0).all() and np.isfinite(got[hub, 0]).all()


@pytest.mark.parametrize("norm_by", ["dst", "src"])
def test_edge_softmax_positional_eids(norm_by):
    rng = np.random.default_rng(17)
    for case in range(20):
        n = int(rng.integers(2, 30))
        e = int(rng.integers(1, 200))
        u, v = rng.integers(0, n, e), rng.integers(0, n, e)
        logits = rng.normal(size=(e, 2, 1))
        eids = rng.choice(e, size=int(rng.integers(1, e + 1)), replace=bool(case % 2))
        g = dgl.graph((u, v), num_nodes=n)
        got = ops.edge_softmax(g, logits, eids=eids, norm_by=norm_by)
        ref = oracle.edge_softmax(u, v, n, logits, eids=eids, norm_by=norm_by)
        close(got, ref, ref, np.float64, "eids case {}".format(case))


@pytest.mark.parametrize("norm_by", ["dst", "src"])
def test_edge_softmax_positional_eids_large_and_on_the_gpu(norm_by):
    """A subset with repeats, hubs split into chunks, ids given as a GPU tensor."""
    rng = np.random.default_rng(46)
    n, e = 2000, 60000
    u, v = rand_graph(n, e, 47)
    v[:5000] = 7
    u[:3000] = 11
    logits = (rng.normal(size=(e, 4, 1)) * 2).astype(np.float32)
    eids = rng.choice(e, size=45000, replace=True)
    g = dgl.graph((u, v), num_nodes=n)
    ref = oracle.edge_softmax(u, v, n, logits, eids=eids, norm_by=norm_by)
    got = ops.edge_softmax(g, torch.from_numpy(logits).cuda(),
                           eids=torch.from_numpy(eids).cuda(), norm_by=norm_by)
    close(got.cpu().numpy(), ref, ref, np.float32, "gpu eids")
    host = ops.edge_softmax(g, logits, eids=eids, norm_by=norm_by)
    np.testing.assert_array_equal(got.cpu().numpy(), host)
    with pytest.raises(dgl.DGLError):
        ops.edge_softmax(g, logits, eids=torch.tensor([0, e], device="cuda"), norm_by=norm_by)


def _positional_abi(ends, eids, n, logits, dtype):
    """mdgl_edge_softmax_positional on GPU copies; numpy results (out,
    endpoint, group_ptr, group_pos, id_range) after waiting on the range
    event the call records."""
    from mojodgl import _lib

    m, d = eids.size, logits.shape[1]
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    et = torch.from_numpy(ends.astype(np.int32)).cuda()
    it = torch.from_numpy(eids.astype(np.int64)).cuda()
    lg = torch.from_numpy(logits).cuda()
    out = torch.zeros((m, d), dtype=tdt, device="cuda")
    endpoint = torch.empty(m, dtype=torch.int32, device="cuda")
    gptr = torch.empty(n + 1, dtype=torch.int32, device="cuda")
    gpos = torch.empty(m, dtype=torch.int32, device="cuda")
    rng_ = torch.empty(2, dtype=torch.int64, device="cuda")
    code = _lib.dtype_code(dtype)
    L = _lib.lib()
    nbytes = L.mdgl_edge_softmax_positional_workspace_bytes(m, n, d, lg.data_ptr(),
                                                            out.data_ptr(), code)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    ev = torch.cuda.Event()
    ev.record()
    rc = L.mdgl_edge_softmax_positional(et.data_ptr(), ends.size, it.data_ptr(), m, n,
                                        lg.data_ptr(), out.data_ptr(), d, endpoint.data_ptr(),
                                        gptr.data_ptr(), gpos.data_ptr(), rng_.data_ptr(),
                                        ev.cuda_event, ws.data_ptr(), nbytes, code,
                                        _lib.stream())
    _lib.check(rc, "edge_softmax_positional")
    ev.synchronize()
    id_range = rng_.cpu().numpy()
    torch.cuda.synchronize()
    return (out.cpu().numpy(), endpoint.cpu().numpy(), gptr.cpu().numpy(), gpos.cpu().numpy(),
            id_range)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", ["mixed", "all-chunked", "all-packed", "one-node", "wide"])
def test_edge_softmax_positional_through_the_abi(dtype, case):
    """The library's positional call: endpoint[i] = ends[eids[i]], the
    grouping equals numpy's stable argsort of the endpoints (group_ptr from
    bincount), id_range the ids' min and max (read once the range event has
    fired), and the softmax the oracle's positional rule; plans with every
    row chunked, every row packed, a single node, and rows wider than one
    64-lane slab (the device figures then hold empty bins)."""
    rng = np.random.default_rng(49)
    n, e, d = {"mixed": (3000, 50000, 8), "all-chunked": (4, 50000, 1),
               "all-packed": (5000, 6000, 4), "one-node": (1, 3000, 3),
               "wide": (500, 20000, 300)}[case]
    u, v = rng.integers(0, n, e), rng.integers(0, n, e)
    if case == "mixed":
        v[:6000] = 17
    if case == "all-packed":
        v = np.arange(e) % n  # degrees of 1 and 2 only
    m = int(0.7 * e)
    eids = rng.choice(e, size=m, replace=True)
    logits = (rng.normal(size=(m, d)) * 2).astype(dtype)
    out, endpoint, gptr, gpos, id_range = _positional_abi(v, eids, n, logits, dtype)
    np.testing.assert_array_equal(endpoint, v[eids])
    np.testing.assert_array_equal(gpos, np.argsort(v[eids], kind="stable"))
    np.testing.assert_array_equal(gptr, np.concatenate([[0], np.cumsum(np.bincount(
        v[eids], minlength=n))]))
    assert list(id_range) == [eids.min(), eids.max()]
    full = np.zeros((e, d), dtype=dtype)
    full[:m] = logits
    ref = oracle.edge_softmax(u, v, n, full, eids=eids, norm_by="dst")[:m]
    close(out, ref, ref, dtype, "positional " + case)
    again = _positional_abi(v, eids, n, logits, dtype)[0]
    np.testing.assert_array_equal(out, again)


def test_edge_softmax_positional_clamps_ids_outside_the_edges():
    """Ids outside [0, E) (the API refuses them from id_range) are clamped
    for every read: the call completes and reports their true range."""
    rng = np.random.default_rng(50)
    n, e = 100, 2000
    v = rng.integers(0, n, e)
    eids = rng.integers(0, e, 500)
    eids[[3, 77]] = [-5, e + 40]
    logits = rng.normal(size=(500, 2)).astype(np.float32)
    out, endpoint, gptr, gpos, id_range = _positional_abi(v, eids, n, logits, np.float32)
    assert list(id_range) == [-5, e + 40]
    np.testing.assert_array_equal(endpoint, v[np.clip(eids, 0, e - 1)])
    assert np.isfinite(out).all()


@pytest.mark.parametrize("slots,chunk_len", [(16, 128), (64, 512), (1, 8)])
def test_softmax_plan_built_on_the_gpu_equals_the_host_plan(slots, chunk_len):
    from mojodgl.ops import _plan

    rng = np.random.default_rng(48)
    deg = np.concatenate([rng.integers(0, 3 * slots, 3000), rng.integers(0, 3 * chunk_len, 50),
                          [0, chunk_len, chunk_len + 1, slots, slots + 1, 1]])
    rng.shuffle(deg)
    indptr = np.concatenate([[0], np.cumsum(deg)])
    eid = rng.permutation(int(indptr[-1])).astype(np.int32)
    for ids in (None, eid):
        host = _plan.SoftmaxPlan(indptr, slots, chunk_len, ordered=True, eid=ids)
        dev = _plan.SoftmaxPlan.from_device(
            torch.from_numpy(indptr).cuda(), slots, chunk_len, ordered=True,
            eid=None if ids is None else torch.from_numpy(ids).cuda())
        np.testing.assert_array_equal(dev.packed.cpu().numpy(), host.packed.cpu().numpy())
        np.testing.assert_array_equal(dev.slot_of_edge.cpu().numpy(),
                                      host.slot_of_edge.cpu().numpy())
        assert dev.table_rows == host.table_rows
    assert dev.num_chunks == host.num_chunks and dev.nbins == host.nbins
    np.testing.assert_array_equal(dev.bounds, host.bounds)
    n = int(host.bounds[-1])
    np.testing.assert_array_equal(dev.order[:n].cpu().numpy(), host.order.cpu().numpy())
    for name in ("chunk_row", "chunk_start", "chunk_first"):
        np.testing.assert_array_equal(getattr(dev, name).cpu().numpy(),
                                      getattr(host, name).cpu().numpy())


# ------------------------------------------------------------------ segments
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("reducer", ["sum", "max", "min", "mean"])
@pytest.mark.parametrize("d", [1, 3, 16, 33])
def test_segment_reduce(dtype, reducer, d):
    rng = np.random.default_rng(18)
    seglen = rng.poisson(20, 3000)
    seglen[::13] = 0
    value = rng.normal(size=(int(seglen.sum()), d)).astype(dtype)
    got = ops.segment_reduce(seglen, value, reducer)
    np.testing.assert_array_equal(got, oracle.segment_reduce(seglen, value, reducer, dtype))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 4, 16, 33])
def test_segment_softmax(dtype, d):
    rng = np.random.default_rng(19)
    seglen = rng.poisson(20, 2000)
    seglen[::11] = 0
    seglen[5] = 3000  # one segment above the workgroup threshold is not special here
    value = (rng.normal(size=(int(seglen.sum()), d)) * 2).astype(dtype)
    got = ops.segment_softmax(seglen, value)
    ref = oracle.segment_softmax(seglen, value, np.float64)
    close(got, ref, ref, dtype, "segment_softmax")


@pytest.mark.parametrize("d", [1, 16, 40])
@pytest.mark.parametrize("mean", [1, 3, 7, 20, 60])
def test_segment_softmax_rows_sharing_wavefronts(mean, d):
    """Segments in their own order: several consecutive segments share a
    wavefront (fewer slots each) when the longest of them fits, and take it
    one after the other when not; with empty segments, outliers that force
    the second way, and a segment count that is no multiple of the sharing."""
    rng = np.random.default_rng(60 + mean)
    seglen = rng.poisson(mean, 1001)
    seglen[::13] = 0
    seglen[[7, 500]] = [8 * mean + 40, 3 * mean + 9]
    value = (rng.normal(size=(int(seglen.sum()), d)) * 2).astype(np.float32)
    got = ops.segment_softmax(seglen, value)
    ref = oracle.segment_softmax(seglen, value, np.float64)
    close(got, ref, ref, np.float32, "segment_softmax shared wavefronts")


@pytest.mark.parametrize("reducer", ["sum", "max", "mean"])
def test_segment_reduce_gpu_lengths(reducer):
    """Lengths given as a GPU tensor: offsets formed and checked on the GPU."""
    rng = np.random.default_rng(40)
    seglen = rng.poisson(9, 700)
    seglen[::7] = 0
    value = rng.normal(size=(int(seglen.sum()), 5)).astype(np.float32)
    got = ops.segment_reduce(torch.from_numpy(seglen).cuda(), torch.from_numpy(value).cuda(),
                             reducer)
    assert isinstance(got, torch.Tensor) and got.is_cuda
    np.testing.assert_array_equal(got.cpu().numpy(),
                                  oracle.segment_reduce(seglen, value, reducer, np.float32))


@pytest.mark.parametrize("d", [1, 16])
def test_segment_softmax_gpu_lengths_with_long_segments(d):
    """GPU lengths, with segments long enough to be split into chunks."""
    rng = np.random.default_rng(41)
    seglen = rng.poisson(12, 900)
    seglen[::17] = 0
    seglen[[3, 400, 899]] = [5000, 1300, 2049]
    value = (rng.normal(size=(int(seglen.sum()), d)) * 2).astype(np.float32)
    got = ops.segment_softmax(torch.from_numpy(seglen).cuda(), torch.from_numpy(value).cuda())
    ref = oracle.segment_softmax(seglen, value, np.float64)
    close(got.cpu().numpy(), ref, ref, np.float32, "segment_softmax gpu lengths")
    host = ops.segment_softmax(seglen, value)
    np.testing.assert_array_equal(got.cpu().numpy(), host)


def test_segment_softmax_degree_plan_through_the_abi():
    """mdgl_segment_softmax served by a degree-binned plan (packed short
    segments, wavefront segments, chunked long ones)."""
    from mojodgl import _lib
    from mojodgl.ops import _plan

    rng = np.random.default_rng(58)
    seglen = np.concatenate([rng.poisson(6, 3000), [0, 0, 700, 3000, 129, 128, 1]])
    rng.shuffle(seglen)
    d = 16
    value = (rng.normal(size=(int(seglen.sum()), d)) * 2).astype(np.float32)
    val = torch.from_numpy(value).cuda()
    out = torch.zeros_like(val)
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(seglen)]).astype(np.int32)).cuda()
    slots, chunk_len = _plan.geometry(d, np.float32, val, out)
    plan = _plan.SoftmaxPlan.from_device(off, slots, chunk_len, ordered=True)
    assert plan.packed is not None
    ws, nbytes = _plan.workspace(plan, d, np.float32)
    ref = oracle.segment_softmax(seglen, value, np.float64)
    results = []
    for packed in (plan.packed, None):  # packed slot list, and the indptr chain
        out.zero_()
        rc = _lib.lib().mdgl_segment_softmax(
            off.data_ptr(), val.data_ptr(), out.data_ptr(), None, seglen.size, d,
            value.shape[0], _lib.ptr(plan.order), plan.bounds_ptr(), plan.nbins,
            _lib.ptr(packed), _lib.ptr(plan.chunk_row), _lib.ptr(plan.chunk_start),
            _lib.ptr(plan.chunk_first), plan.num_chunks, plan.slots, _lib.ptr(ws), nbytes, 0,
            _lib.stream())
        _lib.check(rc, "segment_softmax")
        close(out.cpu().numpy(), ref, ref, np.float32, "segment_softmax degree plan")
        results.append(out.cpu().numpy())
    np.testing.assert_array_equal(results[0], results[1])


def test_segment_gpu_lengths_are_validated():
    value = torch.ones(10, 2, device="cuda")
    for bad in ([3, 3, 3], [12, -2], [4.5, 5.5], []):
        t = torch.tensor(bad, device="cuda")
        with pytest.raises(dgl.DGLError):
            ops.segment_reduce(t, value, "sum")
        with pytest.raises(dgl.DGLError):
            ops.segment_softmax(t, value)
        with pytest.raises(dgl.DGLError):  # the host lengths are refused alike
            ops.segment_reduce(np.array(bad), value.cpu().numpy(), "sum")


@pytest.mark.parametrize("num", [0, 1, 4095, 4096, 4097, 1_000_003])
def test_segment_offsets_through_the_abi(num):
    """mdgl_segment_offsets: offsets equal [0] + cumsum (int32), stats equal
    (min, sum, chunks of the long segments, max) from numpy."""
    from mojodgl import _lib

    rng = np.random.default_rng(70 + num)
    seglen = rng.poisson(5, num).astype(np.int64)
    if num > 10:
        seglen[::7] = 0
        seglen[3] = 700
    L = _lib.lib()
    sl = torch.from_numpy(seglen).cuda()
    off = torch.full((num + 1,), -5, dtype=torch.int32, device="cuda")
    stats = torch.full((4,), -5, dtype=torch.int64, device="cuda")
    nbytes = L.mdgl_segment_offsets_workspace_bytes(num)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    for chunk_len in (0, 64):
        assert L.mdgl_segment_offsets(sl.data_ptr(), num, chunk_len, off.data_ptr(),
                                      stats.data_ptr(), ws.data_ptr(), nbytes,
                                      _lib.stream()) == 0
        want = np.concatenate([[0], np.cumsum(seglen)])
        np.testing.assert_array_equal(off.cpu().numpy(), want)
        heavy = int(np.where(seglen > chunk_len, -(-seglen // chunk_len), 0).sum()) \
            if chunk_len else 0
        assert stats.tolist() == [int(seglen.min()) if num else 0, int(seglen.sum()), heavy,
                                  int(seglen.max()) if num else 0]


def test_wrapping_gpu_lengths_are_refused():
    """GPU lengths whose int64 sum wraps around to the row count: refused from
    the offsets' stats (a length above the row count) before any result is
    returned. Both segment_reduce and segment_softmax read the checks back
    while their first kernels run (those clamp every offset into the rows
    and skip rows that no segment claims) and raise before returning."""
    n = 4
    wrap = np.array([2 ** 62, 2 ** 62, 2 ** 62, 2 ** 62 + n], dtype=np.int64)
    assert int(wrap.sum()) == n  # numpy's int64 sum wraps too
    value = torch.ones(n, 3, device="cuda")
    sl = torch.from_numpy(wrap).cuda()
    for call in (lambda: ops.segment_reduce(sl, value, "sum"),
                 lambda: ops.segment_reduce(sl, value, "max"),
                 lambda: ops.segment_softmax(sl, value)):
        with pytest.raises(dgl.DGLError, match="lengths"):
            call()


def test_read_stream_reads_every_vector():
    """mdgl_read_stream folds every 16-byte vector into its wavefront's XOR
    and writes only a wavefront whose XOR is 0x9e3779b9 in its first word:
    with one such vector planted in zeros, exactly its wavefront's slot is
    written (vector i is read in round i // (2048 * 2048), by workgroup
    (i // 2048) % 2048, lane i % 256), including a vector in the last,
    partial round."""
    from mojodgl import _lib

    L = _lib.lib()
    n16 = 2048 * 2048 * 2 + 1000                     # two full rounds and a partial one
    for i in (0, 5 * 2048 + 3 * 256 + 70, 2048 * 2048 * 2 + 999):
        buf = torch.zeros(n16 * 4, dtype=torch.int32, device="cuda")
        buf[4 * i] = np.int32(np.uint32(0x9e3779b9).view(np.int32))
        sink_bytes = int(L.mdgl_read_stream_sink_bytes(n16 * 16))
        sink = torch.full((sink_bytes // 4,), 7, dtype=torch.int32, device="cuda")
        _lib.check(L.mdgl_read_stream(buf.data_ptr(), n16 * 16, sink.data_ptr(), _lib.stream()),
                   "read_stream")
        got = sink.cpu().numpy().reshape(-1, 4)
        slot = ((i % (2048 * 2048)) // 2048) * 4 + (i % 256) // 64
        want = np.full_like(got, 7)
        want[slot] = [np.uint32(0x9e3779b9).view(np.int32), 0, 0, 0]
        np.testing.assert_array_equal(got, want, err_msg=str(i))


@pytest.mark.parametrize("row_bytes,n,dst_rows", [(1024, 64 * 50 + 17, 0), (1024, 1000, 2500),
                                                   (48, 130, 7), (16, 64, 0)])
def test_read_rows_folds_the_listed_rows(row_bytes, n, dst_rows):
    """mdgl_read_rows: wavefront w (indices [64 w, 64 w + 64)) writes to
    sink[w] the XOR of every 16-byte vector of its rows, skipping indices
    outside the table (negative or past its rows); with dst_rows it writes
    each vector position's XOR over its rows to its share of dst's rows."""
    from mojodgl import _lib

    L = _lib.lib()
    rng = np.random.default_rng(row_bytes + n)
    rows, vecs = 300, row_bytes // 16
    table = rng.integers(-2 ** 31, 2 ** 31, (rows, vecs, 4), dtype=np.int64).astype(np.int32)
    idx = rng.integers(-3, rows + 3, n).astype(np.int32)
    src = torch.from_numpy(table).cuda()
    idt = torch.from_numpy(idx).cuda()
    waves = -(-n // 64)
    assert int(L.mdgl_read_rows_sink_bytes(n)) == waves * 16
    sink = torch.zeros(waves * 4, dtype=torch.int32, device="cuda")
    dst = torch.full((max(dst_rows, 1), vecs, 4), 7, dtype=torch.int32, device="cuda")
    _lib.check(L.mdgl_read_rows(src.data_ptr(), rows, row_bytes, idt.data_ptr(), n,
                                dst.data_ptr(), dst_rows, sink.data_ptr(), _lib.stream()),
               "read_rows")
    want_sink = np.zeros((waves, 4), dtype=np.int32)
    want_dst = np.full((max(dst_rows, 1), vecs, 4), 7, dtype=np.int32)
    for w in range(waves):
        sel = idx[w * 64:(w + 1) * 64]
        sel = sel[(sel >= 0) & (sel < rows)]
        per_pos = np.bitwise_xor.reduce(table[sel], axis=0) if sel.size else \
            np.zeros((vecs, 4), np.int32)
        want_sink[w] = np.bitwise_xor.reduce(per_pos, axis=0)
        for r in range(w * dst_rows // waves, (w + 1) * dst_rows // waves):
            want_dst[r] = per_pos
    np.testing.assert_array_equal(sink.cpu().numpy().reshape(waves, 4), want_sink)
    np.testing.assert_array_equal(dst.cpu().numpy(), want_dst)
    with pytest.raises(dgl.DGLError, match="row_bytes"):
        _lib.check(L.mdgl_read_rows(src.data_ptr(), rows, 24, idt.data_ptr(), n, None, 0,
                                    sink.data_ptr(), _lib.stream()), "read_rows")


# ------------------------------------------------------------------ array helpers
@pytest.mark.parametrize("n", [1, 100, 4095, 4096, 4097, 12289, 1_000_003])
def test_cumsum_clamp_replace_inf_through_the_abi(n):
    """mdgl_cumsum / mdgl_clamp_i64 / mdgl_replace_inf_with_zero (the
    reference's capi helpers) against numpy's cumsum, clip and where: exact."""
    from mojodgl import _lib

    L = _lib.lib()
    rng = np.random.default_rng(80 + n)
    src = rng.integers(-2 ** 40, 2 ** 40, n)
    a = torch.from_numpy(src).cuda()
    out = torch.full_like(a, 7)
    assert L.mdgl_cumsum(a.data_ptr(), out.data_ptr(), n, _lib.stream()) == 0
    np.testing.assert_array_equal(out.cpu().numpy(), np.cumsum(src))
    lo, hi = -2 ** 39, 2 ** 38
    assert L.mdgl_clamp_i64(a.data_ptr(), out.data_ptr(), n, lo, hi, _lib.stream()) == 0
    np.testing.assert_array_equal(out.cpu().numpy(), np.clip(src, lo, hi))
    for dtype, code in ((np.float32, 0), (np.float64, 1)):
        x = rng.normal(size=n).astype(dtype)
        x[::5] = np.inf
        x[1::7] = -np.inf
        x[2::11] = np.nan
        want = np.where(np.isinf(x), 0, x).astype(dtype)
        t = torch.from_numpy(np.concatenate([[dtype(1)], x])).cuda()
        y = torch.zeros_like(t)
        # 16-byte aligned buffers, then views one element in (element loads)
        for src, dst in ((t[1:].clone(), y[1:].clone()), (t[1:], y[1:])):
            assert L.mdgl_replace_inf_with_zero(src.data_ptr(), dst.data_ptr(), n, code,
                                                _lib.stream()) == 0
            np.testing.assert_array_equal(dst.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("width", [1, 2, 3, 4, 6, 8, 12, 16, 33])
def test_gather_rows_and_softmax_grad_through_the_abi(dtype, width):
    """mdgl_gather_rows (dst[i] = src[idx[i]]) and mdgl_edge_softmax_grad
    (a * (g - s[row_of])) against torch indexing and the formula, exact:
    16-byte aligned buffers (the 16-byte chunk path where the width allows,
    with chunks per row a power of two or not) and views one element in (the
    element path)."""
    from mojodgl import _lib

    L = _lib.lib()
    code = 0 if dtype == np.float32 else 1
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    rng = np.random.default_rng(90 + width)
    rows, n = 1000, 7001
    src = torch.from_numpy(rng.normal(size=rows * width + 1).astype(dtype)).cuda()
    idx = torch.from_numpy(rng.integers(0, rows, n).astype(np.int32)).cuda()
    out = torch.zeros(n * width + 1, dtype=tdt, device="cuda")
    for off in (0, 1):
        s_ = src[off:off + rows * width]
        o_ = out[off:off + n * width]
        assert L.mdgl_gather_rows(s_.data_ptr(), idx.data_ptr(), o_.data_ptr(), n, width, code,
                                  _lib.stream()) == 0
        want = s_.reshape(rows, width)[idx.long()].reshape(-1)
        assert torch.equal(o_, want)
    a = torch.from_numpy(rng.random(n * width + 1).astype(dtype)).cuda()
    g = torch.from_numpy(rng.normal(size=n * width + 1).astype(dtype)).cuda()
    for off in (0, 1):
        a_, g_ = a[off:off + n * width], g[off:off + n * width]
        s_ = src[off:off + rows * width]
        o_ = out[off:off + n * width]
        assert L.mdgl_edge_softmax_grad(idx.data_ptr(), a_.data_ptr(), g_.data_ptr(),
                                        s_.data_ptr(), o_.data_ptr(), n, width, code,
                                        _lib.stream()) == 0
        want = (a_.reshape(n, width) * (g_.reshape(n, width)
                                        - s_.reshape(rows, width)[idx.long()])).reshape(-1)
        assert torch.equal(o_, want)


# ------------------------------------------------------------------ dense
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d1,d2,r", [(128, 128, 64), (5, 3, 7), (16, 16, 4), (33, 130, 3),
                                     (1, 1, 2)])
def test_gather_mm(dtype, d1, d2, r):
    rng = np.random.default_rng(20)
    n = 1500
    a = rng.normal(size=(n, d1)).astype(dtype)
    b = (rng.normal(size=(r, d1, d2)) / np.sqrt(d1)).astype(dtype)
    idx = rng.integers(0, r, n)
    got = ops.gather_mm(a, b, idx_b=idx)
    ref = oracle.gather_mm(a, b, idx, np.float64)
    bound = oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64)
    close(got, ref, bound, dtype, "gather_mm")


def test_gather_mm_routes_agree(monkeypatch):
    rng = np.random.default_rng(21)
    a = rng.normal(size=(900, 9)).astype(np.float32)
    b = rng.normal(size=(6, 9, 7)).astype(np.float32)
    idx = rng.integers(0, 6, 900)
    fused = ops.gather_mm(a, b, idx_b=idx)
    monkeypatch.setattr(importlib.import_module("mojodgl.ops.gather_mm"), "_SEGMENT_BLOCK", 0)
    np.testing.assert_array_equal(ops.gather_mm(a, b, idx_b=idx), fused)


@pytest.mark.parametrize("block", [None, 0], ids=["bucketed", "sorted"])
def test_gather_mm_gpu_indices(block, monkeypatch):
    """idx_b as a GPU tensor (checked on the GPU) on both routes."""
    if block is not None:
        monkeypatch.setattr(importlib.import_module("mojodgl.ops.gather_mm"), "_SEGMENT_BLOCK",
                            block)
    rng = np.random.default_rng(42)
    a = rng.normal(size=(20000, 32)).astype(np.float32)
    b = (rng.normal(size=(300, 32, 24)) / 6).astype(np.float32)
    idx = rng.integers(0, 300, 20000)
    got = ops.gather_mm(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(),
                        idx_b=torch.from_numpy(idx).cuda())
    ref = oracle.gather_mm(a, b, idx, np.float64)
    bound = oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64)
    close(got.cpu().numpy(), ref, bound, np.float32, "gather_mm gpu idx")
    np.testing.assert_array_equal(got.cpu().numpy(), ops.gather_mm(a, b, idx_b=idx))
    bad = torch.from_numpy(idx).cuda()
    bad[7] = 300
    with pytest.raises(dgl.DGLError):
        ops.gather_mm(a, b, idx_b=bad)
    with pytest.raises(dgl.DGLError):
        ops.gather_mm(a, b, idx_b=bad[:-1])


def test_gather_mm_many_sort_chunks():
    """More row chunks than the bucketing scan has threads (several per thread)."""
    rng = np.random.default_rng(43)
    n = 2_600_000
    a = rng.normal(size=(n, 4)).astype(np.float32)
    b = rng.normal(size=(37, 4, 3)).astype(np.float32)
    idx = rng.integers(0, 37, n)
    idx[: n // 2] = np.sort(idx[: n // 2])  # long runs of one block as well as mixed rows
    got = ops.gather_mm(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(),
                        idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
    ref = oracle.gather_mm(a, b, idx, np.float64)
    bound = oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64)
    close(got, ref, bound, np.float32, "gather_mm many chunks")


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_segment_mm(dtype):
    rng = np.random.default_rng(22)
    seglen = rng.multinomial(5000, rng.dirichlet(0.5 * np.ones(16)))
    n = 5100  # 100 trailing rows outside every segment stay zero
    a = rng.normal(size=(n, 64)).astype(dtype)
    b = (rng.normal(size=(16, 64, 48)) / 8).astype(dtype)
    got = ops.segment_mm(a, b, seglen)
    ref = oracle.segment_mm(a, b, seglen, np.float64)
    bound = oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64)
    close(got, ref, bound, dtype, "segment_mm")
    assert np.all(np.asarray(got)[5000:] == 0)


# ------------------------------------------------------------------ graph build
def _csr_cases():
    rng = np.random.default_rng(44)
    hub = np.concatenate([np.zeros(30000, dtype=np.int64), rng.integers(0, 70000, 40000)])
    rng.shuffle(hub)
    return [
        ("empty", 0, np.zeros(0, np.int64), np.zeros(0, np.int64)),
        ("no edges", 7, np.zeros(0, np.int64), np.zeros(0, np.int64)),
        ("one node", 1, np.zeros(50, np.int64), np.zeros(50, np.int64)),
        ("256 nodes", 256, rng.integers(0, 256, 10000), rng.integers(0, 256, 10000)),
        ("257 nodes", 257, rng.integers(0, 257, 10000), rng.integers(0, 257, 10000)),
        ("65536 nodes", 65536, rng.integers(0, 65536, 300000), rng.integers(0, 65536, 300000)),
        ("65537 nodes", 65537, rng.integers(0, 65537, 300000), rng.integers(0, 65537, 300000)),
        ("hub", 70000, rng.integers(0, 70000, hub.size), hub),
        ("descending", 5000, np.arange(20000) % 5000, (19999 - np.arange(20000)) // 4),
        ("ends only", 1 << 20, rng.integers(0, 1 << 20, 9000),
         np.where(rng.random(9000) < 0.5, 0, (1 << 20) - 1)),
        ("17M nodes", (1 << 24) + 5, rng.integers(0, (1 << 24) + 5, 200000),
         rng.integers(0, (1 << 24) + 5, 200000)),
    ]


@pytest.mark.parametrize("case", _csr_cases(), ids=lambda c: c[0])
def test_device_csr_build_matches_the_host_sort(case):
    """The GPU radix build equals bincount / cumsum / stable argsort bit for bit."""
    _, n, u, v = case
    ud = torch.from_numpy(u.astype(np.int32)).cuda()
    vd = torch.from_numpy(v.astype(np.int32)).cuda()
    for key, other, by in ((vd, ud, "dst"), (ud, vd, "src")):
        indptr, indices, eid = hg.build_device_csr(key, other, n)
        ref = oracle.csr(u, v, n, by)
        np.testing.assert_array_equal(indptr.cpu().numpy(), ref[0])
        np.testing.assert_array_equal(indices.cpu().numpy(), ref[1])
        np.testing.assert_array_equal(eid.cpu().numpy(), ref[2])


def test_graph_queries_read_the_device_build():
    u, v = rand_graph(3000, 40000, 45)
    g = dgl.graph((u, v), num_nodes=3000)
    g._device_csr("in")
    g._device_csr("out")
    for got, by in ((g._in_csr(), "dst"), (g._out_csr(), "src")):
        for a, b in zip(got, oracle.csr(u, v, 3000, by)):
            np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(g.in_degrees(), np.bincount(v, minlength=3000))
    np.testing.assert_array_equal(g.out_degrees(), np.bincount(u, minlength=3000))


# ------------------------------------------------------------------ dispatcher
@pytest.mark.parametrize("lhs,rhs", list(itertools.permutations("uve", 2)))
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "dot"])
def test_update_all_binary_builtins(lhs, rhs, op):
    n, e = 48, 400
    u, v = rand_graph(n, e, 23)
    rng = np.random.default_rng(24)
    x = rng.normal(size=(n, 6))
    w = rng.normal(size=(e, 6)) + 3
    g = dgl.graph((u, v), num_nodes=n)
    g.ndata["x"] = x
    g.edata["e"] = w
    field = {"u": "x", "v": "x", "e": "e"}
    g.update_all(getattr(fn, "{}_{}_{}".format(lhs, op, rhs))(field[lhs], field[rhs], "m"),
                 fn.sum("m", "h"))
    data = {"u": x, "v": x, "e": w}
    msg = oracle.gsddmm(u, v, n, op, data[lhs], data[rhs], lhs, rhs)
    ref = oracle.gspmm(u, v, n, "copy_rhs", "sum", None, msg)
    close(g.ndata["h"], ref, oracle.gspmm(u, v, n, "copy_rhs", "sum", None, np.abs(msg)),
          np.float64, "update_all " + op)


def test_update_all_fused_max_min_zero_fill_and_udfs():
    u, v = np.array([0, 0, 1]), np.array([1, 1, 2])
    g = dgl.graph((u, v))
    g.ndata["h"] = np.array([[1.0], [2.0], [3.0]])
    want = [[[0.0], [1.0], [2.0]], [[0.0], [0.0], [1.0]], [[0.0], [0.0], [0.0]],
            [[0.0], [0.0], [0.0]]]
    for red, w in zip(("max", "min", "mean", "sum"), want):
        g.update_all(fn.copy_u("h", "m"), getattr(fn, red)("m", "h"))
        np.testing.assert_array_equal(g.ndata["h"], np.array(w))
    n, e = 48, 400
    u, v = rand_graph(n, e, 25)
    rng = np.random.default_rng(26)
    x, w = rng.normal(size=(n, 6)), rng.normal(size=(e, 6))
    g = dgl.graph((u, v), num_nodes=n)
    g.ndata["x"] = x
    g.edata["e"] = w
    g.update_all(lambda edges: {"m": edges.src["x"] * edges.data["e"] + 1.0}, fn.mean("m", "h"))
    ref = oracle.gspmm(u, v, n, "copy_rhs", "mean", None, x[u] * w + 1.0)
    close(g.ndata["h"], ref, oracle.gspmm(u, v, n, "copy_rhs", "mean", None,
                                          np.abs(x[u] * w) + 1.0), np.float64, "udf")
    g.update_all(fn.u_mul_e("x", "e", "m"), lambda nodes: {"s": nodes.mailbox["m"] * 2.0})
    ref = oracle.gspmm(u, v, n, "mul", "sum", x, w) * 2.0
    close(g.ndata["s"], ref, oracle.gspmm(u, v, n, "mul", "sum", np.abs(x), np.abs(w)) * 2.0,
          np.float64, "pre-summed mailbox")


def test_pull_and_readme_vector():
    g = dgl.graph((np.array([0, 1, 2, 0, 1]), np.array([1, 2, 0, 2, 2])))
    g.ndata["h"] = np.array([[1.0, 0.0], [0.0, 1.0], [2.0, 2.0]])
    g.edata["e"] = np.array([[0.5, 0.5], [1.0, 0.0], [0.0, 1.0], [2.0, 1.0], [1.0, 1.0]])
    g.update_all(fn.u_mul_e("h", "e", "m"), fn.mean("m", "z"))
    np.testing.assert_allclose(g.ndata["z"], [[0.0, 2.0], [0.5, 0.0], [2 / 3, 1 / 3]], rtol=1e-15)
    n, e = 48, 400
    u, v = rand_graph(n, e, 27)
    rng = np.random.default_rng(28)
    x, w = rng.normal(size=(n, 6)), rng.normal(size=(e, 6))
    g = dgl.graph((u, v), num_nodes=n)
    g.ndata["x"] = x
    g.edata["e"] = w
    targets = np.array([1, 5, 9, 40])
    g.pull(targets, fn.u_mul_e("x", "e", "m"), fn.sum("m", "h"))
    full = oracle.gspmm(u, v, n, "mul", "sum", x, w)
    want = np.zeros_like(full)
    want[targets] = full[targets]
    close(g.ndata["h"], want, oracle.gspmm(u, v, n, "mul", "sum", np.abs(x), np.abs(w)),
          np.float64, "pull")


@pytest.mark.parametrize("msg,red", [("u_mul_e", "sum"), ("copy_u", "mean"), ("u_add_v", "max"),
                                     ("copy_e", "min"), ("udf", "sum")])
@pytest.mark.parametrize("on_gpu", [False, True])
def test_pull_full_pass_and_subgraph_agree(msg, red, on_gpu, monkeypatch):
    """pull reduces the pulled rows of the graph's own CSR (mdgl_gspmm_rows)
    for a builtin u_op_e / copy message, and otherwise runs a builtin pass
    over every edge when the pulled rows hold many in-edges, or a subgraph of
    their in-edges (selected by the GPU grouping, in edge-id order): all give
    the reference's result (the pulled rows of a full pass, zero elsewhere;
    max / min's +-inf -> 0), bit for bit between them, and a UDF message or
    u_add_v always takes the full pass or the subgraph."""
    n, e = 300, 5000
    u, v = rand_graph(n, e, 29)
    v[:400] = 7
    rng = np.random.default_rng(30)
    x, w = rng.normal(size=(n, 5)), rng.normal(size=(e, 5))
    targets = np.array([3, 7, 8, 100, 299, 7])
    if msg == "udf":
        message = lambda edges: {"m": edges.src["x"] * edges.data["e"]}  # noqa: E731
        ref_msg = ("mul", x, w)
    elif msg == "u_add_v":
        message = fn.u_add_v("x", "x", "m")
        ref_msg = None
    else:
        message = getattr(fn, msg)(*{"u_mul_e": ("x", "e", "m"), "copy_u": ("x", "m"),
                                     "copy_e": ("e", "m")}[msg])
        ref_msg = {"u_mul_e": ("mul", x, w), "copy_u": ("copy_lhs", x, None),
                   "copy_e": ("copy_rhs", None, w)}[msg]
    got = {}
    for mode, full, rows_max in (("full", 10 ** 9, -1), ("subgraph", 0, -1),
                                 ("rows", 0, hg.PULL_ROWS_MAX_DEGREE)):
        monkeypatch.setattr(hg, "PULL_FULL_PASS", full)
        monkeypatch.setattr(hg, "PULL_ROWS_MAX_DEGREE", rows_max)
        g = dgl.graph((u, v), num_nodes=n)
        g.ndata["x"] = torch.from_numpy(x).cuda() if on_gpu else x
        g.edata["e"] = torch.from_numpy(w).cuda() if on_gpu else w
        g.pull(targets, message, getattr(fn, red)("m", "h"))
        h = g.ndata["h"]
        got[mode] = h.cpu().numpy() if isinstance(h, torch.Tensor) else np.asarray(h)
    np.testing.assert_array_equal(got["full"], got["subgraph"])
    np.testing.assert_array_equal(got["rows"], got["subgraph"])
    got[False] = got["subgraph"]
    if ref_msg is None:
        msgs = x[u] + x[v]
        full_ref = oracle.gspmm(u, v, n, "copy_rhs", red, None, msgs)
    else:
        full_ref = oracle.gspmm(u, v, n, ref_msg[0], red, ref_msg[1], ref_msg[2])
    full_ref = np.where(np.isinf(full_ref), 0.0, full_ref)
    want = np.zeros_like(full_ref)
    want[targets] = full_ref[targets]
    close(got[False], want, np.abs(want) + 1e-12, np.float64, "pull {} {}".format(msg, red))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gspmm_rows_reduces_the_listed_rows_whole(dtype):
    """mdgl_gspmm_rows through the C ABI: the listed rows of the graph's CSR,
    each whole (a row four times the chunk length folds in CSR order, bit for
    bit with the oracle for sum / mean / max / min and their args), every
    other row of the output untouched, ids outside the graph skipped and a
    row listed twice written with the same values; pull on such rows goes
    the same way and matches update_all's rows that are not split."""
    from mojodgl import _lib

    n, e = 400, 30000
    u, v = rand_graph(n, e, 61)
    v[:2048] = 5  # a row of more than CHUNK_LEN in-edges: split by update_all, whole here
    rng = np.random.default_rng(62)
    x = rng.normal(size=(n, 12)).astype(dtype)
    w = rng.normal(size=(e, 12)).astype(dtype)
    g = dgl.graph((u, v), num_nodes=n)
    csr = g._device_csr("in")
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    xt, wt = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    listed = np.array([5, 0, 399, 5, -1, 400, 123, 77], dtype=np.int32)  # 5 twice; two outside
    rows_t = torch.from_numpy(listed).cuda()
    keep = np.unique(listed[(listed >= 0) & (listed < n)])
    for red in ("sum", "mean", "max", "min"):
        out = torch.full((n, 12), 7.0, dtype=tdt, device="cuda")
        au = torch.full((n, 12), -9, dtype=torch.int32, device="cuda")
        ae = torch.full((n, 12), -9, dtype=torch.int32, device="cuda")
        rc = _lib.lib().mdgl_gspmm_rows(
            csr.indptr.data_ptr(), csr.indices.data_ptr(), csr.eid.data_ptr(), xt.data_ptr(),
            wt.data_ptr(), out.data_ptr(), n, _lib.BINARY_OPS["mul"], 12, 12, 12,
            _lib.REDUCERS[red], None, 0, None, None, au.data_ptr(), ae.data_ptr(),
            rows_t.data_ptr(), len(listed), 0, _lib.dtype_code(dtype), _lib.stream())
        _lib.check(rc, "gspmm_rows")
        got, gu, ge = out.cpu().numpy(), au.cpu().numpy(), ae.cpu().numpy()
        others = np.setdiff1d(np.arange(n), keep)
        assert np.all(got[others] == 7.0) and np.all(gu[others] == -9) and np.all(ge[others] == -9)
        if red in ("max", "min"):
            want, ru, re_ = oracle.gspmm(u, v, n, "mul", red, x, w, dtype, with_arg=True)
            np.testing.assert_array_equal(gu[keep], ru[keep], err_msg=red)
            np.testing.assert_array_equal(ge[keep], re_[keep], err_msg=red)
        else:
            want = oracle.gspmm(u, v, n, "mul", red, x, w, dtype)
        np.testing.assert_array_equal(got[keep], want[keep], err_msg=red)
    # pull takes the same path: the long row whole, others zero
    g.ndata["x"] = xt
    g.edata["e"] = wt
    g.pull(keep, fn.u_mul_e("x", "e", "m"), fn.sum("m", "h"))
    want = np.zeros((n, 12), dtype=dtype)
    want[keep] = oracle.gspmm(u, v, n, "mul", "sum", x, w, dtype)[keep]
    np.testing.assert_array_equal(g.ndata["h"].cpu().numpy(), want)


def test_graph_from_gpu_ids_is_built_on_the_gpu():
    """GPU endpoint tensors: checked on the GPU, no host copy until a host query."""
    n, e = 700, 9000
    u, v = rand_graph(n, e, 49)
    ud, vd = torch.from_numpy(u).cuda(), torch.from_numpy(v.astype(np.int32)).cuda()
    g = dgl.graph((ud, vd))
    assert g.num_nodes() == int(max(u.max(), v.max())) + 1 and g.num_edges() == e
    assert g._hu is None and g._hv is None  # nothing read back yet
    h = torch.randn(g.num_nodes(), 24, device="cuda")
    w = torch.randn(e, 24, device="cuda")
    got = ops.u_mul_e_max(g, h, w)
    assert g._hu is None and g._hv is None
    ref = ops.u_mul_e_max(dgl.graph((u, v), num_nodes=g.num_nodes()), h, w)
    assert torch.equal(got, ref)
    np.testing.assert_array_equal(g.edges().u, u)
    np.testing.assert_array_equal(g.in_degrees(), np.bincount(v, minlength=g.num_nodes()))
    with pytest.raises(dgl.DGLError):
        dgl.graph((ud, vd), num_nodes=10)
    with pytest.raises(dgl.DGLError):
        dgl.graph((ud - 1, vd))
    with pytest.raises(dgl.DGLError):
        dgl.graph((ud.double(), vd))
    # pull selects the subgraph on the GPU
    g.ndata["x"] = h
    g.edata["w"] = w
    targets = np.array([3, 17, 400])
    g.pull(targets, fn.u_mul_e("x", "w", "m"), fn.sum("m", "z"))
    full = ops.u_mul_e_sum(g, h, w)
    want = torch.zeros_like(full)
    want[targets] = full[targets]
    assert torch.equal(g.ndata["z"], want)


def test_launches_go_to_torchs_current_stream():
    from mojodgl import _lib

    assert _lib.stream() == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert _lib.stream() == side.cuda_stream
        g = dgl.graph(rand_graph(100, 1000, 60), num_nodes=100)
        x = torch.randn(100, 8, device="cuda")
        w = torch.randn(1000, 8, device="cuda")
        out = ops.u_mul_e_sum(g, x, w)
    side.synchronize()
    assert torch.equal(out, ops.u_mul_e_sum(g, x, w))


def test_update_all_replays_from_a_captured_graph():
    """update_all on GPU tensors launches without host syncs, so it can be
    captured in a HIP graph (torch.cuda.CUDAGraph) and replayed; every
    replay, with new input values, equals the eager result."""
    n, e = 3000, 40000
    u, v = rand_graph(n, e, 59)
    g = dgl.graph((u, v), num_nodes=n)
    x = torch.randn(n, 32, device="cuda")
    w = torch.randn(e, 32, device="cuda")
    g.ndata["x"] = x
    g.edata["w"] = w
    for red in ("sum", "max"):  # first calls build the CSR and schedules
        g.update_all(fn.u_mul_e("x", "w", "m"), getattr(fn, red)("m", "z_" + red))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g.update_all(fn.u_mul_e("x", "w", "m"), fn.sum("m", "z_sum"))
        g.update_all(fn.u_mul_e("x", "w", "m"), fn.max("m", "z_max"))
    out_sum, out_max = g.ndata["z_sum"], g.ndata["z_max"]
    for rep in range(3):
        x.copy_(torch.randn(n, 32, device="cuda"))
        w.copy_(torch.randn(e, 32, device="cuda"))
        graph.replay()
        torch.cuda.synchronize()
        want_sum = ops.u_mul_e_sum(dgl.graph((u, v), num_nodes=n), x, w)
        want_max = ops.u_mul_e_max(dgl.graph((u, v), num_nodes=n), x, w)
        want_max = torch.where(torch.isinf(want_max), torch.zeros_like(want_max), want_max)
        torch.cuda.synchronize()
        assert torch.equal(out_sum, want_sum), rep
        assert torch.equal(out_max, want_max), rep


def test_gat_layer_replays_from_a_captured_graph():
    """The GAT layer (gsddmm u_add_v, edge_softmax with its degree plan and
    (max, sum) table, gspmm u_mul_e_sum with a hub split into chunks and
    combined) captured in a HIP graph after the first eager call built the
    plans: every replay, with new inputs, equals the eager result bit for
    bit (no memset nodes, no host syncs inside the ops)."""
    n, e, H, D = 4000, 60000, 4, 16
    u, v = rand_graph(n, e, 61)
    v[:3000] = 7  # a hub of 3000+ in-edges: chunked rows, softmax merge
    g = dgl.graph((u, v), num_nodes=n)
    el = torch.randn(n, H, 1, device="cuda")
    er = torch.randn(n, H, 1, device="cuda")
    h = torch.randn(n, H, D, device="cuda")

    def layer():
        a = ops.edge_softmax(g, torch.nn.functional.leaky_relu(ops.u_add_v(g, el, er), 0.2))
        return ops.u_mul_e_sum(g, h, a)

    layer()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer()
    for rep in range(3):
        for t in (el, er, h):
            t.copy_(torch.randn(t.shape, device="cuda"))
        graph.replay()
        torch.cuda.synchronize()
        want = layer()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep


def test_torch_tensors_stay_on_the_gpu():
    n, e = 500, 8000
    u, v = rand_graph(n, e, 29)
    g = dgl.graph((torch.as_tensor(u), torch.as_tensor(v)), num_nodes=n)
    x = torch.randn(n, 8, 32, device="cuda")
    a = torch.rand(e, 8, 1, device="cuda")
    out = ops.u_mul_e_sum(g, x, a)
    assert isinstance(out, torch.Tensor) and out.is_cuda and out.dtype == torch.float32
    ref = oracle.gspmm(u, v, n, "mul", "sum", x.cpu().numpy(), a.cpu().numpy(), np.float64)
    bound = oracle.gspmm(u, v, n, "mul", "sum", np.abs(x.cpu().numpy()), a.cpu().numpy(),
                         np.float64)
    close(out.cpu().numpy(), ref, bound, np.float32, "torch")


def test_repeat_runs_are_bit_identical():
    """No atomics in the reductions: two runs give the same bits."""
    rng = np.random.default_rng(30)
    n = 2000
    v = rng.permutation(np.repeat(np.arange(n), np.minimum(rng.zipf(2.0, n), 3000)))
    u = rng.integers(0, n, v.size)
    g = dgl.graph((u, v), num_nodes=n)
    x = torch.randn(n, 64, device="cuda")
    w = torch.randn(v.size, 64, device="cuda")
    a = ops.u_mul_e_sum(g, x, w)
    b = ops.u_mul_e_sum(g, x, w)
    assert torch.equal(a, b)
    s1 = ops.edge_softmax(g, w[:, :1])
    s2 = ops.edge_softmax(g, w[:, :1])
    assert torch.equal(s1, s2)


def test_edge_softmax_power_law_and_mask_through_the_abi():
    """Hubs of thousands of edges (many chunks), then the C ABI's mask path
    (all_ones = 0), which the Python API never takes, against the oracle."""
    import ctypes

    from mojodgl import _lib
    from mojodgl.ops import _plan

    rng = np.random.default_rng(31)
    n = 4000
    deg = np.minimum(rng.zipf(1.8, n), 6000)
    v = rng.permutation(np.repeat(np.arange(n), deg))
    u = rng.integers(0, n, v.size)
    e = v.size
    logits = (rng.normal(size=(e, 8, 1)) * 3).astype(np.float32)
    g = dgl.graph((u, v), num_nodes=n)
    got = ops.edge_softmax(g, logits)
    ref = oracle.edge_softmax(u, v, n, logits)
    close(got, ref, ref, np.float32, "power-law edge_softmax")

    mask = (rng.random(e) < 0.6).astype(np.int8)
    csr = g._device_csr("in")
    lg = torch.from_numpy(logits.reshape(e, 8)).cuda()
    out = torch.full((e, 8), -7.0, device="cuda")
    slots, chunk_len = _plan.geometry(8, np.float32, lg, out)
    plan = csr.softmax_plan(slots, chunk_len)
    m = torch.from_numpy(mask).cuda()
    indptr, _, eid = oracle.csr(u, v, n, "dst")
    want = np.full((e, 8), -7.0)
    oracle.lib().oracle_edge_softmax(indptr.ctypes.data, eid.ctypes.data, mask.ctypes.data,
                                     np.ascontiguousarray(logits.reshape(e, 8),
                                                          dtype=np.float64).ctypes.data,
                                     want.ctypes.data, n, 0, 8, 1)
    sel = mask == 1
    assert plan.packed is not None and plan.slot_of_edge is not None
    first = None
    # one-pass and two-pass forms, each with the packed slot list and with
    # the indptr chain: all four write the same values
    for row_of in (None, plan.slot_of_edge):
        for packed in (plan.packed, None):
            out.fill_(-7.0)
            ws, nbytes = _plan.workspace(plan, 8, np.float32,
                                         plan.table_rows if row_of is not None else 0)
            rc = _lib.lib().mdgl_edge_softmax_(
                csr.indptr.data_ptr(), None, csr.eid.data_ptr(), m.data_ptr(), lg.data_ptr(),
                out.data_ptr(), None, n, 0, 8, _lib.ptr(plan.order), plan.bounds_ptr(),
                plan.nbins, _lib.ptr(packed), _lib.ptr(plan.chunk_row),
                _lib.ptr(plan.chunk_start), _lib.ptr(plan.chunk_first), plan.num_chunks,
                plan.slots, _lib.ptr(row_of), e, _lib.ptr(ws), nbytes, 0, _lib.stream())
            assert rc == 0
            got = out.cpu().numpy()
            np.testing.assert_array_equal(got[~sel], -7.0)  # unselected rows untouched
            close(got[sel], want[sel], want[sel], np.float32, "masked")
            if first is None:
                first = got
            np.testing.assert_array_equal(got, first)


@pytest.mark.parametrize("dtype,heads", [(np.float32, 8), (np.float32, 16), (np.float32, 24),
                                         (np.float64, 4), (np.float64, 8)])
def test_edge_softmax_row_pass_write_and_table_pass_agree(dtype, heads, monkeypatch):
    """edge_softmax(ALL) writes rows of whole 64-byte pieces from its row
    pass and other rows through the (max, sum) table and an edge-parallel
    pass: on a power-law graph (hub rows split into chunks, packed rows)
    both forms, forced in turn, give the same bits, within the tolerance
    of the oracle."""
    es = importlib.import_module("mojodgl.ops.edge_softmax")  # the module, not the function

    rng = np.random.default_rng(heads)
    n = 3000
    deg = np.minimum(rng.zipf(1.8, n), 5000)
    v = rng.permutation(np.repeat(np.arange(n), deg))
    u = rng.integers(0, n, v.size)
    logits = (rng.normal(size=(v.size, heads, 1)) * 3).astype(dtype)
    g = dgl.graph((u, v), num_nodes=n)
    lt = torch.from_numpy(logits).cuda()
    got = {}
    for name, row_bytes in (("row pass", 1), ("table pass", 1 << 30)):
        monkeypatch.setattr(es, "TWO_PASS_ROW_BYTES", row_bytes)
        got[name] = ops.edge_softmax(g, lt).cpu().numpy()
    np.testing.assert_array_equal(got["row pass"], got["table pass"])
    ref = oracle.edge_softmax(u, v, n, logits, dtype=np.float64)
    close(got["row pass"], ref, ref, dtype, "edge_softmax {} heads".format(heads))


def test_results_are_deterministic_run_to_run():
    """No atomics anywhere: every op gives the same bits on a second run
    (power-law rows split into chunks, packed softmax rows, grouped GEMM)."""
    rng = np.random.default_rng(90)
    n = 5000
    z = np.minimum(rng.zipf(2.1, n), 3000)
    deg = rng.multinomial(120000, z / z.sum())
    v = rng.permutation(np.repeat(np.arange(n), deg))
    u = rng.integers(0, n, v.size)
    g = dgl.graph((torch.from_numpy(u).cuda(), torch.from_numpy(v).cuda()), num_nodes=n)
    gen = torch.Generator(device="cuda").manual_seed(91)
    h = torch.randn(n, 4, 16, device="cuda", generator=gen)
    el = torch.randn(n, 4, 1, device="cuda", generator=gen)
    seglen = torch.from_numpy(rng.poisson(7, 2000)).cuda()
    val = torch.randn(int(seglen.sum()), 8, device="cuda", generator=gen)
    a = torch.randn(30000, 64, device="cuda", generator=gen)
    b = torch.randn(8, 64, 64, device="cuda", generator=gen)
    idx = torch.randint(0, 8, (30000,), device="cuda", generator=gen)

    def run():
        e = ops.u_add_v(g, el, el)
        att = ops.edge_softmax(g, e)
        return [e, att, ops.u_mul_e_sum(g, h, att), ops.copy_u_max(g, h),
                ops.u_dot_v(g, h, h), ops.segment_reduce(seglen, val, "sum"),
                ops.segment_softmax(seglen, val), ops.gather_mm(a, b, idx_b=idx)]

    first = [t.clone() for t in run()]
    for x, y in zip(first, run()):
        assert torch.equal(x, y)


def test_ops_follow_the_callers_stream():
    """Every op launches on torch's current stream and orders its own side
    copies after it: on a second stream (default priority), with the inputs
    made there by kernels still running when the ops are queued (a chain of
    large products in front of them), the results equal the default
    stream's bit for bit -- the GAT layer, segment ops with GPU lengths,
    edge_softmax over GPU eids, gather_mm and a backward pass."""
    rng = np.random.default_rng(93)
    n = 4000
    z = np.minimum(rng.zipf(2.1, n), 2000)
    deg = rng.multinomial(90000, z / z.sum())
    v = rng.permutation(np.repeat(np.arange(n), deg))
    u = rng.integers(0, n, v.size)
    E = v.size
    g = dgl.graph((torch.from_numpy(u).cuda(), torch.from_numpy(v).cuda()), num_nodes=n)
    seglen_h = rng.poisson(9, 1500)
    eids_h = rng.integers(0, E, E // 3)

    def inputs(busy):
        # the inputs come out of the stream's own queue, behind `busy`
        gen = torch.Generator(device="cuda").manual_seed(94)
        base = torch.randn(6_000_000, device="cuda", generator=gen)
        if busy:
            m = torch.randn(2048, 2048, device="cuda", generator=gen)
            for _ in range(12):
                m = torch.tanh(m @ m)
            base = base + m.sum() * 0
        h = base[:n * 64].reshape(n, 4, 16).clone()
        el = base[n * 64:n * 68].reshape(n, 4, 1).clone()
        x = base[:E * 4].reshape(E, 4, 1).clone()
        seglen = torch.from_numpy(seglen_h).cuda()
        val = base[:int(seglen_h.sum()) * 8].reshape(-1, 8).clone()
        a = base[:20000 * 64].reshape(20000, 64).clone()
        b = base[:8 * 64 * 64].reshape(8, 64, 64).clone()
        idx = torch.from_numpy(rng_idx).cuda()
        return h, el, x, seglen, val, a, b, idx

    rng_idx = rng.integers(0, 8, 20000)

    def run(busy):
        h, el, x, seglen, val, a, b, idx = inputs(busy)
        e = ops.u_add_v(g, el, el)
        att = ops.edge_softmax(g, e)
        hr = h.clone().requires_grad_()
        z = ops.u_mul_e_sum(g, hr, att)
        z.backward(torch.ones_like(z))
        return [e, att, z.detach(), hr.grad, ops.copy_u_max(g, h),
                ops.edge_softmax(g, x, eids=torch.from_numpy(eids_h).cuda()),
                ops.segment_reduce(seglen, val, "max"), ops.segment_softmax(seglen, val),
                ops.gather_mm(a, b, idx_b=idx)]

    want = [t.clone() for t in run(False)]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        got = run(True)
    side.synchronize()
    for i, (x, y) in enumerate(zip(want, got)):
        assert torch.equal(x, y), i


def test_ops_from_several_threads_share_a_graph():
    """Four Python threads, each on its own stream, run the GAT layer, a
    pull, segment ops with GPU lengths and gather_mm over one graph whose
    device CSR, softmax plan and launch cache they build on first use
    concurrently; every result equals the one computed alone on a separate
    graph of the same edges (the library keeps its error text per thread and
    has no other mutable state but the no-alloc scratch)."""
    import threading

    rng = np.random.default_rng(95)
    n = 3000
    z = np.minimum(rng.zipf(2.1, n), 1500)
    deg = rng.multinomial(60000, z / z.sum())
    v = rng.permutation(np.repeat(np.arange(n), deg))
    u = rng.integers(0, n, v.size)
    gen = torch.Generator(device="cuda").manual_seed(96)
    h = torch.randn(n, 4, 16, device="cuda", generator=gen)
    el = torch.randn(n, 4, 1, device="cuda", generator=gen)
    seglen = torch.from_numpy(rng.poisson(6, 1000)).cuda()
    val = torch.randn(int(seglen.sum()), 8, device="cuda", generator=gen)
    a = torch.randn(10000, 64, device="cuda", generator=gen)
    b = torch.randn(8, 64, 64, device="cuda", generator=gen)
    idx = torch.randint(0, 8, (10000,), device="cuda", generator=gen)
    pulled = np.arange(0, n, 3)

    def run(g, tag):
        # features under names of the thread's own
        e = ops.u_add_v(g, el, el)
        att = ops.edge_softmax(g, e)
        g.ndata["h" + tag] = h
        g.edata["a" + tag] = att
        g.pull(pulled, fn.u_mul_e("h" + tag, "a" + tag, "m"), fn.sum("m", "p" + tag))
        return [e, att, ops.u_mul_e_sum(g, h, att), g.ndata["p" + tag], ops.copy_u_max(g, h),
                ops.segment_reduce(seglen, val, "sum"), ops.segment_softmax(seglen, val),
                ops.gather_mm(a, b, idx_b=idx)]

    want = [t.clone() for t in run(dgl.graph((u, v), num_nodes=n), "")]
    torch.cuda.synchronize()
    shared = dgl.graph((u, v), num_nodes=n)
    results, errors = {}, []

    def worker(k):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                outs = [run(shared, str(k)) for _ in range(3)]
                outs = [[t.clone() for t in o] for o in outs]
            s.synchronize()
            results[k] = outs
        except Exception as exc:  # reported below, in the test's thread
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert sorted(results) == [0, 1, 2, 3]
    for k, outs in results.items():
        for rep, got in enumerate(outs):
            for i, (x, y) in enumerate(zip(want, got)):
                assert torch.equal(x, y), (k, rep, i)


@pytest.mark.parametrize("d1", [32, 64, 96, 128])
@pytest.mark.parametrize("d2", [1, 5, 128, 130, 256])
def test_grouped_mm_block_resident_shapes(d1, d2):
    """The float32 kernel on the bf16 matrix cores, which keeps a b block in
    LDS (K a multiple of 32 up to 128, rows of a 16-byte aligned): every
    chunk count, output widths below, at and past one 128-column tile (odd
    widths store element by element), groups that are empty, shorter than a
    256-row tile or span many tiles; segment_mm (consecutive groups) and
    gather_mm (rows through the bucketing permutation) against the oracle,
    and gather_mm against segment_mm on the stably sorted rows bit for bit
    (same kernel, same per-row arithmetic)."""
    rng = np.random.default_rng(d1 * 1000 + d2)
    r = 11
    seglen = np.array([0, 1, 127, 255, 256, 257, 700, 0, 3, 2000, 129])
    n = int(seglen.sum())
    a = rng.normal(size=(n, d1)).astype(np.float32)
    b = (rng.normal(size=(r, d1, d2)) / np.sqrt(d1)).astype(np.float32)
    got = ops.segment_mm(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), seglen)
    got = got.cpu().numpy()
    close(got, oracle.segment_mm(a, b, seglen, np.float64),
          oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64), np.float32,
          "segment_mm d1 {} d2 {}".format(d1, d2))
    idx = np.repeat(np.arange(r), seglen)
    rng.shuffle(idx)
    gm = ops.gather_mm(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(),
                       idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
    close(gm, oracle.gather_mm(a, b, idx, np.float64),
          oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64), np.float32,
          "gather_mm d1 {} d2 {}".format(d1, d2))
    perm = np.argsort(idx, kind="stable")
    want = np.empty_like(gm)
    want[perm] = ops.segment_mm(a[perm], b, np.bincount(idx, minlength=r))
    np.testing.assert_array_equal(gm, want)


@pytest.mark.parametrize("d1", [16, 48, 64, 112, 128])
@pytest.mark.parametrize("d2", [1, 5, 128, 130, 256])
def test_grouped_mm_float64_block_resident_shapes(d1, d2):
    """The float64 kernel that keeps a b block in LDS (K a multiple of 16 up
    to 128, rows of a 16-byte aligned): odd and even chunk counts, output
    widths below, at and past one 128-column tile (columns past the width
    and rows past a group go to the store sink), groups that are empty,
    shorter than a 128-row tile or span many tiles; segment_mm and gather_mm
    against the oracle, and gather_mm against segment_mm on the stably
    sorted rows bit for bit."""
    rng = np.random.default_rng(d1 * 1000 + d2 + 7)
    r = 11
    seglen = np.array([0, 1, 127, 128, 129, 255, 700, 0, 3, 2000, 257])
    n = int(seglen.sum())
    a = rng.normal(size=(n, d1))
    b = rng.normal(size=(r, d1, d2)) / np.sqrt(d1)
    idx = np.repeat(np.arange(r), seglen)
    rng.shuffle(idx)
    at, bt = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    out = torch.full((n + 1, d2), 7.0, dtype=torch.float64, device="cuda")
    seg = ops.segment_mm(at, bt, seglen).cpu().numpy()
    close(seg, oracle.segment_mm(a, b, seglen, np.float64),
          oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64), np.float64,
          "segment_mm d1 {} d2 {}".format(d1, d2))
    gm = ops.gather_mm(at, bt, idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
    close(gm, oracle.gather_mm(a, b, idx, np.float64),
          oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64), np.float64,
          "gather_mm d1 {} d2 {}".format(d1, d2))
    perm = np.argsort(idx, kind="stable")
    want = np.empty_like(gm)
    want[perm] = ops.segment_mm(a[perm], b, np.bincount(idx, minlength=r))
    np.testing.assert_array_equal(gm, want)
    # through the ABI into a buffer one row longer: the row past n is untouched
    from mojodgl import _lib
    L = _lib.lib()
    code = _lib.dtype_code(np.float64)
    ws_n = L.mdgl_segment_mm_workspace_bytes(n, d1, d2, r, code)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    sl = torch.from_numpy(seglen.astype(np.int64)).cuda()
    assert L.mdgl_segment_mm(at.data_ptr(), bt.data_ptr(), out.data_ptr(), sl.data_ptr(), n, d1,
                             r, d2, ws.data_ptr(), ws_n, code, _lib.stream()) == 0
    o = out.cpu().numpy()
    np.testing.assert_array_equal(o[:n], seg)
    assert np.all(o[n] == 7.0)


@pytest.mark.parametrize("case", ["inf_nan", "k_not_16", "unaligned"])
def test_grouped_mm_float64_other_paths(case):
    """float64 beside the block-resident kernel: inf and NaN propagate as in
    IEEE arithmetic (the oracle on the same values), and shapes it does not
    take (K not a multiple of 16, rows of a off a 16-byte boundary) go to the
    general kernel with results within the tolerance rule."""
    rng = np.random.default_rng(73)
    r = 5
    seglen = np.array([300, 0, 129, 1000, 77])
    n = int(seglen.sum())
    k = 24 if case == "k_not_16" else 64
    a = rng.normal(size=(n, k))
    b = rng.normal(size=(r, k, 40)) / np.sqrt(k)
    if case == "inf_nan":
        a[3, 5] = np.inf
        a[10, 0] = -np.inf
        a[20, 7] = np.nan
        b[3, 9, 1] = np.inf
    at = torch.from_numpy(a).cuda()
    if case == "unaligned":
        flat = torch.empty(n * k + 1, dtype=torch.float64, device="cuda")
        at = flat[1:].view(n, k)
        at.copy_(torch.from_numpy(a))
    idx = np.repeat(np.arange(r), seglen)
    seg = ops.segment_mm(at, torch.from_numpy(b).cuda(), seglen).cpu().numpy()
    gat = ops.gather_mm(at, torch.from_numpy(b).cuda(),
                        idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
    with np.errstate(all="ignore"):
        ref = oracle.segment_mm(a, b, seglen, np.float64)
        bound = oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64)
    for got, what in ((seg, "segment_mm"), (gat, "gather_mm")):
        fin = np.isfinite(ref)
        assert np.array_equal(np.isnan(got), np.isnan(ref)), what
        assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)]), what
        close(got[fin], ref[fin], bound[fin], np.float64, what)
    np.testing.assert_array_equal(seg, gat)


def _grouped_both(a, b, seglen, idx):
    """segment_mm and gather_mm of the same rows on the GPU (numpy out)."""
    at, bt = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    seg = ops.segment_mm(at, bt, seglen).cpu().numpy()
    gat = ops.gather_mm(at, bt, idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
    return seg, gat


def test_grouped_mm_non_finite_and_out_of_range_values():
    """Values the bf16 split does not take (inf, NaN, magnitudes from 2^60
    up and below 2^-50 but non-zero) send their chunk of a, or every chunk of
    a group whose b holds one, to float32 MFMAs: inf and NaN land where IEEE
    arithmetic puts them (the oracle in float64 on the same float32 values),
    every finite result stays within the tolerance rule, and rows that share
    a chunk with such a value are unaffected."""
    rng = np.random.default_rng(71)
    k, r = 128, 6
    seglen = np.array([300, 40, 500, 256, 7, 400])
    n = int(seglen.sum())
    a = rng.normal(size=(n, k)).astype(np.float32)
    b = (rng.normal(size=(r, k, k)) / np.sqrt(k)).astype(np.float32)
    a[3, 5] = np.inf           # group 0
    a[10, 0] = -np.inf
    a[20, 77] = np.nan
    a[350, :16] = 1e30         # group 2: huge, finite products
    a[351, 3] = 1e-30          # tiny next to normal values in its chunk
    a[360] *= 1e-30            # a whole row of tiny values
    a[1100:1110] = 0.0         # exact zeros take the bf16 path
    b[1, 9, 1] = np.inf        # group 1: every chunk on float32 MFMAs
    b[3, 0, :] = 1e-30         # group 3: tiny b values
    b[5, 4, 4] = 3e20          # group 5: a huge b value
    idx = np.repeat(np.arange(r), seglen)
    seg, gat = _grouped_both(a, b, seglen, idx)
    with np.errstate(all="ignore"):
        ref = oracle.segment_mm(a, b, seglen, np.float64)
        bound = oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64)
    for got, what in ((seg, "segment_mm"), (gat, "gather_mm")):
        fin = np.isfinite(ref)
        assert np.array_equal(np.isnan(got), np.isnan(ref)), what
        assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)].astype(np.float32)), what
        assert int((~fin).sum()) > 0
        close(got[fin], ref[fin], bound[fin], np.float32, what)
    np.testing.assert_array_equal(seg, gat)


def test_grouped_mm_float32_accuracy():
    """The bf16-split products keep float32 accuracy: against float64, the
    error relative to sum |a b| over 20,000 rows (K = 128) is no larger than
    that of the vendor float32 GEMM (torch.mm, used here only as the
    yardstick) on the same rows, and within float32's unit roundoff
    (2^-24 = 6e-8) on average."""
    rng = np.random.default_rng(72)
    k, r, n = 128, 4, 20000
    seglen = np.full(r, n // r)
    a = rng.normal(size=(n, k)).astype(np.float32)
    b = (rng.normal(size=(r, k, k)) / np.sqrt(k)).astype(np.float32)
    idx = np.repeat(np.arange(r), seglen)
    seg, gat = _grouped_both(a, b, seglen, idx)
    ref = oracle.segment_mm(a, b, seglen, np.float64)
    scale = oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64)
    torch.backends.cuda.matmul.allow_tf32 = False
    at = torch.from_numpy(a).cuda()
    vendor = torch.cat([at[i * (n // r):(i + 1) * (n // r)] @ torch.from_numpy(b[i]).cuda()
                        for i in range(r)]).cpu().numpy()
    e_v = np.abs(vendor - ref) / scale
    for got in (seg, gat):
        e = np.abs(got - ref) / scale
        assert e.mean() <= 1.1 * e_v.mean() and e.mean() < 2 ** -24, (e.mean(), e_v.mean())
        assert e.max() <= 1.5 * e_v.max(), (e.max(), e_v.max())
