"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check uses a method independent of the oracle's own loops: the
reference's printed known answers (tests/golden/reference_vectors.json),
closed forms (bincount / cumsum / stable argsort), numpy's unbuffered
`ufunc.at` (which folds duplicate indices in array order, i.e. ascending edge
id = the CSR order, so sums compare bit for bit), `np.broadcast_to` on
explicitly expanded operands, einsum, and brute-force loops on tiny inputs.
Integer-valued inputs make every sum exact whatever the order, so a wrong
index, operand or target fails them outright.
"""

import itertools
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_vectors.json")
DTYPES = [np.float32, np.float64]


def rand_graph(n, e, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, n, e), rng.integers(0, n, e)


def msg_np(op, x, y):
    return {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide}[op](x, y)


# --------------------------------------------------------------- graph / CSR
def test_csr_matches_closed_form_and_brute_force():
    u, v = rand_graph(37, 300, 1)
    for by, key, other in (("dst", v, u), ("src", u, v)):
        indptr, indices, eid = oracle.csr(u, v, 37, by)
        np.testing.assert_array_equal(np.diff(indptr), np.bincount(key, minlength=37))
        for node in range(37):
            want = [e for e in range(300) if key[e] == node]  # ascending edge id
            got = eid[indptr[node]:indptr[node + 1]].tolist()
            assert got == want
            assert indices[indptr[node]:indptr[node + 1]].tolist() == [int(other[e]) for e in want]


def test_array_primitives_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.integers(-50, 50, 1000)
    np.testing.assert_array_equal(oracle.cumsum(x), np.cumsum(x))
    np.testing.assert_array_equal(oracle.clamp_i64(x, -3, 7), np.clip(x, -3, 7))
    f = rng.normal(size=5000)
    f[::7] = np.inf
    f[::11] = -np.inf
    for dt in DTYPES:
        got = oracle.replace_inf_with_zero(f, dt)
        np.testing.assert_array_equal(got, np.where(np.isinf(f), 0, f).astype(dt))


# --------------------------------------------------------------- gspmm
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_gspmm_sum_mean_bit_exact_against_ufunc_at(dtype, op):
    n, e, d = 50, 700, 5
    u, v = rand_graph(n, e, 2)
    rng = np.random.default_rng(3)
    x = rng.normal(size=(n, d)).astype(dtype)
    w = (rng.random((e, d)) + 0.5).astype(dtype)
    m = msg_np(op, x[u], w)
    want = np.zeros((n, d), dtype=dtype)
    np.add.at(want, v, m)
    got = oracle.gspmm(u, v, n, op, "sum", x, w, dtype)
    np.testing.assert_array_equal(got, want)
    deg = np.maximum(np.bincount(v, minlength=n), 1).astype(dtype)
    got = oracle.gspmm(u, v, n, op, "mean", x, w, dtype)
    np.testing.assert_array_equal(got, want / deg[:, None])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("reduce_op", ["max", "min"])
def test_gspmm_max_min_values_and_args(dtype, reduce_op):
    n, e, d = 30, 400, 4
    u, v = rand_graph(n, e, 4)
    rng = np.random.default_rng(5)
    # small integers make ties frequent, so the tie rule is exercised
    x = rng.integers(-3, 4, (n, d)).astype(dtype)
    w = rng.integers(1, 3, (e, d)).astype(dtype)
    m = x[u] * w
    ident = -np.inf if reduce_op == "max" else np.inf
    want = np.full((n, d), ident, dtype=dtype)
    (np.maximum if reduce_op == "max" else np.minimum).at(want, v, m)
    got, au, ae = oracle.gspmm(u, v, n, "mul", reduce_op, x, w, dtype, with_arg=True)
    np.testing.assert_array_equal(got, want)
    for node in range(n):
        edges = np.nonzero(v == node)[0]  # ascending edge id
        for k in range(d):
            if edges.size == 0:
                assert au[node, k] == -1 and ae[node, k] == -1
                continue
            first = edges[np.nonzero(m[edges, k] == want[node, k])[0][0]]
            assert ae[node, k] == first and au[node, k] == u[first]


@pytest.mark.parametrize("dtype", DTYPES)
def test_gspmm_copy_ops(dtype):
    n, e, d = 40, 333, 3
    u, v = rand_graph(n, e, 6)
    rng = np.random.default_rng(7)
    x = rng.normal(size=(n, d)).astype(dtype)
    w = rng.normal(size=(e, d)).astype(dtype)
    for op, data, src in (("copy_lhs", x, x[u]), ("copy_rhs", w, w)):
        want = np.zeros((n, d), dtype=dtype)
        np.add.at(want, v, src)
        np.testing.assert_array_equal(oracle.gspmm(u, v, n, op, "sum", data if op == "copy_lhs"
                                                   else None, data if op == "copy_rhs" else None,
                                                   dtype), want)


@pytest.mark.parametrize("lshape,rshape", [((8, 4), (8, 1)), ((8, 1), (8, 6)), ((3, 4), (1,)),
                                           ((2, 3, 4), (2, 1, 4)), ((2, 3, 4), (3, 1)),
                                           ((1, 3), (5, 1))])
def test_gspmm_broadcast_equals_explicit_expansion(lshape, rshape):
    n, e = 20, 150
    u, v = rand_graph(n, e, 8)
    rng = np.random.default_rng(9)
    x = rng.normal(size=(n,) + lshape)
    w = rng.normal(size=(e,) + rshape)
    xs, ws = oracle.reshape_lhs_rhs(x.shape, w.shape)
    x2, w2 = x.reshape(xs), w.reshape(ws)
    out_f = np.broadcast_shapes(xs[1:], ws[1:])
    xe = np.ascontiguousarray(np.broadcast_to(x2, (n,) + out_f))
    we = np.ascontiguousarray(np.broadcast_to(w2, (e,) + out_f))
    got = oracle.gspmm(u, v, n, "mul", "sum", x, w)
    want = oracle.gspmm(u, v, n, "mul", "sum", xe, we)
    assert got.shape == (n,) + out_f
    np.testing.assert_array_equal(got, want)
    ref = np.zeros((n,) + out_f)
    np.add.at(ref, v, xe[u] * we)
    np.testing.assert_array_equal(got, ref)


def test_gspmm_zero_in_degree_rows_keep_identity():
    u, v = np.array([0, 1]), np.array([1, 2])
    x = np.ones((5, 3))
    w = np.ones((2, 3))
    assert np.all(oracle.gspmm(u, v, 5, "add", "sum", x, w)[[0, 3, 4]] == 0)
    assert np.all(oracle.gspmm(u, v, 5, "copy_lhs", "max", x, None)[[0, 3, 4]] == -np.inf)
    assert np.all(oracle.gspmm(u, v, 5, "copy_rhs", "min", None, w)[[0, 3, 4]] == np.inf)
    assert np.all(oracle.gspmm(u, v, 5, "mul", "mean", x, w)[[0, 3, 4]] == 0)


# --------------------------------------------------------------- gsddmm
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("lt,rt", list(itertools.permutations("uve", 2)))
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_gsddmm_elementwise_bit_exact(dtype, lt, rt, op):
    n, e, d = 25, 120, 3
    u, v = rand_graph(n, e, 10)
    rng = np.random.default_rng(11)
    data = {"u": rng.normal(size=(n, d)), "v": rng.normal(size=(n, d)) + 3.0,
            "e": rng.normal(size=(e, d)) + 3.0}
    data = {k: a.astype(dtype) for k, a in data.items()}
    rows = {"u": u, "v": v, "e": np.arange(e)}
    want = msg_np(op, data[lt][rows[lt]], data[rt][rows[rt]])
    got = oracle.gsddmm(u, v, n, op, data[lt], data[rt], lt, rt, dtype)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("lt,rt", list(itertools.permutations("uve", 2)))
def test_gsddmm_dot_exact_on_integers_and_close_on_reals(lt, rt):
    n, e = 25, 120
    u, v = rand_graph(n, e, 12)
    rows = {"u": u, "v": v, "e": np.arange(e)}
    rng = np.random.default_rng(13)
    for d in (1, 3, 4, 8, 33):
        ints = {k: rng.integers(-9, 10, (n if k != "e" else e, d)).astype(np.float64)
                for k in "uve"}
        got = oracle.gsddmm(u, v, n, "dot", ints[lt], ints[rt], lt, rt)
        want = np.einsum("ij,ij->i", ints[lt][rows[lt]], ints[rt][rows[rt]])[:, None]
        np.testing.assert_array_equal(got, want)
        reals = {k: rng.normal(size=a.shape) for k, a in ints.items()}
        got = oracle.gsddmm(u, v, n, "dot", reals[lt], reals[rt], lt, rt)
        want = np.einsum("ij,ij->i", reals[lt][rows[lt]], reals[rt][rows[rt]])[:, None]
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_gsddmm_copy_and_broadcast():
    n, e = 12, 60
    u, v = rand_graph(n, e, 14)
    rng = np.random.default_rng(15)
    x = rng.normal(size=(n, 4, 3))
    y = rng.normal(size=(n, 4, 1))
    np.testing.assert_array_equal(oracle.gsddmm(u, v, n, "copy_lhs", x, None, "u"), x[u])
    np.testing.assert_array_equal(oracle.gsddmm(u, v, n, "copy_rhs", None, x, "u", "v"), x[v])
    np.testing.assert_array_equal(oracle.gsddmm(u, v, n, "add", x, y, "u", "v"), x[u] + y[v])
    # multi-head dot contracts the last axis and broadcasts the others
    z = rng.normal(size=(n, 1, 3))
    got = oracle.gsddmm(u, v, n, "dot", x, z, "u", "v")
    assert got.shape == (e, 4, 1)
    np.testing.assert_allclose(got[..., 0], np.einsum("ehk,ehk->eh", x[u], np.broadcast_to(
        z[v], (e, 4, 3))), rtol=1e-12)


# --------------------------------------------------------------- edge_softmax
def _softmax_groups(key, logits, groups_of):
    out = np.zeros_like(logits)
    for members in groups_of:
        w = logits[members]
        ex = np.exp(w - w.max(axis=0))
        out[members] = ex / ex.sum(axis=0)
    return out


@pytest.mark.parametrize("norm_by", ["dst", "src"])
@pytest.mark.parametrize("heads", [1, 3, 8])
def test_edge_softmax_against_brute_force(norm_by, heads):
    n, e = 30, 260
    u, v = rand_graph(n, e, 16)
    logits = np.random.default_rng(17).normal(size=(e, heads, 1)) * 4
    got = oracle.edge_softmax(u, v, n, logits, norm_by=norm_by)
    key = v if norm_by == "dst" else u
    flat = logits.reshape(e, heads)
    want = _softmax_groups(key, flat, [np.nonzero(key == k)[0] for k in range(n)])
    np.testing.assert_allclose(got.reshape(e, heads), want, rtol=1e-13, atol=1e-15)
    sums = np.zeros((n, heads))
    np.add.at(sums, key, got.reshape(e, heads))
    np.testing.assert_allclose(sums[np.bincount(key, minlength=n) > 0], 1.0, atol=1e-13)


@pytest.mark.parametrize("norm_by", ["dst", "src"])
def test_edge_softmax_positional_eids_rule(norm_by):
    """The rule of tests/test_edge_softmax_eids.py:41-71, as a brute-force loop."""
    rng = np.random.default_rng(21)
    for case in range(40):
        n = int(rng.integers(2, 12))
        e = int(rng.integers(1, 40))
        u, v = rng.integers(0, n, e), rng.integers(0, n, e)
        logits = rng.normal(size=(e, 1))
        eids = rng.choice(e, size=int(rng.integers(1, e + 1)), replace=bool(case % 3 == 0))
        key = (v if norm_by == "dst" else u)
        want = np.zeros((e, 1))
        for i in range(len(eids)):
            group = [j for j in range(len(eids)) if key[eids[j]] == key[eids[i]]]
            w = logits[np.array(group)]
            ex = np.exp(w - w.max())
            want[i] = (ex / ex.sum())[group.index(i)]
        got = oracle.edge_softmax(u, v, n, logits, eids=eids, norm_by=norm_by)
        np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-15)


# --------------------------------------------------------------- segments
def _segments(seglen):
    off = np.concatenate([[0], np.cumsum(seglen)])
    return [np.arange(off[i], off[i + 1]) for i in range(len(seglen))]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("reducer", ["sum", "max", "min", "mean"])
def test_segment_reduce_bit_exact(dtype, reducer):
    rng = np.random.default_rng(22)
    seglen = rng.poisson(3, 200)
    seglen[::9] = 0
    value = rng.normal(size=(int(seglen.sum()), 5)).astype(dtype)
    segs = _segments(seglen)
    want = np.zeros((len(seglen), 5), dtype=dtype)
    ids = np.repeat(np.arange(len(seglen)), seglen)
    if reducer in ("sum", "mean"):
        np.add.at(want, ids, value)
        if reducer == "mean":
            want = want / np.maximum(seglen, 1).astype(dtype)[:, None]
    else:
        acc = np.full((len(seglen), 5), -np.inf if reducer == "max" else np.inf, dtype=dtype)
        (np.maximum if reducer == "max" else np.minimum).at(acc, ids, value)
        want = np.where(np.isinf(acc), 0, acc).astype(dtype)
    got = oracle.segment_reduce(seglen, value, reducer, dtype)
    np.testing.assert_array_equal(got, want)
    del segs


@pytest.mark.parametrize("dtype", DTYPES)
def test_segment_softmax_against_brute_force(dtype):
    rng = np.random.default_rng(23)
    seglen = rng.poisson(4, 100)
    seglen[::7] = 0
    value = rng.normal(size=(int(seglen.sum()), 4)).astype(dtype)
    got = oracle.segment_softmax(seglen, value, dtype)
    want = np.zeros_like(value, dtype=np.float64)
    for s in _segments(seglen):
        if s.size:
            w = value[s].astype(np.float64)
            ex = np.exp(w - w.max(axis=0))
            want[s] = ex / ex.sum(axis=0)
    tol = 1e-13 if dtype == np.float64 else 2e-6
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol * 1e-2)


# --------------------------------------------------------------- dense
@pytest.mark.parametrize("d1,d2,r", [(5, 3, 7), (16, 16, 4), (4, 9, 2)])
def test_gather_mm_against_einsum(d1, d2, r):
    rng = np.random.default_rng(24)
    n = 300
    ai = rng.integers(-5, 6, (n, d1)).astype(np.float64)
    bi = rng.integers(-5, 6, (r, d1, d2)).astype(np.float64)
    idx = rng.integers(0, r, n)
    np.testing.assert_array_equal(oracle.gather_mm(ai, bi, idx),
                                  np.einsum("ij,ijk->ik", ai, bi[idx]))
    a, b = rng.normal(size=ai.shape), rng.normal(size=bi.shape)
    np.testing.assert_allclose(oracle.gather_mm(a, b, idx), np.einsum("ij,ijk->ik", a, b[idx]),
                               rtol=1e-12, atol=1e-12)


def test_segment_mm_against_matmul_and_trailing_rows_zero():
    rng = np.random.default_rng(25)
    seglen = np.array([10, 5, 0, 3])
    a = rng.integers(-5, 6, (20, 4)).astype(np.float64)
    b = rng.integers(-5, 6, (4, 4, 3)).astype(np.float64)
    got = oracle.segment_mm(a, b, seglen)
    off = np.concatenate([[0], np.cumsum(seglen)])
    for i in range(4):
        np.testing.assert_array_equal(got[off[i]:off[i + 1]], a[off[i]:off[i + 1]] @ b[i])
    assert np.all(got[18:] == 0)


# --------------------------------------------------------------- threading
def test_worker_split_is_exact():
    """Above PARALLEL_MIN the 32-way split must give bit-identical results."""
    n, e = 9000, 40000
    u, v = rand_graph(n, e, 26)
    rng = np.random.default_rng(27)
    x, w = rng.normal(size=(n, 3)), rng.normal(size=(e, 3))
    old = oracle.set_workers(32)
    try:
        many = oracle.gspmm(u, v, n, "mul", "sum", x, w)
        soft = oracle.edge_softmax(u, v, n, w[:, :1])
        oracle.set_workers(1)
        np.testing.assert_array_equal(oracle.gspmm(u, v, n, "mul", "sum", x, w), many)
        np.testing.assert_array_equal(oracle.edge_softmax(u, v, n, w[:, :1]), soft)
    finally:
        oracle.set_workers(old)


# --------------------------------------------------------------- golden vectors
def _golden():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.mark.parametrize("vec", _golden(), ids=lambda v: v["name"])
def test_reference_vectors(vec):
    op = vec["op"]
    if op == "update_all":
        u, v = np.array(vec["u"]), np.array(vec["v"])
        n = int(max(u.max(), v.max())) + 1
        mname, a, b = vec["message"][0], vec["message"][1], vec["message"][2]
        red = vec["reduce"][0]
        if mname == "copy_u":
            out = oracle.gspmm(u, v, n, "copy_lhs", red, np.array(vec["ndata"][a]), None)
        else:
            binop = mname.split("_")[1]
            out = oracle.gspmm(u, v, n, binop, red, np.array(vec["ndata"][a]),
                               np.array(vec["edata"][b]))
        (key, want), = vec["expect"].items()
        np.testing.assert_allclose(out, np.array(want), rtol=1e-15, atol=1e-15)
    elif op == "update_all_chain":
        u, v = np.array(vec["u"]), np.array(vec["v"])
        h = np.array(vec["x"])
        for red, want in zip(vec["reducers"], vec["expect"]):
            h = oracle.gspmm(u, v, 3, "copy_lhs", red, h, None)
            if red in ("max", "min"):
                h = oracle.replace_inf_with_zero(h)
            np.testing.assert_array_equal(h, np.array(want))
    elif op == "edge_softmax":
        u, v = np.array(vec["u"]), np.array(vec["v"])
        got = oracle.edge_softmax(u, v, 3, np.array(vec["logits"]), eids=vec["eids"],
                                  norm_by=vec["norm_by"])
        np.testing.assert_allclose(got, np.array(vec["expect"]), rtol=1e-15)
    elif op == "segment_reduce":
        got = oracle.segment_reduce(vec["seglen"], np.array(vec["value"]), vec["reducer"])
        np.testing.assert_array_equal(got, np.array(vec["expect"]))
    elif op == "segment_softmax":
        got = oracle.segment_softmax(vec["seglen"], np.array(vec["value"]))
        for row, want in vec["expect_rows"].items():
            np.testing.assert_allclose(got[int(row)], want, rtol=1e-15)
    elif op == "gspmm":
        got = oracle.gspmm(vec["u"], vec["v"], vec["num_nodes"], vec["gspmm_op"],
                           vec["reduce_op"], np.array(vec["lhs"]), np.array(vec["rhs"]))
        np.testing.assert_array_equal(got, np.array(vec["expect"]))
    elif op == "segment_mm":
        got = oracle.segment_mm(np.array(vec["a"]), np.array(vec["b"]), vec["seglen"])
        np.testing.assert_array_equal(got, np.array(vec["expect"]))
    elif op == "gather_mm":
        got = oracle.gather_mm(np.array(vec["a"]), np.array(vec["b"]), vec["idx_b"])
        np.testing.assert_array_equal(got, np.array(vec["expect"]))
    elif op == "reshape_lhs_rhs":
        a, b = oracle.reshape_lhs_rhs(vec["lhs_shape"], vec["rhs_shape"])
        assert [list(a), list(b)] == vec["expect"]
    elif op == "graph":
        u, v = np.array(vec["u"]), np.array(vec["v"])
        indptr, _, eid = oracle.csr(u, v, 3, "dst")
        assert np.diff(indptr).tolist() == vec["in_degrees"]
        outptr, _, oeid = oracle.csr(u, v, 3, "src")
        assert np.diff(outptr).tolist() == vec["out_degrees"]
        assert eid[indptr[1]:indptr[2]].tolist() == vec["in_edges_1"]["eid"]
        assert sorted(oeid[outptr[0]:outptr[1]].tolist()) == vec["out_edges_0"]["eid"]
    else:
        raise AssertionError(op)


# --------------------------------------------------------------- memory safety
def _guarded(n_elems, dtype):
    """A numpy array whose last element ends right before an unreadable page."""
    import ctypes
    import mmap

    page = mmap.PAGESIZE
    nbytes = n_elems * np.dtype(dtype).itemsize
    body = -(-nbytes // page) * page
    buf = mmap.mmap(-1, body + page)
    base = ctypes.addressof(ctypes.c_char.from_buffer(buf))
    libc = ctypes.CDLL(None)
    assert libc.mprotect(ctypes.c_void_p(base + body), page, 0) == 0  # PROT_NONE
    arr = np.frombuffer(buf, dtype=dtype, count=n_elems, offset=body - nbytes)
    return arr, buf


def test_copy_ops_read_only_their_operand():
    """copy_lhs aliases rhs to the node data; reading it at edge ids would run
    past the node rows. With the rows placed right before an unreadable page,
    any such read faults."""
    n, e, d = 20, 500, 3
    u, v = rand_graph(n, e, 31)
    x, keep = _guarded(n * d, np.float64)
    x[:] = np.arange(n * d, dtype=np.float64)
    x = x.reshape(n, d)
    want = np.full((n, d), -np.inf)
    np.maximum.at(want, v, x[u])
    np.testing.assert_array_equal(oracle.gspmm(u, v, n, "copy_lhs", "max", x, None), want)
    # edge data read through copy_rhs by an 'e' target while lhs targets 'u'
    w, keep2 = _guarded(e * d, np.float64)
    w[:] = 1.0
    got = oracle.gsddmm(u, v, n, "copy_rhs", None, w.reshape(e, d), "u", "e")
    np.testing.assert_array_equal(got, np.ones((e, d)))
    del keep, keep2
