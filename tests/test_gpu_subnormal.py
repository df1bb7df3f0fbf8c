"""Subnormal numbers through every kernel family, float32 and float64.

The bit-exact contract (sums folded in the reference's order, correctly
rounded divides, exact max/min) only holds if no kernel flushes subnormal
inputs or results to zero. Every case here feeds or produces values below the
smallest normal number (2^-126 in float32, 2^-1022 in float64):

- gspmm / gsddmm / segment_reduce: messages, products, quotients and sums on
  the subnormal grid. Subnormal sums are exact (fixed-point multiples of the
  smallest subnormal while they stay below 2^-125), so every fold order gives
  the same bits: results are compared bit for bit with the oracle in the same
  precision, split rows and long segments included.
- edge_softmax / segment_softmax: rows spanning more than 85 (float32) or 708
  (float64) in logit value, so exp(x - max) is subnormal. exp and the
  reciprocal multiply round twice on a grid of spacing s (2^-149 / 2^-1074),
  so the bound is tol * |ref| + 2 s against the exact (float64 or long
  double) value; a flush to zero misses it by thousands of s.
- segment_mm / gather_mm (and their gradients): rows of a entirely subnormal,
  on the float32 MFMA fallback (the bf16 split does not take magnitudes below
  2^-50) and on the float64 MFMA kernel: against a float64 (float32 inputs) or
  long double (float64 inputs) sum, within tol * sum|terms| + K s.
"""

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.heterograph as hg
import mojodgl.ops as ops
import oracle

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-5, np.float64: 1e-12}
# the smallest normal exponent and the subnormal spacing of each format
EMIN = {np.float32: -126, np.float64: -1022}
SPACING = {np.float32: 2.0 ** -149, np.float64: 2.0 ** -1074}
# a scale that puts N(0, 1) values on the subnormal grid, and the square root
# of it (two normal operands whose product is subnormal)
SUB = {np.float32: -138, np.float64: -1062}
HALF = {np.float32: -69, np.float64: -531}
# a scale that takes SUB-scaled values back to normal products (2^-40 and
# 2^-200) without overflowing products of ordinary values
BIG = {np.float32: 98, np.float64: 862}


def subnormal(dtype, a):
    """Nonzero entries of a that are subnormal in dtype."""
    a = np.asarray(a)
    return (a != 0) & (np.abs(a) < np.ldexp(1.0, EMIN[dtype]))


def exact_within(got, ref, bound, dtype, slack, what):
    """|got - ref| <= tol * bound + slack * spacing, ref in wider precision."""
    got = np.asarray(got).astype(np.longdouble)
    ref = np.asarray(ref).astype(np.longdouble)
    lim = TOL[dtype] * np.asarray(bound).astype(np.longdouble) + slack * SPACING[dtype]
    err = np.abs(got - ref)
    bad = ~(err <= lim)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - lim, -1)), err.shape)
        raise AssertionError("{}: {} of {} outside; worst at {}: got {!r} ref {!r}".format(
            what, int(bad.sum()), bad.size, i, float(got[i]), float(ref[i])))


@pytest.fixture(params=[None, 4], ids=["whole-rows", "split-rows"])
def chunk_len(request, monkeypatch):
    monkeypatch.setattr(hg, "CHUNK_LEN", request.param if request.param else 2 ** 30)
    return request.param


def hub_graph(n, e, seed):
    rng = np.random.default_rng(seed)
    u, v = rng.integers(0, n, e), rng.integers(0, n, e)
    v[:600] = 9   # a destination hub: split into chunks when chunk_len is set
    u[:300] = 4
    return u, v


# ------------------------------------------------------------------ gspmm
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("op", ["mul", "div", "add", "sub", "copy_u", "copy_e"])
@pytest.mark.parametrize("reduce_op", ["sum", "mean", "max", "min"])
def test_gspmm_subnormal_messages(dtype, op, reduce_op, chunk_len):
    """mul of two normal operands and div of a subnormal by a normal one give
    subnormal products; add / sub / copy move subnormal operands. Sums of
    them are exact, so split rows are bit-exact too; max / min values and
    their args bit-exact against the oracle in the same precision."""
    n, e, d = 250, 3000, 9
    u, v = hub_graph(n, e, 31)
    rng = np.random.default_rng(32)
    if op == "mul":
        x = np.ldexp(rng.normal(size=(n, d)), HALF[dtype]).astype(dtype)
        w = np.ldexp(rng.random((e, d)) + 0.5, HALF[dtype]).astype(dtype)
    elif op == "div":
        x = np.ldexp(rng.normal(size=(n, d)), SUB[dtype]).astype(dtype)
        w = (rng.random((e, d)) + 0.75).astype(dtype)
    else:
        x = np.ldexp(rng.normal(size=(n, d)), SUB[dtype]).astype(dtype)
        w = np.ldexp(rng.normal(size=(e, d)), SUB[dtype]).astype(dtype)
    oop = {"copy_u": "copy_lhs", "copy_e": "copy_rhs"}.get(op, op)
    L = None if op == "copy_e" else x
    R = None if op == "copy_u" else w
    g = dgl.graph((u, v), num_nodes=n)
    got, (au, ae) = ops.spmm._gspmm(g, oop, reduce_op, L, R)
    if chunk_len:
        assert g._device_csr("in").chunks.num_chunks > 0
    arg = reduce_op in ("max", "min")
    want = oracle.gspmm(u, v, n, oop, reduce_op, L, R, dtype, with_arg=arg)
    if arg:
        want, wu, we = want
        np.testing.assert_array_equal(au, wu)
        np.testing.assert_array_equal(ae, we)
    assert subnormal(dtype, want).mean() > 0.3, "the case must produce subnormal results"
    np.testing.assert_array_equal(got, want, err_msg="{} {} {}".format(dtype.__name__, op,
                                                                      reduce_op))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gspmm_subnormal_scalar_weight_and_wide_rows(dtype):
    """The packed scalar-edge-weight path (weights broadcast across lanes) and
    rows wider than one slab (602 columns) with subnormal products."""
    n, e = 300, 5000
    u, v = hub_graph(n, e, 33)
    rng = np.random.default_rng(34)
    g = dgl.graph((u, v), num_nodes=n)
    for d in (16, 602):
        x = np.ldexp(rng.normal(size=(n, d)), HALF[dtype]).astype(dtype)
        w = np.ldexp(rng.random((e, 1)) + 0.5, HALF[dtype]).astype(dtype)
        got = ops.u_mul_e_sum(g, x, w)
        want = oracle.gspmm(u, v, n, "mul", "sum", x, w, dtype)
        assert subnormal(dtype, want).mean() > 0.3
        np.testing.assert_array_equal(got, want, err_msg="d={}".format(d))
        got = ops.copy_u_max(g, np.ldexp(x, SUB[dtype] - HALF[dtype]))
        np.testing.assert_array_equal(got, oracle.gspmm(
            u, v, n, "copy_lhs", "max", np.ldexp(x, SUB[dtype] - HALF[dtype]), None, dtype))


# ------------------------------------------------------------------ gsddmm
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "dot"])
@pytest.mark.parametrize("d", [1, 8, 33, 128])
def test_gsddmm_subnormal_results(dtype, op, d):
    """Elementwise results and dot sums below the smallest normal, bit for bit
    (a dot of subnormal products sums exactly, whatever the lane order)."""
    n, e = 300, 4000
    rng = np.random.default_rng(35 + d)
    u, v = rng.integers(0, n, e), rng.integers(0, n, e)
    if op in ("mul", "dot"):
        x = np.ldexp(rng.normal(size=(n, d)), HALF[dtype]).astype(dtype)
        y = np.ldexp(rng.normal(size=(n, d)), HALF[dtype]).astype(dtype)
    elif op == "div":
        x = np.ldexp(rng.normal(size=(n, d)), SUB[dtype]).astype(dtype)
        y = (rng.random((n, d)) + 0.75).astype(dtype)
    else:
        x = np.ldexp(rng.normal(size=(n, d)), SUB[dtype]).astype(dtype)
        y = np.ldexp(rng.normal(size=(n, d)), SUB[dtype]).astype(dtype)
    g = dgl.graph((u, v), num_nodes=n)
    got = getattr(ops, "u_{}_v".format(op))(g, x, y)
    want = oracle.gsddmm(u, v, n, op, x, y, "u", "v", dtype)
    assert subnormal(dtype, want).mean() > 0.3
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------------ segment_reduce
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("reducer", ["sum", "mean", "max", "min"])
@pytest.mark.parametrize("d", [1, 16, 130])
def test_segment_reduce_subnormal_values(dtype, reducer, d):
    """Segments of subnormal rows, one of them 5,000 rows long (split across
    a workgroup's row streams: its sum is still exact on the subnormal grid),
    host and GPU lengths; bit for bit against the oracle."""
    rng = np.random.default_rng(36 + d)
    seglen = rng.poisson(20, 1500)
    seglen[::17] = 0
    seglen[7] = 5000
    value = np.ldexp(rng.normal(size=(int(seglen.sum()), d)), SUB[dtype]).astype(dtype)
    want = oracle.segment_reduce(seglen, value, reducer, dtype)
    assert subnormal(dtype, want).mean() > 0.3
    np.testing.assert_array_equal(ops.segment_reduce(seglen, value, reducer), want)
    got = ops.segment_reduce(torch.from_numpy(seglen).cuda(), torch.from_numpy(value).cuda(),
                             reducer)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


# ------------------------------------------------------------------ softmaxes
# logit offsets that make exp(x - max) subnormal: exp(-88) = 6.0e-39 (below
# 2^-126 = 1.18e-38) down to exp(-102) = 5.0e-45 (3.6 spacings); in float64
# exp(-709) = 1.2e-308 (below 2^-1022 = 2.2e-308) down to exp(-740) = 4.2e-322
DROP = {np.float32: (88.0, 102.0), np.float64: (709.0, 740.0)}


def spread_logits(rng, shape, dtype):
    """N(0, 1) logits with about half of them lowered by a DROP offset."""
    x = rng.normal(size=shape)
    lo, hi = DROP[dtype]
    low = rng.random(shape[0]) < 0.5
    x[low] -= rng.uniform(lo, hi, size=(int(low.sum()),) + shape[1:])
    return x.astype(dtype)


def exact_softmax(key, x, n):
    """Softmax over the edges of each key value, in long double (x in edge
    order, (E, cols))."""
    x = x.astype(np.longdouble)
    m = np.full((n, x.shape[1]), -np.inf, dtype=np.longdouble)
    np.maximum.at(m, key, x)
    ex = np.exp(x - m[key])
    s = np.zeros((n, x.shape[1]), dtype=np.longdouble)
    np.add.at(s, key, ex)
    return ex / s[key]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("norm_by", ["dst", "src"])
@pytest.mark.parametrize("shape", [(1,), (8, 1), (3, 1)])
def test_edge_softmax_subnormal_weights(dtype, norm_by, shape):
    """Rows of every class (packed bins, wavefront rows, a chunked hub whose
    chunk maxima differ by the DROP offset, so the merge's rescale exp(m_c -
    M) is subnormal too) with subnormal softmax weights; against the exact
    softmax within tol * |ref| + 2 spacings, and against the oracle in the
    same precision within 2 spacings."""
    n, e = 400, 6000
    rng = np.random.default_rng(37)
    u, v = rng.integers(0, n, e), rng.integers(0, n, e)
    v[:700] = 3
    u[:700] = 5
    logits = spread_logits(rng, (e,) + shape, dtype)
    # the hubs' first 550 edges (every chunk of at most 512 slots before the
    # last) far below the rest of their row
    logits[:550] = logits[:550] - DROP[dtype][0]
    g = dgl.graph((u, v), num_nodes=n)
    got = ops.edge_softmax(g, logits, norm_by=norm_by)
    key = v if norm_by == "dst" else u
    ref = exact_softmax(key, logits.reshape(e, -1), n).reshape(logits.shape)
    assert subnormal(dtype, ref.astype(dtype)).mean() > 0.2
    exact_within(got, ref, np.abs(ref), dtype, 2, "edge_softmax vs exact")
    same = oracle.edge_softmax(u, v, n, logits, norm_by=norm_by, dtype=dtype)
    exact_within(got, same, np.abs(same), dtype, 2, "edge_softmax vs oracle")
    # a subset of eids (the mask / positional path) with the same rows
    eids = np.flatnonzero(rng.random(e) < 0.6)
    got = ops.edge_softmax(g, logits, eids=eids, norm_by=norm_by)
    same = oracle.edge_softmax(u, v, n, logits, eids=eids, norm_by=norm_by, dtype=dtype)
    assert subnormal(dtype, same).mean() > 0.1
    exact_within(got, same, np.abs(same), dtype, 2, "edge_softmax eids vs oracle")


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 16, 40])
def test_segment_softmax_subnormal_weights(dtype, d):
    """Staged segments (up to the chunk length), long segments on the CSR
    softmax and rows wider than 32 lanes, with subnormal weights; host and GPU
    lengths."""
    rng = np.random.default_rng(38 + d)
    seglen = rng.poisson(20, 1500)
    seglen[::13] = 0
    seglen[4] = 3000
    value = spread_logits(rng, (int(seglen.sum()), d), dtype)
    key = np.repeat(np.arange(seglen.size), seglen)
    ref = exact_softmax(key, value, seglen.size)
    assert subnormal(dtype, ref.astype(dtype)).mean() > 0.2
    same = oracle.segment_softmax(seglen, value, dtype)
    for got in (ops.segment_softmax(seglen, value),
                ops.segment_softmax(torch.from_numpy(seglen).cuda(),
                                    torch.from_numpy(value).cuda()).cpu().numpy()):
        exact_within(got, ref, np.abs(ref), dtype, 2, "segment_softmax vs exact")
        exact_within(got, same, np.abs(same), dtype, 2, "segment_softmax vs oracle")


# ------------------------------------------------------------------ grouped GEMM
def exact_grouped(a, b, groups):
    """out[i] = a[i] @ b[groups[i]] in long double and sum |a||b| (float64
    products of float32 values are exact; long double keeps float64
    subnormal products to 11 more bits)."""
    a = a.astype(np.longdouble)
    b = b.astype(np.longdouble)
    out = np.einsum("ik,ikj->ij", a, b[groups])
    bound = np.einsum("ik,ikj->ij", np.abs(a), np.abs(b[groups]))
    return out, bound


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_grouped_mm_subnormal_rows(dtype):
    """Rows of a entirely subnormal: with b of ordinary size (subnormal
    results), and with one group's b scaled so the products are normal; a
    flush of subnormal inputs would zero those rows. Float32 takes such rows
    through the float32 MFMA fallback, float64 through its MFMA kernel;
    segment_mm and gather_mm, within tol * sum|terms| + K spacings of the
    exact result."""
    rng = np.random.default_rng(39)
    k, r = 128, 4
    seglen = np.array([300, 257, 40, 500])
    n = int(seglen.sum())
    a = rng.normal(size=(n, k))
    b = rng.normal(size=(r, k, k)) / np.sqrt(k)
    tiny = rng.random(n) < 0.25                       # a quarter of the rows subnormal
    a[tiny] = np.ldexp(a[tiny], SUB[dtype])
    b[2] = np.ldexp(b[2], BIG[dtype])                 # group 2: normal products
    a, b = a.astype(dtype), b.astype(dtype)
    assert subnormal(dtype, a[tiny]).mean() > 0.9
    groups = np.repeat(np.arange(r), seglen)
    ref, bound = exact_grouped(a, b, groups)
    at, bt = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    seg = ops.segment_mm(at, bt, seglen).cpu().numpy()
    perm = rng.permutation(n)
    gat = ops.gather_mm(at[torch.from_numpy(perm).cuda()], bt,
                        idx_b=torch.from_numpy(groups[perm]).cuda()).cpu().numpy()
    assert np.abs(ref[tiny & (groups == 2)]).min() > np.ldexp(1.0, EMIN[dtype])
    for got, rows, what in ((seg, slice(None), "segment_mm"), (gat, perm, "gather_mm")):
        exact_within(got, ref[rows], bound[rows], dtype, k, what)
        z = tiny[rows][:, None] & (np.abs(ref[rows]) > 4 * k * SPACING[dtype])
        assert z.sum() > 1000 and (got[z] != 0).all(), what + ": subnormal rows flushed"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_grouped_mm_gradients_of_subnormal_rows(dtype):
    """Both gradients of segment_mm with subnormal rows of a: db = a^T G runs
    on the float32 / float64 MFMA kernel of the transposed product, with the
    rows as the contracted axis; G scaled so the products are normal."""
    npd = np.float32 if dtype == torch.float32 else np.float64
    rng = np.random.default_rng(40)
    k, r = 64, 3
    seglen = np.array([700, 300, 1100])
    n = int(seglen.sum())
    a = rng.normal(size=(n, k))
    a = np.ldexp(a, SUB[npd])
    b = rng.normal(size=(r, k, k)) / np.sqrt(k)
    G = np.ldexp(rng.normal(size=(n, k)), BIG[npd])
    a, b, G = a.astype(npd), b.astype(npd), G.astype(npd)
    at = torch.from_numpy(a).cuda().requires_grad_()
    bt = torch.from_numpy(b).cuda().requires_grad_()
    ops.segment_mm(at, bt, seglen).backward(torch.from_numpy(G).cuda())
    groups = np.repeat(np.arange(r), seglen)
    al, Gl = a.astype(np.longdouble), G.astype(np.longdouble)
    db = np.zeros((r, k, k), dtype=np.longdouble)
    dbb = np.zeros_like(db)
    for g_ in range(r):
        rows = groups == g_
        db[g_] = al[rows].T @ Gl[rows]
        dbb[g_] = np.abs(al[rows]).T @ np.abs(Gl[rows])
    got = bt.grad.cpu().numpy()
    assert np.abs(db).min() > np.ldexp(1.0, EMIN[npd])
    exact_within(got, db, dbb, npd, n, "db")
    assert (got != 0).all()
