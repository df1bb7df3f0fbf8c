"""The benchmark configurations at full size, on the GPU.

The oracle cannot run the whole of these graphs in seconds, so each op is
checked three ways at full size:
- closed forms computed independently with torch or numpy over every output
  (u_add_v is one IEEE add per element, so it is bit-exact; u_dot_v, segment
  sums and maxima against float64 / exact numpy reductions);
- size-independent invariants over every output (CSR row order, softmax rows
  summing to one, max/min values equal to the message at their arg index);
- the oracle itself on a sample of whole rows (the highest-degree rows, which
  are split across workgroups, plus random rows): unsplit rows bit for bit
  against the oracle in float32, every sampled row against the float64 oracle
  within the tolerance below.

Tolerance (sums and softmaxes): |gpu - ref64| <= 1e-5 * max(|ref64|, T), T the
sum of the absolute terms, in float32, and 1e-12 in float64 (the reference's
own precision; every configuration is also run in float64 below). max/min
values and integer outputs are exact.
"""

import numpy as np
import pytest
import torch

import bench
import mojodgl as dgl
import mojodgl.function as fn
import mojodgl.heterograph as hg
import mojodgl.ops as ops
import oracle
from mojodgl.ops import spmm

pytestmark = pytest.mark.gpu

TOL = 1e-5
TOL64 = 1e-12


def log(*a):
    print("[fullsize]", *a, flush=True)


def within(got, ref, bound, what, tol=TOL):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = np.maximum(np.abs(ref), np.abs(np.asarray(bound, dtype=np.float64)))
    err = np.abs(got - ref)
    ok = err <= tol * bound + 1e-300
    if not ok.all():
        i = np.unravel_index(np.argmax(err - tol * bound), err.shape)
        raise AssertionError("{}: {} of {} outside tolerance; worst at {}: got {} ref {}".format(
            what, int((~ok).sum()), ok.size, i, got[i], ref[i]))


def sample_rows(indptr, seed, hubs=40, rand=2000):
    """The `hubs` highest-degree rows and `rand` random rows, sorted."""
    deg = np.diff(indptr)
    rng = np.random.default_rng(seed)
    top = np.argsort(deg, kind="stable")[-hubs:]
    pick = rng.choice(deg.size, size=min(rand, deg.size), replace=False)
    return np.unique(np.concatenate([top, pick]))


def sub_csr(indptr, indices, eid, rows):
    """The rows' CSR slices: (sub indptr, source ids, original edge ids), in
    the graph's CSR order, so local edge ids keep each row's fold order."""
    deg = indptr[rows + 1] - indptr[rows]
    sub = np.zeros(rows.size + 1, dtype=np.int64)
    np.cumsum(deg, out=sub[1:])
    pos = np.concatenate([np.arange(indptr[r], indptr[r + 1]) for r in rows])
    return sub, indices[pos], eid[pos]


def check_csr(g, u, v, kind):
    """CSR invariants over every edge: degrees are bincounts, rows list edge
    ids in increasing order, and each edge sits in its endpoint's row."""
    indptr, indices, eid = g._in_csr() if kind == "in" else g._out_csr()
    key, other = (v, u) if kind == "in" else (u, v)
    n = g.number_of_nodes()
    np.testing.assert_array_equal(np.diff(indptr), np.bincount(key, minlength=n))
    row = np.repeat(np.arange(n), np.diff(indptr))
    np.testing.assert_array_equal(key[eid], row)
    np.testing.assert_array_equal(other[eid], indices)
    step = np.diff(eid)
    same = row[1:] == row[:-1]
    assert np.all(step[same] > 0)
    assert np.array_equal(np.sort(eid), np.arange(eid.size))


# ------------------------------------------------------------------ C1
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_c1_update_all_whole_graph_bit_exact(dtype):
    N, E, D = 10_000, 100_000, 64
    u, v = bench.uniform_graph(0, N, E)
    rng = np.random.default_rng(0)
    h = rng.standard_normal((N, D), dtype=np.float32).astype(dtype)
    e = rng.random((E, D), dtype=np.float32).astype(dtype)
    g = dgl.graph((u, v), num_nodes=N)
    g.ndata["h"] = torch.from_numpy(h).cuda()
    g.edata["e"] = torch.from_numpy(e).cuda()
    for red in ("sum", "mean", "max", "min"):
        g.update_all(fn.u_mul_e("h", "e", "m"), getattr(fn, red)("m", "z"))
        got = g.ndata["z"].cpu().numpy()
        ref = oracle.gspmm(u, v, N, "mul", red, h, e, dtype)
        if red in ("max", "min"):
            ref = np.where(np.isinf(ref), 0, ref)
        np.testing.assert_array_equal(got, ref, err_msg=red)


# ------------------------------------------------------------------ C2
@pytest.fixture(scope="module")
def c2():
    log("C2: generating the 2.5M-node / 60M-edge power-law graph")
    u, v, stats = bench.power_law_graph(1)
    N = 2_500_000
    g = dgl.graph((u, v), num_nodes=N)
    g._device_csr("in")
    g._device_coo()
    gen = torch.Generator(device="cuda").manual_seed(1)
    el = torch.randn(N, 8, 1, device="cuda", generator=gen)
    er = torch.randn(N, 8, 1, device="cuda", generator=gen)
    h = torch.randn(N, 8, 32, device="cuda", generator=gen)
    log("C2: ready", stats)
    yield {"g": g, "u": u, "v": v, "el": el, "er": er, "h": h, "N": N}
    torch.cuda.empty_cache()


def test_c2_csr_invariants(c2):
    check_csr(c2["g"], c2["u"], c2["v"], "in")


def test_c2_gat_layer(c2):
    g, u, v, el, er, h = (c2[k] for k in ("g", "u", "v", "el", "er", "h"))
    # gsddmm u_add_v: one float32 add per element, bit-exact against torch
    e = ops.u_add_v(g, el, er)
    ud = torch.from_numpy(u).cuda()
    vd = torch.from_numpy(v).cuda()
    assert torch.equal(e, el[ud] + er[vd])
    del ud, vd
    torch.nn.functional.leaky_relu(e, 0.2, inplace=True)
    a = ops.edge_softmax(g, e)
    indptr, indices, eid = g._in_csr()

    # every row of the softmax sums to one (float64 sums of the float32 outputs)
    rows = torch.from_numpy(np.repeat(np.arange(c2["N"]), np.diff(indptr))).cuda()
    sums = torch.zeros(c2["N"], 8, dtype=torch.float64, device="cuda")
    sums.index_add_(0, rows, a.reshape(-1, 8)[torch.from_numpy(eid).cuda()].double())
    deg = torch.from_numpy(np.diff(indptr)).cuda()
    has = deg > 0
    err = (sums[has] - 1).abs().max().item()
    assert err <= TOL, err
    assert torch.all(sums[~has] == 0)
    assert bool(((a >= 0) & (a <= 1)).all())
    del rows, sums

    z = ops.u_mul_e_sum(g, h, a)

    # the oracle on sampled whole rows
    rows = sample_rows(indptr, 5)
    sub, src, eids = sub_csr(indptr, indices, eid, rows)
    local = np.arange(eids.size, dtype=np.int64)
    vloc = np.repeat(np.arange(rows.size), np.diff(sub))
    eidd = torch.from_numpy(eids).cuda()
    logits_s = e.reshape(-1, 8)[eidd].cpu().numpy()
    a_s = a.reshape(-1, 8)[eidd].cpu().numpy()
    ref = oracle.edge_softmax(src, vloc, rows.size, logits_s, dtype=np.float64)
    within(a_s, ref.reshape(a_s.shape), ref.reshape(a_s.shape), "edge_softmax sampled rows")

    hh = h.reshape(c2["N"], 256).cpu().numpy()
    zs = z.reshape(c2["N"], 256)[torch.from_numpy(rows).cuda()].cpu().numpy()
    csr_s = (sub, src, local)
    ref64 = oracle.gspmm(None, None, rows.size, "mul", "sum", hh.reshape(-1, 8, 32),
                         a_s.reshape(-1, 8, 1), np.float64, graph_csr=csr_s).reshape(-1, 256)
    bound = oracle.gspmm(None, None, rows.size, "mul", "sum", np.abs(hh).reshape(-1, 8, 32),
                         a_s.reshape(-1, 8, 1), np.float64, graph_csr=csr_s).reshape(-1, 256)
    within(zs, ref64, bound, "gspmm u_mul_e_sum sampled rows")
    ref32 = oracle.gspmm(None, None, rows.size, "mul", "sum", hh.reshape(-1, 8, 32),
                         a_s.reshape(-1, 8, 1), np.float32, graph_csr=csr_s).reshape(-1, 256)
    whole = np.diff(sub) <= g._device_csr("in").chunks.chunk_len  # rows not split
    log("C2: {} sampled rows, {} not split, max degree {}".format(
        rows.size, int(whole.sum()), int(np.diff(sub).max())))
    np.testing.assert_array_equal(zs[whole], ref32[whole])


def test_c2_gat_layer_float64(c2):
    """The GAT layer in float64: u_add_v bit-exact against torch, softmax
    rows summing to one, sampled rows against the float64 oracle (unsplit
    gspmm rows bit for bit)."""
    g, u, v = c2["g"], c2["u"], c2["v"]
    el, er, h = (c2[k].double() for k in ("el", "er", "h"))
    e = ops.u_add_v(g, el, er)
    ud = torch.from_numpy(u).cuda()
    vd = torch.from_numpy(v).cuda()
    assert torch.equal(e, el[ud] + er[vd])
    del ud, vd
    torch.nn.functional.leaky_relu(e, 0.2, inplace=True)
    a = ops.edge_softmax(g, e)
    indptr, indices, eid = g._in_csr()
    rows = torch.from_numpy(np.repeat(np.arange(c2["N"]), np.diff(indptr))).cuda()
    sums = torch.zeros(c2["N"], 8, dtype=torch.float64, device="cuda")
    sums.index_add_(0, rows, a.reshape(-1, 8)[torch.from_numpy(eid).cuda()])
    has = torch.from_numpy(np.diff(indptr)).cuda() > 0
    err = (sums[has] - 1).abs().max().item()
    assert err <= TOL64, err
    del rows, sums
    z = ops.u_mul_e_sum(g, h, a)

    rows = sample_rows(indptr, 7)
    sub, src, eids = sub_csr(indptr, indices, eid, rows)
    local = np.arange(eids.size, dtype=np.int64)
    vloc = np.repeat(np.arange(rows.size), np.diff(sub))
    eidd = torch.from_numpy(eids).cuda()
    logits_s = e.reshape(-1, 8)[eidd].cpu().numpy()
    a_s = a.reshape(-1, 8)[eidd].cpu().numpy()
    ref = oracle.edge_softmax(src, vloc, rows.size, logits_s, dtype=np.float64)
    within(a_s, ref.reshape(a_s.shape), ref.reshape(a_s.shape), "float64 edge_softmax", TOL64)
    hh = h.reshape(c2["N"], 256).cpu().numpy()
    zs = z.reshape(c2["N"], 256)[torch.from_numpy(rows).cuda()].cpu().numpy()
    csr_s = (sub, src, local)
    ref = oracle.gspmm(None, None, rows.size, "mul", "sum", hh.reshape(-1, 8, 32),
                       a_s.reshape(-1, 8, 1), np.float64, graph_csr=csr_s).reshape(-1, 256)
    bound = oracle.gspmm(None, None, rows.size, "mul", "sum", np.abs(hh).reshape(-1, 8, 32),
                         a_s.reshape(-1, 8, 1), np.float64, graph_csr=csr_s).reshape(-1, 256)
    within(zs, ref, bound, "float64 gspmm u_mul_e_sum", TOL64)
    whole = np.diff(sub) <= g._device_csr("in").chunks.chunk_len
    np.testing.assert_array_equal(zs[whole], ref[whole])


# ------------------------------------------------------------------ C3
@pytest.fixture(scope="module")
def c3():
    log("C3: generating the 230k-node / 114M-edge community graph")
    u, v, N = bench.community_graph()
    g = dgl.graph((u, v), num_nodes=N)
    g._device_csr("in")
    gen = torch.Generator(device="cuda").manual_seed(2)
    h = torch.randn(N, 602, device="cuda", generator=gen)
    indeg = np.maximum(g.in_degrees(), 1).astype(np.float64)
    outdeg = np.maximum(g.out_degrees(), 1).astype(np.float64)
    w = (1.0 / np.sqrt(outdeg[u] * indeg[v])).astype(np.float32).reshape(-1, 1)
    log("C3: ready")
    yield {"g": g, "u": u, "v": v, "h": h, "w": w, "N": N}
    torch.cuda.empty_cache()


def test_c3_aggregations(c3):
    g, h, w, N = c3["g"], c3["h"], c3["w"], c3["N"]
    indptr, indices, eid = g._in_csr()
    rows = sample_rows(indptr, 6, hubs=20, rand=300)
    sub, src, eids = sub_csr(indptr, indices, eid, rows)
    local = np.arange(eids.size, dtype=np.int64)
    csr_s = (sub, src, local)
    hh = h.cpu().numpy()
    rows_d = torch.from_numpy(rows).cuda()
    whole = np.diff(sub) <= g._device_csr("in").chunks.chunk_len  # rows not split

    z = ops.u_mul_e_sum(g, h, torch.from_numpy(w).cuda())[rows_d].cpu().numpy()
    w_s = w[eids]
    ref = oracle.gspmm(None, None, rows.size, "mul", "sum", hh, w_s, np.float64, graph_csr=csr_s)
    bound = oracle.gspmm(None, None, rows.size, "mul", "sum", np.abs(hh), w_s, np.float64,
                         graph_csr=csr_s)
    within(z, ref, bound, "C3 u_mul_e_sum")
    ref32 = oracle.gspmm(None, None, rows.size, "mul", "sum", hh, w_s, np.float32,
                         graph_csr=csr_s)
    np.testing.assert_array_equal(z[whole], ref32[whole])

    m = ops.copy_u_mean(g, h)[rows_d].cpu().numpy()
    ref = oracle.gspmm(None, None, rows.size, "copy_lhs", "mean", hh, None, np.float64,
                       graph_csr=csr_s)
    bound = oracle.gspmm(None, None, rows.size, "copy_lhs", "mean", np.abs(hh), None, np.float64,
                         graph_csr=csr_s)
    within(m, ref, bound, "C3 copy_u_mean")

    out, arg_u, arg_e, _, _ = spmm._run(g, "copy_lhs", "max", h, None, want_arg=True,
                                        arg_dtype=torch.int32)
    # every output of a non-empty row equals the message at its arg index,
    # and the arg edge joins the arg source to the row
    has = torch.from_numpy(np.diff(indptr) > 0).cuda()
    cols = torch.arange(602, device="cuda").expand_as(out)
    assert torch.equal(out[has], h[arg_u.long(), cols][has])
    vd = torch.from_numpy(c3["v"]).cuda()
    ud = torch.from_numpy(c3["u"]).cuda()
    ae = arg_e.long()
    assert torch.equal(vd[ae][has], torch.arange(N, device="cuda")[:, None].expand_as(ae)[has])
    assert torch.equal(ud[ae][has], arg_u.long()[has])
    assert bool((arg_u[~has] == -1).all()) and bool((arg_e[~has] == -1).all())
    # sampled rows: values and arg indices bit-exact against the oracle
    ro, rau, rae = oracle.gspmm(None, None, rows.size, "copy_lhs", "max", hh, None, np.float32,
                                with_arg=True, graph_csr=csr_s)
    full = (np.diff(sub) > 0)[:, None]
    np.testing.assert_array_equal(out[rows_d].cpu().numpy(), ro)
    np.testing.assert_array_equal(arg_u[rows_d].cpu().numpy(), rau)
    np.testing.assert_array_equal(arg_e[rows_d].cpu().numpy(), np.where(full, eids[rae], -1))


def test_c3_aggregations_float64(c3):
    """C3's three ops in float64 (602 columns: five 1 KB slabs of 64 lanes
    on 128-byte line rows): sampled rows against the float64 oracle, unsplit
    rows of the sums bit for bit, max values and arg indices exact."""
    g, N = c3["g"], c3["N"]
    h = c3["h"].double()
    w = c3["w"].astype(np.float64)
    indptr, indices, eid = g._in_csr()
    rows = sample_rows(indptr, 8, hubs=20, rand=300)
    sub, src, eids = sub_csr(indptr, indices, eid, rows)
    csr_s = (sub, src, np.arange(eids.size, dtype=np.int64))
    hh = h.cpu().numpy()
    rows_d = torch.from_numpy(rows).cuda()
    whole = np.diff(sub) <= g._device_csr("in").chunks.chunk_len
    w_s = w[eids]

    z = ops.u_mul_e_sum(g, h, torch.from_numpy(w).cuda())[rows_d].cpu().numpy()
    ref = oracle.gspmm(None, None, rows.size, "mul", "sum", hh, w_s, np.float64, graph_csr=csr_s)
    bound = oracle.gspmm(None, None, rows.size, "mul", "sum", np.abs(hh), w_s, np.float64,
                         graph_csr=csr_s)
    within(z, ref, bound, "float64 C3 u_mul_e_sum", TOL64)
    np.testing.assert_array_equal(z[whole], ref[whole])

    m = ops.copy_u_mean(g, h)[rows_d].cpu().numpy()
    ref = oracle.gspmm(None, None, rows.size, "copy_lhs", "mean", hh, None, np.float64,
                       graph_csr=csr_s)
    bound = oracle.gspmm(None, None, rows.size, "copy_lhs", "mean", np.abs(hh), None,
                         np.float64, graph_csr=csr_s)
    within(m, ref, bound, "float64 C3 copy_u_mean", TOL64)
    np.testing.assert_array_equal(m[whole], ref[whole])

    out, arg_u, arg_e, _, _ = spmm._run(g, "copy_lhs", "max", h, None, want_arg=True,
                                        arg_dtype=torch.int32)
    ro, rau, rae = oracle.gspmm(None, None, rows.size, "copy_lhs", "max", hh, None, np.float64,
                                with_arg=True, graph_csr=csr_s)
    full = (np.diff(sub) > 0)[:, None]
    np.testing.assert_array_equal(out[rows_d].cpu().numpy(), ro)
    np.testing.assert_array_equal(arg_u[rows_d].cpu().numpy(), rau)
    np.testing.assert_array_equal(arg_e[rows_d].cpu().numpy(), np.where(full, eids[rae], -1))


# ------------------------------------------------------------------ C4
def test_c4_u_dot_v_and_segments():
    N, E = 1_000_000, 20_000_000
    u, v = bench.uniform_graph(3, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    gen = torch.Generator(device="cuda").manual_seed(3)
    h = torch.randn(N, 128, device="cuda", generator=gen) * (1.0 / np.sqrt(128))
    s = ops.u_dot_v(g, h, h).reshape(-1)
    ud = torch.from_numpy(u).cuda()
    vd = torch.from_numpy(v).cuda()
    h64 = h.double()
    worst = 0.0
    for lo in range(0, E, 2_000_000):
        a, b = h64[ud[lo:lo + 2_000_000]], h64[vd[lo:lo + 2_000_000]]
        ref = (a * b).sum(1)
        bound = torch.maximum(ref.abs(), (a.abs() * b.abs()).sum(1))
        err = (s[lo:lo + 2_000_000].double() - ref).abs() / bound
        worst = max(worst, err.max().item())
    assert worst <= TOL, worst
    del h64, ud, vd

    rng = np.random.default_rng(3)
    seglen = rng.poisson(20, 1_000_000)
    R = int(seglen.sum())
    val = torch.randn(R, 16, device="cuda", generator=gen)
    vh = val.cpu().numpy()
    sl = torch.from_numpy(seglen).cuda()
    off = np.concatenate([[0], np.cumsum(seglen)])
    full = seglen > 0
    starts = off[:-1][full]

    got = ops.segment_reduce(sl, val, "sum").cpu().numpy()
    ref = np.zeros((seglen.size, 16))
    bound = np.zeros((seglen.size, 16))
    ref[full] = np.add.reduceat(vh.astype(np.float64), starts)
    bound[full] = np.add.reduceat(np.abs(vh).astype(np.float64), starts)
    within(got, ref, bound, "C4 segment sum")
    np.testing.assert_array_equal(
        got[:5000], oracle.segment_reduce(seglen[:5000], vh[:off[5000]], "sum", np.float32))

    got = ops.segment_reduce(sl, val, "max").cpu().numpy()
    ref = np.zeros((seglen.size, 16), dtype=np.float32)
    ref[full] = np.maximum.reduceat(vh, starts)
    np.testing.assert_array_equal(got, ref)

    sm = ops.segment_softmax(sl, val)
    tot = np.zeros((seglen.size, 16))
    tot[full] = np.add.reduceat(sm.cpu().numpy().astype(np.float64), starts)
    assert np.abs(tot[full] - 1).max() <= TOL
    pick = np.sort(rng.choice(seglen.size, 2000, replace=False))
    rows = np.concatenate([np.arange(off[i], off[i + 1]) for i in pick])
    ref = oracle.segment_softmax(seglen[pick], vh[rows], np.float64)
    within(sm[torch.from_numpy(rows).cuda()].cpu().numpy(), ref, ref, "C4 segment softmax")


# ------------------------------------------------------------------ C5
def test_c5_gather_mm_and_segment_mm():
    n, K, R = 10_000_000, 128, 64
    gen = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randn(n, K, device="cuda", generator=gen)
    b = torch.randn(R, K, K, device="cuda", generator=gen) * (1.0 / np.sqrt(K))
    rng = np.random.default_rng(4)
    idx = rng.integers(0, R, n)
    seglen = rng.multinomial(n, rng.dirichlet(0.5 * np.ones(R)))
    sample = np.sort(rng.choice(n, 100_000, replace=False))
    sd = torch.from_numpy(sample).cuda()
    a_s = a[sd].cpu().numpy()
    bh = b.cpu().numpy()

    got = ops.gather_mm(a, b, idx_b=torch.from_numpy(idx).cuda())[sd].cpu().numpy()
    ref = oracle.gather_mm(a_s, bh, idx[sample], np.float64)
    bound = oracle.gather_mm(np.abs(a_s), np.abs(bh), idx[sample], np.float64)
    within(got, ref, bound, "C5 gather_mm")

    got = ops.segment_mm(a, b, seglen)[sd].cpu().numpy()
    group = np.searchsorted(np.cumsum(seglen), sample, side="right")
    ref = oracle.gather_mm(a_s, bh, group, np.float64)
    bound = oracle.gather_mm(np.abs(a_s), np.abs(bh), group, np.float64)
    within(got, ref, bound, "C5 segment_mm")


def test_c4_u_dot_v_and_segments_float64():
    """C4 in float64: u_dot_v against torch's float64 dot, segment sums
    against numpy (the first 5,000 segments bit for bit against the
    oracle), maxima exact, segment_softmax rows summing to one and sampled
    segments against the oracle."""
    N, E = 1_000_000, 20_000_000
    u, v = bench.uniform_graph(3, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    gen = torch.Generator(device="cuda").manual_seed(13)
    h = torch.randn(N, 128, device="cuda", generator=gen, dtype=torch.float64) / np.sqrt(128)
    s = ops.u_dot_v(g, h, h).reshape(-1)
    ud = torch.from_numpy(u).cuda()
    vd = torch.from_numpy(v).cuda()
    worst = 0.0
    for lo in range(0, E, 2_000_000):
        a, b = h[ud[lo:lo + 2_000_000]], h[vd[lo:lo + 2_000_000]]
        ref = (a * b).sum(1)
        bound = torch.maximum(ref.abs(), (a.abs() * b.abs()).sum(1))
        worst = max(worst, ((s[lo:lo + 2_000_000] - ref).abs() / bound).max().item())
    assert worst <= TOL64, worst
    del ud, vd, h

    rng = np.random.default_rng(13)
    seglen = rng.poisson(20, 1_000_000)
    val = torch.randn(int(seglen.sum()), 16, device="cuda", generator=gen, dtype=torch.float64)
    vh = val.cpu().numpy()
    sl = torch.from_numpy(seglen).cuda()
    off = np.concatenate([[0], np.cumsum(seglen)])
    full = seglen > 0
    starts = off[:-1][full]
    got = ops.segment_reduce(sl, val, "sum").cpu().numpy()
    ref = np.zeros((seglen.size, 16))
    bound = np.zeros((seglen.size, 16))
    ref[full] = np.add.reduceat(vh, starts)
    bound[full] = np.add.reduceat(np.abs(vh), starts)
    within(got, ref, bound, "float64 C4 segment sum", TOL64)
    np.testing.assert_array_equal(
        got[:5000], oracle.segment_reduce(seglen[:5000], vh[:off[5000]], "sum", np.float64))
    got = ops.segment_reduce(sl, val, "max").cpu().numpy()
    ref = np.zeros((seglen.size, 16))
    ref[full] = np.maximum.reduceat(vh, starts)
    np.testing.assert_array_equal(got, ref)
    sm = ops.segment_softmax(sl, val)
    tot = np.zeros((seglen.size, 16))
    tot[full] = np.add.reduceat(sm.cpu().numpy(), starts)
    assert np.abs(tot[full] - 1).max() <= TOL64
    pick = np.sort(rng.choice(seglen.size, 2000, replace=False))
    rows = np.concatenate([np.arange(off[i], off[i + 1]) for i in pick])
    ref = oracle.segment_softmax(seglen[pick], vh[rows], np.float64)
    within(sm[torch.from_numpy(rows).cuda()].cpu().numpy(), ref, ref,
           "float64 C4 segment softmax", TOL64)


def test_c5_gather_mm_and_segment_mm_float64():
    """C5 in float64 (v_mfma_f64_16x16x4f64): sampled rows against the
    float64 oracle within 1e-12 of the sum of the absolute terms."""
    n, K, R = 10_000_000, 128, 64
    gen = torch.Generator(device="cuda").manual_seed(14)
    a = torch.randn(n, K, device="cuda", generator=gen, dtype=torch.float64)
    b = torch.randn(R, K, K, device="cuda", generator=gen, dtype=torch.float64) / np.sqrt(K)
    rng = np.random.default_rng(14)
    idx = rng.integers(0, R, n)
    seglen = rng.multinomial(n, rng.dirichlet(0.5 * np.ones(R)))
    sample = np.sort(rng.choice(n, 100_000, replace=False))
    sd = torch.from_numpy(sample).cuda()
    a_s = a[sd].cpu().numpy()
    bh = b.cpu().numpy()
    got = ops.gather_mm(a, b, idx_b=torch.from_numpy(idx).cuda())[sd].cpu().numpy()
    within(got, oracle.gather_mm(a_s, bh, idx[sample], np.float64),
           oracle.gather_mm(np.abs(a_s), np.abs(bh), idx[sample], np.float64),
           "float64 C5 gather_mm", TOL64)
    got = ops.segment_mm(a, b, seglen)[sd].cpu().numpy()
    group = np.searchsorted(np.cumsum(seglen), sample, side="right")
    within(got, oracle.gather_mm(a_s, bh, group, np.float64),
           oracle.gather_mm(np.abs(a_s), np.abs(bh), group, np.float64),
           "float64 C5 segment_mm", TOL64)
