"""Backward passes of gspmm / gsddmm / edge_softmax / segment_reduce /
segment_softmax on the GPU.

The reference has no backward (README.md:110-114), so there is no oracle
vector to match; the gradients are pinned by the mathematics instead:
- against torch's autograd through a float64 restatement of each forward op
  written with plain tensor indexing (index_add_, scatter_reduce), on graphs
  where every node has in- and out-edges and values have no ties;
- against finite differences (torch.autograd.gradcheck, float64).
Tolerance: float64 gradients agree to rtol 1e-9 / atol 1e-12 (sums are
formed in a different order); the float32 GAT chain to rtol 1e-4 / atol 1e-5
of the float64 chain.
"""

import math

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.function as fn
import mojodgl.ops as ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def graph_with_loops(n, e, seed):
    """Random edges plus a self loop on every node (no empty rows)."""
    rng = np.random.default_rng(seed)
    u = np.concatenate([rng.integers(0, n, e), np.arange(n)])
    v = np.concatenate([rng.integers(0, n, e), np.arange(n)])
    perm = rng.permutation(u.size)
    return u[perm], v[perm]


def leaf(shape, seed, positive=False, dtype=torch.float64):
    g = torch.Generator(device=DEV).manual_seed(seed)
    t = torch.randn(shape, generator=g, device=DEV, dtype=dtype)
    if positive:
        t = t.abs() + 0.5
    return t.requires_grad_(True)


def pad(x, nd):
    return x.reshape((x.shape[0],) + (1,) * (nd - x.dim()) + tuple(x.shape[1:]))


def ref_message(op, xu, ye):
    if op == "copy_lhs":
        return xu
    if op == "copy_rhs":
        return ye
    nd = max(xu.dim(), ye.dim())
    xu, ye = pad(xu, nd), pad(ye, nd)
    return {"add": xu + ye, "sub": xu - ye, "mul": xu * ye, "div": xu / ye}[op]


def ref_spmm(u, v, n, op, red, x, y):
    ud = torch.from_numpy(u).to(DEV)
    vd = torch.from_numpy(v).to(DEV)
    m = ref_message(op, x[ud] if x is not None else None, y)
    out = torch.zeros((n,) + tuple(m.shape[1:]), dtype=m.dtype, device=DEV)
    idx = vd.reshape((-1,) + (1,) * (m.dim() - 1)).expand_as(m)
    if red in ("sum", "mean"):
        out = out.index_add(0, vd, m)
        if red == "mean":
            deg = torch.bincount(vd, minlength=n).clamp(min=1).to(m.dtype)
            out = out / deg.reshape((-1,) + (1,) * (m.dim() - 1))
        return out
    return out.scatter_reduce(0, idx, m, "amax" if red == "max" else "amin", include_self=False)


def grads(out, inputs, seed):
    # the weights are drawn in float64 whatever the output dtype, so float32
    # and float64 chains are weighted alike
    w = torch.randn(out.shape, generator=torch.Generator(device=DEV).manual_seed(seed),
                    device=DEV, dtype=torch.float64).to(out.dtype)
    live = [t for t in inputs if t is not None]
    return torch.autograd.grad((out * w).sum(), live)


def assert_grads(got, ref, rtol=1e-9, atol=1e-12):
    assert len(got) == len(ref)
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=rtol, atol=atol)


# ------------------------------------------------------------------ gspmm
# copy_rhs has no broadcast form: only the full edge shape
_OP_YSHAPE = [(op, ys) for op in ["copy_lhs", "copy_rhs", "add", "sub", "mul", "div"]
              for ys in [(3, 4), (3, 1)] if not (op == "copy_rhs" and ys != (3, 4))]


@pytest.mark.parametrize("op,yshape", _OP_YSHAPE,
                         ids=["{}-{}".format(o, "full" if y == (3, 4) else "trailing-broadcast")
                              for o, y in _OP_YSHAPE])
@pytest.mark.parametrize("red", ["sum", "mean", "max", "min"])
def test_gspmm_backward(op, red, yshape):
    n, e = 60, 700
    u, v = graph_with_loops(n, e, 50)
    E = u.size
    g = dgl.graph((u, v), num_nodes=n)
    x = leaf((n, 3, 4), 1) if op != "copy_rhs" else None
    y = leaf((E,) + yshape, 2, positive=(op == "div")) if op != "copy_lhs" else None
    out = ops.gspmm(g, op, red, x, y)
    ref = ref_spmm(u, v, n, op, red, x, y)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    assert_grads(grads(out, [x, y], 3), grads(ref, [x, y], 3))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("xshape,yshape", [((8, 32), (8, 1)), ((4, 16), (4, 1)), ((64,), (1,)),
                                           ((2, 6), (2, 1)), ((3, 128), (3, 1))],
                         ids=["wide-8heads", "packed-4heads", "one-group", "unfusable-6",
                              "slabs-3x128"])
@pytest.mark.parametrize("red", ["sum", "mean"])
def test_gspmm_mul_backward_fused_pass(dtype, xshape, yshape, red):
    """u_mul_e sum / mean with the edge operand constant over x's last axis:
    both gradients come from one pass over the out-CSR (hubs split into
    chunks included). dX equals the separate gspmm bit for bit, dY the
    separate per-head dot to rounding; both against torch autograd in float64
    (shapes the fused kernel does not take fall back to the separate ops)."""
    from mojodgl.ops import spmm

    n, e = 300, 5000
    u, v = graph_with_loops(n, e, 60)
    u[:1200] = 11  # an out-degree hub (chunked in the out-CSR)
    E = u.size
    g = dgl.graph((u, v), num_nodes=n)
    x = leaf((n,) + xshape, 61, dtype=dtype)
    y = leaf((E,) + yshape, 62, dtype=dtype)
    out = ops.gspmm(g, "mul", red, x, y)
    gx, gy = grads(out, [x, y], 63)
    x64, y64 = (t.detach().double().requires_grad_(True) for t in (x, y))
    rx, ry = grads(ref_spmm(u, v, n, "mul", red, x64, y64), [x64, y64], 63)
    # error bound: tol * the sum of the magnitudes of the terms (a hub's
    # gradient folds ~1200 products)
    wabs = torch.randn(out.shape, generator=torch.Generator(device=DEV).manual_seed(63),
                       device=DEV, dtype=torch.float64).abs()
    ud, vd = torch.from_numpy(u).to(DEV), torch.from_numpy(v).to(DEV)
    bx = ref_spmm(v, u, n, "mul", "sum", wabs, y64.detach().abs())
    by = (x64.detach().abs()[ud] * wabs[vd]).sum(-1, keepdim=True).reshape(ry.shape)
    tol = 1e-5 if dtype == torch.float32 else 1e-12

    def within(got, ref, bound):
        assert bool(((got.double() - ref).abs() <= tol * bound + 1e-300).all())

    within(gx, rx, bx.reshape(rx.shape))
    within(gy, ry, by)
    if red == "sum":
        G = torch.randn(out.shape, generator=torch.Generator(device=DEV).manual_seed(63),
                        device=DEV, dtype=torch.float64).to(dtype)
        fused = spmm._mul_sum_dot(g, G, y.detach(), x.detach())
        if xshape[-1] == 6:
            assert fused is None  # 6 columns per group: not a power-of-two lane count
        else:
            dx, dy = fused
            sep = ops.spmm._run(g, "mul", "sum", G, y.detach(), kind="out")[0]
            assert torch.equal(dx, sep.reshape(dx.shape))
            within(dy, ry, by)


def test_gspmm_gradcheck():
    n, e = 12, 40
    u, v = graph_with_loops(n, e, 51)
    g = dgl.graph((u, v), num_nodes=n)
    x = leaf((n, 5), 4)
    y = leaf((u.size, 5), 5)
    assert torch.autograd.gradcheck(lambda a, b: ops.u_mul_e_sum(g, a, b), (x, y))
    assert torch.autograd.gradcheck(lambda a, b: ops.u_add_e_mean(g, a, b), (x, y))
    assert torch.autograd.gradcheck(lambda a, b: ops.u_mul_e_max(g, a, b), (x, y))


# ------------------------------------------------------------------ gsddmm
def ref_sddmm(u, v, op, x, y, tx, ty):
    sel = {"u": torch.from_numpy(u).to(DEV), "v": torch.from_numpy(v).to(DEV)}
    xa = x[sel[tx]] if tx != "e" else x
    ya = y[sel[ty]] if ty != "e" else y
    if op == "dot":
        return (xa * ya).sum(-1, keepdim=True)
    return ref_message(op, xa, ya)


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "dot"])
@pytest.mark.parametrize("tx,ty", [("u", "v"), ("u", "e"), ("e", "v"), ("v", "u"), ("e", "e")])
def test_gsddmm_backward(op, tx, ty):
    n, e = 50, 600
    u, v = graph_with_loops(n, e, 52)
    E = u.size
    g = dgl.graph((u, v), num_nodes=n)
    x = leaf((E if tx == "e" else n, 2, 6), 6)
    y = leaf((E if ty == "e" else n, 2, 6), 7, positive=(op == "div"))
    out = ops.gsddmm(g, op, x, y, lhs_target=tx, rhs_target=ty)
    ref = ref_sddmm(u, v, op, x, y, tx, ty)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    assert_grads(grads(out, [x, y], 8), grads(ref, [x, y], 8))


def test_gsddmm_copy_and_broadcast_backward():
    n, e = 40, 300
    u, v = graph_with_loops(n, e, 53)
    g = dgl.graph((u, v), num_nodes=n)
    x = leaf((n, 4, 3), 9)
    out = ops.copy_u(g, x)
    assert_grads(grads(out, [x], 10), grads(x[torch.from_numpy(u).to(DEV)], [x], 10))
    el = leaf((n, 4, 1), 11)
    er = leaf((n, 4, 1), 12)
    out = ops.u_add_v(g, el, er)
    ref = ref_sddmm(u, v, "add", el, er, "u", "v")
    assert_grads(grads(out, [el, er], 13), grads(ref, [el, er], 13))


# ------------------------------------------------------------------ edge_softmax
def ref_edge_softmax(u, v, n, logits, norm_by):
    key = torch.from_numpy(v if norm_by == "dst" else u).to(DEV)
    flat = logits.reshape(logits.shape[0], math.prod(logits.shape[1:]))
    idx = key[:, None].expand_as(flat)
    mx = torch.full((n, flat.shape[1]), -float("inf"), dtype=flat.dtype, device=DEV)
    mx = mx.scatter_reduce(0, idx, flat, "amax", include_self=True)
    ex = torch.exp(flat - mx[key])
    s = torch.zeros((n, flat.shape[1]), dtype=flat.dtype, device=DEV).index_add(0, key, ex)
    return (ex / s[key]).reshape(logits.shape)


@pytest.mark.parametrize("norm_by", ["dst", "src"])
@pytest.mark.parametrize("shape", [(), (1,), (4, 1)])
def test_edge_softmax_backward(norm_by, shape):
    n, e = 70, 900
    u, v = graph_with_loops(n, e, 54)
    g = dgl.graph((u, v), num_nodes=n)
    logits = leaf((u.size,) + shape, 14)
    out = ops.edge_softmax(g, logits, norm_by=norm_by)
    ref = ref_edge_softmax(u, v, n, logits, norm_by)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-14)
    assert_grads(grads(out, [logits], 15), grads(ref, [logits], 15))
    small_u, small_v = graph_with_loops(10, 30, 55)
    gs = dgl.graph((small_u, small_v), num_nodes=10)
    z = leaf((small_u.size, 2, 1), 16)
    assert torch.autograd.gradcheck(lambda t: ops.edge_softmax(gs, t, norm_by=norm_by), (z,))


@pytest.mark.parametrize("norm_by", ["dst", "src"])
@pytest.mark.parametrize("sel", ["every-third", "repeats", "all-in-order", "empty"])
def test_edge_softmax_subset_backward(norm_by, sel):
    """edge_softmax over a subset of eids (the positional rule: position i
    belongs to the group of eids[i]'s endpoint, rows past len(eids) are zero):
    values and gradients against the float64 restatement applied to the
    selected positions, zero gradient past the selection; with every edge in
    order the gradient equals the eids=ALL one bit for bit; finite differences
    on a small graph."""
    n, e = 70, 900
    u, v = graph_with_loops(n, e, 58)
    g = dgl.graph((u, v), num_nodes=n)
    E = u.size
    rng = np.random.default_rng(59)
    eids = {"every-third": np.arange(0, E, 3),
            "repeats": rng.integers(0, E, E // 2),
            "all-in-order": np.arange(E),
            "empty": np.arange(0)}[sel]
    k = eids.size
    logits = leaf((E, 4, 1), 23)
    out = ops.edge_softmax(g, logits, eids=eids, norm_by=norm_by)
    if k:
        ref = ref_edge_softmax(u[eids], v[eids], n, logits[:k], norm_by)
    else:
        ref = logits[:0] * 0
    ref = torch.cat([ref, logits[k:] * 0])
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-14)
    got = grads(out, [logits], 24)
    assert_grads(got, grads(ref, [logits], 24))
    assert torch.count_nonzero(got[0][k:]) == 0
    if sel == "all-in-order":
        full = ops.edge_softmax(g, logits, norm_by=norm_by)
        assert torch.equal(got[0], grads(full, [logits], 24)[0])
    small_u, small_v = graph_with_loops(10, 30, 60)
    gs = dgl.graph((small_u, small_v), num_nodes=10)
    z = leaf((small_u.size, 2, 1), 25)
    sub = np.arange(0, small_u.size, 2)[::-1].copy()
    assert torch.autograd.gradcheck(
        lambda t: ops.edge_softmax(gs, t, eids=sub, norm_by=norm_by), (z,))


# ------------------------------------------------------------------ segments
SEGLEN = [3, 0, 1, 7, 0, 2, 40, 5, 0, 1, 600, 4]


def ref_segment_ids(seglen):
    sl = torch.as_tensor(seglen, device=DEV)
    return torch.repeat_interleave(torch.arange(len(seglen), device=DEV), sl)


def ref_segment_reduce(seglen, value, reducer):
    ids = ref_segment_ids(seglen)
    flat = value.reshape(value.shape[0], math.prod(value.shape[1:]))
    S, d = len(seglen), flat.shape[1]
    if reducer in ("sum", "mean"):
        out = torch.zeros((S, d), dtype=flat.dtype, device=DEV).index_add(0, ids, flat)
        if reducer == "mean":
            cnt = torch.as_tensor(seglen, device=DEV).clamp(min=1).to(flat.dtype)
            out = out / cnt[:, None]
    else:
        init = -float("inf") if reducer == "max" else float("inf")
        out = torch.full((S, d), init, dtype=flat.dtype, device=DEV)
        out = out.scatter_reduce(0, ids[:, None].expand_as(flat), flat,
                                 "amax" if reducer == "max" else "amin", include_self=True)
        out = torch.where(torch.isinf(out), torch.zeros_like(out), out)
    return out.reshape((S,) + (tuple(value.shape[1:]) if value.dim() > 1 else (1,)))


def ref_segment_softmax(seglen, value):
    ids = ref_segment_ids(seglen)
    flat = value.reshape(value.shape[0], math.prod(value.shape[1:]))
    S = len(seglen)
    mx = torch.full((S, flat.shape[1]), -float("inf"), dtype=flat.dtype, device=DEV)
    mx = mx.scatter_reduce(0, ids[:, None].expand_as(flat), flat, "amax", include_self=True)
    ex = torch.exp(flat - mx[ids])
    s = torch.zeros((S, flat.shape[1]), dtype=flat.dtype, device=DEV).index_add(0, ids, ex)
    return (ex / s[ids]).reshape(value.shape)


@pytest.mark.parametrize("reducer", ["sum", "mean", "max", "min"])
@pytest.mark.parametrize("shape", [(3, 2), ()], ids=["rows-3x2", "1-D"])
@pytest.mark.parametrize("lengths_on", ["host", "gpu"])
def test_segment_reduce_backward(reducer, shape, lengths_on):
    """segment_reduce gradients (sum, mean, max / min through the selected
    row, empty segments included) against torch autograd through the float64
    restatement, and finite differences."""
    n = sum(SEGLEN)
    seglen = SEGLEN if lengths_on == "host" else torch.tensor(SEGLEN, device=DEV)
    value = leaf((n,) + shape, 26)
    out = ops.segment_reduce(seglen, value, reducer)
    ref = ref_segment_reduce(SEGLEN, value, reducer)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    assert_grads(grads(out, [value], 27), grads(ref, [value], 27))
    small = [2, 0, 3, 1]
    z = leaf((sum(small), 2), 28)
    assert torch.autograd.gradcheck(lambda t: ops.segment_reduce(small, t, reducer), (z,))


@pytest.mark.parametrize("shape", [(4,), (2, 3), ()], ids=["rows-4", "rows-2x3", "1-D"])
@pytest.mark.parametrize("lengths_on", ["host", "gpu"])
def test_segment_softmax_backward(shape, lengths_on):
    """segment_softmax gradient against torch autograd through the float64
    restatement (a 600-row segment included) and finite differences."""
    n = sum(SEGLEN)
    seglen = SEGLEN if lengths_on == "host" else torch.tensor(SEGLEN, device=DEV)
    value = leaf((n,) + shape, 29)
    out = ops.segment_softmax(seglen, value)
    ref = ref_segment_softmax(SEGLEN, value)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-14)
    assert_grads(grads(out, [value], 30), grads(ref, [value], 30))
    small = [2, 0, 3, 1]
    z = leaf((sum(small), 2), 31)
    assert torch.autograd.gradcheck(lambda t: ops.segment_softmax(small, t), (z,))


# ------------------------------------------------------------------ segment_mm / gather_mm
def check_by_terms(got, want, bound, dtype):
    """|got - want| <= tol * bound, bound the same sum over absolute terms."""
    tol = 1e-5 if dtype == torch.float32 else 1e-12
    err = (got.double() - want).abs()
    assert bool((err <= tol * bound + 1e-30).all()), float((err / (bound + 1e-300)).max())


def ref_grouped_grads(a, b, groups, G):
    """float64 da, db of out[i] = a[i] @ b[groups[i]] (rows with group -1 give
    zero), and the bounds sum |terms| of each."""
    a64, b64, G64 = a.detach().double(), b.detach().double(), G.double()
    gi = torch.as_tensor(groups, device=DEV)
    live = gi >= 0
    bsel = b64[gi.clamp(min=0)]                                   # n x d1 x d2
    da = torch.bmm(G64[:, None, :], bsel.transpose(1, 2).contiguous())[:, 0] * live[:, None]
    da_b = torch.bmm(G64.abs()[:, None, :], bsel.abs().transpose(1, 2).contiguous())[:, 0]
    outer = a64[:, :, None] * G64[:, None, :] * live[:, None, None]
    db = torch.zeros_like(b64).index_add(0, gi.clamp(min=0), outer)
    db_b = torch.zeros_like(b64).index_add(0, gi.clamp(min=0), outer.abs())
    return da, db, da_b, db_b


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n,d1,d2,r", [(3000, 128, 128, 8), (20000, 16, 16, 2), (900, 5, 3, 7),
                                       (1500, 33, 130, 3), (700, 130, 200, 2)])
def test_segment_mm_backward(dtype, n, d1, d2, r):
    """segment_mm gradients (da = G b^T per segment, db = a^T G summed per
    segment in chunks of rows, empty segments and rows past the segments
    included) against float64 sums, within the term-magnitude tolerance; run
    to run bit-identical."""
    rng = np.random.default_rng(70 + d1 + r)
    seglen = rng.multinomial(n, rng.dirichlet(np.full(r, 0.5)))
    seglen[r // 2] = 0
    rows = int(seglen.sum()) + 37                     # 37 rows in no segment
    a = leaf((rows, d1), 71, dtype=dtype)
    b = leaf((r, d1, d2), 72, dtype=dtype)
    G = torch.randn((rows, d2), generator=torch.Generator(device=DEV).manual_seed(73),
                    device=DEV, dtype=dtype)
    out = ops.segment_mm(a, b, seglen)
    out.backward(G)
    groups = np.concatenate([np.repeat(np.arange(r), seglen), np.full(37, -1)])
    da, db, da_b, db_b = ref_grouped_grads(a, b, groups, G)
    check_by_terms(a.grad, da, da_b, dtype)
    check_by_terms(b.grad, db, db_b, dtype)
    first = (a.grad.clone(), b.grad.clone())
    a.grad = b.grad = None
    ops.segment_mm(a, b, seglen).backward(G)
    assert torch.equal(a.grad, first[0]) and torch.equal(b.grad, first[1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n,d1,d2,r", [(3000, 128, 128, 8), (9000, 16, 16, 3), (900, 5, 3, 7),
                                       (600, 4, 4, 2100)],
                         ids=["128x128", "multi-chunk", "odd", "sorted-route-2100-blocks"])
def test_gather_mm_backward(dtype, n, d1, d2, r):
    """gather_mm gradients (rows bucketed by idx_b, one block unused) against
    float64 sums, and with more blocks than the bucketed route takes (the
    sorted route); run to run bit-identical."""
    rng = np.random.default_rng(80 + d1 + r)
    idx = rng.integers(0, r, n)
    idx[idx == 1] = 0                                  # block 1 unused
    a = leaf((n, d1), 81, dtype=dtype)
    b = leaf((r, d1, d2), 82, dtype=dtype)
    G = torch.randn((n, d2), generator=torch.Generator(device=DEV).manual_seed(83), device=DEV,
                    dtype=dtype)
    idx_t = torch.from_numpy(idx).to(DEV)
    out = ops.gather_mm(a, b, idx_b=idx_t)
    a64, b64 = a.detach().double(), b.detach().double()
    want = torch.bmm(a64[:, None, :], b64[idx_t])[:, 0]
    bound = torch.bmm(a64.abs()[:, None, :], b64[idx_t].abs())[:, 0]
    check_by_terms(out.detach(), want, bound, dtype)
    out.backward(G)
    da, db, da_b, db_b = ref_grouped_grads(a, b, idx, G)
    check_by_terms(a.grad, da, da_b, dtype)
    check_by_terms(b.grad, db, db_b, dtype)
    assert torch.count_nonzero(b.grad[1]) == 0
    first = (a.grad.clone(), b.grad.clone())
    a.grad = b.grad = None
    ops.gather_mm(a, b, idx_b=idx).backward(G)
    assert torch.equal(a.grad, first[0]) and torch.equal(b.grad, first[1])


@pytest.mark.parametrize("route", ["segment", "gather"])
def test_grouped_mm_backward_misaligned_operands(route):
    """a and the output gradient one element off a 16-byte boundary (the
    element loads of both gradient kernels) give the gradients of aligned
    copies: db bit for bit (the same kernel), da to rounding (the aligned
    case may take the bf16-split forward kernel, which orders k differently)."""
    n, d1, d2, r = 2000, 16, 8, 3
    rng = np.random.default_rng(90)
    base = leaf((n * d1 + 1,), 91, dtype=torch.float32)
    b = leaf((r, d1, d2), 92, dtype=torch.float32)
    gbase = torch.randn(n * d2 + 1, device=DEV)
    G = gbase[1:].view(n, d2)
    a = base[1:].view(n, d1)
    if route == "segment":
        seglen = rng.multinomial(n, np.ones(r) / r)
        run = (lambda x, y: ops.segment_mm(x, y, seglen))
    else:
        idx = torch.from_numpy(rng.integers(0, r, n)).to(DEV)
        run = (lambda x, y: ops.gather_mm(x, y, idx_b=idx))
    run(a, b).backward(G)
    got = (base.grad[1:].clone(), b.grad.clone())
    a2 = a.detach().clone().requires_grad_(True)
    b2 = b.detach().clone().requires_grad_(True)
    run(a2, b2).backward(G.clone())
    torch.testing.assert_close(got[0], a2.grad.reshape(-1), rtol=1e-5, atol=1e-5)
    assert torch.equal(got[1], b2.grad)


def test_grouped_mm_backward_values_off_the_fast_path():
    """Gradients through segment_mm when a, b and the output gradient hold
    inf, NaN, tiny and huge values: da's chunks holding them (and every chunk
    of the group whose block of b holds one, read transposed) run on float32
    MFMAs, inf and NaN land where float64 IEEE arithmetic puts them, and every
    finite entry stays within the tolerance."""
    n, d1, d2, r = 3000, 128, 128, 4
    seglen = np.array([1000, 700, 800, 500])
    a = leaf((n, d1), 96, dtype=torch.float32)
    b = leaf((r, d1, d2), 97, dtype=torch.float32)
    G = torch.randn((n, d2), generator=torch.Generator(device=DEV).manual_seed(98), device=DEV)
    with torch.no_grad():
        a[5, 3] = float("inf")
        a[1200, 7] = float("nan")
        a[1800] *= 1e-30
        a[2600, :4] = 1e30
        b[2, 5, 7] = float("inf")
    G[10, 9] = float("-inf")
    G[2000, 0] = 3e20
    ops.segment_mm(a, b, seglen).backward(G)
    da, db, da_b, db_b = ref_grouped_grads(a, b, np.repeat(np.arange(r), seglen), G)
    for got, want, bound in ((a.grad, da, da_b), (b.grad, db, db_b)):
        assert torch.equal(torch.isnan(got), torch.isnan(want))
        inf = torch.isinf(want)
        assert bool(inf.any()) and torch.equal(got[inf], want[inf].float())
        fin = torch.isfinite(want)
        check_by_terms(got[fin], want[fin], bound[fin], torch.float32)


def test_segment_mm_and_gather_mm_gradcheck():
    """Finite differences (float64) through both ops, and a numpy b (no
    gradient for it)."""
    a = leaf((12, 3), 84)
    b = leaf((3, 3, 2), 85)
    seglen = [5, 0, 4]
    assert torch.autograd.gradcheck(lambda x, y: ops.segment_mm(x, y, seglen), (a, b))
    idx = torch.tensor([2, 0, 0, 1, 2, 2, 0, 1, 1, 0, 2, 2], device=DEV)
    assert torch.autograd.gradcheck(lambda x, y: ops.gather_mm(x, y, idx_b=idx), (a, b))
    bn = b.detach().cpu().numpy()
    out = ops.gather_mm(a, bn, idx_b=idx)
    assert out.device == a.device
    (ga,) = torch.autograd.grad(out.sum(), [a])
    # d(sum of a[i] @ b[idx i]) / da[i] = the row sums of b[idx i]
    torch.testing.assert_close(ga, b.detach()[idx].sum(-1), rtol=1e-12, atol=1e-12)


def test_cpu_tensors_take_part_in_autograd():
    """Operands that live on the host (torch CPU tensors requiring grad):
    results and gradients come back on the host, equal to the GPU run."""
    u, v = graph_with_loops(30, 200, 98)
    g = dgl.graph((u, v), num_nodes=30)
    E = u.size
    xg, yg = leaf((30, 2, 4), 99), leaf((E, 2, 1), 100)
    xc = xg.detach().cpu().requires_grad_(True)
    yc = yg.detach().cpu().requires_grad_(True)
    lg = leaf((E, 2, 1), 101)
    lc = lg.detach().cpu().requires_grad_(True)
    for mine in ((xg, yg, lg), (xc, yc, lc)):
        x, y, lo = mine
        a = ops.edge_softmax(g, lo)
        out = ops.u_mul_e_sum(g, x, y * a) + ops.copy_u_max(g, x)
        e = ops.u_dot_v(g, x, x)
        out.sum().backward()
        e.sum().backward()
    for gpu_t, cpu_t in ((xg, xc), (yg, yc), (lg, lc)):
        assert cpu_t.grad.device.type == "cpu"
        torch.testing.assert_close(cpu_t.grad, gpu_t.grad.cpu(), rtol=1e-12, atol=1e-12)
    # segment ops and the grouped GEMMs the same way
    seglen = [3, 0, 5, 2]
    vg, bg = leaf((10, 4), 102), leaf((4, 4, 3), 103)
    vc = vg.detach().cpu().requires_grad_(True)
    bc = bg.detach().cpu().requires_grad_(True)
    idx = [0, 3, 3, 1, 2, 0, 1, 2, 3, 0]
    for v_, b_ in ((vg, bg), (vc, bc)):
        out = (ops.segment_reduce(seglen, v_, "max").sum() + ops.segment_softmax(seglen, v_).sum()
               + (ops.segment_softmax(seglen, v_) * v_).sum()
               + ops.segment_mm(v_, b_, seglen).sum() + ops.gather_mm(v_, b_, idx_b=idx).sum())
        assert out.device == v_.device
        out.backward()
    for gpu_t, cpu_t in ((vg, vc), (bg, bc)):
        assert cpu_t.grad.device.type == "cpu"
        torch.testing.assert_close(cpu_t.grad, gpu_t.grad.cpu(), rtol=1e-12, atol=1e-12)


def test_second_derivatives_raise():
    """The backward passes are not themselves differentiable: asking for a
    second derivative raises instead of returning a silently wrong one."""
    u, v = graph_with_loops(20, 60, 95)
    g = dgl.graph((u, v), num_nodes=20)
    x = leaf((20, 3), 96)
    y = leaf((u.size, 3), 97)
    out = ops.u_mul_e_sum(g, x, y)
    (gx,) = torch.autograd.grad(out.sum(), [x], create_graph=True)
    with pytest.raises(RuntimeError):
        gx.sum().backward()


# ------------------------------------------------------------------ a GAT layer, float32
def test_gat_layer_backward_float32():
    """gsddmm u_add_v -> leaky_relu -> edge_softmax -> gspmm u_mul_e_sum, and
    update_all with a max reducer, against the float64 torch chain."""
    n, e, H, D = 400, 6000, 4, 8
    u, v = graph_with_loops(n, e, 57)
    g = dgl.graph((u, v), num_nodes=n)

    def chain(el, er, h, mine):
        if mine:
            a = ops.edge_softmax(g, torch.nn.functional.leaky_relu(ops.u_add_v(g, el, er), 0.2))
            return ops.u_mul_e_sum(g, h, a)
        ev = ref_sddmm(u, v, "add", el, er, "u", "v")
        a = ref_edge_softmax(u, v, n, torch.nn.functional.leaky_relu(ev, 0.2), "dst")
        return ref_spmm(u, v, n, "mul", "sum", h, a)

    el, er, h = leaf((n, H, 1), 18, dtype=torch.float32), leaf((n, H, 1), 19,
                                                             dtype=torch.float32), \
        leaf((n, H, D), 20, dtype=torch.float32)
    got = grads(chain(el, er, h, True), [el, er, h], 21)
    el64, er64, h64 = (t.detach().double().requires_grad_(True) for t in (el, er, h))
    ref = grads(chain(el64, er64, h64, False), [el64, er64, h64], 21)
    for a, b in zip(got, ref):
        torch.testing.assert_close(a.double(), b, rtol=1e-4, atol=1e-5)

    x = leaf((n, 6), 22)
    g.ndata["x"] = x
    g.edata["w"] = leaf((u.size, 6), 23)
    g.update_all(fn.u_mul_e("x", "w", "m"), fn.max("m", "z"))
    z = g.ndata["z"]
    ref = ref_spmm(u, v, n, "mul", "max", x, g.edata["w"])
    assert_grads(grads(z, [x, g.edata["w"]], 24), grads(ref, [x, g.edata["w"]], 24))


# ------------------------------------------------------------------ max / min without a selection
def brute_max_min_grads(u, v, n, red, x, y):
    """Gradients of sum(gspmm(u_mul_e, red)) by brute force: each output
    element's first message (row order) reaching its value, if any beats the
    identity, passes y[e] to x[u[e]] and x[u[e]] to y[e]; no other term."""
    x, y = x.detach().cpu().numpy(), y.detach().cpu().numpy()
    gx, gy = np.zeros_like(x), np.zeros_like(y)
    for node in range(n):
        edges = np.nonzero(v == node)[0]
        for k in range(x.shape[1]):
            best, arg = (-np.inf if red == "max" else np.inf), -1
            for e in edges:
                m = x[u[e], k] * y[e, k]
                if (m > best) if red == "max" else (m < best):
                    best, arg = m, e
            if arg >= 0:
                gx[u[arg], k] += y[arg, k]
                gy[arg, k] += x[u[arg], k]
    return gx, gy


@pytest.mark.parametrize("red", ["max", "min"])
def test_max_min_gradient_reaches_no_edge_without_a_selection(red):
    """A row whose messages never beat the identity (all -inf for max, all
    +inf for min, or NaN) has no selected edge: no gradient term comes from
    any of its edges -- in particular none reaches edge 0, which lies in
    that row, and none is 0 times an infinite operand -- while every other
    output passes its gradient through its selected edge (brute force)."""
    n = 6
    u = np.array([1, 2, 3, 0, 4, 5, 1, 2])
    v = np.array([0, 0, 0, 1, 1, 2, 2, 3])  # edge 0 is in row 0
    bad = np.inf if red == "min" else -np.inf
    x = leaf((n, 3), 401, positive=True)
    yv = torch.randn((u.size, 3), generator=torch.Generator(device=DEV).manual_seed(402),
                     device=DEV, dtype=torch.float64).abs() + 0.5
    yv[:3, 1] = bad            # row 0, column 1: only identity-valued messages
    yv[:3, 2] = float("nan")   # row 0, column 2: only NaN messages
    y = yv.requires_grad_(True)
    out = ops.gspmm(dgl.graph((u, v), num_nodes=n), "mul", red, x, y)
    assert torch.isinf(out[0, 1]) and torch.isinf(out[0, 2])
    gx, gy = torch.autograd.grad(out[torch.isfinite(out)].sum(), (x, y))
    wx, wy = brute_max_min_grads(u, v, n, red, x, y)
    np.testing.assert_array_equal(gy.cpu().numpy(), wy)
    np.testing.assert_array_equal(gx.cpu().numpy(), wx)
    assert torch.all(gy[:3, 1:] == 0)


@pytest.mark.parametrize("red", ["max", "min"])
def test_update_all_gradient_is_zero_where_inf_became_zero(red):
    """update_all replaces a +-inf max / min with 0 (reference
    heterograph.py:232-239): that output is a constant, so the edge whose
    infinite message produced it receives no gradient; the rest as without
    the replacement."""
    n = 5
    u = np.array([0, 1, 2, 3, 4, 0, 1])
    v = np.array([1, 1, 2, 2, 3, 4, 4])
    sign = np.inf if red == "max" else -np.inf
    x = leaf((n, 2), 411, positive=True)
    yv = torch.randn((u.size, 2), generator=torch.Generator(device=DEV).manual_seed(412),
                     device=DEV, dtype=torch.float64).abs() + 0.5
    yv[2, 0] = sign  # row 2, column 0: an infinite message wins
    y = yv.requires_grad_(True)
    g = dgl.graph((u, v), num_nodes=n)
    g.ndata["x"] = x
    g.edata["y"] = y
    g.update_all(fn.u_mul_e("x", "y", "m"), getattr(fn, red)("m", "z"))
    z = g.ndata["z"]
    assert z[2, 0] == 0 and z[0, 0] == 0 and z[0, 1] == 0  # replaced inf; node 0 has no in-edge
    gx, gy = torch.autograd.grad(z.sum(), (x, y))
    assert gy[2, 0] == 0 and gx[u[2], 0] == 0
    # every other selected edge gets its row's gradient
    xd, yd = x.detach(), y.detach()
    plain = ops.gspmm(g, "mul", red, xd, yd)
    for e in range(u.size):
        for k in range(2):
            if (e, k) == (2, 0):
                continue
            sel = float(plain[v[e], k]) == float(xd[u[e], k] * yd[e, k]) and np.isfinite(
                float(plain[v[e], k]))
            first = sel and all(not (float(xd[u[f], k] * yd[f, k]) == float(plain[v[e], k]))
                                for f in range(e) if v[f] == v[e])
            want = float(xd[u[e], k]) if first else 0.0
            assert float(gy[e, k]) == want, (e, k)


# ------------------------------------------------------------------ randomized gradients
_RANDOM_XY = [((3, 4), (3, 4)), ((3, 4), (3, 1)), ((8, 32), (8, 1)), ((4, 16), (4, 1)),
              ((64,), (1,)), ((5,), (5,)), ((2, 6), (2, 1)), ((3, 130), (3, 1)), ((300,), (300,)),
              ((1,), (1,))]


def _random_graph(rng, distinct_with_loops):
    """Random edges (some graphs with a hub or with no edges at all); for
    max / min, distinct non-loop edges plus a loop on every node, so no row
    is empty and no two messages of a row tie."""
    n = int(rng.integers(1, 500))
    e = int(rng.integers(0, 5000)) if rng.random() > 0.05 else 0
    u, v = rng.integers(0, n, e), rng.integers(0, n, e)
    if e and rng.random() < 0.4:
        v[: int(rng.integers(1, e + 1))] = rng.integers(0, n)
    if distinct_with_loops:
        pairs = np.unique(np.stack([u, v], 1), axis=0) if e else np.zeros((0, 2), np.int64)
        pairs = pairs[pairs[:, 0] != pairs[:, 1]]
        u = np.concatenate([pairs[:, 0], np.arange(n)])
        v = np.concatenate([pairs[:, 1], np.arange(n)])
        p = rng.permutation(u.size)
        u, v = u[p], v[p]
    return n, u.astype(np.int64), v.astype(np.int64)


def _random_leaf(shape, rng, positive=False):
    t = torch.from_numpy(rng.standard_normal(shape)).to(DEV)
    return (t.abs() + 0.5 if positive else t).requires_grad_(True)


def _check_pair(out, ref, inputs, seed, tag, fwd_atol=1e-12):
    torch.testing.assert_close(out, ref, rtol=1e-11, atol=fwd_atol,
                               msg=lambda m: "{} forward: {}".format(tag, m))
    for a, b in zip(grads(out, inputs, seed), grads(ref, inputs, seed)):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-11,
                                   msg=lambda m: "{} gradient: {}".format(tag, m))


def _random_gradient_case(seed):
    rng = np.random.default_rng(77000 + seed)
    op = ["copy_lhs", "copy_rhs", "add", "sub", "mul", "div"][rng.integers(6)]
    red = ["sum", "mean", "max", "min"][rng.integers(4)]
    n, u, v = _random_graph(rng, red in ("max", "min"))
    E = u.size
    g = dgl.graph((u, v), num_nodes=n)
    xs, ys = _RANDOM_XY[rng.integers(len(_RANDOM_XY))]
    ys = xs if op == "copy_rhs" else ys
    tag = "seed {} n {} E {} {} {} {} {}".format(seed, n, E, op, red, xs, ys)
    x = _random_leaf((n,) + xs, rng) if op != "copy_rhs" else None
    y = _random_leaf((E,) + ys, rng, positive=(op == "div")) if op != "copy_lhs" else None
    _check_pair(ops.gspmm(g, op, red, x, y), ref_spmm(u, v, n, op, red, x, y), [x, y], seed,
                tag)

    tx, ty = ["u", "v", "e"][rng.integers(3)], ["u", "v", "e"][rng.integers(3)]
    sop = ["add", "sub", "mul", "div", "dot"][rng.integers(5)]
    xs2, ys2 = _RANDOM_XY[rng.integers(len(_RANDOM_XY))]
    ys2 = xs2 if sop == "dot" else ys2
    x2 = _random_leaf(((E if tx == "e" else n),) + xs2, rng)
    y2 = _random_leaf(((E if ty == "e" else n),) + ys2, rng, positive=(sop == "div"))
    _check_pair(ops.gsddmm(g, sop, x2, y2, lhs_target=tx, rhs_target=ty),
                ref_sddmm(u, v, sop, x2, y2, tx, ty), [x2, y2], seed + 1,
                "{} | gsddmm {} {} {} {} {}".format(tag, sop, tx, ty, xs2, ys2))

    heads = [(), (1,), (4, 1), (8, 1), (2, 3, 1)][rng.integers(5)]
    norm_by = ["dst", "src"][rng.integers(2)]
    scale = float(rng.choice([1.0, 3.0, 30.0]))  # 30: exp(x - max) underflows in places
    lg = (torch.from_numpy(rng.standard_normal((E,) + heads)).to(DEV) * scale).requires_grad_(True)
    _check_pair(ops.edge_softmax(g, lg, norm_by=norm_by), ref_edge_softmax(u, v, n, lg, norm_by),
                [lg], seed + 2, "{} | edge_softmax {} {}".format(tag, heads, norm_by),
                fwd_atol=1e-13)

    S = int(rng.integers(0, 300))
    seglen = rng.poisson(float(rng.choice([0.5, 3, 20, 700])), S)
    d = [(3, 2), (), (5,), (17,)][rng.integers(4)]
    vals = _random_leaf((int(seglen.sum()),) + d, rng)
    sred = ["sum", "mean", "max", "min"][rng.integers(4)]
    sl = torch.from_numpy(seglen).to(DEV) if rng.random() < 0.5 else seglen
    stag = "{} | segment {} S {} {}".format(tag, sred, S, d)
    out = ops.segment_reduce(sl, vals, sred)
    _check_pair(out, ref_segment_reduce(seglen, vals, sred).reshape(out.shape), [vals], seed + 3,
                stag)
    _check_pair(ops.segment_softmax(sl, vals), ref_segment_softmax(seglen, vals), [vals],
                seed + 4, stag + " softmax", fwd_atol=1e-13)


@pytest.mark.parametrize("block", range(4))
def test_random_gradient_cases(block):
    """Fixed-seed random cases through every differentiable op, float64,
    against torch's autograd over the restatements above: graphs with hubs,
    empty rows or no edges, every message op and reducer, broadcast edge
    operands (the fused u_mul_e pass among them), all target pairs of
    gsddmm, softmax heads and underflowing logits, empty and long
    segments with lengths on the host or the GPU."""
    for seed in range(block * 50, (block + 1) * 50):
        _random_gradient_case(seed)
