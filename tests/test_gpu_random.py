"""Randomized parity: random graphs (some with a hub), feature shapes
(broadcast included), ops, reducers, dtypes, softmax layouts and segment
lengths against the oracle, under the tolerance rule of test_gpu_parity.py
(max / min bit-exact in the same precision). Seeds are fixed, so a failure
names a reproducible case."""

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.ops as ops
import oracle
from test_gpu_parity import close

pytestmark = pytest.mark.gpu

SHAPES = [((4,), (4,)), ((3, 4), (3, 1)), ((3, 4), (1, 4)), ((8, 32), (8, 1)), ((1,), (1,)),
          ((5,), (1,)), ((2, 3, 4), (2, 1, 4)), ((64,), (64,)), ((130,), (130,))]


def random_graph(rng):
    n = int(rng.integers(1, 3000))
    e = int(rng.integers(0, 30000))
    u, v = rng.integers(0, n, e), rng.integers(0, n, e)
    if e and rng.random() < 0.5:
        v[: int(rng.integers(1, e + 1))] = rng.integers(0, n)  # a hub
    return n, u, v


def check_case(seed):
    rng = np.random.default_rng(1000 + seed)
    n, u, v = random_graph(rng)
    E = len(u)
    g = dgl.graph((u, v), num_nodes=n)
    dtype = np.float32 if rng.random() < 0.7 else np.float64
    ls, rs = SHAPES[rng.integers(len(SHAPES))]
    if rng.random() < 0.5:
        ls, rs = rs, ls
    x = rng.standard_normal((n,) + ls).astype(dtype)
    y = rng.random((E,) + rs).astype(dtype) + 0.5
    op = ["add", "sub", "mul", "div", "copy_lhs", "copy_rhs"][rng.integers(6)]
    red = ["sum", "max", "min", "mean"][rng.integers(4)]
    case = "seed {} n {} E {} {} {} {} {} {}".format(seed, n, E, dtype.__name__, ls, rs, op, red)
    xo = None if op == "copy_rhs" else x
    yo = None if op == "copy_lhs" else y
    got = ops.gspmm(g, op, red, None if xo is None else torch.from_numpy(xo).cuda(),
                    None if yo is None else torch.from_numpy(yo).cuda()).cpu().numpy()
    if red in ("max", "min"):
        np.testing.assert_array_equal(got, oracle.gspmm(u, v, n, op, red, xo, yo, dtype),
                                      err_msg=case)
    else:
        ref = oracle.gspmm(u, v, n, op, red, xo, yo, np.float64)
        bound = oracle.gspmm(u, v, n, {"sub": "add"}.get(op, op), red,
                             None if xo is None else np.abs(xo),
                             None if yo is None else np.abs(yo), np.float64)
        close(got, ref, bound, dtype, case)

    lt, rt = ["u", "v", "e"][rng.integers(3)], ["u", "v", "e"][rng.integers(3)]
    sop = ["add", "sub", "mul", "div", "dot"][rng.integers(5)]
    lsh, rsh = (ls, ls) if sop == "dot" else (ls, rs)
    L = rng.standard_normal(((n if lt != "e" else E),) + lsh).astype(dtype)
    Rr = rng.random(((n if rt != "e" else E),) + rsh).astype(dtype) + 0.5
    got = ops.gsddmm(g, sop, torch.from_numpy(L).cuda(), torch.from_numpy(Rr).cuda(),
                     lhs_target=lt, rhs_target=rt).cpu().numpy()
    ref = oracle.gsddmm(u, v, n, sop, L, Rr, lt, rt, np.float64)
    bound = oracle.gsddmm(u, v, n, "add" if sop == "sub" else sop, np.abs(L), np.abs(Rr), lt, rt,
                          np.float64)
    close(got, ref, bound, dtype, "{}: gsddmm {} {} {}".format(case, sop, lt, rt))

    heads = [(), (1,), (4, 1), (8, 1)][rng.integers(4)]
    logits = rng.standard_normal((E,) + heads).astype(dtype) * 3
    norm_by = ["dst", "src"][rng.integers(2)]
    eids = rng.integers(0, E, int(rng.integers(0, E + 1))) if E and rng.random() < 0.3 else None
    lt_ = torch.from_numpy(logits).cuda()
    got = (ops.edge_softmax(g, lt_, norm_by=norm_by) if eids is None
           else ops.edge_softmax(g, lt_, eids=eids, norm_by=norm_by)).cpu().numpy()
    ref = oracle.edge_softmax(u, v, n, logits, eids=eids, norm_by=norm_by, dtype=np.float64)
    close(got, ref, ref, dtype, "{}: edge_softmax {} {}".format(case, heads, norm_by))

    S = int(rng.integers(0, 2000))
    seglen = rng.poisson(float(rng.choice([1, 5, 20, 200])), S)
    if S and rng.random() < 0.2:
        seglen[rng.integers(S)] = int(rng.integers(600, 5000))
    d = int(rng.choice([1, 3, 16, 33]))
    val = rng.standard_normal((int(seglen.sum()), d)).astype(dtype)
    sred = ["sum", "max", "min", "mean"][rng.integers(4)]
    sl = torch.from_numpy(seglen).cuda() if rng.random() < 0.5 else seglen
    vt = torch.from_numpy(val).cuda()
    got = ops.segment_reduce(sl, vt, sred).cpu().numpy()
    ref = oracle.segment_reduce(seglen, val, sred, dtype=np.float64)
    bound = oracle.segment_reduce(seglen, np.abs(val), sred if sred != "min" else "max",
                                  dtype=np.float64)
    close(got, ref, np.abs(bound), dtype, "{}: segment_reduce {} S {} d {}".format(case, sred, S,
                                                                                   d))
    got = ops.segment_softmax(sl, vt).cpu().numpy()
    ref = oracle.segment_softmax(seglen, val, dtype=np.float64)
    close(got, ref, ref, dtype, "{}: segment_softmax S {} d {}".format(case, S, d))


@pytest.mark.parametrize("block", range(4))
def test_random_cases(block):
    for seed in range(block * 50, (block + 1) * 50):
        check_case(seed)


@pytest.mark.parametrize("block", range(2))
def test_random_grouped_mm(block):
    """gather_mm (both routes) and segment_mm over random row counts, widths
    (odd, not multiples of 4, past one 128-wide tile) and block counts."""
    for seed in range(block * 40, (block + 1) * 40):
        rng = np.random.default_rng(5000 + seed)
        dtype = np.float32 if rng.random() < 0.7 else np.float64
        n = int(rng.integers(0, 6000))
        d1 = int(rng.choice([1, 3, 4, 16, 32, 64, 96, 128, 130, 200]))
        d2 = int(rng.choice([1, 2, 5, 16, 64, 128, 129, 256]))
        r = int(rng.integers(1, 80))
        a = rng.standard_normal((n, d1)).astype(dtype)
        b = rng.standard_normal((r, d1, d2)).astype(dtype)
        idx = rng.integers(0, r, n)
        case = "seed {} {} n {} d1 {} d2 {} r {}".format(seed, dtype.__name__, n, d1, d2, r)
        at, bt = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        got = ops.gather_mm(at, bt, idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
        close(got, oracle.gather_mm(a, b, idx, np.float64),
              oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64), dtype, "gather " + case)
        seglen = rng.multinomial(int(n * rng.random()), np.ones(r) / r)
        got = ops.segment_mm(at, bt, seglen).cpu().numpy()
        close(got, oracle.segment_mm(a, b, seglen, np.float64),
              oracle.segment_mm(np.abs(a), np.abs(b), seglen, np.float64), dtype,
              "segment " + case)
