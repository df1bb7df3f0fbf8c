"""Features that start off a 16-byte boundary, and apply_node_func.

Views one element into their allocation (as the reference's
tests/test_ops.py:369-399 makes with numpy, here GPU tensors used in place):
the load mode of each operand, the dot's lane width and the softmax lane
layout are all chosen from the buffers' alignment, so every op is run on
such views, compared with the oracle under the tolerance rule of
test_gpu_parity.py, and compared with the same op on aligned copies (bit
for bit where both fold in the same order).

update_all / pull with an apply_node_func (reference
tests/test_function.py:115-125).
"""

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.function as fn
import mojodgl.ops as ops
import oracle
from test_gpu_parity import close

pytestmark = pytest.mark.gpu

N, E = 300, 4000


def graph(seed):
    rng = np.random.default_rng(seed)
    u, v = rng.integers(0, N, E), rng.integers(0, N, E)
    v[:700] = 7  # a row long enough to be split into chunks
    return u, v


def offset_view(a: np.ndarray) -> torch.Tensor:
    """`a` on the GPU as a contiguous view whose data pointer is one element
    past a 256-byte aligned allocation."""
    buf = torch.empty(a.size + 1, dtype=torch.float32 if a.dtype == np.float32
                      else torch.float64, device="cuda")
    view = buf[1:].view(a.shape)
    view.copy_(torch.from_numpy(a))
    assert view.is_contiguous() and view.data_ptr() % 16 != 0
    return view


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("width", [5, 8, 64])
def test_ops_on_offset_views(dtype, width):
    u, v = graph(71)
    g = dgl.graph((u, v), num_nodes=N)
    rng = np.random.default_rng(72)
    x = rng.standard_normal((N, width)).astype(dtype)
    e = rng.standard_normal((E, width)).astype(dtype)
    xv, ev = offset_view(x), offset_view(e)
    xa, ea = torch.from_numpy(x).cuda(), torch.from_numpy(e).cuda()
    what = "{} width {}".format(dtype.__name__, width)

    got = ops.u_add_e_sum(g, xv, ev)
    ref = oracle.gspmm(u, v, N, "add", "sum", x, e, np.float64)
    close(got.cpu().numpy(), ref, oracle.gspmm(u, v, N, "add", "sum", np.abs(x), np.abs(e),
                                                np.float64), dtype, "u_add_e_sum " + what)
    assert torch.equal(got, ops.u_add_e_sum(g, xa, ea)), "u_add_e_sum aligned " + what

    got = ops.copy_u_max(g, xv)
    np.testing.assert_array_equal(got.cpu().numpy(),
                                  oracle.gspmm(u, v, N, "copy_lhs", "max", x, None, dtype),
                                  err_msg="copy_u_max " + what)

    got = ops.u_dot_v(g, xv, xv)
    ref = oracle.gsddmm(u, v, N, "dot", x, x, "u", "v", np.float64)
    bound = oracle.gsddmm(u, v, N, "dot", np.abs(x), np.abs(x), "u", "v", np.float64)
    close(got.cpu().numpy(), ref, bound, dtype, "u_dot_v " + what)
    close(ops.u_dot_v(g, xa, xa).cpu().numpy(), ref, bound, dtype, "u_dot_v aligned " + what)

    heads = e[:, :1] if width == 5 else e.reshape(E, -1, 1)[:, :8]
    logits = np.ascontiguousarray(heads)
    lv = offset_view(logits)
    got = ops.edge_softmax(g, lv)
    ref = oracle.edge_softmax(u, v, N, logits, dtype=np.float64)
    close(got.cpu().numpy(), ref, ref, dtype, "edge_softmax " + what)
    close(ops.edge_softmax(g, torch.from_numpy(logits).cuda()).cpu().numpy(), ref, ref, dtype,
          "edge_softmax aligned " + what)

    seglen = rng.poisson(9, 400)
    seglen[3] = 0
    seglen[11] = 900  # longer than one wavefront's chunk
    R = int(seglen.sum())
    val = rng.standard_normal((R, width)).astype(dtype)
    vv = offset_view(val)
    for red in ("sum", "max"):
        got = ops.segment_reduce(seglen, vv, red).cpu().numpy()
        if red == "max":
            np.testing.assert_array_equal(got, oracle.segment_reduce(seglen, val, red, dtype),
                                          err_msg="segment_reduce max " + what)
        else:
            ref = oracle.segment_reduce(seglen, val, red, dtype=np.float64)
            close(got, ref, oracle.segment_reduce(seglen, np.abs(val), red, dtype=np.float64),
                  dtype, "segment_reduce sum " + what)
    got = ops.segment_softmax(seglen, vv).cpu().numpy()
    ref = oracle.segment_softmax(seglen, val, dtype=np.float64)
    close(got, ref, ref, dtype, "segment_softmax " + what)


def test_update_all_with_apply_node_func():
    u, v = graph(73)
    rng = np.random.default_rng(74)
    x = rng.standard_normal((N, 6))
    w = rng.standard_normal((E, 6))
    for as_torch in (False, True):
        g = dgl.graph((u, v), num_nodes=N)
        g.ndata["x"] = torch.from_numpy(x).cuda() if as_torch else x
        g.edata["e"] = torch.from_numpy(w).cuda() if as_torch else w
        g.update_all(fn.copy_u("x", "m"), fn.sum("m", "h"),
                     lambda nodes: {"h": nodes.data["h"] * 0.5 + 2.0})
        s = oracle.gspmm(u, v, N, "copy_lhs", "sum", x, None, np.float64)
        got = g.ndata["h"]
        got = got.cpu().numpy() if as_torch else got
        close(got, s * 0.5 + 2.0, np.abs(oracle.gspmm(u, v, N, "copy_lhs", "sum", np.abs(x),
                                                       None, np.float64)) * 0.5 + 2.0,
              np.float64, "apply_node_func")
        # the apply function may write another field; the reduced one is then not stored
        g.update_all(fn.u_mul_e("x", "e", "m"), fn.max("m", "r"),
                     lambda nodes: {"w": nodes.data["r"] + 1})
        assert "r" not in g.ndata
        mx = oracle.gspmm(u, v, N, "mul", "max", x, w, np.float64)
        mx = np.where(np.isinf(mx), 0, mx)
        got = g.ndata["w"]
        np.testing.assert_array_equal(got.cpu().numpy() if as_torch else got, mx + 1)
    # pull: the apply function sees the pulled subgraph's result; the rows
    # outside the pulled nodes are zero
    g = dgl.graph((u, v), num_nodes=N)
    g.ndata["x"] = x
    targets = np.array([0, 7, 100, 299])
    g.pull(targets, fn.copy_u("x", "m"), fn.mean("m", "h"),
           lambda nodes: {"h": nodes.data["h"] - 1.0})
    full = oracle.gspmm(u, v, N, "copy_lhs", "mean", x, None, np.float64) - 1.0
    want = np.zeros_like(full)
    want[targets] = full[targets]
    close(g.ndata["h"], want, np.abs(want) + 1.0, np.float64, "pull apply_node_func")
