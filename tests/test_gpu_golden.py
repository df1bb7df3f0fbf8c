"""The reference's printed known answers (tests/golden/reference_vectors.json,
each entry citing the reference file:line it comes from) through the product
API on the GPU: the HIP path, with GPU tensors and, where the answer is exact
in float32 as well, in both precisions.

Tolerance: results that are exact in binary floating point (sums of ones,
integer-valued products, 1/2) must match bit for bit; the others within
1e-12 relative in float64 and 1e-6 in float32 (thirds and the mean's
divide round)."""

import json
import os

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.function as fn
import mojodgl.ops as ops

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_vectors.json")


def _vectors():
    with open(GOLDEN) as f:
        return {v["name"]: v for v in json.load(f)}


VEC = _vectors()


def gpu(x, dtype):
    return torch.tensor(np.asarray(x), dtype=dtype, device="cuda")


def ids(x):
    return torch.tensor(np.asarray(x, dtype=np.int64), device="cuda")


def check(got, want, dtype):
    got = got.detach().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    want = np.asarray(want, dtype=np.float64)
    rtol = 1e-12 if dtype == torch.float64 else 1e-6
    np.testing.assert_allclose(got, want, rtol=rtol, atol=0)
    exact = want == np.round(want * 4) / 4  # quarters and integers are exact in both
    np.testing.assert_array_equal(got[exact], want[exact])


DTYPES = [torch.float32, torch.float64]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("name", ["readme_u_mul_e_mean", "update_all_copy_u_sum_docstring"])
def test_update_all_vectors(name, dtype):
    vec = VEC[name]
    g = dgl.graph((ids(vec["u"]), ids(vec["v"])))
    for k, x in vec["ndata"].items():
        g.ndata[k] = gpu(x, dtype)
    for k, x in vec["edata"].items():
        g.edata[k] = gpu(x, dtype)
    msg = getattr(fn, vec["message"][0])(*vec["message"][1:])
    red = getattr(fn, vec["reduce"][0])(*vec["reduce"][1:])
    g.update_all(msg, red)
    (key, want), = vec["expect"].items()
    check(g.ndata[key], want, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_update_all_zero_degree_chain(dtype):
    """max, then min, mean and sum of copy_u over 0->1, 0->1, 1->2: node 0
    has no in-edge, so max / min give 0 there, not the identity."""
    vec = VEC["update_all_zero_degree_chain"]
    g = dgl.graph((ids(vec["u"]), ids(vec["v"])), num_nodes=3)
    g.ndata["h"] = gpu(vec["x"], dtype)
    for red, want in zip(vec["reducers"], vec["expect"]):
        g.update_all(fn.copy_u("h", "m"), getattr(fn, red)("m", "h"))
        check(g.ndata["h"], want, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("name", ["edge_softmax_docstring_dst", "edge_softmax_docstring_src",
                                  "edge_softmax_docstring_eids"])
def test_edge_softmax_vectors(name, dtype):
    vec = VEC[name]
    g = dgl.graph((ids(vec["u"]), ids(vec["v"])))
    logits = gpu(vec["logits"], dtype)
    if vec["eids"] is None:
        got = ops.edge_softmax(g, logits, norm_by=vec["norm_by"])
    else:
        got = ops.edge_softmax(g, logits, eids=ids(vec["eids"]), norm_by=vec["norm_by"])
    check(got, vec["expect"], dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("lengths_on", ["host", "gpu"])
def test_segment_vectors(dtype, lengths_on):
    vec = VEC["segment_reduce_docstring"]
    seglen = vec["seglen"] if lengths_on == "host" else ids(vec["seglen"])
    check(ops.segment_reduce(seglen, gpu(vec["value"], dtype), vec["reducer"]), vec["expect"],
          dtype)
    vec = VEC["segment_softmax_docstring_rows"]
    seglen = vec["seglen"] if lengths_on == "host" else ids(vec["seglen"])
    got = ops.segment_softmax(seglen, gpu(vec["value"], dtype)).cpu().numpy()
    for row, want in vec["expect_rows"].items():
        check(got[int(row)], want, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_zero_degree_mean_vector(dtype):
    """u_add_e mean over two parallel edges into node 1: zero-degree rows
    are 0, not the mean's divisor."""
    vec = VEC["zero_degree_mean"]
    g = dgl.graph((ids(vec["u"]), ids(vec["v"])), num_nodes=vec["num_nodes"])
    got = ops.gspmm(g, vec["gspmm_op"], vec["reduce_op"], gpu(vec["lhs"], dtype),
                    gpu(vec["rhs"], dtype))
    check(got, vec["expect"], dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_grouped_mm_vectors(dtype):
    vec = VEC["segment_mm_ones"]
    check(ops.segment_mm(gpu(vec["a"], dtype), gpu(vec["b"], dtype), vec["seglen"]),
          vec["expect"], dtype)
    vec = VEC["gather_mm_2pow53"]  # 2^53 * 2^53 * 2: exact in both precisions
    got = ops.gather_mm(gpu(vec["a"], dtype), gpu(vec["b"], dtype), idx_b=ids(vec["idx_b"]))
    check(got, vec["expect"], dtype)


def test_graph_query_vector():
    """Degrees and in/out-edges of a graph built from GPU ids."""
    vec = VEC["graph_queries"]
    g = dgl.graph((ids(vec["u"]), ids(vec["v"])))
    assert g.in_degrees().tolist() == vec["in_degrees"]
    assert g.out_degrees().tolist() == vec["out_degrees"]
    e = g.in_edges(1)
    for k in ("u", "v", "eid"):
        assert getattr(e, k).tolist() == vec["in_edges_1"][k], k
    e = g.out_edges(0)
    for k in ("u", "v", "eid"):
        assert getattr(e, k).tolist() == vec["out_edges_0"][k], k
