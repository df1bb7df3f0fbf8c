"""Host-side logic of mojodgl that needs no GPU: the API surface, graph
construction and queries, argument validation (which runs before anything is
copied to the GPU), the gspmm heavy-row schedule, and the refusal to run
without a GPU."""

import itertools

import numpy as np
import pytest
import torch

import mojodgl as dgl
import mojodgl.function as fn
import mojodgl.heterograph as hg
import mojodgl.ops as ops
import mojodgl.ops.sddmm as sddmm_mod

U = np.array([2, 0, 1, 0])
V = np.array([1, 2, 0, 1])


def test_api_surface_matches_the_reference():
    # 64 names in ops: 34 from sddmm, 25 from spmm, 5 others (reference README.md:51-52)
    assert len(ops.__all__) == 64
    expected = {"{}_{}_{}".format(a, op, b) for a, b in itertools.permutations("uve", 2)
                for op in ("add", "sub", "mul", "div", "dot")}
    assert expected <= set(dir(fn)) and expected <= set(dir(ops))
    for b in ("add", "sub", "mul", "div"):
        for r in ("sum", "max", "min", "mean"):
            assert callable(getattr(ops, "u_{}_e_{}".format(b, r)))
    for r in ("sum", "max", "min", "mean"):
        assert callable(getattr(ops, "copy_u_" + r)) and callable(getattr(ops, "copy_e_" + r))
    for name in ("gspmm", "gsddmm", "segment_reduce", "segment_softmax", "segment_mm",
                 "gather_mm", "edge_softmax", "copy_u", "copy_v", "copy_e"):
        assert callable(getattr(ops, name))
    import mojodgl.nn.functional as nnf

    assert nnf.edge_softmax is ops.edge_softmax
    for name in expected:
        assert getattr(ops, name).__doc__


def test_builtin_descriptors():
    for name in ("u_add_v", "u_mul_e", "v_div_u", "e_dot_v", "u_sub_e"):
        msg = getattr(fn, name)("a", "b", "m")
        assert msg.name == name
        assert (msg.lhs_field, msg.rhs_field, msg.out_field) == ("a", "b", "m")
    assert fn.copy_u("a", "m").name == "copy_u" and fn.copy_e("a", "m").name == "copy_e"
    for name in ("sum", "max", "min", "mean"):
        red = getattr(fn, name)("m", "h")
        assert red.name == name and red.msg_field == "m" and red.out_field == "h"


def test_graph_queries():
    g = dgl.graph((U, V))
    assert g.num_nodes() == 3 and g.num_edges() == 4
    np.testing.assert_array_equal(g.edges().u, U)
    np.testing.assert_array_equal(g.edges().eid, np.arange(4))
    np.testing.assert_array_equal(g.in_degrees(), [1, 2, 1])
    np.testing.assert_array_equal(g.out_degrees(), [2, 1, 1])
    np.testing.assert_array_equal(g.in_degrees([0, 2]), [1, 1])
    e = g.in_edges(1)
    assert e.u.tolist() == [2, 0] and e.eid.tolist() == [0, 3]
    assert dgl.graph((U, V), num_nodes=10).number_of_nodes() == 10
    assert list(g.canonical_etypes) == [("_N", "_E", "_N")]
    empty = dgl.graph((np.array([], dtype=np.int64), np.array([], dtype=np.int64)))
    assert empty.num_nodes() == 0 and empty.num_edges() == 0
    import scipy.sparse as sp

    m = sp.csr_matrix(np.array([[0, 1, 0], [0, 0, 1], [1, 0, 0]], dtype=np.float64))
    gs = dgl.graph(m)
    assert sorted(zip(gs.edges().u.tolist(), gs.edges().v.tolist())) == [(0, 1), (1, 2), (2, 0)]
    gt = dgl.graph((torch.tensor([0, 1]), torch.tensor([1, 2])))
    assert gt.num_nodes() == 3


def test_idtype_sets_the_dtype_of_returned_ids():
    g32 = dgl.graph((U, V), idtype=np.int32)
    g64 = dgl.graph((U, V))
    assert g64.idtype is np.int64 and g32.idtype is np.int32
    for g, dt in ((g32, np.int32), (g64, np.int64)):
        e = g.edges()
        assert e.u.dtype == dt and e.v.dtype == dt and e.eid.dtype == dt
        assert g.in_degrees().dtype == dt and g.out_degrees([0]).dtype == dt
        assert g.in_edges(1).eid.dtype == dt
    np.testing.assert_array_equal(g32.edges().u, U)
    assert dgl.graph((U, V), idtype=torch.int32).idtype is np.int32
    assert dgl.graph((U, V), idtype="int64").idtype is np.int64
    with pytest.raises(dgl.DGLError):
        dgl.graph((U, V), idtype=np.float32)


def test_graph_validation():
    with pytest.raises(dgl.DGLError):
        dgl.graph(([0, 1], [1, 5]), num_nodes=3)
    with pytest.raises(dgl.DGLError):
        dgl.graph(([-1, 1], [1, 2]))
    with pytest.raises(dgl.DGLError):
        dgl.graph((np.array([0.5]), np.array([1.0])))
    g = dgl.graph((U, V))
    with pytest.raises(ValueError):
        g.ndata["h"] = np.ones((2, 3))
    with pytest.raises(KeyError):
        g.ndata["missing"]


def test_feature_store_keeps_dtypes():
    g = dgl.graph((U, V))
    g.ndata["a"] = np.ones((3, 2), dtype=np.float32)
    g.ndata["b"] = np.ones((3, 2), dtype=np.int32)
    g.ndata["c"] = torch.ones(3, 2, dtype=torch.float32)
    assert g.ndata["a"].dtype == np.float32
    assert g.ndata["b"].dtype == np.float64
    assert isinstance(g.ndata["c"], torch.Tensor)


def test_reshape_lhs_rhs():
    a, b = sddmm_mod.reshape_lhs_rhs(np.zeros((4, 3, 1)), np.zeros((5, 3, 3, 4)))
    assert a.shape == (4, 1, 3, 1) and b.shape == (5, 3, 3, 4)
    assert sddmm_mod.out_feat_shape((4, 1, 3, 1), (5, 3, 3, 4)) == (3, 3, 4)
    assert sddmm_mod.out_feat_shape((4, 8, 32), (5, 8, 32), dot=True) == (8, 1)


def test_validation_errors_come_before_the_gpu():
    g = dgl.graph((U, V))
    x = np.ones((3, 4))
    e = np.ones((4, 4))
    for call in (lambda: ops.u_add_e_sum(g, np.ones((2, 4)), e),
                 lambda: ops.copy_e_sum(g, e[:-1]),
                 lambda: ops.u_add_v(g, np.ones((2, 4)), x),
                 lambda: ops.gspmm(g, "dot", "sum", x, e),
                 lambda: ops.gspmm(g, "mul", "median", x, e),
                 lambda: ops.gsddmm(g, "add", x, x, lhs_target="w"),
                 lambda: ops.u_dot_v(g, np.ones((3, 4)), np.ones((3, 5))),
                 lambda: ops.u_add_v(g, np.ones((3, 4)), np.ones((3, 5))),
                 lambda: ops.u_mul_e_sum(g, np.ones((3, 2), dtype=np.complex128),
                                         np.ones((4, 2))),
                 lambda: ops.segment_reduce(np.array([3, 3]), np.ones((4, 2))),
                 lambda: ops.segment_reduce(np.array([6, -2]), np.ones((4, 2))),
                 lambda: ops.segment_reduce(np.array([4]), np.ones((4, 1)), "median"),
                 lambda: ops.segment_softmax(np.array([3]), np.ones((4, 1))),
                 lambda: ops.segment_mm(np.ones((6, 3)), np.ones((4, 3, 2)), np.array([2, 2, 2])),
                 lambda: ops.segment_mm(np.ones((6, 3)), np.ones((4, 3, 2)),
                                        np.array([-3, 3, 3, 3])),
                 lambda: ops.segment_mm(np.ones((6, 3)), np.ones((4, 3, 2)),
                                        np.array([10, 0, 0, 0])),
                 lambda: ops.gather_mm(np.ones((4, 3)), np.ones((2, 3, 5)),
                                       idx_b=np.array([0, 1, 2, 5])),
                 lambda: ops.gather_mm(np.ones((4, 3)), np.ones((2, 3, 5)),
                                       idx_b=np.array([0, 1, 2, -1])),
                 lambda: ops.gather_mm(np.ones((5, 9)), np.ones((2, 2, 3)),
                                       idx_b=np.array([0, 1, 0, 1, 0])),
                 lambda: ops.gather_mm(np.ones((4, 3)), np.ones((2, 3, 5)),
                                       idx_b=np.array([0, 1, 2])),
                 lambda: ops.gather_mm(np.full((4, 2), 2 ** 53 + 1, dtype=np.uint64),
                                       np.ones((2, 2, 3)), idx_b=np.zeros(4, dtype=np.int64)),
                 lambda: ops.edge_softmax(g, np.ones((4, 3))),
                 lambda: ops.edge_softmax(g, np.ones(4), norm_by="edge"),
                 lambda: ops.edge_softmax(g, np.ones(4), eids=np.array([0, 4])),
                 lambda: ops.edge_softmax(g, np.ones(3)),
                 lambda: ops.edge_softmax(g, np.ones(4, dtype=np.complex128))):
        with pytest.raises(dgl.DGLError):
            call()


def test_wrapping_host_lengths_are_refused():
    """Lengths whose int64 sum wraps around to the row count (each above the
    row count): refused on the host before anything reaches the GPU."""
    n = 4
    wrap = np.array([2 ** 62, 2 ** 62, 2 ** 62, 2 ** 62 + n], dtype=np.int64)
    assert int(wrap.sum()) == n
    for call in (lambda: ops.segment_reduce(wrap, np.ones((n, 2)), "sum"),
                 lambda: ops.segment_reduce(wrap, np.ones((n, 2)), "mean"),
                 lambda: ops.segment_softmax(wrap, np.ones((n, 2))),
                 lambda: ops.segment_mm(np.ones((n, 3)), np.ones((4, 3, 2)), wrap),
                 lambda: ops.segment_mm(np.ones((n, 3)), np.ones((2, 3, 2)),
                                        np.array([2 ** 63 - 1, 2], dtype=np.int64))):
        with pytest.raises(dgl.DGLError, match="lengths"):
            call()


def test_no_gpu_means_a_loud_error():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    g = dgl.graph((U, V))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.u_mul_e_sum(g, np.ones((3, 2)), np.ones((4, 2)))


def test_split_length_leaves_rows_a_quarter_over_a_chunk_whole():
    def ip(deg):
        return np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)

    assert hg.split_length(ip([3, 512, 640, 7]), 512) == 640  # none split
    assert hg.split_length(ip([3, 512, 641, 7]), 512) == 512  # rows > 512 split
    assert hg.split_length(ip([3, 512, 20000]), 512) == 512
    assert hg.split_length(ip([3, 500]), 512) == 512  # nothing to split
    assert hg.split_length(ip([5, 4]), 4) == 5
    assert hg.split_length(ip([6, 4]), 4) == 4
    assert hg.split_length(np.zeros(1, dtype=np.int64), 512) == 512  # no rows
    heavy, _, _, _ = hg.chunk_plan(ip([3, 512, 640, 7]), hg.split_length(ip([3, 512, 640, 7]), 512))
    assert heavy.size == 0


def test_chunk_plan():
    rng = np.random.default_rng(0)
    deg = rng.integers(0, 40, 200)
    deg[7] = 1000
    indptr = np.concatenate([[0], np.cumsum(deg)])
    heavy, ptr, row, start = hg.chunk_plan(indptr, 16)
    np.testing.assert_array_equal(heavy, np.nonzero(deg > 16)[0])
    # the chunks of each heavy row tile its slots exactly, in order
    for h, r in enumerate(heavy):
        starts = start[ptr[h]:ptr[h + 1]]
        assert np.all(row[ptr[h]:ptr[h + 1]] == r)
        np.testing.assert_array_equal(starts, np.arange(indptr[r], indptr[r + 1], 16))
    assert row.size == sum((d + 15) // 16 for d in deg if d > 16)


def test_packed_softmax_slots_list_each_rows_edges():
    """The packed edge list of a softmax plan: for the rows of bin k (in plan
    order), 2^k entries each, the edge ids of the row's CSR slots then -1."""
    from mojodgl.ops._plan import _packed_bin

    rng = np.random.default_rng(3)
    deg = rng.integers(0, 9, 50)
    indptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    eid = rng.permutation(int(indptr[-1]))
    for k in range(4):
        rows = np.nonzero((deg > (1 << k) // 2) & (deg <= (1 << k)))[0]
        rows = rng.permutation(rows)
        for ids in (None, eid):
            got = _packed_bin(rows, indptr, k, ids, np)
            want = []
            for r in rows:
                for s in range(1 << k):
                    j = indptr[r] + s
                    want.append(-1 if s >= deg[r] else (j if ids is None else ids[j]))
            np.testing.assert_array_equal(got, np.array(want, dtype=np.int64))
    torch_rows = torch.tensor([3, 1, 4])
    got = _packed_bin(torch_rows, torch.from_numpy(indptr), 3, torch.from_numpy(eid), torch)
    np.testing.assert_array_equal(got.numpy(), _packed_bin(np.array([3, 1, 4]), indptr, 3, eid,
                                                           np))


def test_softmax_table_slots_of_edges():
    """Two-pass edge_softmax table slots: an ordered row's slot is its
    position in the row order, a chunked row's is len(order) + its first
    chunk; every edge gets its row's slot (brute force over the CSR)."""
    from mojodgl.ops._plan import _edge_slots

    rng = np.random.default_rng(5)
    deg = rng.integers(0, 7, 40)
    deg[[3, 17]] = [25, 11]  # chunked at chunk_len 8
    indptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    E = int(indptr[-1])
    eid = rng.permutation(E)
    ordered = rng.permutation(np.nonzero((deg > 0) & (deg <= 8))[0])
    heavy = np.nonzero(deg > 8)[0]
    per = (deg[heavy] + 7) // 8
    chunk_row = np.repeat(heavy, per)
    firsts = np.concatenate([[0], np.cumsum(per)[:-1]])
    chunk_first = np.repeat(firsts, per)
    for ids in (None, eid):
        got = _edge_slots(ordered, chunk_row, chunk_first, indptr, ids)
        want = np.full(E, -1)
        for r in range(deg.size):
            if deg[r] == 0:
                continue
            slot = (int(np.nonzero(ordered == r)[0][0]) if r in ordered
                    else ordered.size + int(firsts[list(heavy).index(r)]))
            for j in range(indptr[r], indptr[r + 1]):
                want[j if ids is None else ids[j]] = slot
        np.testing.assert_array_equal(got, want)
    t = _edge_slots(torch.from_numpy(ordered), torch.from_numpy(chunk_row),
                    torch.from_numpy(chunk_first), torch.from_numpy(indptr), torch.from_numpy(eid))
    np.testing.assert_array_equal(t.numpy(), _edge_slots(ordered, chunk_row, chunk_first,
                                                         indptr, eid))


def test_fused_backward_takes_trailing_group_operands_only():
    """The one-pass u_mul_e backward applies when the edge operand is x's
    feature shape with the last axis collapsed to one."""
    from mojodgl.ops._autograd import _trailing_groups

    x = torch.zeros(5, 8, 32)
    assert _trailing_groups(x, torch.zeros(9, 8, 1))
    assert not _trailing_groups(x, torch.zeros(9, 8, 32))  # elementwise
    assert not _trailing_groups(x, torch.zeros(9, 1, 1))   # broadcast over heads too
    assert not _trailing_groups(x, torch.zeros(9, 8))      # other rank
    assert _trailing_groups(torch.zeros(5, 64), torch.zeros(9, 1))
    assert _trailing_groups(torch.zeros(5, 64), torch.zeros(9))
    assert not _trailing_groups(torch.zeros(5, 1), torch.zeros(9, 1))


def test_udf_batches_on_host_features():
    g = dgl.graph((U, V))
    x = np.arange(6, dtype=np.float64).reshape(3, 2)
    w = np.arange(4, dtype=np.float32).reshape(4, 1) + 10
    g.ndata["x"] = x
    g.edata["w"] = w
    edges = dgl.EdgeBatch(g, np.arange(4))
    np.testing.assert_array_equal(edges.src["x"], x[U])
    np.testing.assert_array_equal(edges.dst["x"], x[V])
    np.testing.assert_array_equal(edges.data["w"], w)
    assert "x" in edges.src and "w" in edges.data and "w" not in edges.src
    assert set(edges.src) == {"x"} and len(edges.data) == 1
    assert edges.number_of_edges == 4 and edges.number_of_nodes == 3
    assert edges.batch_num_edges() == [4] and edges.batch_num_nodes() == [3]
    sub = dgl.EdgeBatch(g, np.array([3, 3, 1]))  # a selection, repeats kept
    np.testing.assert_array_equal(sub.src["x"], x[U[[3, 3, 1]]])
    np.testing.assert_array_equal(sub.data["w"], w[[3, 3, 1]])
    t = dgl.EdgeBatch(g, np.array([2, 0]))
    g.ndata["y"] = torch.arange(6.0).reshape(3, 2)  # tensors are gathered as tensors
    got = t.dst["y"]
    assert isinstance(got, torch.Tensor)
    np.testing.assert_array_equal(got.numpy(), np.arange(6.0).reshape(3, 2)[V[[2, 0]]])
    nodes = dgl.NodeBatch(data={"h": x}, mailbox={"h": x + 1, "m": x * 2}, num_nodes=3)
    np.testing.assert_array_equal(nodes["h"], x + 1)  # the mailbox is looked at first
    np.testing.assert_array_equal(nodes["m"], x * 2)
    np.testing.assert_array_equal(nodes.data["h"], x)
    assert nodes.num_nodes() == 3 and nodes.batch_num_nodes() == [3]
    with pytest.raises(KeyError):
        nodes["missing"]
    empty = dgl.NodeBatch(num_nodes=2)
    assert dict(empty.mailbox) == {} and dict(empty.data) == {}


def test_feature_store_mapping():
    g = dgl.graph((U, V))
    g.ndata["a"] = [[1], [2], [3]]
    g.edata["b"] = np.ones((4, 2), dtype=np.float32)
    assert len(g.ndata) == 1 and list(g.ndata) == ["a"] and "a" in g.ndata
    assert g.ndata["a"].flags["C_CONTIGUOUS"] and g.ndata["a"].dtype == np.float64
    assert set(g.edata.keys()) == {"b"} and len(g.edata.items()) == 1
    assert g.ndata.pop("a").shape == (3, 1) and "a" not in g.ndata
    assert g.ndata.pop("a", None) is None
    g.ndata["c"] = np.zeros((3, 2))
    del g.ndata["c"]
    with pytest.raises(KeyError):
        g.ndata["c"]
    with pytest.raises(ValueError):
        g.edata["b"] = np.ones((3, 2))
    with pytest.raises(ValueError):
        g.ndata["s"] = 1.0
    with pytest.raises(ValueError):
        g.ndata["t"] = torch.ones(2, 2)


def test_library_build_stamp_matches_the_sources():
    from mojodgl import _lib

    path = _lib.build()  # builds only when missing or stale
    assert path == _lib.LIB and _lib.is_current()
    with open(path + ".sources") as f:
        assert f.read().strip() == _lib._sources_digest()


def test_stale_stamp_that_make_sees_as_current_rebuilds_everything(tmp_path):
    """When make finds nothing out of date but the source digest differs (a
    source deleted, renamed, or restored with an older time), build() runs
    make once more with -B instead of failing with an empty log. `make` is
    replaced on PATH by a stand-in that logs its arguments and, only under
    -B, writes the library and its stamp."""
    import os
    import stat
    import subprocess
    import sys

    pkg = os.path.dirname(os.path.dirname(dgl.__file__))
    fake = tmp_path / "bin" / "make"
    fake.parent.mkdir()
    log = tmp_path / "make.log"
    fake.write_text(
        "#!{py}\nimport sys\nsys.path.insert(0, {pkg!r})\nfrom mojodgl import _lib\n"
        "args = sys.argv[1:]\nopen({log!r}, 'a').write(' '.join(args) + '\\n')\n"
        "out = [a[4:] for a in args if a.startswith('OUT=')][0]\n"
        "if '-B' in args:\n"
        "    open(out, 'w').write('lib')\n"
        "    open(out + '.sources', 'w').write(_lib._sources_digest())\n".format(
            py=sys.executable, pkg=pkg, log=str(log)))
    fake.chmod(fake.stat().st_mode | stat.S_IEXEC)
    target = tmp_path / "libmdgl.so"
    target.write_text("old")
    (tmp_path / "libmdgl.so.sources").write_text("a digest of other sources")
    env = dict(os.environ, MOJODGL_LIB=str(target),
               PATH=str(fake.parent) + os.pathsep + os.environ["PATH"])
    code = ("import sys; sys.path.insert(0, {!r})\nfrom mojodgl import _lib\n"
            "print(_lib.build() == {!r}, _lib.is_current())\n").format(pkg, str(target))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.stdout.strip() == "True True", out.stdout + out.stderr
    calls = log.read_text().splitlines()
    assert len(calls) == 2 and "-B" not in calls[0].split() and "-B" in calls[1].split()


def test_missing_library_at_mojodgl_lib_is_built_or_refused(tmp_path):
    """MOJODGL_LIB names the library (reference _lib.py:16); a missing one
    is built there on first use (_lib.py:116-124), and a failed build is a
    BuildError naming it. Here the compiler is replaced by /bin/false, so
    the build must fail loudly and nothing is loaded."""
    import os
    import subprocess
    import sys

    target = tmp_path / "nowhere" / "libmdgl.so"
    env = dict(os.environ, MOJODGL_LIB=str(target), HIPCC="/bin/false")
    code = ("import sys; sys.path.insert(0, {!r})\n"
            "from mojodgl import _lib\n"
            "try:\n"
            "    _lib.lib()\n"
            "except _lib.BuildError as exc:\n"
            "    print('BuildError', {!r} in str(exc))\n"
            "else:\n"
            "    print('loaded')\n").format(os.path.dirname(os.path.dirname(dgl.__file__)),
                                            str(target))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.stdout.strip() == "BuildError True", out.stdout + out.stderr
    assert not target.exists()


def test_bench_measures_one_gpu_only():
    """bench.py --gpus N with N above 1 exits with a message instead of
    measuring: there is no multi-GPU path."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_bench_host_accounting_counts_library_calls():
    """bench.py's per-call accounting stands in for the library handle and
    counts its mdgl_* calls by name, passing everything else through."""
    import bench

    class Fake:
        other = 5

        def mdgl_a(self, x):
            return x + 1

        def mdgl_b(self):
            return "b"

    c = bench._CountingLib(Fake())
    assert c.mdgl_a(1) == 2 and c.mdgl_a(2) == 3 and c.mdgl_b() == "b" and c.other == 5
    assert c.calls == {"mdgl_a": 2, "mdgl_b": 1}
