"""Homogeneous graph and the message-passing dispatcher (reference
python/mojodgl/heterograph.py).

Edges keep the order they were given. The two CSR views (by destination for
gspmm / edge_softmax(dst), by source for edge_softmax(src)) are the
reference's -- bincount, cumsum, stable argsort by endpoint
(heterograph.py:69-86), so inside a row the slots are in edge-id order, which
fixes the fold order and the max/min tie order -- built once per graph and
only when first needed, on the GPU (mdgl_build_csr, a stable radix sort) from
the int32 edge endpoints. Host queries read that build back; with no GPU
build yet they sort on the host the reference's way. The GPU CSRs are cached
with two schedules:

* gspmm: rows longer than CHUNK_LEN are split into CHUNK_LEN-slot chunks
  whose partials are folded in order, so a power-law hub is spread over
  many wavefronts without atomics;
* softmax: rows sorted by degree (packed several to a wavefront when short,
  one wavefront each when longer, chunks when longer still), per lane layout.

`update_all` / `pull` route builtins exactly as the reference does
(heterograph.py:206-290): copy_u, copy_e and u_{add,sub,mul,div}_e with a
builtin reducer run as one fused gspmm; every other message is computed by
gsddmm and reduced by gspmm(copy_rhs); max/min results get +-inf -> 0
(done in the gspmm epilogue here, a separate pass in the reference).
"""

from __future__ import annotations

from collections import namedtuple

import numpy as np
import torch

from . import _lib
from ._lib import i64
from .base import DGLError, is_all
from .function.base import TargetCode
from .function.message import BinaryMessageFunction, CopyMessageFunction, MessageFunction
from .function.reducer import ReduceFunction
from .ops import _autograd
from .ops import spmm as _spmm
from .ops._plan import SoftmaxPlan
from .ops.sddmm import gsddmm
from .udf import EdgeBatch, FeatureDict, NodeBatch

__all__ = ["DGLGraph"]

_EdgeTuple = namedtuple("EdgeTuple", "u v eid")
_Code2Str = TargetCode.CODE2STR

# rows of more in-edges than this are split into chunks of this many for gspmm
CHUNK_LEN = 512
# pull reduces the pulled rows of the graph's own CSR (mdgl_gspmm_rows, each
# row whole) for a builtin u_op_e / copy message with a builtin reducer when
# no pulled row has more in-edges than this; otherwise it runs a builtin pass
# over every edge (no subgraph) when the pulled rows hold at least
# 1 / PULL_FULL_PASS of the edges, else a subgraph of their in-edges
PULL_ROWS_MAX_DEGREE = 4096
PULL_FULL_PASS = 8
# a graph is local when at least LOCAL_FRACTION of its edges join nodes whose
# ids differ by less than LOCAL_WINDOW (the rows whose 512-byte column slabs
# fill an XCD's 4 MB L2); gspmm then cuts wide rows into narrower slabs
LOCAL_WINDOW = 4096
LOCAL_FRACTION = 0.5


def chunk_plan(indptr: np.ndarray, chunk_len: int):
    """gspmm heavy-row schedule of a CSR, on the host.

    Returns (heavy_rows, heavy_ptr, chunk_row, chunk_start): the rows with
    more than `chunk_len` slots, and their chunks of `chunk_len` slots (the
    last one shorter) in CSR order; chunks heavy_ptr[h]..heavy_ptr[h+1] are
    row heavy_rows[h]'s.
    """
    deg = np.diff(indptr)
    heavy = np.nonzero(deg > chunk_len)[0].astype(np.int64)
    per = (deg[heavy] + chunk_len - 1) // chunk_len
    ptr = np.zeros(heavy.size + 1, dtype=np.int64)
    np.cumsum(per, out=ptr[1:])
    row = np.repeat(heavy, per)
    local = np.arange(int(ptr[-1]), dtype=np.int64) - np.repeat(ptr[:-1], per)
    start = indptr[row] + local * chunk_len
    return heavy, ptr, row, start


def split_length(indptr: np.ndarray, chunk_len: int) -> int:
    """The chunk length of a CSR's gspmm schedule: `chunk_len`, or, when no
    row is more than a quarter longer than that, the longest row's length, so
    that no row is split. A row a little over one chunk then ends at most a
    quarter after its chunks would, and saves the write of its partials and
    their fold (a 50-block community graph whose longest rows hold 513-593
    slots: 3-4 % faster unsplit)."""
    longest = int((indptr[1:] - indptr[:-1]).max()) if indptr.size > 1 else 0
    if chunk_len < longest <= chunk_len + chunk_len // 4:
        return longest
    return int(chunk_len)


class _Chunks:
    """gspmm heavy-row schedule of one CSR, on the GPU."""

    def __init__(self, indptr: np.ndarray, chunk_len: int):
        heavy, ptr, row, start = chunk_plan(indptr, chunk_len)
        self.chunk_len = int(chunk_len)
        self.num_heavy = int(heavy.size)
        self.num_chunks = int(row.size)
        if heavy.size == 0:
            self.chunk_row = self.chunk_start = self.heavy_rows = self.heavy_ptr = None
            return
        self.chunk_row = _lib.i32_device(row)
        self.chunk_start = _lib.i32_device(start)
        self.heavy_rows = _lib.i32_device(heavy)
        self.heavy_ptr = _lib.i32_device(ptr)
        _lib.settle()  # cached by its CSR, possibly read from another stream


def build_device_csr(key: torch.Tensor, other, num_rows: int):
    """COO -> CSR grouped by `key` on the GPU (int32 tensors in edge-id order):
    (indptr, indices, eid) int32 GPU tensors, the reference's bincount /
    cumsum / stable argsort (heterograph.py:69-86) bit for bit. With `other`
    None only the grouping is made (indices is None)."""
    dev = _lib.device()
    key = key.contiguous()
    E = int(key.numel())
    L = _lib.lib()
    indptr = torch.empty(num_rows + 1, dtype=torch.int32, device=dev)
    indices = torch.empty(E, dtype=torch.int32, device=dev) if other is not None else None
    eid = torch.empty(E, dtype=torch.int32, device=dev)
    nbytes = L.mdgl_build_csr_workspace_bytes(E, num_rows)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes > 0 else None
    rc = L.mdgl_build_csr(key.data_ptr(), _lib.ptr(other), E, num_rows, indptr.data_ptr(),
                          _lib.ptr(indices), eid.data_ptr(), _lib.ptr(ws), max(nbytes, 0),
                          _lib.stream())
    _lib.check(rc, "build_csr")
    return indptr, indices, eid


class _DeviceCSR:
    """A CSR view on the GPU (int32) with its gspmm and softmax schedules;
    the host keeps indptr (int64) for the schedules."""

    def __init__(self, arrays, chunk_len):
        self.host_indptr, self.indptr, self.indices, self.eid = arrays
        self.chunks = _Chunks(self.host_indptr, split_length(self.host_indptr, chunk_len))
        self.params = int(chunk_len)
        self._softmax = {}
        self._slot_of_eid = None
        self._split = {}

    def chunks_for(self, chunk_len):
        """The heavy-row schedule for another chunk length (cached)."""
        if int(chunk_len) == self.chunks.chunk_len:
            return self.chunks
        got = self._split.get(int(chunk_len))
        if got is None:
            got = self._split[int(chunk_len)] = _Chunks(self.host_indptr, int(chunk_len))
        return got

    def slot_of_eid(self):
        """The inverse of `eid`: the CSR slot of every edge id (cached)."""
        if self._slot_of_eid is None:
            E = self.eid.shape[0]
            pos = torch.empty(E, dtype=torch.int32, device=self.eid.device)
            pos[self.eid.to(torch.int64)] = torch.arange(E, dtype=torch.int32,
                                                         device=self.eid.device)
            _lib.settle()
            self._slot_of_eid = pos
        return self._slot_of_eid

    def softmax_plan(self, slots, chunk_len):
        """Degree-sorted row order, packed edge ids and chunks for a softmax
        lane layout (cached)."""
        key = (int(slots), int(chunk_len))
        if key not in self._softmax:
            plan = SoftmaxPlan.from_device(self.indptr, slots, chunk_len, ordered=True,
                                           eid=self.eid)
            _lib.settle()
            self._softmax[key] = plan
        return self._softmax[key]


_IDTYPES = {None: np.int64, np.int64: np.int64, np.int32: np.int32, "int64": np.int64,
            "int32": np.int32, torch.int64: np.int64, torch.int32: np.int32}


def _idtype(idtype):
    try:
        return _IDTYPES[idtype]
    except (KeyError, TypeError):
        pass
    try:
        return _IDTYPES[np.dtype(idtype).type]
    except (KeyError, TypeError):
        raise DGLError("idtype must be int32 or int64, got {}".format(idtype)) from None


def _on_gpu(a):
    return isinstance(a, torch.Tensor) and a.device.type == "cuda"


class DGLGraph(object):
    """A homogeneous graph whose message passing runs on the GPU.

    Node ids given as GPU tensors stay on the GPU: they are checked there
    (one small read back), converted to int32 in place of an upload, and the
    host copy used by host-side queries is read back only when one asks.
    `idtype` (int32 or int64) is the dtype of the ids the queries return.
    """

    def __init__(self, u, v, num_nodes=None, idtype=np.int64):
        self.idtype = _idtype(idtype)
        self._hu = self._hv = None
        self._dcoo = None
        if _on_gpu(u) and _on_gpu(v):
            if u.is_floating_point() or v.is_floating_point() or u.is_complex() or v.is_complex():
                raise DGLError("node ids must be integers")
            u = u.detach().reshape(-1)
            v = v.detach().reshape(-1)
            if u.shape != v.shape:
                raise DGLError("u and v must have the same length")
            E = int(u.numel())
            lo = hi = 0
            if E:
                lo, hi = torch.stack((torch.minimum(u.min(), v.min()),
                                      torch.maximum(u.max(), v.max()))).tolist()
            if num_nodes is None:
                num_nodes = 0 if E == 0 else hi + 1
            num_nodes = int(num_nodes)
            if num_nodes < 0:
                raise DGLError("num_nodes must be non-negative, got {}".format(num_nodes))
            if E and (hi >= num_nodes or lo < 0):
                raise DGLError("node ids must be in [0, {}), got [{}, {}]".format(
                    num_nodes, lo, hi))
            self._E = E
            self._num_nodes = num_nodes
            self._check_int32()
            dev = _lib.device()
            self._dcoo = (u.to(device=dev, dtype=torch.int32).contiguous(),
                          v.to(device=dev, dtype=torch.int32).contiguous())
            _lib.settle()
        else:
            u = i64(u)
            v = i64(v)
            if u.shape != v.shape:
                raise DGLError("u and v must have the same length")
            if num_nodes is None:
                num_nodes = 0 if u.size == 0 else int(max(u.max(), v.max())) + 1
            num_nodes = int(num_nodes)
            if num_nodes < 0:
                raise DGLError("num_nodes must be non-negative, got {}".format(num_nodes))
            if u.size and (int(u.max()) >= num_nodes or int(v.max()) >= num_nodes
                           or int(u.min()) < 0 or int(v.min()) < 0):
                raise DGLError("node ids must be in [0, {}), got [{}, {}]".format(
                    num_nodes, int(min(u.min(), v.min())), int(max(u.max(), v.max()))))
            self._hu = u.reshape(-1)
            self._hv = v.reshape(-1)
            self._E = int(self._hu.size)
            self._num_nodes = num_nodes
        self._nstore = {}
        self._estore = {}
        self.ndata = FeatureDict(self._nstore, self._num_nodes, "ndata")
        self.edata = FeatureDict(self._estore, self._E, "edata")
        self._csr = {}
        self._draw = {}
        self._dcsr = {}
        self._locality = None
        self._launches = {}  # gspmm call shapes seen on this graph (ops/spmm.py)

    def _source_locality(self):
        """Fraction of the edges whose source id lies within LOCAL_WINDOW of
        their destination id (once per graph, counted on the GPU by
        mdgl_coo_locality): high on graphs whose node ids follow their
        communities, where narrower gspmm column slabs of a block of
        neighbouring rows stay in cache."""
        if self._locality is None:
            if self._E == 0:
                self._locality = 0.0
            else:
                u, v = self._device_coo()
                part = torch.empty(_lib.COO_LOCALITY_BLOCKS, dtype=torch.int64, device=u.device)
                _lib.check(_lib.lib().mdgl_coo_locality(u.data_ptr(), v.data_ptr(), self._E,
                                                        LOCAL_WINDOW, part.data_ptr(),
                                                        _lib.stream()), "coo_locality")
                self._locality = int(part.cpu().numpy().sum()) / self._E
        return self._locality

    def _local(self):
        """Whether gspmm should cut wide rows into narrower column slabs."""
        return self._source_locality() >= LOCAL_FRACTION

    @property
    def _u(self):
        """Host int64 source ids (read back once from a GPU-built graph)."""
        if self._hu is None:
            self._hu = self._dcoo[0].cpu().numpy().astype(np.int64)
        return self._hu

    @property
    def _v(self):
        """Host int64 destination ids (read back once from a GPU-built graph)."""
        if self._hv is None:
            self._hv = self._dcoo[1].cpu().numpy().astype(np.int64)
        return self._hv

    def _ids(self, a):
        return np.ascontiguousarray(a, dtype=self.idtype)

    # ------------------------------------------------------------------ csr
    def _build(self, kind):
        key, other = (self._v, self._u) if kind == "in" else (self._u, self._v)
        deg = np.bincount(key, minlength=self._num_nodes).astype(np.int64)
        indptr = np.zeros(self._num_nodes + 1, dtype=np.int64)
        np.cumsum(deg, out=indptr[1:])
        order = np.argsort(key, kind="stable").astype(np.int64)
        self._csr[kind] = (indptr, np.ascontiguousarray(other[order]), order, deg)

    def _host_csr(self, kind):
        if kind not in self._csr:
            raw = self._draw.get(kind)
            if raw is not None:
                # read back the GPU build rather than sorting again on the host
                indptr, indices, eid = raw[0], raw[2].cpu().numpy(), raw[3].cpu().numpy()
                self._csr[kind] = (indptr, indices.astype(np.int64), eid.astype(np.int64),
                                   np.diff(indptr))
            else:
                self._build(kind)
        return self._csr[kind]

    def _in_csr(self):
        return self._host_csr("in")[:3]

    def _out_csr(self):
        return self._host_csr("out")[:3]

    def _check_int32(self):
        if self._E >= 2 ** 31 or self._num_nodes >= 2 ** 31:
            raise DGLError("graphs with 2**31 or more nodes or edges are not supported on the GPU")

    def _device_raw(self, kind):
        """(host int64 indptr, GPU indptr, indices, eid) of the in ("in") or
        out ("out") CSR, built once on the GPU from the edge endpoints."""
        raw = self._draw.get(kind)
        if raw is None:
            u, v = self._device_coo()
            key, other = (v, u) if kind == "in" else (u, v)
            indptr, indices, eid = build_device_csr(key, other, self._num_nodes)
            host = indptr.cpu().numpy().astype(np.int64)
            raw = (host, indptr, indices, eid)
            self._draw[kind] = raw
        return raw

    def _current_csr(self, kind):
        """The GPU CSR of `kind` if it is built and has the schedules for the
        current CHUNK_LEN (what _device_csr would return), else None."""
        cached = self._dcsr.get(kind)
        return cached if cached is not None and cached.params == int(CHUNK_LEN) else None

    def _device_csr(self, kind):
        """The GPU CSR of `kind` with the schedules for the current CHUNK_LEN."""
        params = int(CHUNK_LEN)
        cached = self._dcsr.get(kind)
        if cached is None or cached.params != params:
            if cached is not None:
                self._launches.clear()  # replays of the old schedules (they hold its CSR)
            cached = _DeviceCSR(self._device_raw(kind), params)
            self._dcsr[kind] = cached
        return cached

    def _device_coo(self):
        """int32 GPU copies of the edge endpoints, in edge-id order."""
        self._check_int32()
        if self._dcoo is None:
            coo = (_lib.i32_device(self._u), _lib.i32_device(self._v))
            _lib.settle()
            self._dcoo = coo
        return self._dcoo

    # -------------------------------------------------------------- queries
    def number_of_nodes(self, ntype=None):
        return self._num_nodes

    def number_of_src_nodes(self, ntype=None):
        return self._num_nodes

    def number_of_dst_nodes(self, ntype=None):
        return self._num_nodes

    @property
    def canonical_etypes(self):
        return (("_N", "_E", "_N"),)

    def number_of_edges(self, etype=None):
        return self._E

    def num_nodes(self):
        return self._num_nodes

    def num_edges(self):
        return self._E

    def num_src_nodes(self):
        return self._num_nodes

    def num_dst_nodes(self):
        return self._num_nodes

    def __len__(self):
        return self._num_nodes

    def __repr__(self):
        return "Graph(num_nodes={}, num_edges={},)".format(self._num_nodes, self.num_edges())

    def __str__(self):
        return self.__repr__()

    def edges(self, form="uv", order="eid", etype=None):
        """All edges as a named tuple of (u, v, eid), in edge-id order."""
        if form not in ("uv", "all"):
            raise DGLError("form must be 'uv' or 'all'")
        if order != "eid":
            raise DGLError("only order='eid' is supported")
        return _EdgeTuple(self._ids(self._u), self._ids(self._v),
                          np.arange(self._E, dtype=self.idtype))

    def _select(self, ids, order, on_src):
        if is_all(ids):
            sel = np.arange(self._u.size)
        else:
            key = self._u if on_src else self._v
            sel = np.nonzero(np.isin(key, i64(ids)))[0]
        if order == "srcid":
            sel = sel[np.argsort(self._u[sel], kind="stable")]
        elif order == "dstid":
            sel = sel[np.argsort(self._v[sel], kind="stable")]
        sel = sel.astype(np.int64)
        return _EdgeTuple(self._ids(self._u[sel]), self._ids(self._v[sel]), self._ids(sel))

    def in_edges(self, v, form="uv", order="eid", etype=None):
        """All in-edges of `v` (every node when `v` is ALL), in edge-id order."""
        return self._select(v, order, False)

    def out_edges(self, u, form="uv", order="eid", etype=None):
        """All out-edges of `u` (every node when `u` is ALL), in edge-id order."""
        return self._select(u, order, True)

    def in_degrees(self, v=None):
        deg = self._host_csr("in")[3]
        return self._ids(deg if v is None else deg[i64(v)])

    def out_degrees(self, u=None):
        deg = self._host_csr("out")[3]
        return self._ids(deg if u is None else deg[i64(u)])

    # ------------------------------------------------------- message passing
    def _builtin_message(self, message_func):
        """Per-edge messages of a builtin message function (gsddmm)."""
        if isinstance(message_func, CopyMessageFunction):
            target = _Code2Str[message_func.target]
            if target == "e":
                return self.edata[message_func.in_field]
            return gsddmm(self, "copy_lhs", self.ndata[message_func.in_field], None,
                          lhs_target=target)
        if not isinstance(message_func, BinaryMessageFunction):
            raise DGLError("unrecognised message function {}".format(message_func))
        lhs = _Code2Str[message_func.lhs]
        rhs = _Code2Str[message_func.rhs]
        lhs_data = self.edata[message_func.lhs_field] if lhs == "e" \
            else self.ndata[message_func.lhs_field]
        rhs_data = self.edata[message_func.rhs_field] if rhs == "e" \
            else self.ndata[message_func.rhs_field]
        return gsddmm(self, message_func.binary_op, lhs_data, rhs_data, lhs_target=lhs,
                      rhs_target=rhs)

    def _fusable(self, message_func):
        """(op, lhs field, rhs field) when gspmm computes message and reduce at once."""
        if isinstance(message_func, CopyMessageFunction):
            target = _Code2Str[message_func.target]
            if target == "u":
                return "copy_lhs", message_func.in_field, None
            if target == "e":
                return "copy_rhs", None, message_func.in_field
            return None
        if not isinstance(message_func, BinaryMessageFunction):
            return None
        if message_func.binary_op == "dot":
            return None
        if _Code2Str[message_func.lhs] != "u" or _Code2Str[message_func.rhs] != "e":
            return None
        return message_func.binary_op, message_func.lhs_field, message_func.rhs_field

    def _reduce(self, op, reduce_op, lhs, rhs):
        """gspmm whose max/min results get +-inf -> 0, as message passing wants."""
        replace_inf = reduce_op in ("max", "min")
        if _autograd.needs_grad(lhs, rhs):
            return _autograd.GSpMM.apply(self, op, reduce_op, lhs, rhs, replace_inf)
        out, _, _, as_torch, dev = _spmm._run(self, op, reduce_op, lhs, rhs,
                                              replace_inf=replace_inf)
        return _lib.give_back(out, as_torch, dev)

    def _pass(self, message_func, reduce_func, apply_node_func, write=True):
        """One message-passing round; returns the new node features.

        `write=False` leaves the feature store untouched (for `pull`).
        """
        num_nodes = self._num_nodes
        fused = self._fusable(message_func) if isinstance(message_func, MessageFunction) \
            else None
        if fused is not None and isinstance(reduce_func, ReduceFunction):
            op, lhs_field, rhs_field = fused
            lhs_data = self.ndata[lhs_field] if lhs_field is not None else None
            rhs_data = self.edata[rhs_field] if rhs_field is not None else None
            result = {reduce_func.out_field: self._reduce(op, reduce_func.name, lhs_data,
                                                          rhs_data)}
        else:
            if isinstance(message_func, MessageFunction):
                messages = {message_func.out_field: self._builtin_message(message_func)}
            else:
                edges = EdgeBatch(self, np.arange(self._E, dtype=np.int64))
                messages = dict(message_func(edges))
            if isinstance(reduce_func, ReduceFunction):
                key = next(iter(messages))
                result = {reduce_func.out_field: self._reduce("copy_rhs", reduce_func.name, None,
                                                              messages[key])}
            else:
                # the reduce UDF sees each message field pre-summed over in-edges
                mailbox = {k: self._reduce("copy_rhs", "sum", None, m)
                           for k, m in messages.items()}
                nodes = NodeBatch(data=self._nstore, mailbox=mailbox, num_nodes=num_nodes)
                result = dict(reduce_func(nodes))
        if apply_node_func is not None:
            nodes = NodeBatch(data=result, mailbox=None, num_nodes=num_nodes)
            result = dict(apply_node_func(nodes))
        if write:
            for key, value in result.items():
                self.ndata[key] = value
        return result

    def update_all(self, message_func, reduce_func, apply_node_func=None, etype=None):
        """Send messages along all the edges and update all the nodes.

        Parameters
        ----------
        message_func : builtin message function or callable(EdgeBatch) -> dict
        reduce_func : builtin reduce function or callable(NodeBatch) -> dict
        apply_node_func : callable(NodeBatch) -> dict, optional
        etype : str or (str, str, str), optional

        Nodes without in-edges get zero from every builtin reducer.
        """
        if etype is not None and etype not in self.canonical_etypes:
            raise DGLError("etype {} not in {}".format(etype, self.canonical_etypes))
        self._pass(message_func, reduce_func, apply_node_func)

    def pull(self, v, message_func, reduce_func, apply_node_func=None, etype=None):
        """Pull messages from the in-edges of nodes `v` and update only those rows.

        The written feature is zero outside `v` (reference heterograph.py:318-347).
        """
        if etype is not None and etype not in self.canonical_etypes:
            raise DGLError("etype {} not in {}".format(etype, self.canonical_etypes))
        v = np.unique(i64(v))
        if v.size == 0:
            return
        if int(v[0]) < 0 or int(v[-1]) >= self._num_nodes:
            raise DGLError("node ids must be in [0, {}), got [{}, {}]".format(
                self._num_nodes, int(v[0]), int(v[-1])))
        csr = self._device_csr("in")
        ip = csr.host_indptr
        degs = ip[v + 1] - ip[v]  # in-edges of v, known on the host
        pulled = int(degs.sum())
        builtin = (isinstance(message_func, MessageFunction)
                   and isinstance(reduce_func, ReduceFunction) and apply_node_func is None)
        fused = self._fusable(message_func) if builtin else None
        if fused is not None and int(degs.max()) <= PULL_ROWS_MAX_DEGREE:
            op, lhs_field, rhs_field = fused
            lhs = self.ndata[lhs_field] if lhs_field is not None else None
            rhs = self.edata[rhs_field] if rhs_field is not None else None
            if not _autograd.needs_grad(lhs, rhs):
                # the pulled rows of the graph's CSR, every other row zero
                red = reduce_func.name
                out, _, _, as_torch, dev = _spmm._run(
                    self, op, red, lhs, rhs, replace_inf=red in ("max", "min"),
                    rows=_lib.i32_device(v))
                self.ndata[reduce_func.out_field] = _lib.give_back(out, as_torch, dev)
                return
        if builtin and pulled * PULL_FULL_PASS >= self._E:
            # a builtin output row depends on its own in-edges only, so a pass
            # over every edge gives the subgraph's rows for v; taken when v's
            # in-edges are a large share of the graph (no subgraph to build)
            result = self._pass(message_func, reduce_func, None, write=False)
            self._write_pulled(result, v)
            return
        # the in-edges of `v` in edge-id order, selected on the GPU: a stable
        # grouping of the edges by whether their destination is pulled puts
        # them last, `pulled` of them; the subgraph is built from them there
        du, dv = self._device_coo()
        flag = torch.zeros(self._num_nodes, dtype=torch.int32, device=du.device)
        flag[torch.from_numpy(v).to(du.device)] = 1
        _, _, grouped = build_device_csr(flag[dv.long()], None, 2)
        sel = grouped[self._E - pulled:].long()
        sub = DGLGraph(du[sel], dv[sel], num_nodes=self._num_nodes)
        for key, value in self._nstore.items():
            sub.ndata[key] = value
        for key, value in self._estore.items():
            if isinstance(value, torch.Tensor):
                sub.edata[key] = value[sel.to(value.device)]
            else:
                sub.edata[key] = value[sel.cpu().numpy()]
        result = sub._pass(message_func, reduce_func, apply_node_func, write=False)
        self._write_pulled(result, v)

    def _write_pulled(self, result, v):
        """Store each result feature with the rows outside `v` zeroed
        (reference heterograph.py:344-347)."""
        for key, value in result.items():
            if isinstance(value, torch.Tensor):
                rows = torch.zeros_like(value)
                idx = torch.as_tensor(v, device=value.device)
                rows[idx] = value[idx]
            else:
                value = np.asarray(value)
                rows = np.zeros_like(value)
                rows[v] = value[v]
            self.ndata[key] = rows
