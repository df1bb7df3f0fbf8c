"""Feature store and the arguments of user-defined functions.

Public surface as in the reference (python/mojodgl/udf.py): `FeatureDict` is
`g.ndata` / `g.edata`; a message UDF receives an `EdgeBatch` whose `src`,
`dst` and `data` give the node features of every edge's endpoints and the
edge features; a reduce or apply UDF receives a `NodeBatch` whose
`mailbox` holds the messages (pre-summed per node, a documented divergence of
the reference) and whose `data` holds node features.

Differences from the reference's store: float32 and float64 values keep
their dtype (the reference turns every assignment into float64,
udf.py:18-26) and torch tensors stay tensors on their device, so GPU features
are never copied between calls. Every other dtype becomes float64.

Design: the store is a `MutableMapping` that validates on assignment; the
three per-edge views of an `EdgeBatch` are one read-only `Mapping` type,
`RowSelection`, which gathers the rows of a feature by an index array
(converted once to a device tensor the first time a tensor feature asks).
"""

from __future__ import annotations

from collections.abc import Mapping, MutableMapping

import numpy as np
import torch

__all__ = ["FeatureDict", "NodeBatch", "EdgeBatch"]


def _admit(value, num_rows: int, label: str):
    """`value` as stored: tensors as given, arrays float32 or float64,
    C-contiguous; its leading axis must have `num_rows` entries."""
    if not isinstance(value, torch.Tensor):
        value = np.asarray(value)
        keep = value.dtype if value.dtype == np.float32 else np.float64
        value = np.ascontiguousarray(value, dtype=keep)
    shape = tuple(value.shape)
    if not shape or shape[0] != num_rows:
        raise ValueError("{} expects {} rows, got shape {}".format(label, num_rows, shape))
    return value


class FeatureDict(MutableMapping):
    """Feature name -> array or tensor with one row per node (`ndata`) or per
    edge (`edata`). Writes are checked for the row count; reads raise
    KeyError for a missing name."""

    def __init__(self, store: dict, num_rows: int, what: str):
        # `store` is the graph's own dict: the dispatcher reads it directly
        self._features = store
        self.num_rows = int(num_rows)
        self.label = what

    def __setitem__(self, name, value):
        self._features[name] = _admit(value, self.num_rows, self.label)

    def __getitem__(self, name):
        if name not in self._features:
            raise KeyError("{} has no feature {!r}".format(self.label, name))
        return self._features[name]

    def __delitem__(self, name):
        del self._features[name]

    def __iter__(self):
        return iter(self._features)

    def __len__(self):
        return len(self._features)

    def __repr__(self):
        return "{}({})".format(self.label, dict(self._features))


class RowSelection(Mapping):
    """Read-only view of a feature mapping restricted to the rows `index`
    (in that order, repeats allowed): `view[name]` is `features[name][index]`
    for numpy arrays and `index_select` for tensors."""

    def __init__(self, features: Mapping, index: np.ndarray, name: str):
        self._features = features
        self._index = index
        self._dev_index = {}
        self.name = name

    def _on(self, device) -> torch.Tensor:
        idx = self._dev_index.get(device)
        if idx is None:
            idx = torch.as_tensor(self._index, dtype=torch.int64, device=device)
            self._dev_index[device] = idx
        return idx

    def __getitem__(self, key):
        value = self._features[key]
        if isinstance(value, torch.Tensor):
            return value.index_select(0, self._on(value.device))
        return value[self._index]

    def __iter__(self):
        return iter(self._features)

    def __len__(self):
        return len(self._features)

    def __contains__(self, key):
        return key in self._features

    def __repr__(self):
        return self.name


class NodeBatch:
    """Argument of a reduce or apply-node UDF. `nodes[name]` looks in the
    mailbox first, then in the node data."""

    def __init__(self, data=None, mailbox=None, num_nodes: int = 0, batch_num_nodes=None):
        self.data = {} if data is None else data
        self.mailbox = {} if mailbox is None else mailbox
        self._count = int(num_nodes)

    def __getitem__(self, key):
        source = self.mailbox if key in self.mailbox else self.data
        return source[key]

    def num_nodes(self, ntype=None) -> int:
        return self._count

    def batch_num_nodes(self, ntype=None):
        return [self._count]

    def __repr__(self):
        names = [*self.mailbox, *self.data]
        return "NodeBatch(num_nodes={}, keys={})".format(self._count, names)


class EdgeBatch:
    """Argument of a message UDF over the edges `eids` (edge-id order):
    `src` / `dst` are the node features of their endpoints, `data` the edge
    features."""

    def __init__(self, graph, eids: np.ndarray):
        self._graph = graph
        self._eids = np.asarray(eids)
        self.src = RowSelection(graph.ndata, graph._u[self._eids], "src")
        self.dst = RowSelection(graph.ndata, graph._v[self._eids], "dst")
        self.data = RowSelection(graph.edata, self._eids, "data")

    @property
    def number_of_nodes(self) -> int:
        return self._graph.number_of_nodes()

    @property
    def number_of_edges(self) -> int:
        return int(self._eids.size)

    def batch_num_nodes(self, ntype=None):
        return [self.number_of_nodes]

    def batch_num_edges(self, etype=None):
        return [self.number_of_edges]

    def __repr__(self):
        return "EdgeBatch(num_edges={})".format(self.number_of_edges)
