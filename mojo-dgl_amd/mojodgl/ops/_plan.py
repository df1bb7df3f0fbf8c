"""Host-side work plans for the softmax kernels (rows served by degree).

A softmax call on the GPU serves rows in three ways (csrc/softmax_impl.h):
rows of degree <= `slots` packed several to a wavefront by degree bin, rows of
degree <= `chunk_len` one wavefront each, longer rows as chunks of
`chunk_len` edges. `slots` and `chunk_len` come from mdgl_softmax_geometry
for the buffers of the call.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from .. import _lib


def _packed_bin(rows, indptr, k, eid, xp):
    """Edge ids of bin k's rows slot by slot: 2^k per row, -1 past the degree
    (`xp` is numpy or torch; `eid` None means the slot index itself)."""
    width = 1 << k
    start = indptr[rows]
    deg = indptr[rows + 1] - start
    if xp is np:
        slot = np.arange(width, dtype=np.int64)
    else:
        slot = torch.arange(width, dtype=torch.int64, device=rows.device)
    valid = slot[None, :] < deg[:, None]
    j = xp.where(valid, start[:, None] + slot[None, :], 0)
    val = j if eid is None else eid[j]
    if xp is not np:
        val = val.to(torch.int64)
    return xp.where(valid, val, -1).reshape(-1)


def _edge_slots(ordered_rows, chunk_row, chunk_first, indptr, eid):
    """Table slot of every edge's row for the two-pass edge_softmax: a row's
    position in the row order, or len(order) + the index of its first chunk
    for a chunked row. Indexed by edge id (by CSR slot when `eid` is None).
    numpy arrays give a numpy result, GPU tensors a GPU tensor (int32)."""
    nord = ordered_rows.shape[0]
    n_rows = indptr.shape[0] - 1
    if isinstance(indptr, np.ndarray):
        slot_of_row = np.full(n_rows, -1, dtype=np.int64)
        slot_of_row[ordered_rows] = np.arange(nord)
        if chunk_row is not None and chunk_row.shape[0]:
            heads = np.nonzero(chunk_first == np.arange(chunk_row.shape[0]))[0]
            slot_of_row[chunk_row[heads]] = nord + heads
        per_slot = slot_of_row[np.repeat(np.arange(n_rows), np.diff(indptr))]
        if eid is None:
            return per_slot.astype(np.int32)
        out = np.empty(per_slot.shape[0], dtype=np.int32)
        out[np.asarray(eid, dtype=np.int64)] = per_slot
        return out
    dev = indptr.device
    ip = indptr.to(torch.int64)
    slot_of_row = torch.full((n_rows,), -1, dtype=torch.int64, device=dev)
    slot_of_row[ordered_rows.to(torch.int64)] = torch.arange(nord, device=dev)
    if chunk_row is not None and chunk_row.shape[0]:
        heads = torch.nonzero(chunk_first.to(torch.int64)
                              == torch.arange(chunk_row.shape[0], device=dev)).squeeze(1)
        slot_of_row[chunk_row[heads].to(torch.int64)] = nord + heads
    n_slots = int(eid.shape[0]) if eid is not None else int(ip[-1].item())
    rows = torch.repeat_interleave(torch.arange(n_rows, device=dev), ip[1:] - ip[:-1],
                                   output_size=n_slots)
    per_slot = slot_of_row[rows].to(torch.int32)
    if eid is None:
        return per_slot
    out = torch.empty(n_slots, dtype=torch.int32, device=dev)
    out[eid.to(torch.int64)] = per_slot
    return out


class SoftmaxPlan:
    """Plan arrays on the GPU (order / packed edge ids / chunks / table slot
    of every edge) and the host bin bounds."""

    def __init__(self, indptr: np.ndarray, slots: int, chunk_len: int, ordered: bool,
                 eid: np.ndarray | None = None):
        deg = np.diff(indptr)
        self.slots = int(slots)
        self.chunk_len = int(chunk_len)
        self.nbins = int(np.log2(slots)) + 1
        heavy = np.nonzero(deg > chunk_len)[0]
        per = (deg[heavy] + chunk_len - 1) // chunk_len
        first = np.zeros(heavy.size + 1, dtype=np.int64)
        np.cumsum(per, out=first[1:])
        row = np.repeat(heavy, per)
        cfirst = np.repeat(first[:-1], per)
        local = np.arange(row.size, dtype=np.int64) - cfirst
        start = indptr[row] + local * chunk_len
        self.num_chunks = int(row.size)
        if self.num_chunks:
            self.chunk_row = _lib.i32_device(row)
            self.chunk_start = _lib.i32_device(start)
            self.chunk_first = _lib.i32_device(cfirst)
        else:
            self.chunk_row = self.chunk_start = self.chunk_first = None
        self.order = None
        self.bounds = None
        self.packed = None
        self.slot_of_edge = None
        self.table_rows = int(deg.shape[0])
        if ordered:
            rows = np.nonzero((deg > 0) & (deg <= chunk_len))[0]
            d = deg[rows]
            key = np.where(d <= slots, np.ceil(np.log2(np.maximum(d, 1))), self.nbins)
            key = key.astype(np.uint8)
            perm = np.argsort(key, kind="stable")
            ordered_rows = rows[perm]
            self.order = _lib.i32_device(ordered_rows)
            counts = np.bincount(key, minlength=self.nbins + 1)
            self.bounds = np.zeros(self.nbins + 2, dtype=np.int64)
            np.cumsum(counts, out=self.bounds[1:])
            ip = np.asarray(indptr, dtype=np.int64)
            parts = [_packed_bin(ordered_rows[self.bounds[k]:self.bounds[k + 1]], ip, k,
                                 None if eid is None else np.asarray(eid, dtype=np.int64), np)
                     for k in range(self.nbins) if self.bounds[k + 1] > self.bounds[k]]
            if parts:
                self.packed = _lib.i32_device(np.concatenate(parts))
            self.table_rows = int(ordered_rows.size) + self.num_chunks
            self.slot_of_edge = _lib.i32_device(_edge_slots(
                ordered_rows, row if self.num_chunks else None, cfirst, ip, eid))

    @classmethod
    def from_device(cls, indptr: torch.Tensor, slots: int, chunk_len: int, ordered: bool,
                    num_chunks: int | None = None, eid: torch.Tensor | None = None):
        """The same plan built on the GPU from GPU offsets (int32 or int64):
        chunks of the long rows, and with `ordered` the rows with
        0 < degree <= chunk_len grouped by degree bin, stably (ascending row
        id inside a bin), through the radix grouping of mdgl_build_csr, the
        packed rows' edge ids slot by slot (`eid` the CSR's edge ids, or None
        for the slot index) and the two-pass table slot of every edge
        (`slot_of_edge`, `table_rows`). `num_chunks`, when the caller knows
        it, saves a read back."""
        from ..heterograph import build_device_csr

        self = cls.__new__(cls)
        self.slots = int(slots)
        self.chunk_len = int(chunk_len)
        self.nbins = int(np.log2(slots)) + 1
        ip = indptr.to(torch.int64)
        deg = ip[1:] - ip[:-1]
        cl = self.chunk_len
        if num_chunks is None:
            num_chunks = int(torch.where(deg > cl, (deg + cl - 1) // cl, 0).sum().item())
        self.num_chunks = int(num_chunks)
        self.chunk_row = self.chunk_start = self.chunk_first = None
        if self.num_chunks:
            heavy = torch.nonzero(deg > cl).squeeze(1)
            per = (deg[heavy] + cl - 1) // cl
            first = torch.cumsum(per, 0) - per
            row = torch.repeat_interleave(heavy, per, output_size=self.num_chunks)
            cfirst = torch.repeat_interleave(first, per, output_size=self.num_chunks)
            local = torch.arange(self.num_chunks, dtype=torch.int64, device=ip.device) - cfirst
            self.chunk_row = row.to(torch.int32)
            self.chunk_start = (ip[row] + local * cl).to(torch.int32)
            self.chunk_first = cfirst.to(torch.int32)
        self.order = None
        self.bounds = None
        self.packed = None
        self.slot_of_edge = None
        self.table_rows = int(deg.shape[0])
        if ordered:
            nb = self.nbins
            # bin k (ceil(log2(degree))) for degree <= slots, bin nb for the
            # wavefront rows, nb + 1 (past the bounds) for empty and long rows
            bits = torch.zeros_like(deg)
            for j in range(nb - 1):
                bits += (deg > (1 << j)).to(torch.int64)
            key = torch.where(deg <= slots, bits, torch.full_like(deg, nb))
            key = torch.where((deg == 0) | (deg > cl), torch.full_like(deg, nb + 1), key)
            ptr, _, order = build_device_csr(key.to(torch.int32), None, nb + 2)
            self.order = order
            self.bounds = ptr[: nb + 2].cpu().numpy().astype(np.int64)
            b = self.bounds
            parts = [_packed_bin(order[b[k]:b[k + 1]].to(torch.int64), ip, k, eid, torch)
                     for k in range(nb) if b[k + 1] > b[k]]
            if parts:
                self.packed = torch.cat(parts).to(torch.int32)
            nord = int(b[nb + 1])
            self.table_rows = nord + self.num_chunks
            self.slot_of_edge = _edge_slots(order[:nord], self.chunk_row, self.chunk_first, ip,
                                            eid)
        return self

    def bounds_ptr(self):
        return None if self.bounds is None else self.bounds.ctypes.data


def geometry(d, dtype, logits: torch.Tensor, out: torch.Tensor):
    slots = ctypes.c_int64()
    chunk = ctypes.c_int64()
    rc = _lib.lib().mdgl_softmax_geometry(d, _lib.dtype_code(dtype), logits.data_ptr(),
                                          out.data_ptr(), ctypes.byref(slots),
                                          ctypes.byref(chunk))
    _lib.check(rc, "softmax_geometry")
    return slots.value, chunk.value


def workspace(plan: SoftmaxPlan, d, dtype, table_rows=0):
    n = _lib.lib().mdgl_softmax_workspace_bytes(plan.num_chunks, table_rows, d,
                                                _lib.dtype_code(dtype))
    if not n:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=_lib.device()), n
