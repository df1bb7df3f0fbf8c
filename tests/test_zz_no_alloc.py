"""mdgl_gspmm_noalloc (heavy-row partials in the library's device scratch)
against mdgl_gspmm (partials in a caller workspace), through the C ABI.

Both run the same kernels in the same order, so values and arg indices must
be bit-identical. Two calls in a row, the second smaller, so the scratch
keeps the first call's partials when the second one starts; sum, mean and
max with arg outputs; a call whose partials exceed the scratch is refused
before anything is launched.
"""

import numpy as np
import pytest
import torch

import mojodgl as dgl
from mojodgl import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # MDGL_NOALLOC_SCRATCH_BYTES of include/mdgl.h


def power_graph(n, e, hubs, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, n, e)
    v = rng.integers(0, n, e)
    for h in range(hubs):
        v[h::hubs * 3] = h * 7  # a third of the edges go to `hubs` rows
    return u, v


def call(entry, g, x, y, red, chunk_len, with_ws):
    """One gspmm u_mul_e over g's in-CSR with heavy rows cut into chunk_len-slot
    chunks; returns (out, arg_u, arg_e)."""
    L = _lib.lib()
    csr = g._device_csr("in")
    sched = csr.chunks_for(chunk_len)
    n, d = g.number_of_nodes(), x.shape[1]
    out = torch.full((n, d), float("nan"), dtype=x.dtype, device="cuda")
    arg = red in (_lib.REDUCE_MAX, _lib.REDUCE_MIN)
    au = torch.full((n, d), -7, dtype=torch.int32, device="cuda") if arg else None
    ae = torch.full((n, d), -7, dtype=torch.int32, device="cuda") if arg else None
    dt = _lib.dtype_code(np.float32 if x.dtype == torch.float32 else np.float64)
    args = [csr.indptr.data_ptr(), csr.indices.data_ptr(), csr.eid.data_ptr(), x.data_ptr(),
            y.data_ptr(), out.data_ptr(), n, _lib.OP_MUL, d, d, d, red, None, 0, None, None,
            _lib.ptr(au), _lib.ptr(ae), _lib.ptr(sched.chunk_row), _lib.ptr(sched.chunk_start),
            sched.num_chunks, sched.chunk_len, _lib.ptr(sched.heavy_rows),
            _lib.ptr(sched.heavy_ptr), sched.num_heavy]
    if with_ws:
        nbytes = L.mdgl_gspmm_workspace_bytes(sched.num_chunks, d, red, dt)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        args += [ws.data_ptr(), nbytes]
    rc = entry(*args, 0, dt, _lib.stream())
    _lib.check(rc, entry.__name__)
    torch.cuda.synchronize()
    return out, au, ae, sched.num_chunks


def test_noalloc_matches_the_workspace_entry_point_twice():
    L = _lib.lib()
    cases = [(power_graph(20_000, 200_000, 3, 1), 64, torch.float32, 8),
             (power_graph(3_000, 30_000, 2, 2), 16, torch.float64, 8)]
    for (u, v), d, dtype, chunk_len in cases:
        g = dgl.graph((u, v), num_nodes=int(max(u.max(), v.max())) + 1)
        gen = torch.Generator(device="cuda").manual_seed(d)
        x = torch.randn(g.number_of_nodes(), d, device="cuda", dtype=dtype, generator=gen)
        y = torch.randn(g.number_of_edges(), d, device="cuda", dtype=dtype, generator=gen)
        for red in (_lib.REDUCE_SUM, _lib.REDUCE_MEAN, _lib.REDUCE_MAX):
            want = call(L.mdgl_gspmm, g, x, y, red, chunk_len, True)
            got = call(L.mdgl_gspmm_noalloc, g, x, y, red, chunk_len, False)
            case = "d {} {} red {} chunks {}".format(d, dtype, red, want[3])
            assert want[3] > 1000, case  # the partials really pass through the scratch
            assert torch.equal(got[0], want[0]), case
            assert not torch.isnan(got[0]).any(), case
            if red == _lib.REDUCE_MAX:
                assert torch.equal(got[1], want[1]) and torch.equal(got[2], want[2]), case


def test_noalloc_refuses_partials_beyond_the_scratch():
    L = _lib.lib()
    d = 4096
    chunks = SCRATCH_BYTES // (4 * d) + 1
    assert L.mdgl_gspmm_workspace_bytes(chunks, d, _lib.REDUCE_SUM, _lib.FLOAT32) > SCRATCH_BYTES
    # no buffers at all: the size check comes before anything else is looked at
    rc = L.mdgl_gspmm_noalloc(None, None, None, None, None, None, 10, _lib.OP_MUL, d, d, d,
                              _lib.REDUCE_SUM, None, 0, None, None, None, None, None, None,
                              chunks, 8, None, None, 1, 0, _lib.FLOAT32, None)
    assert rc == _lib.EWORKSPACE
    assert b"scratch" in L.mdgl_last_error()
