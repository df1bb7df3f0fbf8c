"""Row grouping of gather_mm's sorted route on libmdgl (no vendor sort or
index kernels): the grouping equals numpy's stable argsort of idx_b (the
reference's gather_mm.py:79-87) bit for bit, gathering and scattering rows
by it are exact inverses through the C ABI, and gather_mm with more blocks
than the bucketed route takes matches the oracle and segment_mm on the
sorted rows."""

import numpy as np
import pytest
import torch

import mojodgl.ops as ops
import oracle
from mojodgl import _lib
from mojodgl.ops.gather_mm import group_rows, move_rows
from test_gpu_parity import close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,r", [(0, 3), (1, 1), (5000, 1), (70001, 7), (300000, 3000),
                                 (123457, 70000)])
def test_group_rows_is_numpy_stable_argsort(n, r):
    rng = np.random.default_rng(n + r)
    idx = rng.integers(0, r, n)
    if n > 100:
        idx[: n // 3] = np.sort(idx[: n // 3])  # runs as well as mixed rows
    perm, seglen = group_rows(torch.from_numpy(idx).cuda(), r)
    np.testing.assert_array_equal(perm.cpu().numpy(), np.argsort(idx, kind="stable"))
    np.testing.assert_array_equal(seglen.cpu().numpy(), np.bincount(idx, minlength=r))
    assert perm.dtype == torch.int32 and seglen.dtype == torch.int64


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("width", [1, 3, 4, 8, 33, 128])
@pytest.mark.parametrize("offset", [0, 1])
def test_gather_and_scatter_rows_are_inverse(dtype, width, offset):
    n = 5003
    rng = np.random.default_rng(width * 7 + offset)
    perm = torch.from_numpy(rng.permutation(n).astype(np.int32)).cuda()
    base = torch.randn(n * width + offset, dtype=dtype, device="cuda")
    x = base[offset:].view(n, width)
    got = move_rows(x, perm)
    assert torch.equal(got, x[perm.long()])
    back = torch.full_like(x, float("nan"))
    code = _lib.FLOAT32 if dtype == torch.float32 else _lib.FLOAT64
    rc = _lib.lib().mdgl_scatter_rows(got.data_ptr(), perm.data_ptr(), back.data_ptr(), n, width,
                                      code, _lib.stream())
    _lib.check(rc, "scatter_rows")
    assert torch.equal(back, x)
    assert torch.equal(move_rows(got, perm, scatter=True), x)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gather_mm_with_more_blocks_than_buckets(dtype):
    """R = 2100 > 2048 blocks: the grouped (sorted) route; equal to the oracle
    and, bit for bit, to segment_mm on the rows sorted by numpy's stable
    argsort and put back in place (the reference's sorted route,
    gather_mm.py:79-87)."""
    rng = np.random.default_rng(11)
    n, d1, d2, r = 6000, 12, 8, 2100
    a = rng.normal(size=(n, d1)).astype(dtype)
    b = (rng.normal(size=(r, d1, d2)) / 4).astype(dtype)
    idx = rng.integers(0, r, n)
    got = ops.gather_mm(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(),
                        idx_b=torch.from_numpy(idx).cuda()).cpu().numpy()
    close(got, oracle.gather_mm(a, b, idx, np.float64),
          oracle.gather_mm(np.abs(a), np.abs(b), idx, np.float64), dtype, "gather_mm r 2100")
    perm = np.argsort(idx, kind="stable")
    want = np.empty_like(got)
    want[perm] = ops.segment_mm(a[perm], b, np.bincount(idx, minlength=r))
    np.testing.assert_array_equal(got, want)
