"""segment_reduce's kernels: rows staged through LDS (narrow rows), row
streams (wide rows) and the split pass for segments longer than
MDGL_SEGMENT_SPLIT_ROWS, against the oracle under the tolerance rule of
test_gpu_parity.py.

Segments folded row by row (every segment when none is longer than the
split threshold) are bit-identical to the oracle in the same precision;
split segments are exact for max / min and their arg rows and within the
tolerance for sums. The arg row is pinned by brute force: the first row of
the segment holding the selected value (NaN never selected)."""

import numpy as np
import pytest
import torch

import mojodgl.ops as ops
import oracle
from mojodgl import _lib
from test_gpu_parity import close

pytestmark = pytest.mark.gpu

SPLIT = 4096  # MDGL_SEGMENT_SPLIT_ROWS


def lengths(rng, S, mean, long_rows=()):
    seglen = rng.poisson(mean, S)
    seglen[::11] = 0
    for i, n in enumerate(long_rows):
        seglen[(i * 37 + 5) % S] = n
    return seglen


def first_arg(seglen, value, reducer):
    """Row of the first max / min of each segment and column (-1 when none
    is selected)."""
    off = np.concatenate([[0], np.cumsum(seglen)])
    d = value.shape[1]
    out = np.full((seglen.size, d), -1, dtype=np.int64)
    for s in range(seglen.size):
        rows = value[off[s]:off[s + 1]]
        if rows.shape[0] == 0:
            continue
        for k in range(d):
            col = rows[:, k]
            ok = ~np.isnan(col)
            if not ok.any():
                continue
            best = np.max(col[ok]) if reducer == "max" else np.min(col[ok])
            if np.isinf(best) and (best < 0 if reducer == "max" else best > 0):
                continue  # never beats the identity
            out[s, k] = off[s] + int(np.nonzero(col == best)[0][0])
    return out


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 2, 3, 5, 16, 33, 64, 130, 602])
@pytest.mark.parametrize("reducer", ["sum", "max", "mean"])
def test_segment_reduce_widths_bit_exact(dtype, d, reducer):
    """No segment above the split threshold: every kernel folds row by row."""
    rng = np.random.default_rng(d * 3 + len(reducer))
    S = 1500 if d < 100 else 300
    seglen = lengths(rng, S, 20, long_rows=(SPLIT, 1000))
    value = rng.standard_normal((int(seglen.sum()), d)).astype(dtype)
    for lens in (seglen, torch.from_numpy(seglen).cuda()):
        got = ops.segment_reduce(lens, torch.from_numpy(value).cuda(), reducer)
        np.testing.assert_array_equal(got.cpu().numpy(),
                                      oracle.segment_reduce(seglen, value, reducer, dtype),
                                      err_msg="{} d {}".format(reducer, d))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 3, 16, 40, 300])
def test_segment_reduce_long_segments_split(dtype, d):
    """Segments above the split threshold (one of them 1M rows for narrow
    rows) among short ones: max / min exact, sums within the tolerance,
    the short segments still bit-identical."""
    rng = np.random.default_rng(100 + d)
    big = (1_000_000, SPLIT + 1, 9000) if d <= 16 else (SPLIT + 1, 20000)
    seglen = lengths(rng, 700, 15, long_rows=big)
    value = rng.standard_normal((int(seglen.sum()), d)).astype(dtype)
    vt = torch.from_numpy(value).cuda()
    short = seglen <= SPLIT
    for lens in (seglen, torch.from_numpy(seglen).cuda()):
        for reducer in ("sum", "mean", "max", "min"):
            got = ops.segment_reduce(lens, vt, reducer).cpu().numpy()
            same = oracle.segment_reduce(seglen, value, reducer, dtype)
            if reducer in ("max", "min"):
                np.testing.assert_array_equal(got, same, err_msg=reducer)
            else:
                np.testing.assert_array_equal(got[short], same[short], err_msg=reducer)
                ref = oracle.segment_reduce(seglen, value, reducer, np.float64)
                bound = oracle.segment_reduce(seglen, np.abs(value), reducer, np.float64)
                close(got, ref, bound, dtype, "segment_reduce {} d {}".format(reducer, d))


@pytest.mark.parametrize("d", [1, 4, 16, 33, 200])
def test_segment_reduce_arg_rows(d):
    """mdgl_segment_reduce_arg: the selected row is the first reaching the
    value, in folded and in split segments, with ties and NaN present."""
    rng = np.random.default_rng(200 + d)
    seglen = lengths(rng, 400, 12, long_rows=(SPLIT + 300, 7000))
    n = int(seglen.sum())
    value = np.round(rng.standard_normal((n, d)) * 2).astype(np.float32)  # many ties
    value[rng.random((n, d)) < 0.05] = np.nan
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(seglen)]).astype(np.int32)).cuda()
    vt = torch.from_numpy(value).cuda()
    L = _lib.lib()
    for reducer in ("max", "min"):
        for flags in (0, _lib.SEGMENTS_SHORT):  # split pass, or every segment folded whole
            out = torch.empty(seglen.size, d, device="cuda")
            arg = torch.full((seglen.size, d), -9, dtype=torch.int32, device="cuda")
            rc = L.mdgl_segment_reduce_arg(off.data_ptr(), vt.data_ptr(), out.data_ptr(),
                                           arg.data_ptr(), seglen.size, d,
                                           _lib.REDUCERS[reducer], n, flags, _lib.FLOAT32,
                                           _lib.stream())
            _lib.check(rc, "segment_reduce_arg")
            want = oracle.segment_reduce(seglen, value, reducer, np.float32)
            got = out.cpu().numpy()
            got = np.where(np.isinf(got), 0, got)  # the oracle's +-inf -> 0
            np.testing.assert_array_equal(got, want, err_msg="{} {}".format(reducer, flags))
            np.testing.assert_array_equal(arg.cpu().numpy(), first_arg(seglen, value, reducer),
                                          err_msg="{} args {}".format(reducer, flags))


def test_short_segment_hint_is_only_a_hint():
    """MDGL_SEGMENTS_SHORT with a segment above the threshold: that segment is
    folded whole, in row order (bit-identical), not skipped."""
    rng = np.random.default_rng(300)
    seglen = lengths(rng, 300, 10, long_rows=(20000,))
    n = int(seglen.sum())
    value = rng.standard_normal((n, 8)).astype(np.float32)
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(seglen)]).astype(np.int32)).cuda()
    vt = torch.from_numpy(value).cuda()
    out = torch.full((seglen.size, 8), float("nan"), device="cuda")
    rc = _lib.lib().mdgl_segment_reduce(off.data_ptr(), vt.data_ptr(), out.data_ptr(), seglen.size,
                                        8, _lib.REDUCERS["sum"], n, _lib.SEGMENTS_SHORT,
                                        _lib.FLOAT32, _lib.stream())
    _lib.check(rc, "segment_reduce")
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  oracle.segment_reduce(seglen, value, "sum", np.float32))


def test_segment_reduce_clamps_offsets_into_the_rows():
    """Offsets past the row count (here only through the C ABI: the API
    refuses them) read as segments clipped to the rows, never beyond."""
    rng = np.random.default_rng(301)
    n, d = 5000, 16
    value = rng.standard_normal((n, d)).astype(np.float32)
    raw = np.array([0, 100, 4000, 6000, 9000, 200], dtype=np.int32)  # ends past n, one backwards
    off = torch.from_numpy(raw).cuda()
    out = torch.empty(raw.size - 1, d, device="cuda")
    rc = _lib.lib().mdgl_segment_reduce(off.data_ptr(), torch.from_numpy(value).cuda().data_ptr(),
                                        out.data_ptr(), raw.size - 1, d, _lib.REDUCERS["max"], n, 0,
                                        _lib.FLOAT32, _lib.stream())
    _lib.check(rc, "segment_reduce")
    clipped = np.clip(raw.astype(np.int64), 0, n)
    lens = np.maximum(np.diff(clipped), 0)
    lens[-1] = 0
    starts = clipped[:-1]
    got = out.cpu().numpy()
    for s in range(raw.size - 1):
        rows = value[starts[s]:starts[s] + lens[s]]
        want = rows.max(axis=0) if lens[s] else np.full(d, -np.inf, dtype=np.float32)
        np.testing.assert_array_equal(got[s], want, err_msg=str(s))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 16])
def test_segment_softmax_short_with_backward_offsets(dtype, d):
    """Offsets that run backwards (only through the C ABI: GPU lengths are
    checked after this call, and the API then raises) leave rows inside a
    staged window that no segment claims: [10, 12, 0, 2, 2, 5] gives the
    segments [10, 12), [0, 2) and [2, 5) in one window of rows [0, 12), with
    rows 5-9 in none. Those rows, and the rows past the segments, are left as
    they were; the claimed rows hold their segment's softmax."""
    rng = np.random.default_rng(302 + d)
    n = 40
    value = rng.standard_normal((n, d)).astype(dtype)
    raw = np.array([10, 12, 0, 2, 2, 5], dtype=np.int32)
    off = torch.from_numpy(raw).cuda()
    out = torch.full((n, d), 7.0, dtype=torch.float32 if dtype == np.float32 else torch.float64,
                     device="cuda")
    rc = _lib.lib().mdgl_segment_softmax_short(
        off.data_ptr(), torch.from_numpy(value).cuda().data_ptr(), out.data_ptr(), raw.size - 1,
        d, n, _lib.FLOAT32 if dtype == np.float32 else _lib.FLOAT64, _lib.stream())
    _lib.check(rc, "segment_softmax_short")
    got = out.cpu().numpy()
    want = np.full((n, d), 7.0, dtype=dtype)
    for lo, hi in ((10, 12), (0, 2), (2, 5)):
        want[lo:hi] = oracle.segment_softmax(np.array([hi - lo]), value[lo:hi], dtype)
    tol = 1e-6 if dtype == np.float32 else 1e-15
    np.testing.assert_allclose(got, want, rtol=tol, atol=0)
    np.testing.assert_array_equal(got[5:10], 7.0)
    np.testing.assert_array_equal(got[12:], 7.0)


@pytest.mark.parametrize("d", [3, 16, 40])
def test_skip_long_then_long_only_equals_one_call(d):
    """MDGL_SEGMENTS_SKIP_LONG leaves the segments above the split threshold
    unwritten and MDGL_SEGMENTS_LONG_ONLY writes only those: the two calls
    together write what one call without either flag writes, values and
    arg rows alike (the order segment_reduce uses for GPU lengths, whose
    longest length is known only after the first call is queued)."""
    rng = np.random.default_rng(400 + d)
    seglen = lengths(rng, 500, 14, long_rows=(SPLIT + 1, 12000, SPLIT))
    n = int(seglen.sum())
    value = np.round(rng.standard_normal((n, d)) * 3).astype(np.float32)
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(seglen)]).astype(np.int32)).cuda()
    vt = torch.from_numpy(value).cuda()
    long_ = seglen > SPLIT
    L = _lib.lib()
    for reducer in ("sum", "max"):
        red = _lib.REDUCERS[reducer]
        results = []
        for passes in ((0,), (_lib.SEGMENTS_SKIP_LONG, _lib.SEGMENTS_LONG_ONLY)):
            out = torch.full((seglen.size, d), 12345.0, device="cuda")
            arg = torch.full((seglen.size, d), -9, dtype=torch.int32, device="cuda")
            for i, flags in enumerate(passes):
                if reducer == "max":
                    rc = L.mdgl_segment_reduce_arg(off.data_ptr(), vt.data_ptr(), out.data_ptr(),
                                                   arg.data_ptr(), seglen.size, d, red, n, flags,
                                                   _lib.FLOAT32, _lib.stream())
                else:
                    rc = L.mdgl_segment_reduce(off.data_ptr(), vt.data_ptr(), out.data_ptr(),
                                               seglen.size, d, red, n, flags, _lib.FLOAT32,
                                               _lib.stream())
                _lib.check(rc, "segment_reduce")
                if flags == _lib.SEGMENTS_SKIP_LONG:
                    first = out.cpu().numpy()
                    assert (first[long_] == 12345.0).all(), "long segments written by SKIP_LONG"
                    assert (first[~long_] != 12345.0).all()
                    if reducer == "max":
                        assert (arg.cpu().numpy()[long_] == -9).all()
            results.append((out.cpu().numpy(), arg.cpu().numpy()))
        np.testing.assert_array_equal(results[0][0], results[1][0], err_msg=reducer)
        if reducer == "max":
            np.testing.assert_array_equal(results[0][1], results[1][1], err_msg="args")


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("d", [1, 16, 33])
def test_segment_softmax_short_leaves_long_segments(dtype, d):
    """mdgl_segment_softmax_short: the rows of segments of at most chunk_len
    rows are the softmax (against the oracle), the rows of longer segments
    are left as they were."""
    from mojodgl.ops import _plan

    rng = np.random.default_rng(500 + d)
    probe = torch.zeros(4, d, dtype=torch.float32 if dtype == np.float32 else torch.float64,
                        device="cuda")
    slots, chunk_len = _plan.geometry(d, dtype, probe, torch.zeros_like(probe))
    seglen = rng.poisson(10, 800)
    seglen[::13] = 0
    seglen[[5, 300]] = [chunk_len + 1, 3 * chunk_len]
    seglen[[6, 301]] = [chunk_len, 1]
    n = int(seglen.sum())
    value = (rng.normal(size=(n, d)) * 2).astype(dtype)
    val = torch.from_numpy(value).cuda()
    out = torch.full_like(val, 7.0)
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(seglen)]).astype(np.int32)).cuda()
    rc = _lib.lib().mdgl_segment_softmax_short(off.data_ptr(), val.data_ptr(), out.data_ptr(),
                                               seglen.size, d, n, _lib.dtype_code(dtype),
                                               _lib.stream())
    V = 16 // np.dtype(dtype).itemsize
    if (d // V if d % V == 0 else d) > 32:  # wider than the staged kernel takes
        assert rc == _lib.ENOTSUP
        return
    _lib.check(rc, "segment_softmax_short")
    got = out.cpu().numpy()
    row_long = np.repeat(seglen > chunk_len, seglen)
    assert (got[row_long] == 7.0).all()
    ref = oracle.segment_softmax(seglen, value, np.float64)
    close(got[~row_long], ref[~row_long], ref[~row_long], dtype, "segment_softmax_short")
