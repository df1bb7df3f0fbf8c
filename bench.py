#!/usr/bin/env python3
"""Benchmark of the message-passing kernel layer on one MI355X.

Headline workload (one "step"): the GAT attention layer on the power-law
graph -- N = 2,500,000 nodes, E = 60,000,000 edges, in-degrees Zipf(2.1)
capped at 20,000, uniform sources, H = 8 heads of 32 features, float32:

    e = gsddmm u_add_v(el, er)            (E, 8, 1)
    e = leaky_relu(e, 0.2)                (the caller's op: torch, in place)
    a = edge_softmax(g, e, norm_by='dst') (E, 8, 1)
    z = gspmm u_mul_e_sum(h, a)           (N, 8, 32)

All inputs and the graph's GPU CSR are resident in HBM before timing.
`value` is GEdge*feat/s of the whole step (E * 8 + E * 8 + E * 256 edge-feature
units per step, the three library ops' output widths). The JSON line also
carries the roofline of the dominant kernel (gspmm, timed with HIP events on
the stream it is launched on) and the CPU baseline (the oracle, a C++
restatement of the reference's kernels, timed on this host on a sample).

After the headline the default run measures every other configuration and
adds them under "configs" (each op: HIP-event median and best over
repetitions that each start with the L2 and the 256 MB MALL flushed by a
512 MB write, algorithmic bytes or flops, the fraction of the HBM or MFMA
peak, and the oracle's CPU rate on a stated sample):

  c1  update_all u_mul_e + sum / mean / max / min, uniform 10k-node graph
  c2_f64  gspmm u_mul_e_sum of the headline graph in float64
  c3  GCN aggregation on a 50-block community graph (114M edges x 602)
  c4  gsddmm u_dot_v (20M edges x 128), segment_reduce, segment_softmax
  c5  gather_mm and segment_mm (1e7 rows, 128 x 128, 64 relations) on MFMA

--workload c1|c3|c4|c5 runs one of them alone as its own line, and
--workload gat_train the headline layer with autograd (forward + backward).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mojo-dgl_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_F64_PEAK_TFLOPS = 78.6
FLUSH_BYTES = 512 << 20
# Fabric read requests leave the L2 as 32-, 64- or 128-byte transactions. On
# this GPU the 128-byte count (TCC_BUBBLE) reads 0, which makes FETCH_SIZE
# report half of a plain copy; the bytes are therefore formed from the total
# and the 32- and 64-byte counts (a 1 GiB copy reads 8.39M requests = 1 GiB).
# Writes are 32- or 64-byte transactions (WRITE_SIZE's own formula).
READ_COUNTERS = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum")
WRITE_COUNTERS = ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum")


def read_bytes(c):
    """Fabric read bytes from the request counts (READ_COUNTERS)."""
    total, r32, r64 = (c.get(k, 0.0) for k in READ_COUNTERS)
    return 128.0 * (total - r32 - r64) + 64.0 * r64 + 32.0 * r32


def write_bytes(c):
    """Fabric write bytes from the transaction counts (WRITE_COUNTERS)."""
    total, w64 = (c.get(k, 0.0) for k in WRITE_COUNTERS)
    return 32.0 * (total - w64) + 64.0 * w64


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- generators
def power_law_graph(seed=1, n=2_500_000, e=60_000_000, a=2.1, cap=20_000):
    """Destination degrees ~ Zipf(a) capped at `cap` (excess redistributed over
    uncapped nodes by multinomial until none exceeds it); sources uniform."""
    rng = np.random.default_rng(seed)
    z = np.minimum(rng.zipf(a, n), cap).astype(np.float64)
    deg = rng.multinomial(e, z / z.sum())
    while deg.max() > cap:
        excess = int(np.maximum(deg - cap, 0).sum())
        deg = np.minimum(deg, cap)
        free = deg < cap
        p = np.where(free, z, 0.0)
        deg += rng.multinomial(excess, p / p.sum())
    v = np.repeat(np.arange(n, dtype=np.int64), deg)
    v = v[rng.permutation(e)]
    u = rng.integers(0, n, e, dtype=np.int64)
    stats = {"max_in_degree": int(deg.max()), "nodes_at_cap": int((deg == cap).sum()),
             "zero_in_degree": int((deg == 0).sum())}
    return u, v, stats


def uniform_graph(seed, n, e):
    rng = np.random.default_rng(seed)
    return rng.integers(0, n, e, dtype=np.int64), rng.integers(0, n, e, dtype=np.int64)


def community_graph(seed=2, blocks=50, per_block=4_600, e=114_000_000, intra=0.95):
    rng = np.random.default_rng(seed)
    n = blocks * per_block
    e_in = int(e * intra) // blocks * blocks
    per = e_in // blocks
    b = np.repeat(np.arange(blocks, dtype=np.int64), per) * per_block
    u = np.concatenate([b + rng.integers(0, per_block, e_in), rng.integers(0, n, e - e_in)])
    v = np.concatenate([b + rng.integers(0, per_block, e_in), rng.integers(0, n, e - e_in)])
    perm = rng.permutation(e)
    return u[perm], v[perm], n


# ---------------------------------------------------------------- counters
TRAFFIC_CALLS = 3


def workload_gspmm_traffic(args):
    """The headline graph's gspmm u_mul_e_sum, TRAFFIC_CALLS calls and nothing
    else of the library: run under rocprofv3 --pmc by measure_traffic."""
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops

    N, E, H, D = args.nodes, args.edges, 8, 32
    u, v, _ = power_law_graph(1, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    g._device_csr("in")
    gen = torch.Generator(device="cuda").manual_seed(1)
    h = torch.randn(N, H, D, device="cuda", generator=gen)
    a = torch.rand(E, H, 1, device="cuda", generator=gen)
    torch.cuda.synchronize()
    for _ in range(TRAFFIC_CALLS):
        ops.u_mul_e_sum(g, h, a)
    torch.cuda.synchronize()
    return {"calls": TRAFFIC_CALLS}


def pmc_totals(db_path, kernel_substr):
    """{counter: sum over the dispatches of kernels whose name holds
    kernel_substr} from a rocprofv3 database, and the dispatch count."""
    import sqlite3

    con = sqlite3.connect(db_path)
    sums, disp = {}, set()
    for d, name, cname, val in con.execute(
            "select dispatch_id, kernel_name, counter_name, value from counters_collection"):
        if kernel_substr in name:
            sums[cname] = sums.get(cname, 0.0) + float(val)
            disp.add(d)
    con.close()
    return sums, len(disp)


def measure_traffic(args):
    """Fabric bytes per gspmm u_mul_e_sum call on the headline graph, live:
    two child runs of this script (--workload gspmm_traffic) under
    rocprofv3 --pmc, one per counter group, each under its own time limit
    (the whole process group is killed past it). Started before this process
    touches the GPU. Returns the traffic entry, with the reason when a pass
    fails (then no bytes)."""
    import shutil
    import signal
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    tmp = tempfile.mkdtemp(prefix="mdgl_traffic_")
    totals, dispatches = {}, {}
    for name, counters in (("read", READ_COUNTERS), ("write", WRITE_COUNTERS)):
        cmd = [exe, "--pmc", *counters, "--kernel-include-regex", "gspmm_kernel", "-d", tmp,
               "-o", name, "--", sys.executable, os.path.abspath(__file__), "--workload",
               "gspmm_traffic", "--nodes", str(args.nodes), "--edges", str(args.edges)]
        log("rocprofv3 pass ({}): {}".format(name, " ".join(counters)))
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                                start_new_session=True)
        try:
            out, err = proc.communicate(timeout=args.traffic_timeout)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.communicate()
            return {"bytes": None, "reason": "rocprofv3 pass {} passed {} s".format(
                name, args.traffic_timeout)}
        db = os.path.join(tmp, name + "_results.db")
        if '"calls"' not in out or not os.path.exists(db):
            return {"bytes": None, "reason": "rocprofv3 pass {} ended with status {}: {}".format(
                name, proc.returncode, (err or out).strip()[-300:])}
        sums, nd = pmc_totals(db, "gspmm_kernel")
        totals.update(sums)
        dispatches[name] = nd
    rd, wr = read_bytes(totals), write_bytes(totals)
    shutil.rmtree(tmp, ignore_errors=True)
    return {"bytes": round((rd + wr) / TRAFFIC_CALLS), "read_bytes": round(rd / TRAFFIC_CALLS),
            "write_bytes": round(wr / TRAFFIC_CALLS),
            "requests": {k: round(v / TRAFFIC_CALLS) for k, v in totals.items()},
            "gspmm_kernel_dispatches_per_call": dispatches["read"] / TRAFFIC_CALLS,
            "source": "this run: rocprofv3 --pmc {} and {} over {} calls of gspmm u_mul_e_sum on "
                      "the same graph in a child process; bytes = 128 x (requests - 32B - 64B) + "
                      "64 x 64B + 32 x 32B reads, 32 x (transactions - 64B) + 64 x 64B "
                      "writes".format(" ".join(READ_COUNTERS), " ".join(WRITE_COUNTERS),
                                      TRAFFIC_CALLS)}


# ---------------------------------------------------------------- timing
class OpTimer:
    """HIP events around each op on torch's current stream, where libmdgl
    launches (the stream handle is passed through the C ABI)."""

    def __init__(self):
        import torch

        self.torch = torch
        self.pending = {}
        self.totals = {}
        self.counts = {}

    def __call__(self, name, fn):
        torch = self.torch
        s = torch.cuda.Event(enable_timing=True)
        t = torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn()
        t.record()
        self.pending.setdefault(name, []).append((s, t))
        return out

    def collect(self):
        for name, evs in self.pending.items():
            for s, t in evs:
                self.totals[name] = self.totals.get(name, 0.0) + s.elapsed_time(t)
                self.counts[name] = self.counts.get(name, 0) + 1
        self.pending = {}

    def avg_ms(self, name):
        return self.totals[name] / self.counts[name]


def run_steps(step, steps, warmup, timer):
    """ms per step over `steps` timed steps (after `warmup`), bracketed by
    synchronizations; then the same number of steps again with HIP events
    around each op for `timer`'s per-op figures (kept out of the step's
    clock: a launch-bound step would otherwise carry the events' host
    cost)."""
    import torch

    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(None)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        step(timer)
    torch.cuda.synchronize()
    timer.collect()
    return (t1 - t0) * 1e3 / steps


class _CountingLib:
    """Stands in for the loaded libmdgl handle and counts its mdgl_* calls."""

    def __init__(self, real):
        self._real = real
        self.calls = {}

    def __getattr__(self, name):
        attr = getattr(self._real, name)
        if not name.startswith("mdgl_"):
            return attr

        def counted(*a):
            self.calls[name] = self.calls.get(name, 0) + 1
            return attr(*a)
        return counted


def host_accounting(calls, reps):
    """Host-side cost of each public call (the reference's profile_deep.py
    counts ctypes calls and allocations per op; bench/analysis.md:84 its
    glue time): the libmdgl entry points one call makes, by name; the device
    allocations it asks torch's caching allocator for (requests and bytes;
    the allocator serves them from its cache after the first call); the host
    time until the call returns (its GPU work enqueued, not finished), median
    of `reps`; and the time per call when `reps` calls run back to back (HIP
    events), which the host time bounds for small ops. Each call runs once
    first, so the graph's one-time set-up (CSR build, schedules) is not
    counted."""
    import torch

    from mojodgl import _lib

    out = {}
    real = _lib.lib()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    for name, fn_ in calls.items():
        fn_()
        torch.cuda.synchronize()
        proxy = _CountingLib(real)
        m0 = torch.cuda.memory_stats()
        _lib._lib = proxy
        try:
            fn_()
        finally:
            _lib._lib = real
        m1 = torch.cuda.memory_stats()
        torch.cuda.synchronize()
        host = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn_()
            host.append(time.perf_counter() - t0)
        torch.cuda.synchronize()
        s.record()
        for _ in range(reps):
            fn_()
        t.record()
        torch.cuda.synchronize()
        out[name] = {
            "lib_calls": sum(proxy.calls.values()),
            "entry_points": dict(sorted(proxy.calls.items())),
            "device_allocations": int(m1.get("allocation.all.allocated", 0)
                                      - m0.get("allocation.all.allocated", 0)),
            "device_alloc_bytes": int(m1.get("allocated_bytes.all.allocated", 0)
                                      - m0.get("allocated_bytes.all.allocated", 0)),
            "host_us": round(float(np.median(host)) * 1e6, 1),
            "back_to_back_us": round(s.elapsed_time(t) * 1e3 / reps, 1),
        }
    return out


class ColdTimer:
    """Per-op GPU time: `warmup` untimed calls, then `reps` calls, each
    between two HIP events on torch's current stream (where libmdgl
    launches) and each after a 512 MB write that evicts the L2 and the
    256 MB MALL; returns the median and the best in ms."""

    def __init__(self, reps, warmup):
        import torch

        self.torch = torch
        self.reps = max(1, int(reps))
        self.warmup = max(0, int(warmup))
        self.flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda")

    def __call__(self, fn, flush=True):
        torch = self.torch
        for _ in range(self.warmup):
            fn()
        s = torch.cuda.Event(enable_timing=True)
        t = torch.cuda.Event(enable_timing=True)
        times = []
        for _ in range(self.reps):
            if flush:
                self.flush.fill_(1)
            s.record()
            fn()
            t.record()
            t.synchronize()
            times.append(s.elapsed_time(t))
        return {"median_ms": round(float(np.median(times)), 4), "best_ms": round(min(times), 4)}


def hbm_entry(times, nbytes, units=None, cache_note=False):
    """One op's line: times, algorithmic bytes, GB/s and fraction of the
    8 TB/s HBM peak at the median (and the edge-feature rate)."""
    med = times["median_ms"]
    out = dict(times)
    out["bytes"] = int(nbytes)
    gbs = nbytes / med / 1e6
    out["GBps"] = round(gbs, 1)
    out["frac"] = round(gbs / HBM_PEAK_GBS, 4)
    if units is not None:
        out["GEdge_feat_s"] = round(units / med / 1e6, 2)
    if cache_note and gbs > HBM_PEAK_GBS:
        out["cache_assisted"] = True
    return out


def mfma_entry(times, flops, nbytes, peak_tflops):
    med = times["median_ms"]
    out = dict(times)
    out["flops"] = int(flops)
    out["bytes"] = int(nbytes)
    tf = flops / med / 1e9
    out["TFLOPs"] = round(tf, 1)
    out["frac"] = round(tf / peak_tflops, 4)
    out["GBps"] = round(nbytes / med / 1e6, 1)
    out["hbm_frac"] = round(nbytes / med / 1e6 / HBM_PEAK_GBS, 4)
    return out


def cpu_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_rate(once, units, seconds, unit, sample, cores, scale=1e9):
    """The oracle's rate on a sample: one warm-up, then repetitions until
    `seconds` have passed (at least 3), best and median (the reference's
    method, bench/profile_deep.py:29-34)."""
    once()
    times = []
    while (sum(times) < seconds or len(times) < 3) and len(times) < 500:
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    best, med = min(times), float(np.median(times))
    return {"value": round(units / best / scale, 4), "median_value": round(units / med / scale, 4),
            "unit": unit, "cores": cores, "kind": "port",
            "sample": "{}; best of {} repetitions ({:.1f} s)".format(sample, len(times),
                                                                    sum(times)),
            "host": {"cpus_available": cpu_cores(), "model": cpu_model()}}


def oracle_setup():
    """The oracle with its static split at min(32, host cores) workers, as the
    reference's 32 workers capped at what this host gives the process."""
    import oracle

    cores = min(32, cpu_cores())
    oracle.set_workers(cores)
    return oracle, oracle.lib(), cores


def _p(a):
    return None if a is None else a.ctypes.data


def csr_sample(g, fraction):
    """The first rows of g's in-CSR holding about `fraction` of the edges:
    (rows, slots, indptr, indices, eid) as host int64 arrays."""
    indptr, indices, eid = g._in_csr()
    target = int(indices.size * fraction)
    S = max(1, int(np.searchsorted(indptr, target)))
    nnz = int(indptr[S])
    return (S, nnz, np.ascontiguousarray(indptr[:S + 1]), np.ascontiguousarray(indices[:nnz]),
            np.ascontiguousarray(eid[:nnz]))


def free_gpu():
    import torch

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- headline
def workload_gat(args):
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops

    N, E, H, D = args.nodes, args.edges, 8, 32
    log("generating power-law graph N={} E={}".format(N, E))
    u, v, gstats = power_law_graph(1, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    log("building GPU CSR")
    g._device_csr("in")
    g._device_coo()
    gen = torch.Generator(device="cuda").manual_seed(1)
    el = torch.randn(N, H, 1, device="cuda", generator=gen)
    er = torch.randn(N, H, 1, device="cuda", generator=gen)
    h = torch.randn(N, H, D, device="cuda", generator=gen)
    torch.cuda.synchronize()

    def step(t):
        run = t if t is not None else (lambda name, fn: fn())
        e = run("gsddmm_u_add_v", lambda: ops.u_add_v(g, el, er))
        run("leaky_relu", lambda: torch.nn.functional.leaky_relu(e, 0.2, inplace=True))
        a = run("edge_softmax", lambda: ops.edge_softmax(g, e))
        return run("gspmm_u_mul_e_sum", lambda: ops.u_mul_e_sum(g, h, a))

    log("timing the step")
    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    units = E * H + E * H + E * H * D
    spmm_bytes = 4 * (N + 1) + 8 * E + 4 * E * H * D + 4 * E * H + 4 * N * H * D
    sddmm_bytes = 8 * E + 4 * E * H * 2 + 4 * E * H
    soft_bytes = 4 * (N + 1) + 4 * E + 4 * E * H * 2
    spmm_ms = timer.avg_ms("gspmm_u_mul_e_sum")
    achieved = spmm_bytes / (spmm_ms * 1e-3) / 1e9
    breakdown = {k: round(timer.avg_ms(k), 4) for k in timer.totals}
    kernels = {
        "gspmm_u_mul_e_sum": {"ms": round(spmm_ms, 4), "bytes": spmm_bytes,
                              "GBps": round(achieved, 1)},
        "gsddmm_u_add_v": {"ms": round(timer.avg_ms("gsddmm_u_add_v"), 4), "bytes": sddmm_bytes,
                           "GBps": round(sddmm_bytes / timer.avg_ms("gsddmm_u_add_v") / 1e6, 1)},
        "edge_softmax": {"ms": round(timer.avg_ms("edge_softmax"), 4), "bytes": soft_bytes,
                         "GBps": round(soft_bytes / timer.avg_ms("edge_softmax") / 1e6, 1)},
    }
    result = {
        "metric": "gSpMM/gSDDMM GEdge·feat/s + achieved HBM GB/s (% of peak), fp32, 1 GPU",
        "value": round(units / (ms * 1e-3) / 1e9, 2),
        "unit": "GEdge·feat/s",
        "ms_per_step": round(ms, 4),
        "dtype": "f32",
        "config": {"workload": "GAT layer on a power-law graph: gsddmm u_add_v -> leaky_relu -> "
                               "edge_softmax(dst) -> gspmm u_mul_e_sum",
                   "num_nodes": N, "num_edges": E, "heads": H, "head_dim": D,
                   "edge_feat_units_per_step": units, **gstats},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (args.traffic_result or {}).get("bytes"),
                     "traffic_detail": args.traffic_result,
                     "kernel": "gspmm u_mul_e_sum", "algorithmic_bytes": spmm_bytes,
                     "avg_ms": round(spmm_ms, 4)},
        "breakdown_ms": breakdown,
        "kernels": kernels,
    }
    if not args.step_only:
        log("host-side cost per call of the step's ops")
        e0 = ops.u_add_v(g, el, er)
        a0 = ops.edge_softmax(g, e0)
        result["host_accounting"] = host_accounting({
            "gsddmm_u_add_v": lambda: ops.u_add_v(g, el, er),
            "edge_softmax": lambda: ops.edge_softmax(g, e0),
            "gspmm_u_mul_e_sum": lambda: ops.u_mul_e_sum(g, h, a0)}, 5)
        del e0, a0
        log("the step's ops alone with cold caches")
        result["cold_caches"] = time_gat_ops_cold(g, el, er, h, N, E, H, D, args)
        log("outside the step: graph build, edge_softmax over a subset, forward + backward")
        result["graph_build"] = time_graph_build(g, u, v, N, args)
        result["edge_softmax_subset"] = time_subset_softmax(g, el, er, E, args)
        result["forward_backward"] = time_gat_backward(g, el, er, h)
        result["gather_ceilings"] = time_gather_ceilings(g, N, E, H, args)
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle) of the step on a sample")
        result["cpu_baseline"] = cpu_baseline_gat(g, el, er, h, args)
    if not args.headline_only:
        del el, er
        free_gpu()
        result["c2_f64"] = section_c2_f64(g, h, args)
    del g, h
    free_gpu()
    return result


def time_gat_ops_cold(g, el, er, h, N, E, H, D, args):
    """The step's three libmdgl ops one at a time, each after a 512 MB write
    that evicts the L2 and the MALL (median and best of --reps, HIP events),
    with the same algorithmic bytes as the step's figures; and copy_u_sum
    over the same graph and node table, outside the step."""
    import torch

    import mojodgl.ops as ops

    cold = ColdTimer(args.reps, 1)
    e = torch.nn.functional.leaky_relu(ops.u_add_v(g, el, er), 0.2)
    a = ops.edge_softmax(g, e)
    ops_ = (
        ("gsddmm_u_add_v", lambda: ops.u_add_v(g, el, er), 8 * E + 4 * E * H * 2 + 4 * E * H,
         E * H),
        ("edge_softmax", lambda: ops.edge_softmax(g, e), 4 * (N + 1) + 4 * E + 4 * E * H * 2,
         E * H),
        ("gspmm_u_mul_e_sum", lambda: ops.u_mul_e_sum(g, h, a),
         4 * (N + 1) + 8 * E + 4 * E * H * D + 4 * E * H + 4 * N * H * D, E * H * D),
    )
    out = {name: hbm_entry(cold(fn), nbytes, units) for name, fn, nbytes, units in ops_}
    # not in the step: the same gspmm without the edge operand (the source
    # rows, their ids and the output only), beside the read_rows ceilings
    out["gspmm_copy_u_sum_not_in_step"] = hbm_entry(
        cold(lambda: ops.copy_u_sum(g, h)), 4 * (N + 1) + 4 * E + 4 * E * H * D + 4 * N * H * D,
        E * H * D)
    del e, a
    return out


def time_gather_ceilings(g, N, E, H, args):
    """The access patterns of gsddmm u_add_v and of edge_softmax's two passes
    alone, through mdgl_gather_rows (rows of a table gathered by an index,
    written in index order; no arithmetic), cold caches, median of reps:
      * rows_32B_by_edge_id: 32-byte rows (H float32) of an (E, H) table by
        a random permutation of the edges (the row pass reading the logits
        of a row's edges);
      * rows_32B_by_node: 32-byte rows of an (N, H) table by each edge's
        destination, twice the bytes of one gsddmm operand;
      * rows_64B_by_node: 64-byte rows of an (N, 2H) table by each edge's
        destination (the write pass reading a row's (max, sum));
      * rows_1KB_by_source: 1 KB rows (the H x D floats of a node) of an
        (N, H * D) table by N random edge sources (gspmm's source-row reads);
      * rows_1KB_in_order: the same table by 0 .. N - 1, a streaming copy;
      * rows_1KB_streamed: the same table read once in order and hardly
        written (segment_reduce sum over runs of 64 rows): a streaming read;
      * stream_read_1.28GB / _2.56GB: a bare one-pass read (mdgl_read_stream,
        a persistent grid of 16-byte nontemporal loads), the read ceiling of
        this GPU;
      * read_rows_1KB_by_csr_source: the 1 KB rows of an (N, H * D) table
        read by the in-CSR's sources in slot order and not written
        (mdgl_read_rows): gspmm's source-row reads with nothing else;
      * read_rows_1KB_by_csr_source_out_written: the same reads beside a
        write of N 1 KB rows (gspmm's output volume).
    Each figure is GB/s of bytes moved per launch (4 index + gathered + written
    per row; read + written for the streaming reads)."""
    import torch

    from mojodgl import _lib

    L = _lib.lib()
    cold = ColdTimer(max(3, args.reps // 2), 1)
    gen = torch.Generator(device="cuda").manual_seed(9)
    perm = torch.randperm(E, device="cuda", generator=gen).to(torch.int32)
    ud, vd = g._device_coo()
    in_order = torch.arange(N, dtype=torch.int32, device="cuda")
    out = {}
    for name, rows, width, idx in (("rows_32B_by_edge_id", E, H, perm),
                                   ("rows_32B_by_node", N, H, vd),
                                   ("rows_64B_by_node", N, 2 * H, vd),
                                   ("rows_1KB_by_source", N, 256, ud[:N]),
                                   ("rows_1KB_in_order", N, 256, in_order)):
        table = torch.randn(rows, width, device="cuda", generator=gen)
        n_idx = idx.numel()
        dst = torch.empty(n_idx, width, device="cuda")

        def run():
            _lib.check(L.mdgl_gather_rows(table.data_ptr(), idx.data_ptr(), dst.data_ptr(), n_idx,
                                          width, _lib.FLOAT32, _lib.stream()), "gather_rows")

        t = cold(run)
        nbytes = n_idx * (4 + 8 * width)
        out[name] = dict(t, bytes=nbytes, GBps=round(nbytes / t["median_ms"] / 1e6, 1),
                         table_MB=round(rows * width * 4 / 1e6, 1))
        del table, dst
    del perm, in_order
    import mojodgl.ops as ops

    table = torch.randn(N, 256, device="cuda", generator=gen)
    runs = torch.full((N // 64,), 64, dtype=torch.int64, device="cuda")
    rows = int(runs.numel()) * 64
    view = table[:rows]

    def stream():
        ops.segment_reduce(runs, view, "sum")

    t = cold(stream)
    nbytes = rows * 1024 + runs.numel() * 1024
    out["rows_1KB_streamed"] = dict(t, bytes=nbytes, GBps=round(nbytes / t["median_ms"] / 1e6, 1),
                                    table_MB=round(rows * 1024 / 1e6, 1))
    del table, runs, view
    # gspmm's source-row reads alone, then beside its output's write volume
    indices = g._device_csr("in").indices
    assert indices.numel() == E
    table = torch.randn(N, 256, device="cuda", generator=gen)
    dst = torch.empty(N, 256, device="cuda")
    sink = torch.empty(int(L.mdgl_read_rows_sink_bytes(E)) // 4, device="cuda")
    for name, dst_rows in (("read_rows_1KB_by_csr_source", 0),
                           ("read_rows_1KB_by_csr_source_out_written", N)):
        def read_rows():
            _lib.check(L.mdgl_read_rows(table.data_ptr(), N, 1024, indices.data_ptr(), E,
                                        dst.data_ptr(), dst_rows, sink.data_ptr(),
                                        _lib.stream()), "read_rows")

        t = cold(read_rows)
        nbytes = E * (4 + 1024) + dst_rows * 1024
        out[name] = dict(t, bytes=nbytes, GBps=round(nbytes / t["median_ms"] / 1e6, 1),
                         table_MB=round(N * 1024 / 1e6, 1))
    del table, dst, sink
    # the one-pass streaming read the bandwidth figures are judged against
    # (mdgl_read_stream: 2,048 workgroups striding with 16-byte nontemporal
    # loads, 32 KB per workgroup and round, next to nothing written), at the
    # size of C4's values and of the GAT node table
    for name, nbytes in (("stream_read_1.28GB", 1_280_000_000),
                         ("stream_read_2.56GB", 2_560_000_000)):
        buf = torch.ones(nbytes // 4, device="cuda")
        sink_bytes = int(L.mdgl_read_stream_sink_bytes(nbytes))
        sink = torch.empty(sink_bytes // 4, device="cuda")

        def read():
            _lib.check(L.mdgl_read_stream(buf.data_ptr(), nbytes, sink.data_ptr(),
                                          _lib.stream()), "read_stream")

        t = cold(read)
        moved = nbytes + sink_bytes
        out[name] = dict(t, bytes=moved, GBps=round(moved / t["median_ms"] / 1e6, 1))
        del buf, sink
    free_gpu()
    return out


def time_gat_backward(g, el, er, h):
    """The same layer with autograd (el, er, h requiring grad): forward plus
    backward, not part of a step (HIP events, average of 3). The backward
    reductions run on the forward kernels over the in- and out-CSR."""
    import torch

    import mojodgl.ops as ops

    el_, er_, h_ = (t.clone().requires_grad_(True) for t in (el, er, h))
    gen = torch.Generator(device="cuda").manual_seed(5)
    grad = torch.randn(h.shape, device="cuda", generator=gen)

    def fb():
        for t in (el_, er_, h_):
            t.grad = None  # as an optimizer's zero_grad(set_to_none=True)
        e = torch.nn.functional.leaky_relu(ops.u_add_v(g, el_, er_), 0.2)
        out = ops.u_mul_e_sum(g, h_, ops.edge_softmax(g, e))
        out.backward(grad)

    fb()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(3):
        fb()
    t.record()
    torch.cuda.synchronize()
    return {"ms": round(s.elapsed_time(t) / 3, 3)}


def time_grouped_backward(fn, a, b, grad, steps):
    """Average ms of the backward of fn(a, b) (both gradients, no
    accumulation into .grad), HIP events over `steps` calls."""
    import torch

    a_, b_ = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    out = fn(a_, b_)
    torch.autograd.grad(out, [a_, b_], grad, retain_graph=True)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        torch.autograd.grad(out, [a_, b_], grad, retain_graph=True)
    t.record()
    torch.cuda.synchronize()
    return s.elapsed_time(t) / steps


def time_subset_softmax(g, el, er, E, args):
    """edge_softmax over a subset of edge ids (every other edge, a GPU
    tensor), not part of a step: the positional grouping by endpoint and its
    plan are built on the GPU for each call (HIP events, average of 3)."""
    import torch

    import mojodgl.ops as ops

    eids = torch.arange(0, E, 2, device="cuda")
    logits = ops.u_add_v(g, el, er)[: eids.numel()].contiguous()
    ops.edge_softmax(g, logits, eids=eids)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(3):
        ops.edge_softmax(g, logits, eids=eids)
    t.record()
    torch.cuda.synchronize()
    return {"ms": round(s.elapsed_time(t) / 3, 3), "selected_edges": int(eids.numel())}


def time_graph_build(g, u, v, N, args):
    """The in-CSR build (not part of a step): on the GPU from the resident
    int32 endpoints (mdgl_build_csr, HIP events, average of 3), and the
    reference's host method (numpy bincount / cumsum / stable argsort, once)."""
    import torch

    from mojodgl.heterograph import build_device_csr

    ud, vd = g._device_coo()
    build_device_csr(vd, ud, N)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(3):
        build_device_csr(vd, ud, N)
    t.record()
    torch.cuda.synchronize()
    out = {"gpu_ms": round(s.elapsed_time(t) / 3, 3)}
    if not args.no_cpu_baseline:
        import oracle

        t0 = time.perf_counter()
        oracle.csr(u, v, N, "dst")
        out["host_numpy_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    return out


def cpu_baseline_gat(g, el, er, h, args):
    """The oracle (C++ restatement of the reference's kernels, float32, its
    32-way static split capped at this host's cores) on the first rows of the
    destination CSR: their in-edges through gsddmm u_add_v, edge_softmax and
    gspmm u_mul_e_sum, kernel-only (prebuilt CSR, preallocated outputs)."""
    oracle, L, cores = oracle_setup()
    N = g.number_of_nodes()
    S, nnz, ip, src, _ = csr_sample(g, args.cpu_fraction)
    E = g.number_of_edges()
    H, D = 8, 32
    elh = el.reshape(N, H).cpu().numpy()
    erh = er.reshape(N, H).cpu().numpy()
    hh = h.reshape(N, H * D).cpu().numpy()
    dst = np.repeat(np.arange(S, dtype=np.int64), np.diff(ip))
    local = np.arange(nnz, dtype=np.int64)
    logits = np.empty((nnz, H), dtype=np.float32)
    soft = np.empty((nnz, H), dtype=np.float32)
    out = np.empty((S, H * D), dtype=np.float32)
    _, loff, roff, _ = oracle.bcast((N, H, D), (nnz, H, 1))
    deg = np.diff(ip)
    mask = np.ones(1, dtype=np.int8)

    def once():
        L.oracle_gsddmm(_p(src), _p(dst), _p(elh), _p(erh), _p(logits), nnz, 0, 1, 0, H, H, H,
                        None, None, 1, 0)
        np.maximum(logits, 0.2 * logits, out=logits)  # leaky_relu
        L.oracle_edge_softmax(_p(ip), _p(local), _p(mask), _p(logits), _p(soft), S, 1, H, 0)
        L.oracle_gspmm(_p(ip), _p(src), _p(local), _p(hh), _p(soft), _p(out), S, 2, H * D, H,
                       H * D, 0, _p(deg), _p(loff), _p(roff), None, None, 0)

    return cpu_rate(once, nnz * (H + H + H * D), args.cpu_seconds, "GEdge·feat/s",
                    "the in-edges of the first {} destination rows ({} edges, {:.1%} of E) "
                    "through gsddmm u_add_v, leaky_relu, edge_softmax and gspmm u_mul_e_sum in "
                    "float32".format(S, nnz, nnz / E), cores)


# ---------------------------------------------------------------- configs
def section_c1(args):
    """update_all u_mul_e with sum / mean / max / min on the uniform graph
    (N = 10,000, E = 100,000, 64 features): warm back-to-back calls (the
    step), each call alone with cold caches, the step replayed from a HIP
    graph, and pull / numpy-input variants outside the step."""
    import torch

    import mojodgl as dgl
    import mojodgl.function as fn

    N, E, D = 10_000, 100_000, 64
    u, v = uniform_graph(0, N, E)
    rng = np.random.default_rng(0)
    hx = rng.standard_normal((N, D), dtype=np.float32)
    ex = rng.random((E, D), dtype=np.float32)
    g = dgl.graph((u, v), num_nodes=N)
    g.ndata["h"] = torch.from_numpy(hx).cuda()
    g.edata["e"] = torch.from_numpy(ex).cuda()
    reds = ("sum", "mean", "max", "min")

    def c1_bytes(red, es):
        # indptr, (src, eid) per edge, the source and edge rows, the output
        # rows, and the two int32 arg rows of max / min
        return (4 * (N + 1) + 8 * E + es * E * D + es * E * D + es * N * D
                + (8 * N * D if red in ("max", "min") else 0))

    def call(red):
        g.update_all(fn.u_mul_e("h", "e", "m"), getattr(fn, red)("m", "z"))

    def step(t):
        run = t if t is not None else (lambda name, fn_: fn_())
        for red in reds:
            run("update_all_" + red, lambda: call(red))

    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    units = E * D
    cold = ColdTimer(args.reps, 3)
    ops_out = {}
    for red in reds:
        ent = hbm_entry(cold(lambda: call(red)), c1_bytes(red, 4), units)
        ent["warm_ms"] = round(timer.avg_ms("update_all_" + red), 4)
        ops_out["update_all_u_mul_e_" + red] = ent
    # the four calls captured once in a HIP graph and replayed: the launches
    # without the Python dispatch (update_all makes no host syncs)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(None)
    graph.replay()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        graph.replay()
    t.record()
    torch.cuda.synchronize()
    gms = s.elapsed_time(t) / args.steps
    pull_nodes = np.arange(0, N, 2)
    g2 = dgl.graph((u, v), num_nodes=N)
    g2.ndata["h"] = hx
    g2.edata["e"] = ex
    extra = {}
    for name, f in (("pull_u_mul_e_sum", lambda: g.pull(pull_nodes, fn.u_mul_e("h", "e", "m"),
                                                         fn.sum("m", "z"))),
                    ("update_all_sum_numpy_inputs",
                     lambda: g2.update_all(fn.u_mul_e("h", "e", "m"), fn.sum("m", "z")))):
        f()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            f()
        torch.cuda.synchronize()
        extra[name] = round((time.perf_counter() - t0) * 1e3 / args.steps, 4)
    acct = {"update_all_u_mul_e_" + red: (lambda r=red: call(r)) for red in reds}
    acct["pull_u_mul_e_sum"] = lambda: g.pull(pull_nodes, fn.u_mul_e("h", "e", "m"),
                                              fn.sum("m", "z"))
    acct["update_all_sum_numpy_inputs"] = lambda: g2.update_all(fn.u_mul_e("h", "e", "m"),
                                                                fn.sum("m", "z"))
    accounting = host_accounting(acct, 200)
    out = {"workload": "update_all u_mul_e + sum/mean/max/min, uniform graph, float32",
           "num_nodes": N, "num_edges": E, "feat": D,
           "note": "cache-resident and launch-bound: 55-60 MB of algorithmic bytes per call",
           "step_ms": round(ms, 4), "value": round(4 * units / ms / 1e6, 2),
           "unit": "GEdge·feat/s", "ops": ops_out,
           "graph_replay": {"ms_per_step": round(gms, 4),
                            "value": round(4 * units / gms / 1e6, 2)},
           "outside_step_ms": extra, "host_accounting": accounting}
    if not args.no_cpu_baseline:
        oracle, L, cores = oracle_setup()
        indptr, indices, eid = oracle.csr(u, v, N, "dst")
        deg = np.diff(indptr)
        z = np.empty((N, D), dtype=np.float32)
        zr = np.empty_like(z)

        def once():
            for red in range(4):
                L.oracle_gspmm(_p(indptr), _p(indices), _p(eid), _p(hx), _p(ex), _p(z), N, 2, D,
                               D, D, red, _p(deg), None, None, None, None, 0)
                if red in (1, 2):  # update_all's +-inf -> 0, a separate pass there
                    L.oracle_replace_inf_with_zero(_p(z), _p(zr), z.size, 0)

        out["cpu_baseline"] = cpu_rate(once, 4 * units, args.cpu_seconds_extra, "GEdge·feat/s",
                                       "the whole graph, the four update_all reductions "
                                       "kernel-only (gspmm, then +-inf -> 0 for max / min)",
                                       cores)
    # float64, the reference's precision, on the same graph and values
    h64, e64 = hx.astype(np.float64), ex.astype(np.float64)
    g.ndata["h"] = torch.from_numpy(h64).cuda()
    g.edata["e"] = torch.from_numpy(e64).cuda()
    ops64 = {"update_all_u_mul_e_" + red: hbm_entry(cold(lambda: call(red)), c1_bytes(red, 8),
                                                    units) for red in reds}
    f64 = {"workload": "update_all u_mul_e + sum/mean/max/min, uniform graph, float64 (the "
                       "reference's precision)",
           "num_nodes": N, "num_edges": E, "feat": D, "ops": ops64}
    if not args.no_cpu_baseline:
        z64 = np.empty((N, D), dtype=np.float64)
        zr64 = np.empty_like(z64)

        def once64():
            for red in range(4):
                L.oracle_gspmm(_p(indptr), _p(indices), _p(eid), _p(h64), _p(e64), _p(z64), N,
                               2, D, D, D, red, _p(deg), None, None, None, None, 1)
                if red in (1, 2):
                    L.oracle_replace_inf_with_zero(_p(z64), _p(zr64), z64.size, 1)

        f64["cpu_baseline"] = cpu_rate(once64, 4 * units, args.cpu_seconds_extra,
                                       "GEdge·feat/s", "the whole graph, the four update_all "
                                       "reductions kernel-only, float64", cores)
    out["f64"] = f64
    return out


def section_c2_f64(g, h32, args):
    """The headline graph's ops in float64, the reference's precision:
    gspmm u_mul_e_sum h (N, 8, 32) x a (E, 8, 1), gsddmm u_add_v and
    edge_softmax alone (cold caches), and the whole GAT step."""
    import torch

    import mojodgl.ops as ops

    N, E, H, D = g.number_of_nodes(), g.number_of_edges(), 8, 32
    log("float64 gspmm on the power-law graph")
    h = h32.to(torch.float64)
    gen = torch.Generator(device="cuda").manual_seed(6)
    a = torch.rand(E, H, 1, device="cuda", dtype=torch.float64, generator=gen)
    cold = ColdTimer(args.reps, 2)
    nbytes = 4 * (N + 1) + 8 * E + 8 * E * H * D + 8 * E * H + 8 * N * H * D
    el = torch.randn(N, H, 1, device="cuda", dtype=torch.float64, generator=gen)
    er = torch.randn(N, H, 1, device="cuda", dtype=torch.float64, generator=gen)
    logits = ops.u_add_v(g, el, er)
    sddmm_bytes = 8 * E + 8 * E * H * 2 + 8 * E * H
    soft_bytes = 4 * (N + 1) + 4 * E + 8 * E * H * 2
    out = {"workload": "the GAT layer's ops in float64 (the reference's precision) on the "
                       "power-law graph: gsddmm u_add_v, edge_softmax (E, 8, 1), gspmm "
                       "u_mul_e_sum h (N, 8, 32) x a (E, 8, 1)",
           "num_nodes": N, "num_edges": E,
           "ops": {"gspmm_u_mul_e_sum": hbm_entry(cold(lambda: ops.u_mul_e_sum(g, h, a)), nbytes,
                                                  E * H * D),
                   "gsddmm_u_add_v": hbm_entry(cold(lambda: ops.u_add_v(g, el, er)), sddmm_bytes,
                                               E * H),
                   "edge_softmax": hbm_entry(cold(lambda: ops.edge_softmax(g, logits)),
                                             soft_bytes, E * H)}}
    del logits

    def step(t):
        e = ops.u_add_v(g, el, er)
        torch.nn.functional.leaky_relu(e, 0.2, inplace=True)
        return ops.u_mul_e_sum(g, h, ops.edge_softmax(g, e))

    ms = run_steps(step, max(3, args.steps // 2), args.warmup, OpTimer())
    units = E * H + E * H + E * H * D
    out["step"] = {"ms": round(ms, 4), "GEdge_feat_s": round(units / (ms * 1e-3) / 1e9, 2),
                   "note": "the headline step (gsddmm u_add_v, leaky_relu, edge_softmax, gspmm "
                           "u_mul_e_sum) with float64 features, warm, as the headline"}
    del el, er
    if not args.no_cpu_baseline:
        oracle, L, cores = oracle_setup()
        S, nnz, ip, src, eid = csr_sample(g, args.cpu_fraction)
        hh = h.reshape(N, H * D).cpu().numpy()
        ah = a.reshape(E, H).cpu().numpy()
        z = np.empty((S, H * D), dtype=np.float64)
        _, loff, roff, _ = oracle.bcast((N, H, D), (E, H, 1))
        deg = np.diff(ip)

        def once():
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh), _p(ah), _p(z), S, 2, H * D, H,
                           H * D, 0, _p(deg), _p(loff), _p(roff), None, None, 1)

        out["cpu_baseline"] = cpu_rate(
            once, nnz * H * D, args.cpu_seconds_extra, "GEdge·feat/s",
            "the in-edges of the first {} destination rows ({} edges, {:.1%} of E) through gspmm "
            "u_mul_e_sum in float64 (restated kernel + broadcast extension)".format(S, nnz,
                                                                                 nnz / E), cores)
    del h, a
    free_gpu()
    return out


def section_c3(args):
    """GCN aggregation on the community graph: u_mul_e_sum with
    w = 1/sqrt(outdeg(u) indeg(v)) (E, 1), copy_u_mean, copy_u_max with
    arg_u / arg_e."""
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops
    from mojodgl.ops import spmm

    log("generating community graph")
    u, v, N = community_graph()
    E = u.size
    F = args.c3_feat
    g = dgl.graph((u, v), num_nodes=N)
    g._device_csr("in")
    indeg = np.maximum(np.bincount(v, minlength=N), 1).astype(np.float64)
    outdeg = np.maximum(np.bincount(u, minlength=N), 1).astype(np.float64)
    wh = (1.0 / np.sqrt(outdeg[u] * indeg[v])).astype(np.float32).reshape(E, 1)
    w = torch.from_numpy(wh).cuda()
    gen = torch.Generator(device="cuda").manual_seed(2)
    h = torch.randn(N, F, device="cuda", generator=gen)
    calls = {
        "u_mul_e_sum": lambda: ops.u_mul_e_sum(g, h, w),
        "copy_u_mean": lambda: ops.copy_u_mean(g, h),
        "copy_u_max_arg": lambda: spmm._run(g, "copy_lhs", "max", h, None, want_arg=True,
                                            arg_dtype=torch.int32),
    }
    def c3_bytes(es):
        # u_mul_e_sum, copy_u_mean, copy_u_max (+ int32 arg_u)
        mean = 4 * (N + 1) + 4 * E + es * E * F + es * N * F
        return (4 * (N + 1) + 8 * E + es * E * F + es * E + es * N * F, mean, mean + 4 * N * F)

    cold = ColdTimer(args.reps, 2)
    log("timing c3")
    ops_out = {name: hbm_entry(cold(fn_), b, E * F, cache_note=True)
               for (name, fn_), b in zip(calls.items(), c3_bytes(4))}
    # the cache-level ceiling of this access pattern: the same kernels over
    # the same CSR (destination rows, degrees, slot order, edge weights) with
    # every source folded into the first 1,024 nodes (a 2.4 MB table, which
    # each XCD's 4 MB L2 holds) or into the first block's 4,600 nodes (11 MB,
    # which the 256 MB MALL holds): the rate of the gathers when they hit.
    # The folded graph keeps the original's lane layout (its locality, which
    # picks the column slab width), so only where the sources sit changes.
    log("c3 cache-resident ceilings")
    ceilings = {}
    for label, fold in (("l2_resident_1024_rows", 1024), ("mall_resident_4600_rows", 4600)):
        gc = dgl.graph((u % fold, v), num_nodes=N)
        gc._locality = g._source_locality()
        gc._device_csr("in")
        ccalls = {
            "u_mul_e_sum": lambda: ops.u_mul_e_sum(gc, h, w),
            "copy_u_mean": lambda: ops.copy_u_mean(gc, h),
            "copy_u_max_arg": lambda: spmm._run(gc, "copy_lhs", "max", h, None, want_arg=True,
                                                arg_dtype=torch.int32),
        }
        ceilings[label] = {name: cold(fn_) for name, fn_ in ccalls.items()}
        del gc, ccalls
        free_gpu()
    for name, ent in ops_out.items():
        c = ceilings["l2_resident_1024_rows"][name]["median_ms"]
        ent["ceiling_ms"] = c
        ent["ceiling_frac"] = round(c / ent["median_ms"], 4)
    out = {"workload": "GCN aggregation on a 50-block community graph, float32",
           "num_nodes": N, "num_edges": E, "feat": F,
           "note": "95% of the edges stay inside 4,600-node blocks, so the L2 and the MALL serve "
                   "most source rows: rates above the HBM peak are cache-assisted "
                   "(compulsory bytes 2.48 GB); ceiling_frac = the same op over the same CSR "
                   "with its sources folded into an L2-resident table, divided by the op",
           "ops": ops_out, "cache_ceilings": ceilings}
    if not args.no_cpu_baseline:
        oracle, L, cores = oracle_setup()
        S, nnz, ip, src, eid = csr_sample(g, args.cpu_fraction_c3)
        hh = h.cpu().numpy()
        deg = np.diff(ip)
        z = np.empty((S, F), dtype=np.float32)
        zr = np.empty_like(z)
        au = np.empty((S, F), dtype=np.int64)
        ae = np.empty((S, F), dtype=np.int64)
        loff = np.arange(F, dtype=np.int64)
        roff = np.zeros(F, dtype=np.int64)

        def once():
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh), _p(wh), _p(z), S, 2, F, 1, F, 0,
                           _p(deg), _p(loff), _p(roff), None, None, 0)
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh), _p(hh), _p(z), S, 5, F, F, F, 3,
                           _p(deg), None, None, None, None, 0)
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh), _p(hh), _p(z), S, 5, F, F, F, 1,
                           _p(deg), None, None, _p(au), _p(ae), 0)
            L.oracle_replace_inf_with_zero(_p(z), _p(zr), z.size, 0)

        out["cpu_baseline"] = cpu_rate(
            once, 3 * nnz * F, args.cpu_seconds_extra, "GEdge·feat/s",
            "the in-edges of the first {} destination rows ({} edges, {:.1%} of E) through "
            "u_mul_e_sum (restated kernel + broadcast extension: w is (E, 1)), copy_u_mean and "
            "copy_u_max with arg outputs, float32".format(S, nnz, nnz / E), cores)
    # float64, the reference's precision, on the same graph
    h64, w64 = h.double(), w.double()
    calls64 = {
        "u_mul_e_sum": lambda: ops.u_mul_e_sum(g, h64, w64),
        "copy_u_mean": lambda: ops.copy_u_mean(g, h64),
        "copy_u_max_arg": lambda: spmm._run(g, "copy_lhs", "max", h64, None, want_arg=True,
                                            arg_dtype=torch.int32),
    }
    log("timing c3 in float64")
    f64 = {"workload": "GCN aggregation on a 50-block community graph, float64 (the reference's "
                       "precision)",
           "num_nodes": N, "num_edges": E, "feat": F,
           "ops": {name: hbm_entry(cold(fn_), b, E * F, cache_note=True)
                   for (name, fn_), b in zip(calls64.items(), c3_bytes(8))}}
    if not args.no_cpu_baseline:
        hh64 = hh.astype(np.float64)
        wh64 = wh.astype(np.float64)
        z64 = np.empty((S, F), dtype=np.float64)
        zr64 = np.empty_like(z64)

        def once64():
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh64), _p(wh64), _p(z64), S, 2, F, 1, F,
                           0, _p(deg), _p(loff), _p(roff), None, None, 1)
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh64), _p(hh64), _p(z64), S, 5, F, F, F,
                           3, _p(deg), None, None, None, None, 1)
            L.oracle_gspmm(_p(ip), _p(src), _p(eid), _p(hh64), _p(hh64), _p(z64), S, 5, F, F, F,
                           1, _p(deg), None, None, _p(au), _p(ae), 1)
            L.oracle_replace_inf_with_zero(_p(z64), _p(zr64), z64.size, 1)

        f64["cpu_baseline"] = cpu_rate(
            once64, 3 * nnz * F, args.cpu_seconds_extra, "GEdge·feat/s",
            "the in-edges of the first {} destination rows ({} edges, {:.1%} of E) through the "
            "three ops, float64".format(S, nnz, nnz / E), cores)
    out["f64"] = f64
    del g, h, w, h64, w64, calls, calls64
    free_gpu()
    return out


def section_c4(args):
    """gsddmm u_dot_v on a uniform graph (N = 1e6, E = 2e7, 128 features),
    segment_reduce sum / max and segment_softmax over 1e6 Poisson(20)
    segments of 16 columns, and the reference's array helpers at those
    sizes."""
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops
    from mojodgl import _lib

    N, E, F = 1_000_000, 20_000_000, 128
    log("generating uniform graph and segments")
    u, v = uniform_graph(3, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    g._device_coo()
    gen = torch.Generator(device="cuda").manual_seed(3)
    h = torch.randn(N, F, device="cuda", generator=gen) * (1.0 / np.sqrt(F))
    rng = np.random.default_rng(3)
    seglen = rng.poisson(20, 1_000_000)
    S = seglen.size
    R = int(seglen.sum())
    val = torch.randn(R, 16, device="cuda", generator=gen)
    seglen_d = torch.from_numpy(seglen).cuda()  # lengths resident on the GPU like the values
    calls = {
        "u_dot_v": (lambda: ops.u_dot_v(g, h, h), 8 * E + 4 * E * F * 2 + 4 * E, E * F),
        "segment_reduce_sum": (lambda: ops.segment_reduce(seglen_d, val, "sum"),
                               4 * (S + 1) + 4 * R * 16 + 4 * S * 16, R * 16),
        "segment_reduce_max": (lambda: ops.segment_reduce(seglen_d, val, "max"),
                               4 * (S + 1) + 4 * R * 16 + 4 * S * 16, R * 16),
        "segment_softmax": (lambda: ops.segment_softmax(seglen_d, val),
                            4 * (S + 1) + 4 * R * 16 * 2, R * 16),
    }
    cold = ColdTimer(args.reps, 3)
    log("timing c4")
    ops_out = {name: hbm_entry(cold(fn_), b, units) for name, (fn_, b, units) in calls.items()}
    # the reference's array helpers at the same sizes: cumsum and clamp over
    # the 1M int64 lengths, replace_inf over the values
    L = _lib.lib()
    lens = seglen_d.to(torch.int64).contiguous()
    ibuf = torch.empty_like(lens)
    fbuf = torch.empty_like(val)
    helpers = {
        "cumsum": (lambda: L.mdgl_cumsum(lens.data_ptr(), ibuf.data_ptr(), S, _lib.stream()),
                   16 * S),
        "clamp_i64": (lambda: L.mdgl_clamp_i64(lens.data_ptr(), ibuf.data_ptr(), S, 1, R,
                                               _lib.stream()), 16 * S),
        "replace_inf_with_zero": (lambda: L.mdgl_replace_inf_with_zero(
            val.data_ptr(), fbuf.data_ptr(), R * 16, 0, _lib.stream()), 8 * R * 16),
    }
    for name, (fn_, b) in helpers.items():
        assert fn_() == 0
        ops_out[name] = hbm_entry(cold(fn_), b)
    out = {"workload": "u_dot_v link scoring + segment_reduce sum/max + segment_softmax, float32",
           "num_nodes": N, "num_edges": E, "segments": S, "rows": R, "ops": ops_out}
    if not args.no_cpu_baseline:
        oracle, Lo, cores = oracle_setup()
        ne = int(E * args.cpu_fraction_c4)
        hh = h.cpu().numpy()
        us, vs = np.ascontiguousarray(u[:ne]), np.ascontiguousarray(v[:ne])
        score = np.empty((ne, 1), dtype=np.float32)
        ns = int(S * args.cpu_fraction_c4)
        offs = oracle.offsets_of(seglen[:ns])
        nr = int(offs[-1])
        vh = val[:nr].cpu().numpy()
        sred = np.empty((ns, 16), dtype=np.float32)
        sres = np.empty_like(sred)
        ssm = np.zeros((nr, 16), dtype=np.float32)

        def once_dot():
            Lo.oracle_gsddmm(_p(us), _p(vs), _p(hh), _p(hh), _p(score), ne, 0, 1, 4, F, F, 1,
                             None, None, F, 0)

        def once_seg():
            Lo.oracle_segment_reduce(_p(offs), _p(vh), _p(sred), ns, 16, 0, nr, 0)
            Lo.oracle_segment_reduce(_p(offs), _p(vh), _p(sred), ns, 16, 1, nr, 0)
            Lo.oracle_replace_inf_with_zero(_p(sred), _p(sres), sred.size, 0)
            Lo.oracle_segment_softmax(_p(offs), _p(vh), _p(ssm), ns, 16, nr, 0)

        out["cpu_baseline"] = {
            "u_dot_v": cpu_rate(once_dot, ne * F, args.cpu_seconds_extra, "GEdge·feat/s",
                                "the first {} edges ({:.0%} of E), float32".format(
                                    ne, ne / E), cores),
            "segments": cpu_rate(once_seg, 3 * nr * 16, args.cpu_seconds_extra,
                                 "G row·feat/s",
                                 "the first {} segments ({} rows) through segment_reduce sum, "
                                 "max (+ replace_inf) and segment_softmax, float32".format(ns, nr),
                                 cores)}
    del ibuf, fbuf, helpers
    # float64, the reference's precision, on the same graph and segments
    h64, val64 = h.double(), val.double()
    calls64 = {
        "u_dot_v": (lambda: ops.u_dot_v(g, h64, h64), 8 * E + 8 * E * F * 2 + 8 * E, E * F),
        "segment_reduce_sum": (lambda: ops.segment_reduce(seglen_d, val64, "sum"),
                               4 * (S + 1) + 8 * R * 16 + 8 * S * 16, R * 16),
        "segment_reduce_max": (lambda: ops.segment_reduce(seglen_d, val64, "max"),
                               4 * (S + 1) + 8 * R * 16 + 8 * S * 16, R * 16),
        "segment_softmax": (lambda: ops.segment_softmax(seglen_d, val64),
                            4 * (S + 1) + 8 * R * 16 * 2, R * 16),
    }
    log("timing c4 in float64")
    f64 = {"workload": "u_dot_v link scoring + segment_reduce sum/max + segment_softmax, "
                       "float64 (the reference's precision)",
           "num_nodes": N, "num_edges": E, "segments": S, "rows": R,
           "ops": {name: hbm_entry(cold(fn_), b, units)
                   for name, (fn_, b, units) in calls64.items()}}
    if not args.no_cpu_baseline:
        hh64 = hh.astype(np.float64)
        vh64 = vh.astype(np.float64)
        score64 = np.empty((ne, 1), dtype=np.float64)
        sred64 = np.empty((ns, 16), dtype=np.float64)
        sres64 = np.empty_like(sred64)
        ssm64 = np.zeros((nr, 16), dtype=np.float64)

        def once_dot64():
            Lo.oracle_gsddmm(_p(us), _p(vs), _p(hh64), _p(hh64), _p(score64), ne, 0, 1, 4, F, F,
                             1, None, None, F, 1)

        def once_seg64():
            Lo.oracle_segment_reduce(_p(offs), _p(vh64), _p(sred64), ns, 16, 0, nr, 1)
            Lo.oracle_segment_reduce(_p(offs), _p(vh64), _p(sred64), ns, 16, 1, nr, 1)
            Lo.oracle_replace_inf_with_zero(_p(sred64), _p(sres64), sred64.size, 1)
            Lo.oracle_segment_softmax(_p(offs), _p(vh64), _p(ssm64), ns, 16, nr, 1)

        f64["cpu_baseline"] = {
            "u_dot_v": cpu_rate(once_dot64, ne * F, args.cpu_seconds_extra, "GEdge·feat/s",
                                "the first {} edges ({:.0%} of E), float64".format(ne, ne / E),
                                cores),
            "segments": cpu_rate(once_seg64, 3 * nr * 16, args.cpu_seconds_extra,
                                 "G row·feat/s",
                                 "the first {} segments ({} rows) through segment_reduce sum, "
                                 "max (+ replace_inf) and segment_softmax, float64".format(ns, nr),
                                 cores)}
    out["f64"] = f64
    del g, h, val, h64, val64, seglen_d, lens, calls, calls64
    free_gpu()
    return out


def section_c5(args):
    """gather_mm and segment_mm: a (1e7, 128), b (64, 128, 128), idx_b
    uniform, seglen multinomial over Dirichlet(0.5) weights; the vendor BLAS
    on one block of the same shape beside them; both gradients."""
    import torch

    import mojodgl.ops as ops

    n, K, R = 10_000_000, 128, 64
    gen = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randn(n, K, device="cuda", generator=gen)
    b = torch.randn(R, K, K, device="cuda", generator=gen) * (1.0 / np.sqrt(K))
    rng = np.random.default_rng(4)
    idx_h = rng.integers(0, R, n)
    idx = torch.from_numpy(idx_h).cuda()
    seglen = rng.multinomial(n, rng.dirichlet(0.5 * np.ones(R)))
    flops = 2.0 * n * K * K
    cold = ColdTimer(args.reps, 3)
    log("timing c5")
    ops_out = {
        "gather_mm": mfma_entry(cold(lambda: ops.gather_mm(a, b, idx_b=idx)), flops,
                                4 * n * K * 2 + 8 * n + 4 * R * K * K, MFMA_F32_PEAK_TFLOPS),
        "segment_mm": mfma_entry(cold(lambda: ops.segment_mm(a, b, seglen)), flops,
                                 4 * n * K * 2 + 4 * R * K * K + 8 * R, MFMA_F32_PEAK_TFLOPS),
    }
    # the vendor BLAS (torch.mm, full float32) on the same shape with one
    # weight block and no grouping, for comparison
    torch.backends.cuda.matmul.allow_tf32 = False
    w0 = b[0].contiguous()
    dst = torch.empty(n, K, device="cuda")
    blas = mfma_entry(cold(lambda: torch.mm(a, w0, out=dst)), flops, 4 * n * K * 2 + 4 * K * K,
                      MFMA_F32_PEAK_TFLOPS)
    del dst
    gg = torch.randn(n, K, device="cuda", generator=gen)
    for name, fn_ in (("gather_mm", lambda x, y: ops.gather_mm(x, y, idx_b=idx)),
                      ("segment_mm", lambda x, y: ops.segment_mm(x, y, seglen))):
        m = time_grouped_backward(fn_, a, b, gg, args.steps)
        ops_out[name]["backward"] = {"ms": round(m, 3), "TFLOPs": round(2 * flops / m / 1e9, 1)}
    del gg
    out = {"workload": "RGCN relation transform: gather_mm + segment_mm, float32",
           "rows": n, "d1": K, "d2": K, "relations": R, "ops": ops_out,
           "arithmetic": "float32 in and out; each product formed from exact three-way bf16 "
                         "splits of both operands (six part products on "
                         "v_mfma_f32_32x32x16_bf16, float32 accumulation); frac is against "
                         "the 157.3 TFLOP/s float32 MFMA peak, hbm_frac against 8 TB/s",
           "vendor_blas_one_block": blas}
    if not args.no_cpu_baseline:
        oracle, L, cores = oracle_setup()
        ng = args.cpu_rows_c5
        ah = a[:ng].cpu().numpy()
        bh = b.cpu().numpy()
        ih = np.ascontiguousarray(idx_h[:ng])
        og = np.empty((ng, K), dtype=np.float32)
        sl = (seglen * (args.cpu_rows_c5_serial / n)).astype(np.int64)
        ns = int(sl.sum())
        os_ = np.zeros((ns, K), dtype=np.float32)
        ahs = np.ascontiguousarray(ah[:ns]) if ns <= ng else a[:ns].cpu().numpy()

        def once_g():
            L.oracle_gather_mm(_p(ah), _p(bh), _p(ih), _p(og), ng, K, K, 0)

        def once_s():
            L.oracle_segment_mm(_p(ahs), _p(bh), _p(os_), _p(sl), ns, K, R, K, 0)

        out["cpu_baseline"] = {
            "gather_mm": cpu_rate(once_g, 2.0 * ng * K * K, args.cpu_seconds_extra, "GFLOP/s",
                                  "the first {} rows, float32".format(ng), cores),
            "segment_mm": cpu_rate(once_s, 2.0 * ns * K * K, args.cpu_seconds_extra, "GFLOP/s",
                                   "{} rows in 64 segments of the same proportions, float32; "
                                   "serial, as the reference's kernel".format(ns), 1)}
    del w0
    # float64, the reference's precision, on the float64 matrix cores
    # (v_mfma_f64_16x16x4f64), same rows, blocks and groups
    a64, b64 = a.double(), b.double()
    del a, b
    free_gpu()
    log("timing c5 in float64")
    f64 = {"workload": "RGCN relation transform: gather_mm + segment_mm, float64 (the "
                       "reference's precision)",
           "rows": n, "d1": K, "d2": K, "relations": R,
           "ops": {"gather_mm": mfma_entry(cold(lambda: ops.gather_mm(a64, b64, idx_b=idx)),
                                           flops, 8 * n * K * 2 + 8 * n + 8 * R * K * K,
                                           MFMA_F64_PEAK_TFLOPS),
                   "segment_mm": mfma_entry(cold(lambda: ops.segment_mm(a64, b64, seglen)),
                                            flops, 8 * n * K * 2 + 8 * R * K * K + 8 * R,
                                            MFMA_F64_PEAK_TFLOPS)},
           "arithmetic": "float64 in and out on v_mfma_f64_16x16x4f64; frac is against the "
                         "78.6 TFLOP/s float64 MFMA peak"}
    if not args.no_cpu_baseline:
        ah64 = ah.astype(np.float64)
        bh64 = bh.astype(np.float64)
        og64 = np.empty((ng, K), dtype=np.float64)
        ahs64 = ahs.astype(np.float64)
        os64 = np.zeros((ns, K), dtype=np.float64)

        def once_g64():
            L.oracle_gather_mm(_p(ah64), _p(bh64), _p(ih), _p(og64), ng, K, K, 1)

        def once_s64():
            L.oracle_segment_mm(_p(ahs64), _p(bh64), _p(os64), _p(sl), ns, K, R, K, 1)

        f64["cpu_baseline"] = {
            "gather_mm": cpu_rate(once_g64, 2.0 * ng * K * K, args.cpu_seconds_extra, "GFLOP/s",
                                  "the first {} rows, float64".format(ng), cores),
            "segment_mm": cpu_rate(once_s64, 2.0 * ns * K * K, args.cpu_seconds_extra, "GFLOP/s",
                                   "{} rows in 64 segments of the same proportions, float64; "
                                   "serial, as the reference's kernel".format(ns), 1)}
    out["f64"] = f64
    del a64, b64, idx
    free_gpu()
    return out


def workload_gat_train(args):
    """The GAT layer with autograd on el, er and h: one step is the forward
    and the backward (gradients set to None before each, as an optimizer's
    zero_grad). Per-op times: the forward ops, then `backward` for the whole
    backward pass."""
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops

    N, E, H, D = args.nodes, args.edges, 8, 32
    log("generating power-law graph N={} E={}".format(N, E))
    u, v, gstats = power_law_graph(1, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    g._device_csr("in")
    g._device_csr("out")
    g._device_coo()
    gen = torch.Generator(device="cuda").manual_seed(1)
    el = torch.randn(N, H, 1, device="cuda", generator=gen).requires_grad_(True)
    er = torch.randn(N, H, 1, device="cuda", generator=gen).requires_grad_(True)
    h = torch.randn(N, H, D, device="cuda", generator=gen).requires_grad_(True)
    grad = torch.randn(N, H, D, device="cuda", generator=gen)
    torch.cuda.synchronize()

    def step(t):
        run = t if t is not None else (lambda name, fn: fn())
        for x in (el, er, h):
            x.grad = None
        e = run("gsddmm_u_add_v", lambda: ops.u_add_v(g, el, er))
        e = run("leaky_relu", lambda: torch.nn.functional.leaky_relu(e, 0.2))
        a = run("edge_softmax", lambda: ops.edge_softmax(g, e))
        out = run("gspmm_u_mul_e_sum", lambda: ops.u_mul_e_sum(g, h, a))
        run("backward", lambda: out.backward(grad))

    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    units = E * H + E * H + E * H * D
    return {"metric": "GAT layer forward + backward, fp32, 1 GPU",
            "value": round(units / (ms * 1e-3) / 1e9, 2), "unit": "GEdge·feat/s (forward units)",
            "ms_per_step": round(ms, 4), "dtype": "f32",
            "config": {"workload": "GAT layer forward + backward on a power-law graph",
                       "num_nodes": N, "num_edges": E, "heads": H, "head_dim": D, **gstats},
            "breakdown_ms": {k: round(timer.avg_ms(k), 4) for k in timer.totals}}


SECTIONS = {"c1": section_c1, "c3": section_c3, "c4": section_c4, "c5": section_c5}


def workload_c5_phases(args):
    """segment_mm of the RGCN configuration in a loop, phase by phase, for a
    power and clock sampler running beside it (amd-smi in another process):
    the bf16-split kernel, the same call with every group forced onto the
    float32 MFMA path (one b value out of the split's range), the vendor BLAS
    on one block, and segment_mm in float64. Each phase prints its wall-clock
    bounds."""
    import torch

    import mojodgl.ops as ops

    n, K, R = 10_000_000, 128, 64
    gen = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randn(n, K, device="cuda", generator=gen)
    b = torch.randn(R, K, K, device="cuda", generator=gen) * (1.0 / np.sqrt(K))
    rng = np.random.default_rng(4)
    seglen = rng.multinomial(n, rng.dirichlet(0.5 * np.ones(R)))
    forced = b.clone()
    forced[:, 0, 0] = 1e30
    w0 = b[0].contiguous()
    dst = torch.empty(n, K, device="cuda")
    torch.backends.cuda.matmul.allow_tf32 = False
    phases = []
    a64, b64 = a.double(), b.double()
    for name, fn_ in (("segment_mm_bf16_split", lambda: ops.segment_mm(a, b, seglen)),
                      ("segment_mm_float32_mfma", lambda: ops.segment_mm(a, forced, seglen)),
                      ("torch_mm_one_block", lambda: torch.mm(a, w0, out=dst)),
                      ("segment_mm_float64", lambda: ops.segment_mm(a64, b64, seglen))):
        fn_()
        torch.cuda.synchronize()
        t0 = time.time()
        calls = 0
        while time.time() - t0 < args.phase_seconds:
            for _ in range(10):
                fn_()
            torch.cuda.synchronize()
            calls += 10
        t1 = time.time()
        phases.append({"phase": name, "start": round(t0, 3), "end": round(t1, 3), "calls": calls,
                       "ms_per_call": round((t1 - t0) * 1e3 / calls, 4)})
        log("phase", name, round(t0, 3), round(t1, 3))
        time.sleep(0.5)
    return {"metric": "ms per call by phase", "value": phases[0]["ms_per_call"],
            "unit": "ms", "ms_per_step": phases[0]["ms_per_call"], "dtype": "f32",
            "config": {"workload": "RGCN segment_mm phases for a power sampler"},
            "phases": phases}


def workload_section(name):
    """One configuration alone, printed as its own line."""

    def run(args):
        sec = SECTIONS[name](args)
        ops_out = sec["ops"]
        first = next(iter(ops_out.values()))
        rate = ("TFLOPs", "TFLOP/s") if "TFLOPs" in first else ("GBps", "GB/s")
        return {"metric": "{} per op, 1 GPU".format(rate[1]), "value": first[rate[0]],
                "unit": rate[1], "ms_per_step": first["median_ms"], "dtype": "f32",
                "config": {"workload": sec.pop("workload")}, **sec}

    return run


WORKLOADS = {"gat": workload_gat, "gat_train": workload_gat_train,
             "gspmm_traffic": workload_gspmm_traffic, "c5_phases": workload_c5_phases,
             **{k: workload_section(k) for k in SECTIONS}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="gat", choices=sorted(WORKLOADS))
    ap.add_argument("--nodes", type=int, default=2_500_000)
    ap.add_argument("--edges", type=int, default=60_000_000)
    ap.add_argument("--reps", type=int, default=20,
                    help="cold-cache repetitions per op in the configuration sections")
    ap.add_argument("--headline-only", action="store_true",
                    help="measure the GAT step only (no configuration sections)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--step-only", action="store_true",
                    help="skip the measurements outside the step (graph build, edge_softmax "
                         "over a subset, forward + backward), so a profile holds the step's "
                         "kernels only")
    ap.add_argument("--cpu-fraction", type=float, default=0.1)
    ap.add_argument("--cpu-fraction-c3", type=float, default=0.01)
    ap.add_argument("--c3-feat", type=int, default=602,
                    help="node feature width of the community-graph section (the config: 602)")
    ap.add_argument("--chunk-len", type=int, default=None,
                    help="gspmm heavy-row chunk length (mojodgl.heterograph.CHUNK_LEN; "
                         "default 512)")
    ap.add_argument("--cpu-fraction-c4", type=float, default=0.05)
    ap.add_argument("--cpu-rows-c5", type=int, default=100_000)
    ap.add_argument("--cpu-rows-c5-serial", type=int, default=20_000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-seconds-extra", type=float, default=3.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="finish with a 1 GiB device-to-device copy (counter calibration)")
    ap.add_argument("--phase-seconds", type=float, default=4.0,
                    help="length of each phase of --workload c5_phases")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the live rocprofv3 measurement of the headline gspmm's bytes")
    ap.add_argument("--traffic-timeout", type=float, default=150.0,
                    help="time limit of each rocprofv3 counter pass (seconds)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: mojodgl runs on a single MI355X and has no "
              "multi-GPU path (--gpus {} requested)".format(args.gpus), file=sys.stderr)
        sys.exit(2)
    t_start = time.perf_counter()
    args.traffic_result = None
    if args.workload == "gat" and not args.no_traffic:
        # child processes, before this one touches the GPU
        args.traffic_result = measure_traffic(args)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs the GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.chunk_len is not None:
        import mojodgl.heterograph as hg

        hg.CHUNK_LEN = args.chunk_len
    res = WORKLOADS[args.workload](args)
    if args.workload == "gspmm_traffic":
        print(json.dumps(res), flush=True)
        return
    if args.workload == "gat" and not args.headline_only:
        configs = {"c2_f64": res.pop("c2_f64")}
        for name, fn_ in SECTIONS.items():
            log("section", name)
            configs[name] = fn_(args)
        res["configs"] = {"c1": configs["c1"], "c2_f64": configs["c2_f64"],
                          "c3": configs["c3"], "c4": configs["c4"], "c5": configs["c5"]}
        for name in ("c1", "c3", "c4", "c5"):
            res["configs"][name + "_f64"] = configs[name].pop("f64")
    res["bench_wall_s"] = round(time.perf_counter() - t_start, 1)
    if args.calibrate_copy:
        # a plain device copy of 1 GiB, for scaling rocprofv3 byte counters
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    line = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"),
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": res.pop("ms_per_step"), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": res.pop("dtype"),
            "data": "synthetic (seeded numpy graphs, torch.randn features on the GPU)",
            "config": res.pop("config")}
    line.update(res)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
