#!/usr/bin/env python3
"""Benchmark of the message-passing kernel layer on one MI355X.

Default workload (one "step"): the GAT attention layer on the power-law
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

Other workloads (--workload c1|c3|c4|c5) print their own line; they are
measurement runs for the other configurations, not the headline, and so is
--workload gat_train (the same layer with autograd: forward + backward).
"""

from __future__ import annotations

import argparse
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
# HBM bytes per launch of the gspmm kernel on the default workload, from
# rocprofv3 FETCH_SIZE / WRITE_SIZE scaled by a 1 GiB copy (profiles/gat_power_law_kernels.md)
GSPMM_TRAFFIC_BYTES = 72.35e9
MFMA_F32_PEAK_TFLOPS = 157.3


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
    import torch

    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(timer)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    timer.collect()
    return (t1 - t0) * 1e3 / steps


def cpu_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# ---------------------------------------------------------------- workloads
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
                     "traffic": args.traffic, "kernel": "gspmm u_mul_e_sum",
                     "algorithmic_bytes": spmm_bytes, "avg_ms": round(spmm_ms, 4)},
        "breakdown_ms": breakdown,
        "kernels": kernels,
    }
    if not args.step_only:
        result["graph_build"] = time_graph_build(g, u, v, N, args)
        result["edge_softmax_subset"] = time_subset_softmax(g, el, er, E, args)
        result["forward_backward"] = time_gat_backward(g, el, er, h)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_gat(g, el, er, h, args)
    return result


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
    import oracle

    indptr, indices, eid = g._in_csr()
    N = g.number_of_nodes()
    target = int(indices.size * args.cpu_fraction)
    S = int(np.searchsorted(indptr, target))
    nnz = int(indptr[S])
    H, D = 8, 32
    elh = el.reshape(N, H).cpu().numpy()
    erh = er.reshape(N, H).cpu().numpy()
    hh = h.reshape(N, H * D).cpu().numpy()
    src = np.ascontiguousarray(indices[:nnz])
    dst = np.repeat(np.arange(S, dtype=np.int64), np.diff(indptr[:S + 1]))
    ip = np.ascontiguousarray(indptr[:S + 1])
    local = np.arange(nnz, dtype=np.int64)
    cores = min(32, cpu_cores())
    oracle.set_workers(cores)
    L = oracle.lib()
    logits = np.empty((nnz, H), dtype=np.float32)
    soft = np.empty((nnz, H), dtype=np.float32)
    out = np.empty((S, H * D), dtype=np.float32)
    _, loff, roff, _ = oracle.bcast((N, H, D), (nnz, H, 1))
    deg = np.diff(ip)
    mask = np.ones(1, dtype=np.int8)
    p = lambda a: a.ctypes.data  # noqa: E731

    def once():
        L.oracle_gsddmm(p(src), p(dst), p(elh), p(erh), p(logits), nnz, 0, 1, 0, H, H, H, None,
                        None, 1, 0)
        np.maximum(logits, 0.2 * logits, out=logits)  # leaky_relu
        L.oracle_edge_softmax(p(ip), p(local), p(mask), p(logits), p(soft), S, 1, H, 0)
        L.oracle_gspmm(p(ip), p(src), p(local), p(hh), p(soft), p(out), S, 2, H * D, H, H * D, 0,
                       p(deg), p(loff), p(roff), None, None, 0)

    once()  # warm-up
    reps, t = 0, 0.0
    while t < args.cpu_seconds and reps < 100:
        t0 = time.perf_counter()
        once()
        t += time.perf_counter() - t0
        reps += 1
    units = nnz * (H + H + H * D)
    return {"value": round(units * reps / t / 1e9, 4), "unit": "GEdge·feat/s", "cores": cores,
            "kind": "port",
            "sample": "the in-edges of the first {} destination rows ({} edges, {:.1%} of E) "
                      "through gsddmm u_add_v, leaky_relu, edge_softmax and gspmm u_mul_e_sum in "
                      "float32, {} repetitions, {:.1f} s".format(S, nnz, nnz / indices.size,
                                                                  reps, t)}


def workload_c1(args):
    import torch

    import mojodgl as dgl
    import mojodgl.function as fn

    N, E, D = 10_000, 100_000, 64
    u, v = uniform_graph(0, N, E)
    rng = np.random.default_rng(0)
    g = dgl.graph((u, v), num_nodes=N)
    g.ndata["h"] = torch.from_numpy(rng.standard_normal((N, D), dtype=np.float32)).cuda()
    g.edata["e"] = torch.from_numpy(rng.random((E, D), dtype=np.float32)).cuda()

    def step(t):
        run = t if t is not None else (lambda name, fn_: fn_())
        for red in ("sum", "mean", "max", "min"):
            run("update_all_" + red, lambda: g.update_all(fn.u_mul_e("h", "e", "m"),
                                                          getattr(fn, red)("m", "z")))

    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    units = 4 * E * D
    # the same step captured once in a HIP graph and replayed: the launches
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
    # each op again with cold caches: a 512 MB write before every call evicts
    # L2 and the 256 MB MALL (the four calls above run cache-resident)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    cold = {}
    for red in ("sum", "mean", "max", "min"):
        tot = 0.0
        for _ in range(args.steps):
            flush.fill_(1)
            s.record()
            g.update_all(fn.u_mul_e("h", "e", "m"), getattr(fn, red)("m", "z"))
            t.record()
            torch.cuda.synchronize()
            tot += s.elapsed_time(t)
        cold["update_all_" + red] = round(tot / args.steps, 4)
    # pull on every other node (the in-edges selected and the subgraph built
    # on the GPU), and update_all with numpy features (copies to and from the
    # GPU inside each call), outside the step
    pull_nodes = np.arange(0, N, 2)
    g2 = dgl.graph((u, v), num_nodes=N)
    g2.ndata["h"] = g.ndata["h"].cpu().numpy()
    g2.edata["e"] = g.edata["e"].cpu().numpy()
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
    return {"metric": "gSpMM GEdge·feat/s, fp32, 1 GPU", "value": round(units / ms / 1e6, 2),
            "unit": "GEdge·feat/s", "ms_per_step": round(ms, 4), "dtype": "f32",
            "config": {"workload": "update_all u_mul_e + sum/mean/max/min, uniform graph",
                       "num_nodes": N, "num_edges": E, "feat": D},
            "breakdown_ms": {k: round(timer.avg_ms(k), 4) for k in timer.totals},
            "graph_replay": {"ms_per_step": round(gms, 4),
                             "value": round(units / gms / 1e6, 2)},
            "cold_caches_ms": cold,
            "outside_step_ms": extra}


def workload_c3(args):
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops
    from mojodgl.ops import spmm

    log("generating community graph")
    u, v, N = community_graph()
    E = u.size
    F = 602
    g = dgl.graph((u, v), num_nodes=N)
    g._device_csr("in")
    indeg = np.maximum(g.in_degrees(), 1).astype(np.float64)
    outdeg = np.maximum(g.out_degrees(), 1).astype(np.float64)
    w = torch.from_numpy((1.0 / np.sqrt(outdeg[u] * indeg[v])).astype(np.float32)
                         .reshape(E, 1)).cuda()
    gen = torch.Generator(device="cuda").manual_seed(2)
    h = torch.randn(N, F, device="cuda", generator=gen)

    def step(t):
        run = t if t is not None else (lambda name, fn_: fn_())
        run("u_mul_e_sum", lambda: ops.u_mul_e_sum(g, h, w))
        run("copy_u_mean", lambda: ops.copy_u_mean(g, h))
        run("copy_u_max_arg", lambda: spmm._run(g, "copy_lhs", "max", h, None, want_arg=True,
                                                arg_dtype=torch.int32))

    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    units = 3 * E * F
    b_mul = 4 * (N + 1) + 8 * E + 4 * E * F + 4 * E + 4 * N * F
    b_mean = 4 * (N + 1) + 4 * E + 4 * E * F + 4 * N * F
    b_max = b_mean + 4 * N * F
    kern = {}
    for name, b in (("u_mul_e_sum", b_mul), ("copy_u_mean", b_mean), ("copy_u_max_arg", b_max)):
        m = timer.avg_ms(name)
        kern[name] = {"ms": round(m, 3), "bytes": b, "GBps_algorithmic": round(b / m / 1e6, 1)}
    return {"metric": "gSpMM GEdge·feat/s, fp32, 1 GPU", "value": round(units / ms / 1e6, 2),
            "unit": "GEdge·feat/s", "ms_per_step": round(ms, 4), "dtype": "f32",
            "config": {"workload": "GCN aggregation on a 50-block community graph",
                       "num_nodes": N, "num_edges": E, "feat": F},
            "kernels": kern}


def workload_c4(args):
    import torch

    import mojodgl as dgl
    import mojodgl.ops as ops

    N, E = 1_000_000, 20_000_000
    u, v = uniform_graph(3, N, E)
    g = dgl.graph((u, v), num_nodes=N)
    g._device_coo()
    gen = torch.Generator(device="cuda").manual_seed(3)
    h = torch.randn(N, 128, device="cuda", generator=gen) * (1.0 / np.sqrt(128))
    rng = np.random.default_rng(3)
    seglen = rng.poisson(20, 1_000_000)
    R = int(seglen.sum())
    val = torch.randn(R, 16, device="cuda", generator=gen)
    seglen_d = torch.from_numpy(seglen).cuda()  # lengths resident on the GPU like the values

    def step(t):
        run = t if t is not None else (lambda name, fn_: fn_())
        run("u_dot_v", lambda: ops.u_dot_v(g, h, h))
        run("segment_sum", lambda: ops.segment_reduce(seglen_d, val, "sum"))
        run("segment_max", lambda: ops.segment_reduce(seglen_d, val, "max"))
        run("segment_softmax", lambda: ops.segment_softmax(seglen_d, val))

    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    S = seglen.size
    kern = {}
    for name, b in (("u_dot_v", 8 * E + 4 * E * 128 * 2 + 4 * E),
                    ("segment_sum", 4 * (S + 1) + 4 * R * 16 + 4 * S * 16),
                    ("segment_max", 4 * (S + 1) + 4 * R * 16 + 4 * S * 16),
                    ("segment_softmax", 4 * (S + 1) + 4 * R * 16 * 2)):
        m = timer.avg_ms(name)
        kern[name] = {"ms": round(m, 4), "bytes": b, "GBps": round(b / m / 1e6, 1)}
    units = E * 128 + 3 * R * 16
    # the reference's array helpers at the same sizes, outside the step:
    # cumsum and clamp over the 1M int64 lengths, replace_inf over the values
    from mojodgl import _lib

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
        torch.cuda.synchronize()
        s_ = torch.cuda.Event(enable_timing=True)
        t_ = torch.cuda.Event(enable_timing=True)
        s_.record()
        for _ in range(args.steps):
            fn_()
        t_.record()
        torch.cuda.synchronize()
        m = s_.elapsed_time(t_) / args.steps
        kern[name] = {"ms": round(m, 4), "bytes": b, "GBps": round(b / m / 1e6, 1)}
    return {"metric": "gSDDMM / segment GEdge·feat/s, fp32, 1 GPU",
            "value": round(units / ms / 1e6, 2), "unit": "GEdge·feat/s",
            "ms_per_step": round(ms, 4), "dtype": "f32",
            "config": {"workload": "u_dot_v link scoring + segment_reduce sum/max + "
                                   "segment_softmax", "num_nodes": N, "num_edges": E,
                       "segments": S, "rows": R},
            "kernels": kern}


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


def workload_c5(args):
    import torch

    import mojodgl.ops as ops

    n, K, R = 10_000_000, 128, 64
    gen = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randn(n, K, device="cuda", generator=gen)
    b = torch.randn(R, K, K, device="cuda", generator=gen) * (1.0 / np.sqrt(K))
    rng = np.random.default_rng(4)
    idx = torch.from_numpy(rng.integers(0, R, n)).cuda()
    seglen = rng.multinomial(n, rng.dirichlet(0.5 * np.ones(R)))

    def step(t):
        run = t if t is not None else (lambda name, fn_: fn_())
        run("gather_mm", lambda: ops.gather_mm(a, b, idx_b=idx))
        run("segment_mm", lambda: ops.segment_mm(a, b, seglen))

    timer = OpTimer()
    ms = run_steps(step, args.steps, args.warmup, timer)
    flops = 2.0 * n * K * K
    # the vendor BLAS (torch.mm) on the same shape with one weight block and
    # no grouping, for comparison (not part of the step)
    torch.backends.cuda.matmul.allow_tf32 = False  # full float32, like the step
    w0 = b[0].contiguous()
    dst = torch.empty(n, K, device="cuda")
    torch.mm(a, w0, out=dst)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    t = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        torch.mm(a, w0, out=dst)
    t.record()
    torch.cuda.synchronize()
    blas_ms = s.elapsed_time(t) / args.steps
    kern = {}
    for name in ("gather_mm", "segment_mm"):
        m = timer.avg_ms(name)
        kern[name] = {"ms": round(m, 3), "TFLOPs": round(flops / m / 1e9, 1),
                      "mfma_frac": round(flops / m / 1e9 / MFMA_F32_PEAK_TFLOPS, 4)}
    # backward (not part of the step): both gradients, da = G b^T and
    # db = a^T G per relation, 2 * flops
    gg = torch.randn(n, K, device="cuda", generator=gen)
    for name, fn_ in (("gather_mm", lambda x, y: ops.gather_mm(x, y, idx_b=idx)),
                      ("segment_mm", lambda x, y: ops.segment_mm(x, y, seglen))):
        m = time_grouped_backward(fn_, a, b, gg, args.steps)
        kern[name]["backward"] = {"ms": round(m, 3), "TFLOPs": round(2 * flops / m / 1e9, 1)}
    return {"metric": "gather_mm / segment_mm TFLOP/s, fp32, 1 GPU",
            "value": round(2 * flops / ms / 1e9, 2), "unit": "TFLOP/s",
            "ms_per_step": round(ms, 4), "dtype": "f32",
            "config": {"workload": "RGCN relation transform: gather_mm + segment_mm",
                       "rows": n, "d1": K, "d2": K, "relations": R},
            "kernels": kern,
            "vendor_blas_one_block": {"ms": round(blas_ms, 3),
                                      "TFLOPs": round(flops / blas_ms / 1e9, 1)}}


WORKLOADS = {"gat": workload_gat, "gat_train": workload_gat_train, "c1": workload_c1,
             "c3": workload_c3, "c4": workload_c4, "c5": workload_c5}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="gat", choices=sorted(WORKLOADS))
    ap.add_argument("--nodes", type=int, default=2_500_000)
    ap.add_argument("--edges", type=int, default=60_000_000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--step-only", action="store_true",
                    help="skip the measurements outside the step (graph build, edge_softmax "
                         "over a subset, forward + backward), so a profile holds the step's "
                         "kernels only")
    ap.add_argument("--cpu-fraction", type=float, default=0.1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="finish with a 1 GiB device-to-device copy (counter calibration)")
    ap.add_argument("--traffic", type=float, default=GSPMM_TRAFFIC_BYTES,
                    help="HBM bytes per gspmm launch measured by rocprofv3 (reported as is)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: mojodgl runs on a single MI355X and has no "
              "multi-GPU path (--gpus {} requested)".format(args.gpus), file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs the GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    res = WORKLOADS[args.workload](args)
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
