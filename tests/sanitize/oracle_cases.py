"""Runs the oracle's functions on small seeded cases and saves the results
(argv[1], an .npz). tests/test_sanitize.py runs it twice: against the
sanitizer build of the oracle (AddressSanitizer and UndefinedBehaviorSanitizer
preloaded) and against the regular build, and compares the two."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", ".."))
import oracle  # noqa: E402

rng = np.random.default_rng(0)
out = {}
n, e = 40, 300
u, v = rng.integers(0, n, e), rng.integers(0, n, e)
v[:80] = 3  # a long row
x = rng.standard_normal((n, 2, 3))
w = rng.standard_normal((e, 2, 1)) + 2.0
for op in ("add", "sub", "mul", "div", "copy_lhs", "copy_rhs"):
    for red in ("sum", "max", "min", "mean"):
        lhs = None if op == "copy_rhs" else x
        rhs = None if op == "copy_lhs" else w
        r, au, ae = oracle.gspmm(u, v, n, op, red, lhs, rhs, np.float64, with_arg=True)
        out["gspmm_%s_%s" % (op, red)] = r
        out["gspmm_%s_%s_args" % (op, red)] = np.stack([au, ae])
for op in ("add", "sub", "mul", "div", "dot"):
    for lt, rt in (("u", "v"), ("e", "u"), ("v", "e")):
        L = x if lt != "e" else rng.standard_normal((e, 2, 3))
        R = (x if rt != "e" else rng.standard_normal((e, 2, 3))) + 3.0
        out["gsddmm_%s_%s%s" % (op, lt, rt)] = oracle.gsddmm(u, v, n, op, L, R, lt, rt,
                                                             np.float32)
logits = rng.standard_normal((e, 4, 1))
out["edge_softmax_dst"] = oracle.edge_softmax(u, v, n, logits)
out["edge_softmax_src"] = oracle.edge_softmax(u, v, n, logits, norm_by="src")
out["edge_softmax_eids"] = oracle.edge_softmax(u, v, n, logits, eids=rng.integers(0, e, 120))
seglen = rng.poisson(6, 50)
seglen[::5] = 0
val = rng.standard_normal((int(seglen.sum()), 5))
for red in ("sum", "max", "min", "mean"):
    out["segment_" + red] = oracle.segment_reduce(seglen, val, red, np.float32)
out["segment_softmax"] = oracle.segment_softmax(seglen, val)
a = rng.standard_normal((97, 7))
b = rng.standard_normal((4, 7, 5))
out["gather_mm"] = oracle.gather_mm(a, b, rng.integers(0, 4, 97))
out["segment_mm"] = oracle.segment_mm(a, b, np.array([30, 0, 40, 20]))
out["cumsum"] = oracle.cumsum(rng.integers(-5, 9, 1000))
out["clamp"] = oracle.clamp_i64(rng.integers(-50, 50, 100), -3, 7)
out["replace_inf"] = oracle.replace_inf_with_zero(np.array([1.0, np.inf, -np.inf, np.nan, 2.0]))
np.savez(sys.argv[1], **out)
print("oracle cases:", len(out))
