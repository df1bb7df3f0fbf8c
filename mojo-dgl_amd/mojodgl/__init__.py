"""mojodgl -- DGL's graph message-passing kernels on AMD Instinct MI355X.

The names are DGL's: `graph`, `ops`, `function`, `g.update_all` with
`fn.copy_u('h', 'm')` and `fn.sum('m', 'h')` mean what they mean upstream.
Every kernel runs on the GPU through libmdgl.so (hand-written HIP for
gfx950); numpy inputs are copied to the GPU and results come back as numpy,
torch tensors on the GPU stay there.
"""

from . import function, nn, ops  # noqa: F401
from ._lib import build  # noqa: F401
from .base import ALL, EID, ETYPE, NID, NTYPE, DGLError  # noqa: F401
from .convert import graph  # noqa: F401
from .function import *  # noqa: F401,F403
from .heterograph import DGLGraph  # noqa: F401
from .ops import *  # noqa: F401,F403
from .udf import EdgeBatch, NodeBatch  # noqa: F401

__version__ = "0.1.0"

__all__ = [
    "DGLGraph", "graph", "DGLError", "ALL", "EID", "ETYPE", "NID", "NTYPE",
    "EdgeBatch", "NodeBatch", "build",
    "function", "ops", "nn",
] + ops.__all__
