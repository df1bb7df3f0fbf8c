"""`nn.functional.edge_softmax` is `ops.edge_softmax` itself."""

from ...ops import edge_softmax  # noqa: F401
