"""Neural-network helpers (only `functional.edge_softmax`, as the reference)."""

from . import functional  # noqa: F401
