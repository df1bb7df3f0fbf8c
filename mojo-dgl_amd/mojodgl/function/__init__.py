"""Builtin message and reduce functions (the `dgl.function` names)."""

# pylint: disable=redefined-builtin
from .base import *  # noqa: F401,F403
from .message import *  # noqa: F401,F403
from .reducer import *  # noqa: F401,F403
