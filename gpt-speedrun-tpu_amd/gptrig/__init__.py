"""gptrig: the GPT speedrun rig's training-step hot path on MI355X (gfx950).

Operator API mirrors the reference's ``rig.kernels`` / ``rig.nn`` /
``rig.attention``; the compute is the C-ABI library ``libgptrig.so`` built
from ``csrc/`` (see ``include/gptrig.h``).
"""

from . import _lib  # noqa: F401
from ._lib import version  # noqa: F401

__all__ = ("version",)
