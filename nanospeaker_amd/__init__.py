"""
nanospeaker_amd: nanoSpeaker's dropless MoE hot path (routing, dispatch, grouped SwiGLU
experts, combine, backward) as hand-written HIP kernels for MI355X (gfx950), behind a
C ABI (include/nsmoe.h) and the reference's Python interface (MoEBlock, TopKRouter,
moe_kernel ops).
"""

from .glu import GLUFeedForward, glu_hidden_dim, make_glu
from .moe import AUTO_CAPACITY, MoEBlock
from .router import TopKRouter
from .utils import ACTIVATIONS, resolve_activation

__all__ = [
    "ACTIVATIONS", "AUTO_CAPACITY", "GLUFeedForward", "MoEBlock", "TopKRouter",
    "glu_hidden_dim", "make_glu", "resolve_activation",
]
