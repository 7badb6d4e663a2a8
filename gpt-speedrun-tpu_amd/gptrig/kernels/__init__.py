"""gfx950 kernels behind the reference's operator API (``rig/kernels/__init__.py:8-34``)."""

from .flash_attention import (
    AttentionConfig,
    AttentionTiles,
    attention_tile_candidates,
    causal_attention,
    make_causal_attention,
    select_attention_tiles,
)
from .linear_cross_entropy import (
    DEFAULT_VOCAB_TILE_SIZE,
    tiled_tied_cross_entropy,
    tiled_tied_cross_entropy_losses,
)

__all__ = (
    "DEFAULT_VOCAB_TILE_SIZE",
    "AttentionConfig",
    "AttentionTiles",
    "attention_tile_candidates",
    "causal_attention",
    "make_causal_attention",
    "select_attention_tiles",
    "tiled_tied_cross_entropy",
    "tiled_tied_cross_entropy_losses",
)
