"""Attention runtime plumbing, mirroring ``rig/attention.py``.

On one GPU the reference's data-axis ``shard_map`` (``:165-202``) collapses to
the local callable, so ``make_mesh_attention`` returns the HIP attention
directly.  Tile plans are compile-time constants of the HIP kernels.
"""

from __future__ import annotations

from typing import Callable

import torch

from .kernels import AttentionConfig, AttentionTiles, make_causal_attention

AttentionCallable = Callable[..., torch.Tensor]


def attention_softmax_scale(rule: str, head_dim: int) -> float:
    """``attention_softmax_scale`` (``rig/attention.py:55-62``)."""

    if rule == "inverse_head_dim":
        return 1.0 / float(head_dim)
    if rule == "inverse_sqrt_head_dim":
        return head_dim ** -0.5
    raise ValueError(f"unsupported attention scale {rule!r}")


def make_mesh_attention(*, backend: str, mesh=None, tiles: AttentionTiles | None, softmax_scale: float,
                        document_masking: bool) -> AttentionCallable | None:
    """``make_mesh_attention`` (``rig/attention.py:165-202``) for one device."""

    if backend == "dense":
        return None
    if tiles is None:
        raise ValueError("non-dense attention requires a resolved tile plan")
    return make_causal_attention(AttentionConfig(backend="auto", tiles=tiles, softmax_scale=softmax_scale))


def document_segments(tokens: torch.Tensor, boundary_token: int) -> torch.Tensor:
    """``document_segments`` (``rig/attention.py:205-208``)."""

    return torch.cumsum((tokens == boundary_token).to(torch.int32), dim=1).to(torch.int32)
