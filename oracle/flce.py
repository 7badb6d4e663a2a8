"""Tiled linear cross-entropy restated from ``rig/kernels/linear_cross_entropy.py``.

Test infrastructure only (see ``oracle/__init__.py``).

The forward walks the (zero-padded) vocabulary in ``vocab_tile_size`` tiles with
an online (max, sum-exp) pair; the backward recomputes each tile's logits from
the saved log-normaliser.  Matmul operands are rounded to ``compute_dtype``;
logits, probabilities and accumulators are float32.
"""

from __future__ import annotations

import math

import torch

from .nn import F32

DEFAULT_VOCAB_TILE_SIZE = 2_048


def validate_inputs(hidden, embedding, targets, semantic_vocab_size: int, vocab_tile_size: int) -> None:
    """``_validate_inputs`` (``linear_cross_entropy.py:45-76``)."""

    if hidden.ndim < 1:
        raise ValueError("hidden must have at least one dimension")
    if embedding.ndim != 2:
        raise ValueError("embedding must have shape [storage_vocab, width]")
    if hidden.shape[-1] != embedding.shape[1]:
        raise ValueError("hidden width must match the embedding width")
    if tuple(targets.shape) != tuple(hidden.shape[:-1]):
        raise ValueError("targets must match hidden's leading dimensions")
    if targets.dtype.is_floating_point or targets.dtype == torch.bool:
        raise TypeError(f"targets must have an integer dtype, got {targets.dtype}")
    if not 0 < semantic_vocab_size <= embedding.shape[0]:
        raise ValueError("semantic_vocab_size must be in [1, storage_vocab]")
    if vocab_tile_size <= 0:
        raise ValueError(f"vocab_tile_size must be positive, got {vocab_tile_size}")


def _padded(embedding: torch.Tensor, tile: int) -> tuple[torch.Tensor, int]:
    """``_padded_embedding`` (``:79-89``)."""

    storage = embedding.shape[0]
    count = (storage + tile - 1) // tile
    padded = count * tile
    if padded == storage:
        return embedding, count
    pad = torch.zeros((padded - storage, embedding.shape[1]), dtype=embedding.dtype)
    return torch.cat([embedding, pad], 0), count


def _tile_logits(h_c: torch.Tensor, w_pad: torch.Tensor, index: int, tile: int, cdt) -> torch.Tensor:
    """``_tile_logits`` (``:92-112``): float32-accumulated ``h W_tile^T``."""

    w = w_pad[index * tile:(index + 1) * tile].to(cdt).to(F32)
    return h_c @ w.T


def losses_and_lse(hidden, embedding, targets, *, semantic_vocab_size: int,
                   vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE, compute_dtype=torch.bfloat16):
    """``_losses_and_residual`` (``:115-179``): per-target losses and the LSE."""

    validate_inputs(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size)
    flat_h = hidden.reshape(-1, hidden.shape[-1])
    flat_t = targets.reshape(-1).to(torch.int64)
    h_c = flat_h.to(compute_dtype).to(F32)
    w_pad, count = _padded(embedding, vocab_tile_size)
    positions = torch.arange(vocab_tile_size)
    running_max = torch.full((flat_h.shape[0],), -math.inf, dtype=F32)
    running_sum = torch.zeros((flat_h.shape[0],), dtype=F32)
    for index in range(count):
        start = index * vocab_tile_size
        logits = _tile_logits(h_c, w_pad, index, vocab_tile_size, compute_dtype)
        valid = (start + positions) < semantic_vocab_size
        logits = torch.where(valid[None, :], logits, torch.tensor(-math.inf))
        tile_max = logits.max(dim=1).values
        next_max = torch.maximum(running_max, tile_max)
        scaled = running_sum * torch.exp(running_max - next_max)
        scaled = torch.where(torch.isnan(scaled), torch.zeros_like(scaled), scaled)
        running_sum = scaled + torch.exp(logits - next_max[:, None]).sum(dim=1)
        running_max = next_max
    lse = running_max + torch.log(running_sum)
    valid_target = (flat_t >= 0) & (flat_t < semantic_vocab_size)
    safe = flat_t.clamp(0, semantic_vocab_size - 1)
    tw = embedding[safe].to(compute_dtype).to(F32)
    target_logits = (h_c * tw).sum(-1)
    losses = torch.where(valid_target, lse - target_logits, torch.tensor(math.inf))
    return losses.reshape(targets.shape), lse


def losses_backward(hidden, embedding, targets, lse, cotangent, *, semantic_vocab_size: int,
                    vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE, compute_dtype=torch.bfloat16):
    """``_tiled_losses_bwd`` (``:220-302``): dh (hidden dtype), dW (embedding dtype).

    Invalid targets get a zero cotangent (``:236-240``); storage rows at or
    above ``semantic_vocab_size`` get exactly zero gradient (``:263-267``).
    """

    flat_h = hidden.reshape(-1, hidden.shape[-1])
    flat_t = targets.reshape(-1).to(torch.int64)
    h_c = flat_h.to(compute_dtype).to(F32)
    w_pad, count = _padded(embedding, vocab_tile_size)
    positions = torch.arange(vocab_tile_size)
    valid_target = (flat_t >= 0) & (flat_t < semantic_vocab_size)
    ct = torch.where(valid_target, cotangent.reshape(-1).to(F32), torch.zeros((), dtype=F32))
    grad_h = torch.zeros(flat_h.shape, dtype=F32)
    grad_w = torch.zeros((w_pad.shape[0], embedding.shape[1]), dtype=F32)
    for index in range(count):
        start = index * vocab_tile_size
        w_c = w_pad[start:start + vocab_tile_size].to(compute_dtype).to(F32)
        logits = h_c @ w_c.T
        ids = start + positions
        valid = ids < semantic_vocab_size
        p = torch.where(valid[None, :], torch.exp(logits - lse[:, None]), torch.zeros((), dtype=F32))
        onehot = (flat_t[:, None] == ids[None, :]).to(F32)
        g = ((p - onehot) * ct[:, None]).to(compute_dtype).to(F32)
        grad_h += g @ w_c
        grad_w[start:start + vocab_tile_size] = g.T @ h_c
    dh = grad_h.reshape(hidden.shape).to(hidden.dtype)
    dw = grad_w[: embedding.shape[0]].to(embedding.dtype)
    return dh, dw


def dense_losses(hidden, embedding, targets, semantic_vocab_size: int, compute_dtype) -> torch.Tensor:
    """Dense log-softmax oracle used by the reference's own FLCE tests
    (``tests/test_linear_cross_entropy.py:21-37``); differentiable."""

    logits = hidden.to(compute_dtype).to(F32) @ embedding[:semantic_vocab_size].to(compute_dtype).to(F32).T
    logp = torch.log_softmax(logits, dim=-1)
    return -torch.gather(logp, -1, targets.to(torch.int64)[..., None])[..., 0]


class TiledLosses(torch.autograd.Function):
    """Per-token losses with the reference's custom VJP."""

    @staticmethod
    def forward(ctx, hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype):
        losses, lse = losses_and_lse(hidden, embedding, targets, semantic_vocab_size=semantic_vocab_size,
                                     vocab_tile_size=vocab_tile_size, compute_dtype=compute_dtype)
        ctx.save_for_backward(hidden, embedding, targets, lse)
        ctx.cfg = (semantic_vocab_size, vocab_tile_size, compute_dtype)
        return losses

    @staticmethod
    def backward(ctx, ct):
        hidden, embedding, targets, lse = ctx.saved_tensors
        sv, tile, cdt = ctx.cfg
        dh, dw = losses_backward(hidden, embedding, targets, lse, ct, semantic_vocab_size=sv,
                                 vocab_tile_size=tile, compute_dtype=cdt)
        return dh, dw, None, None, None, None


def tiled_tied_cross_entropy_losses(hidden, embedding, targets, *, semantic_vocab_size: int,
                                    vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE,
                                    compute_dtype=torch.bfloat16) -> torch.Tensor:
    """``tiled_tied_cross_entropy_losses`` (``:308-346``)."""

    validate_inputs(hidden, embedding, targets, int(semantic_vocab_size), int(vocab_tile_size))
    return TiledLosses.apply(hidden, embedding, targets, int(semantic_vocab_size), int(vocab_tile_size), compute_dtype)


def tiled_tied_cross_entropy(hidden, embedding, targets, *, semantic_vocab_size: int,
                             vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE,
                             compute_dtype=torch.bfloat16) -> torch.Tensor:
    """``tiled_tied_cross_entropy`` (``:349-368``): float32 mean."""

    losses = tiled_tied_cross_entropy_losses(hidden, embedding, targets, semantic_vocab_size=semantic_vocab_size,
                                             vocab_tile_size=vocab_tile_size, compute_dtype=compute_dtype)
    return losses.to(F32).mean()
