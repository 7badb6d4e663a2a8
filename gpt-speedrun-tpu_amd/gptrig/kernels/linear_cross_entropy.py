"""Fused linear cross-entropy on gfx950, mirroring ``rig/kernels/linear_cross_entropy.py``.

``tiled_tied_cross_entropy_losses`` / ``tiled_tied_cross_entropy`` keep the
reference's keyword signature and validation (``_validate_inputs``, ``:45-76``):
ValueError/TypeError before any launch.  The forward never materialises the
``[tokens, vocab]`` logits; the backward recomputes them one vocabulary chunk
at a time (``vocab_tile_size`` rounded up to a multiple of 256 is that chunk).
Matmul operands are bfloat16 (the reference's default ``compute_dtype``);
logits, the online log-sum-exp, probabilities and accumulation are float32.
"""

from __future__ import annotations

import torch

from .. import _lib

DEFAULT_VOCAB_TILE_SIZE = 2_048


def _validate_inputs(hidden, embedding, targets, semantic_vocab_size: int, vocab_tile_size: int) -> None:
    if hidden.ndim < 1:
        raise ValueError("hidden must have at least one dimension")
    if embedding.ndim != 2:
        raise ValueError(f"embedding must have shape [storage_vocab, width], got {tuple(embedding.shape)}")
    if hidden.shape[-1] != embedding.shape[1]:
        raise ValueError(
            f"hidden width must match the embedding width; got {hidden.shape[-1]} and {embedding.shape[1]}"
        )
    if tuple(targets.shape) != tuple(hidden.shape[:-1]):
        raise ValueError(
            f"targets must match hidden's leading dimensions; got {tuple(targets.shape)} and {tuple(hidden.shape[:-1])}"
        )
    if targets.dtype.is_floating_point or targets.dtype == torch.bool or targets.dtype.is_complex:
        raise TypeError(f"targets must have an integer dtype, got {targets.dtype}")
    if not 0 < semantic_vocab_size <= embedding.shape[0]:
        raise ValueError(
            f"semantic_vocab_size must be in [1, storage_vocab]; got {semantic_vocab_size} for {embedding.shape[0]} rows"
        )
    if vocab_tile_size <= 0:
        raise ValueError(f"vocab_tile_size must be positive, got {vocab_tile_size}")


def _normalize_compute_dtype(compute_dtype) -> torch.dtype:
    if not isinstance(compute_dtype, torch.dtype) or not compute_dtype.is_floating_point:
        raise TypeError(f"compute_dtype must be floating point, got {compute_dtype}")
    if compute_dtype != torch.bfloat16:
        raise TypeError(f"the HIP kernels compute in bfloat16; got compute_dtype={compute_dtype}")
    return compute_dtype


def chunk_for(vocab_rows: int) -> int:
    """A backward vocabulary chunk of at least ``vocab_rows`` rows (whole 256-row tiles)."""

    return max(256, (int(vocab_rows) + 255) // 256 * 256)


# The backward's one large buffer is the bf16 softmax-gradient chunk G^T
# (tokens x chunk rows).  The chunk is the whole vocabulary unless that buffer
# would pass this budget; then the fewest equal chunks that fit.  One chunk
# measured fastest on MI355X (720 TFLOP/s at 16384 tokens against 694 with two
# and 395 with 2048-row chunks; 828 against 810 at 65536 tokens).
GRAD_CHUNK_BUDGET_BYTES = 8 << 30


def grad_chunk(n_tokens: int, vocab: int) -> int:
    parts = max(1, -(-(2 * int(n_tokens) * int(vocab)) // GRAD_CHUNK_BUDGET_BYTES))
    return chunk_for(-(-int(vocab) // parts))


def flce_forward(h2: torch.Tensor, w: torch.Tensor, t1: torch.Tensor, semantic_vocab_size: int):
    """Per-token losses and LSE (both f32 [n]) for bf16 ``h2 [n,d]``, ``w [V,d]``."""

    n, d = h2.shape
    V = w.shape[0]
    losses = torch.empty(n, dtype=torch.float32, device=h2.device)
    lse = torch.empty(n, dtype=torch.float32, device=h2.device)
    ws = _lib.workspace(_lib.query("gptrig_flce_fwd_workspace_bytes", n, d, V), h2.device)
    _lib.call("gptrig_flce_fwd", h2.data_ptr(), w.data_ptr(), t1.data_ptr(), losses.data_ptr(), lse.data_ptr(),
              ws.data_ptr(), ws.numel(), n, d, V, int(semantic_vocab_size), _lib.stream())
    return losses, lse


def flce_backward(h2, w, t1, lse, cotangent, cotangent_scale: float, semantic_vocab_size: int, chunk: int,
                  dweight: torch.Tensor | None = None, accumulate: bool = False):
    """dh (bf16 [n,d]) and dW (f32 [V,d]); ``cotangent`` None means every token
    gets ``cotangent_scale``."""

    n, d = h2.shape
    V = w.shape[0]
    dh = torch.empty((n, d), dtype=torch.bfloat16, device=h2.device)
    if dweight is None:
        dweight = torch.empty((V, d), dtype=torch.float32, device=h2.device)
        accumulate = False
    ws = _lib.workspace(_lib.query("gptrig_flce_bwd_workspace_bytes", n, d, V, chunk), h2.device)
    _lib.call("gptrig_flce_bwd", h2.data_ptr(), w.data_ptr(), t1.data_ptr(), lse.data_ptr(), _lib.ptr(cotangent),
              float(cotangent_scale), dh.data_ptr(), dweight.data_ptr(), int(accumulate), ws.data_ptr(), ws.numel(),
              n, d, V, int(semantic_vocab_size), int(chunk), _lib.stream())
    return dh, dweight


def _flatten(hidden, embedding, targets):
    """bf16 ``[n8, d]`` hidden, bf16 weight and int32 targets, rows padded to a
    multiple of 8 with target -1 (an invalid target: no loss, no gradient)."""

    d = hidden.shape[-1]
    h2 = hidden.reshape(-1, d).to(torch.bfloat16)
    t1 = targets.reshape(-1).to(torch.int32)
    n = h2.shape[0]
    n8 = (n + 7) // 8 * 8
    if n8 != n:
        h2 = torch.cat([h2, h2.new_zeros((n8 - n, d))])
        t1 = torch.cat([t1, t1.new_full((n8 - n,), -1)])
    return h2.contiguous(), embedding.to(torch.bfloat16).contiguous(), t1.contiguous(), n


class _TiledLosses(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, embedding, targets, semantic_vocab_size, chunk):
        h2, w, t1, n = _flatten(hidden, embedding, targets)
        losses, lse = flce_forward(h2, w, t1, semantic_vocab_size)
        ctx.save_for_backward(h2, w, t1, lse)
        ctx.cfg = (semantic_vocab_size, chunk, hidden.shape, hidden.dtype, embedding.dtype, n)
        return losses[:n].reshape(targets.shape)

    @staticmethod
    def backward(ctx, ct):
        h2, w, t1, lse = ctx.saved_tensors
        sv, chunk, hshape, hdtype, edtype, n = ctx.cfg
        cot = torch.zeros(h2.shape[0], dtype=torch.float32, device=h2.device)
        cot[:n] = ct.reshape(-1).to(torch.float32)
        dh, dw = flce_backward(h2, w, t1, lse, cot, 0.0, sv, chunk)
        return dh[:n].reshape(hshape).to(hdtype), dw.to(edtype), None, None, None


class _TiledMean(torch.autograd.Function):
    """Mean loss with the constant 1/n cotangent folded into the backward kernel."""

    @staticmethod
    def forward(ctx, hidden, embedding, targets, semantic_vocab_size, chunk):
        h2, w, t1, n = _flatten(hidden, embedding, targets)
        losses, lse = flce_forward(h2, w, t1, semantic_vocab_size)
        ctx.save_for_backward(h2, w, t1, lse)
        ctx.cfg = (semantic_vocab_size, chunk, hidden.shape, hidden.dtype, embedding.dtype, n)
        return losses[:n].mean()

    @staticmethod
    def backward(ctx, ct):
        h2, w, t1, lse = ctx.saved_tensors
        sv, chunk, hshape, hdtype, edtype, n = ctx.cfg
        # ct is a device scalar; spread ct/n on the device (no host sync).
        cot = torch.zeros(h2.shape[0], dtype=torch.float32, device=h2.device)
        cot[:n] = ct.to(torch.float32) / n
        dh, dw = flce_backward(h2, w, t1, lse, cot, 0.0, sv, chunk)
        return dh[:n].reshape(hshape).to(hdtype), dw.to(edtype), None, None, None


def _prepare(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype):
    semantic_vocab_size = int(semantic_vocab_size)
    vocab_tile_size = int(vocab_tile_size)
    _normalize_compute_dtype(compute_dtype)
    _validate_inputs(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size)
    _lib.require_device(hidden, embedding, targets)
    if hidden.shape[-1] % 64:
        raise ValueError(f"the HIP kernels need width % 64 == 0; got {hidden.shape[-1]}")
    # vocab_tile_size is validated as the reference does; the HIP kernels tile
    # the vocabulary themselves, and the backward chunk follows the memory budget.
    n_tokens = hidden.numel() // max(hidden.shape[-1], 1)
    return semantic_vocab_size, grad_chunk(n_tokens, embedding.shape[0])


def tiled_tied_cross_entropy_losses(hidden, embedding, targets, *, semantic_vocab_size: int,
                                    vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE,
                                    compute_dtype=torch.bfloat16) -> torch.Tensor:
    """One float32 cross-entropy value per target (``:308-346``); invalid
    targets give +inf and no gradient."""

    sv, chunk = _prepare(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype)
    return _TiledLosses.apply(hidden, embedding, targets, sv, chunk)


def tiled_tied_cross_entropy(hidden, embedding, targets, *, semantic_vocab_size: int,
                             vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE,
                             compute_dtype=torch.bfloat16) -> torch.Tensor:
    """Mean tiled cross entropy in float32 (``:349-368``)."""

    sv, chunk = _prepare(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype)
    return _TiledMean.apply(hidden, embedding, targets, sv, chunk)
