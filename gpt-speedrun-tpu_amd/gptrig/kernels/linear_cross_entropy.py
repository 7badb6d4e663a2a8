"""Fused linear cross-entropy on gfx950, mirroring ``rig/kernels/linear_cross_entropy.py``.

``tiled_tied_cross_entropy_losses`` / ``tiled_tied_cross_entropy`` keep the
reference's keyword signature and validation (``_validate_inputs``, ``:45-76``):
ValueError/TypeError before any launch.  Neither direction materialises the
``[tokens, vocab]`` logits.  The backward recomputes them one vocabulary chunk
at a time, and ``vocab_tile_size`` (rounded up to a multiple of 256, the
kernels' tile) is that chunk: its bf16 softmax-gradient buffer is at most
``[tokens, chunk]``, the bound of the reference's ``[tokens, vocab_tile_size]``
live logits (``:1-24``).  With ``compute_dtype=torch.bfloat16`` (the
reference's default) the matmul operands are bfloat16; logits, the online
log-sum-exp, probabilities and accumulation are float32.  Any width is
accepted: widths that are not a multiple of 64 are zero-padded, which leaves
every logit unchanged.  With ``compute_dtype=torch.float32`` every product and
sum is float32 (``gptrig_flce32_*``: the same tiled algorithm on float32
operands, a float32 ``[tokens, chunk]`` logit-gradient workspace); gradients
come back in the inputs' dtypes, as the reference casts them (``:297-302``).
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
    if compute_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"the HIP kernels compute in bfloat16 or float32; got compute_dtype={compute_dtype}")
    return compute_dtype


def chunk_for(vocab_rows: int) -> int:
    """The backward's vocabulary chunk for a requested tile: the smallest
    multiple of 256 rows that is at least ``vocab_rows``."""

    return max(256, (int(vocab_rows) + 255) // 256 * 256)


def workspace_bytes(n_tokens: int, width: int, vocab: int, vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE) -> int:
    """Device workspace of the backward for ``vocab_tile_size``: the bf16
    ``[tokens, chunk]`` softmax gradient, the float32 ``[tokens, width]`` dh
    accumulator (the reference's ``grad_hidden`` carry, ``:247``) and the
    work-queue counters."""

    d = (int(width) + 63) // 64 * 64
    n = (int(n_tokens) + 7) // 8 * 8
    return int(_lib.query("gptrig_flce_bwd_workspace_bytes", n, d, int(vocab), chunk_for(vocab_tile_size)))


# The trainer's opt-in: one chunk covering the whole vocabulary while its bf16
# G^T fits this budget (then the fewest equal chunks that fit).  With the
# memory of one MI355X this is the fastest choice for the 125M step (no fp32 dh
# accumulator passes); the public API never takes it implicitly.
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


def flce_forward_keep(h2: torch.Tensor, w: torch.Tensor, t1: torch.Tensor, semantic_vocab_size: int,
                      keep: torch.Tensor | None = None):
    """``flce_forward`` that also keeps the probabilities for
    ``flce_backward_keep`` (``gptrig_flce_fwd_keep``): returns ``(losses, lse,
    keep)``, ``keep`` a uint8 device buffer of ``gptrig_flce_keep_bytes``
    (passed in to reuse one)."""

    n, d = h2.shape
    V = w.shape[0]
    losses = torch.empty(n, dtype=torch.float32, device=h2.device)
    lse = torch.empty(n, dtype=torch.float32, device=h2.device)
    nbytes = _lib.query("gptrig_flce_keep_bytes", n, V)
    if keep is None or keep.numel() < nbytes:
        keep = _lib.workspace(nbytes, h2.device)
    ws = _lib.workspace(_lib.query("gptrig_flce_fwd_workspace_bytes", n, d, V), h2.device)
    _lib.call("gptrig_flce_fwd_keep", h2.data_ptr(), w.data_ptr(), t1.data_ptr(), losses.data_ptr(), lse.data_ptr(),
              keep.data_ptr(), keep.numel(), ws.data_ptr(), ws.numel(), n, d, V, int(semantic_vocab_size),
              _lib.stream())
    return losses, lse, keep


def flce_backward_keep(h2, w, t1, lse, keep, cotangent, cotangent_scale: float, semantic_vocab_size: int,
                       dweight: torch.Tensor | None = None, accumulate: bool = False):
    """``flce_backward`` from ``flce_forward_keep``'s buffer (consumed)."""

    n, d = h2.shape
    V = w.shape[0]
    dh = torch.empty((n, d), dtype=torch.bfloat16, device=h2.device)
    if dweight is None:
        dweight = torch.empty((V, d), dtype=torch.float32, device=h2.device)
        accumulate = False
    if t1.data_ptr() % 16:  # the backward reads the targets 16 bytes at a time
        t1 = t1.clone()
    ws = _lib.workspace(_lib.query("gptrig_flce_bwd_keep_workspace_bytes", n, d), h2.device)
    _lib.call("gptrig_flce_bwd_keep", h2.data_ptr(), w.data_ptr(), t1.data_ptr(), lse.data_ptr(),
              _lib.ptr(cotangent), float(cotangent_scale), dh.data_ptr(), dweight.data_ptr(), int(accumulate),
              keep.data_ptr(), keep.numel(), ws.data_ptr(), ws.numel(), n, d, V, int(semantic_vocab_size),
              _lib.stream())
    return dh, dweight


def _flatten(hidden, embedding, targets):
    """bf16 ``[n8, d64]`` hidden, bf16 ``[V, d64]`` weight and int32 targets:
    rows padded to a multiple of 8 with target -1 (an invalid target: no loss,
    no gradient), columns zero-padded to a multiple of 64 (zero columns add
    nothing to any logit)."""

    d = hidden.shape[-1]
    d64 = (d + 63) // 64 * 64
    h2 = hidden.reshape(-1, d).to(torch.bfloat16)
    w = embedding.to(torch.bfloat16)
    if d64 != d:
        h2 = torch.nn.functional.pad(h2, (0, d64 - d))
        w = torch.nn.functional.pad(w, (0, d64 - d))
    t1 = targets.reshape(-1).to(torch.int32)
    n = h2.shape[0]
    n8 = (n + 7) // 8 * 8
    if n8 != n:
        h2 = torch.cat([h2, h2.new_zeros((n8 - n, d64))])
        t1 = torch.cat([t1, t1.new_full((n8 - n,), -1)])
    return h2.contiguous(), w.contiguous(), t1.contiguous(), n


def _unflatten(dh, dw, n, hshape, hdtype, edtype):
    d = hshape[-1]
    return dh[:n, :d].reshape(hshape).to(hdtype), dw[:, :d].to(edtype)


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
        return (*_unflatten(dh, dw, n, hshape, hdtype, edtype), None, None, None)


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
        return (*_unflatten(dh, dw, n, hshape, hdtype, edtype), None, None, None)


def flce32_forward(h: torch.Tensor, w: torch.Tensor, t1: torch.Tensor, semantic_vocab_size: int):
    """Per-token losses and LSE (f32 [n]) with float32 compute, for f32 ``h [n,d]``, ``w [V,d]``."""

    n, d = h.shape
    V = w.shape[0]
    losses = torch.empty(n, dtype=torch.float32, device=h.device)
    lse = torch.empty(n, dtype=torch.float32, device=h.device)
    ws = _lib.workspace(_lib.query("gptrig_flce32_fwd_workspace_bytes", n, d, V), h.device)
    _lib.call("gptrig_flce32_fwd", h.data_ptr(), w.data_ptr(), t1.data_ptr(), losses.data_ptr(), lse.data_ptr(),
              ws.data_ptr(), ws.numel(), n, d, V, int(semantic_vocab_size), _lib.stream())
    return losses, lse


def flce32_backward(h, w, t1, lse, cotangent, cotangent_scale: float, semantic_vocab_size: int, vocab_chunk: int):
    """``(dh f32 [n, d], dW f32 [V, d])`` with float32 compute."""

    n, d = h.shape
    V = w.shape[0]
    dh = torch.empty((n, d), dtype=torch.float32, device=h.device)
    dw = torch.empty((V, d), dtype=torch.float32, device=h.device)
    ws = _lib.workspace(_lib.query("gptrig_flce32_bwd_workspace_bytes", n, d, V, int(vocab_chunk)), h.device)
    _lib.call("gptrig_flce32_bwd", h.data_ptr(), w.data_ptr(), t1.data_ptr(), lse.data_ptr(), _lib.ptr(cotangent),
              float(cotangent_scale), dh.data_ptr(), dw.data_ptr(), 0, ws.data_ptr(), ws.numel(), n, d, V,
              int(semantic_vocab_size), int(vocab_chunk), _lib.stream())
    return dh, dw


def _flatten32(hidden, embedding, targets):
    d = hidden.shape[-1]
    return (hidden.reshape(-1, d).to(torch.float32).contiguous(), embedding.to(torch.float32).contiguous(),
            targets.reshape(-1).to(torch.int32).contiguous())


class _TiledLosses32(torch.autograd.Function):
    """``tiled_tied_cross_entropy_losses`` with ``compute_dtype=float32``."""

    @staticmethod
    def forward(ctx, hidden, embedding, targets, semantic_vocab_size, chunk):
        h, w, t1 = _flatten32(hidden, embedding, targets)
        losses, lse = flce32_forward(h, w, t1, semantic_vocab_size)
        ctx.save_for_backward(h, w, t1, lse)
        ctx.cfg = (semantic_vocab_size, chunk, hidden.shape, hidden.dtype, embedding.dtype)
        return losses.reshape(targets.shape)

    @staticmethod
    def backward(ctx, ct):
        h, w, t1, lse = ctx.saved_tensors
        sv, chunk, hshape, hdtype, edtype = ctx.cfg
        cot = ct.reshape(-1).to(torch.float32).contiguous()
        dh, dw = flce32_backward(h, w, t1, lse, cot, 0.0, sv, chunk)
        return dh.reshape(hshape).to(hdtype), dw.to(edtype), None, None, None


class _TiledMean32(torch.autograd.Function):
    """``tiled_tied_cross_entropy`` with ``compute_dtype=float32``."""

    @staticmethod
    def forward(ctx, hidden, embedding, targets, semantic_vocab_size, chunk):
        h, w, t1 = _flatten32(hidden, embedding, targets)
        losses, lse = flce32_forward(h, w, t1, semantic_vocab_size)
        ctx.save_for_backward(h, w, t1, lse)
        ctx.cfg = (semantic_vocab_size, chunk, hidden.shape, hidden.dtype, embedding.dtype)
        return losses.mean()

    @staticmethod
    def backward(ctx, ct):
        h, w, t1, lse = ctx.saved_tensors
        sv, chunk, hshape, hdtype, edtype = ctx.cfg
        n = h.shape[0]
        cot = (ct.to(torch.float32) / n).expand(n).contiguous()
        dh, dw = flce32_backward(h, w, t1, lse, cot, 0.0, sv, chunk)
        return dh.reshape(hshape).to(hdtype), dw.to(edtype), None, None, None


def _prepare(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype):
    semantic_vocab_size = int(semantic_vocab_size)
    vocab_tile_size = int(vocab_tile_size)
    dtype = _normalize_compute_dtype(compute_dtype)
    _validate_inputs(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size)
    _lib.require_device(hidden, embedding, targets)
    if dtype == torch.float32:
        return semantic_vocab_size, int(vocab_tile_size), True
    return semantic_vocab_size, chunk_for(vocab_tile_size), False


def tiled_tied_cross_entropy_losses(hidden, embedding, targets, *, semantic_vocab_size: int,
                                    vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE,
                                    compute_dtype=torch.bfloat16) -> torch.Tensor:
    """One float32 cross-entropy value per target (``:308-346``); invalid
    targets give +inf and no gradient."""

    sv, chunk, f32 = _prepare(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype)
    return (_TiledLosses32 if f32 else _TiledLosses).apply(hidden, embedding, targets, sv, chunk)


def tiled_tied_cross_entropy(hidden, embedding, targets, *, semantic_vocab_size: int,
                             vocab_tile_size: int = DEFAULT_VOCAB_TILE_SIZE,
                             compute_dtype=torch.bfloat16) -> torch.Tensor:
    """Mean tiled cross entropy in float32 (``:349-368``)."""

    sv, chunk, f32 = _prepare(hidden, embedding, targets, semantic_vocab_size, vocab_tile_size, compute_dtype)
    return (_TiledMean32 if f32 else _TiledMean).apply(hidden, embedding, targets, sv, chunk)
