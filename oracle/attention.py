"""Causal attention restated from ``rig/kernels/tpu_flash_attention.py``.

Test infrastructure only (see ``oracle/__init__.py``).

Layout is the reference's BHSD ``[batch, heads, sequence, head_dim]``.  Scores
are float32 (bf16 products are exact in float32, sums are float32) and the
mask adds ``-0.7 * float32_max`` (``tpu_flash_attention.py:71,311-319``).  Two
forwards, which differ only in what the bf16 probabilities are:

* :func:`flash_attention_forward`, the Pallas forward kernel the training
  step runs (``:236-349``): per ``block_kv_compute`` keys, the unnormalised
  ``exp(s - running max)`` is rounded to ``v.dtype`` for the PV product and
  the float32 accumulator is rescaled; the output is rounded once at the end.
  :class:`DenseAttention` (the model's attention) uses it.
* :func:`attention_forward` / :func:`reference_causal_attention`, the
  kernel's own test oracle (``:171-207``): the normalised softmax is rounded
  to ``v.dtype`` before the PV product.

The backward kernels (``:479-701``) use one formula for both.
"""

from __future__ import annotations

import torch

from .nn import F32

MASK_VALUE = -0.7 * float(torch.finfo(torch.float32).max)


def validate_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """``_validate_qkv`` (``tpu_flash_attention.py:145-168``)."""

    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must use BHSD rank-4 layout")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("dense causal self-attention requires identical q/k/v shapes")
    if not all(q.shape):
        raise ValueError(f"q/k/v dimensions must be nonzero, got {tuple(q.shape)}")
    if q.shape[-1] > 128 or q.shape[-1] % 8:
        raise ValueError("the kernel requires head_dim <= 128 and divisible by 8")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k, and v dtypes must match")
    if not q.dtype.is_floating_point:
        raise TypeError("q, k, and v must be floating point")


def visibility(sequence: int, segment_ids: torch.Tensor | None, valid_sequence: int | None = None) -> torch.Tensor:
    """Boolean ``[B or 1, 1, S, S]`` mask: causal, same document, key < valid."""

    row = torch.arange(sequence)[:, None]
    col = torch.arange(sequence)[None, :]
    visible = col <= row
    if valid_sequence is not None:
        visible = visible & (col < valid_sequence)
    visible = visible[None, None]
    if segment_ids is not None:
        same = segment_ids[:, None, :, None] == segment_ids[:, None, None, :]
        visible = visible & same
    return visible


def _scores(q: torch.Tensor, k: torch.Tensor, scale: float) -> torch.Tensor:
    return torch.matmul(q.to(F32), k.to(F32).transpose(-1, -2)) * scale


def reference_causal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    segment_ids: torch.Tensor | None = None,
) -> torch.Tensor:
    """``reference_causal_attention`` (``tpu_flash_attention.py:171-207``)."""

    return attention_forward(q, k, v, softmax_scale=softmax_scale, segment_ids=segment_ids)[0]


def attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    segment_ids: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Output and natural-log LSE ``[B,H,S]`` float32.

    The LSE is what ``_tpu_flash_forward_kernel`` stores
    (``log(l) + m``, ``tpu_flash_attention.py:344-348``) and what the backward
    kernels subtract (``:556-558``).
    """

    validate_qkv(q, k, v)
    scale = float(q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale)
    scores = _scores(q, k, scale)
    visible = visibility(q.shape[2], segment_ids)
    scores = torch.where(visible, scores, torch.tensor(MASK_VALUE, dtype=F32))
    lse = torch.logsumexp(scores, dim=-1)
    probabilities = torch.softmax(scores, dim=-1).to(v.dtype)
    out = torch.matmul(probabilities.to(F32), v.to(F32)).to(q.dtype)
    return out, lse


# Tile shapes the kernel's tile choice ranks (``rig/kernels/autotune.py:906-916``).
_FLASH_TILE_SHAPES = ((128, 128, 128), (128, 256, 128), (256, 256, 128), (256, 512, 128), (512, 512, 128),
                      (512, 512, 256), (256, 1024, 256), (512, 1024, 256), (1024, 1024, 128))


def flash_tiles(sequence: int) -> tuple[int, int, int]:
    """``(block_q, block_kv, block_kv_compute)`` as ``select_attention_tiles``
    (``tpu_flash_attention.py:112-142``) picks them: among the shapes that tile
    the sequence padded to a multiple of 128 (``autotune.py:752-760``), the one
    nearest to (512, 512, 256), ties to the larger compute block, then block_q,
    then block_kv.  (The VMEM bound of ``autotune.py:762-790`` admits every
    shape here for head_dim <= 128.)  512/512/256 at S = 1024.
    """

    extent = -(-sequence // 128) * 128
    legal = [t for t in _FLASH_TILE_SHAPES if extent % t[0] == 0 and extent % t[1] == 0]
    return min(legal, key=lambda t: (abs(t[0] - 512) + abs(t[1] - 512) + abs(t[2] - 256), -t[2], -t[0], -t[1]))


def flash_attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    segment_ids: torch.Tensor | None = None,
    probability_dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Output and LSE of the Pallas forward kernel (``tpu_flash_attention.py:236-349``).

    Keys are visited in ``block_kv_compute`` chunks of the ``block_kv`` blocks
    that ``_below_or_on_diagonal`` (``:210-218``) admits for the row's
    ``block_q`` block, past the sequence end masked (``:311-313``, the
    wrapper's right padding).  Per chunk (``:293-343``): ``s`` masked,
    ``m' = max(m, rowmax s)``, ``p = exp(s - m')``, ``c = exp(m - m') l``,
    ``l' = rowsum p + c``, ``acc = acc * (c / l') + (p.astype(v) @ v) / l'``
    (reciprocal ``1 / l'``, 1 where ``l' = 0``); output ``acc`` rounded to
    ``q.dtype`` and LSE ``log l + m`` (``:344-348``).  ``probability_dtype``
    (default ``v.dtype``) is the rounding of ``p``; float32 leaves it
    unrounded, which makes the result the exact softmax average.
    """

    validate_qkv(q, k, v)
    batch, heads, sequence, head_dim = q.shape
    scale = float(head_dim ** -0.5 if softmax_scale is None else softmax_scale)
    pdt = v.dtype if probability_dtype is None else probability_dtype
    block_q, block_kv, chunk = flash_tiles(sequence)
    extent = -(-sequence // 128) * 128
    qf = q.to(F32)
    kf = torch.zeros((batch, heads, extent, head_dim), dtype=F32)
    vf = torch.zeros((batch, heads, extent, head_dim), dtype=F32)
    kf[:, :, :sequence] = k.to(F32)
    vf[:, :, :sequence] = v.to(F32)
    rows = torch.arange(sequence)
    last_row = (rows // block_q + 1) * block_q - 1
    m = torch.full((batch, heads, sequence, 1), -float("inf"), dtype=F32)
    l = torch.zeros((batch, heads, sequence, 1), dtype=F32)  # noqa: E741
    acc = torch.zeros((batch, heads, sequence, head_dim), dtype=F32)
    mask_value = torch.tensor(MASK_VALUE, dtype=F32)
    zero = torch.zeros((), dtype=F32)
    for kv_block in range(extent // block_kv):
        visit = (last_row >= kv_block * block_kv)[:, None]
        for start in range(kv_block * block_kv, (kv_block + 1) * block_kv, chunk):
            cols = torch.arange(start, start + chunk)
            scores = torch.matmul(qf, kf[:, :, start:start + chunk].transpose(-1, -2)) * scale
            mask = (cols[None, :] <= rows[:, None]) & (cols[None, :] < sequence)
            mask = mask[None, None]
            if segment_ids is not None:
                kv_seg = torch.full((batch, chunk), -1, dtype=segment_ids.dtype)
                inside = cols < sequence
                kv_seg[:, inside] = segment_ids[:, cols[inside]]
                mask = mask & (segment_ids[:, None, :, None] == kv_seg[:, None, None, :])
            scores = scores + torch.where(mask, zero, mask_value)
            m_next = torch.maximum(m, scores.max(dim=-1, keepdim=True).values)
            p = torch.exp(scores - m_next)
            corrected = torch.exp(m - m_next) * l
            l_next = p.sum(dim=-1, keepdim=True) + corrected
            inverse = torch.where(l_next == 0.0, torch.ones_like(l_next), 1.0 / l_next)
            contribution = torch.matmul(p.to(pdt).to(F32), vf[:, :, start:start + chunk])
            acc_next = acc * (corrected * inverse) + contribution * inverse
            acc = torch.where(visit, acc_next, acc)
            m = torch.where(visit, m_next, m)
            l = torch.where(visit, l_next, l)  # noqa: E741
    return acc.to(q.dtype), (torch.log(l) + m)[..., 0]


def attention_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    do: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    segment_ids: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """dQ, dK, dV as the reference's two backward kernels compute them.

    * Delta = rowsum(float32(O) * float32(dO))          (``:532-535``)
    * P = exp(scale*QK^T - LSE), zero where masked       (``:556-560``)
    * dP = dO V^T (float32)                               (``:561-566``)
    * dS = (dP - Delta) * P * scale                       (``:567-568``)
    * dQ = bf16(dS) K,  dK = bf16(dS)^T Q,  dV = bf16(P)^T dO   (``:569-573,680-698``)

    Accumulation is float32; the results are rounded to the input dtype.
    """

    scale = float(q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale)
    cdt = q.dtype
    delta = (o.to(F32) * do.to(F32)).sum(-1, keepdim=True)
    scores = _scores(q, k, scale)
    visible = visibility(q.shape[2], segment_ids)
    p = torch.where(visible, torch.exp(scores - lse[..., None]), torch.zeros((), dtype=F32))
    dp = torch.matmul(do.to(F32), v.to(F32).transpose(-1, -2))
    ds = (dp - delta) * p * scale
    ds_c = ds.to(cdt).to(F32)
    p_c = p.to(cdt).to(F32)
    dq = torch.matmul(ds_c, k.to(F32)).to(cdt)
    dk = torch.matmul(ds_c.transpose(-1, -2), q.to(F32)).to(cdt)
    dv = torch.matmul(p_c.transpose(-1, -2), do.to(F32)).to(cdt)
    return dq, dk, dv


def document_segments(tokens: torch.Tensor, boundary_token: int) -> torch.Tensor:
    """``document_segments`` (``rig/attention.py:205-208``)."""

    return torch.cumsum((tokens == boundary_token).to(torch.int32), dim=1).to(torch.int32)


def attention_softmax_scale(rule: str, head_dim: int) -> float:
    """``attention_softmax_scale`` (``rig/attention.py:55-62``)."""

    if rule == "inverse_head_dim":
        return 1.0 / float(head_dim)
    if rule == "inverse_sqrt_head_dim":
        return head_dim ** -0.5
    raise ValueError(f"unsupported attention scale {rule!r}")


class DenseAttention(torch.autograd.Function):
    """The training step's attention: the Pallas kernel's forward numerics
    (:func:`flash_attention_forward`) and its custom-VJP backward formulas."""

    @staticmethod
    def forward(ctx, q, k, v, scale, segment_ids):
        o, lse = flash_attention_forward(q, k, v, softmax_scale=scale, segment_ids=segment_ids)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale
        ctx.segment_ids = segment_ids
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = attention_backward(
            q, k, v, o, lse, do.contiguous(), softmax_scale=ctx.scale, segment_ids=ctx.segment_ids
        )
        return dq, dk, dv, None, None
