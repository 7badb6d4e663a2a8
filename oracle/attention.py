"""Causal attention restated from ``rig/kernels/tpu_flash_attention.py``.

Test infrastructure only (see ``oracle/__init__.py``).

Layout is the reference's BHSD ``[batch, heads, sequence, head_dim]``.  Scores
are float32 (bf16 products are exact in float32, sums are float32), the mask
adds ``-0.7 * float32_max`` (``tpu_flash_attention.py:71,311-319``),
probabilities are rounded to ``v.dtype`` before the PV product
(``:201``) and the output is rounded to ``q.dtype`` (``:202-207``).
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
    """Dense attention with the reference's custom-VJP backward formulas."""

    @staticmethod
    def forward(ctx, q, k, v, scale, segment_ids):
        o, lse = attention_forward(q, k, v, softmax_scale=scale, segment_ids=segment_ids)
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
