"""Causal flash attention on gfx950, mirroring ``rig/kernels/tpu_flash_attention.py``.

Same operator API as the reference: ``make_causal_attention(AttentionConfig)``
returns ``attention(q, k, v, segment_ids=None)`` over BHSD tensors, validated
before any launch (``_validate_qkv``, ``tpu_flash_attention.py:145-168``), with
the default scale ``head_dim ** -0.5`` (``:992-996``) and a custom backward
that saves ``(q, k, v, o, lse, segments)`` (``:1103-1159``).  ``backend="hip"``
(or ``"auto"``) runs the kernels of ``csrc/attention.hip``; sequences of any
length are handled in-kernel (keys past the end never exist), so no padding
to 128 is needed.  Head dims other than 64/128 (<= 128, multiple of 8) are
zero-padded to the next kernel size, which leaves scores unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Literal

import torch

from .. import _lib

Backend = Literal["auto", "hip"]
_KERNEL_DIMS = (64, 128)


@dataclass(frozen=True)
class AttentionTiles:
    """Tile plan of the HIP kernels.

    The tiles are fixed at compile time per head dim, so a plan describes
    the kernels rather than choosing among them (``kernel_tiles``).  Field
    names follow the reference's ``AttentionTilePlan``
    (``rig/kernels/autotune.py:84-157``); ``*_compute`` is the sub-tile one
    wave (one MFMA row block) handles.  The defaults are the head_dim 64 plan.
    """

    block_q: int = 128  # forward: queries per workgroup (4 waves x 32)
    block_kv: int = 64  # forward: keys per LDS tile
    block_kv_compute: int = 32  # forward: keys per online-softmax half-step
    block_q_dkv: int = 64  # backward: queries per step
    block_q_dkv_compute: int = 32
    block_kv_dkv: int = 256  # backward: keys per workgroup (8 waves x 32)
    block_kv_dkv_compute: int = 32
    block_q_dq: int = 64  # dQ is accumulated by the same (key-owned) workgroups
    block_kv_dq: int = 256
    block_kv_dq_compute: int = 32

    @property
    def has_backward_tiles(self) -> bool:
        return True

    def to_dict(self) -> dict:
        return dict(self.__dict__)


def kernel_tiles(head_dim: int) -> AttentionTiles:
    """The plan the kernels run for ``head_dim`` (padded up to 64 or 128):
    the head_dim 128 backward owns 128 keys per workgroup (4 waves x 32)."""

    if head_dim <= 0 or head_dim > _KERNEL_DIMS[-1]:
        raise ValueError(f"head_dim must be in (0, {_KERNEL_DIMS[-1]}]; got {head_dim}")
    if head_dim <= 64:
        return AttentionTiles()
    return AttentionTiles(block_kv_dkv=128, block_kv_dq=128)


def attention_tile_candidates(*, sequence: int, head_dim: int, training: bool = True) -> tuple[AttentionTiles, ...]:
    """The candidate list has one entry: the kernels' fixed plan."""

    return (kernel_tiles(head_dim),)


def select_attention_tiles(*, sequence: int, head_dim: int, training: bool = True) -> AttentionTiles:
    return kernel_tiles(head_dim)


@dataclass(frozen=True)
class AttentionConfig:
    """Static configuration (``tpu_flash_attention.py:75-97``)."""

    backend: Backend = "auto"
    tiles: AttentionTiles | None = None
    softmax_scale: float | None = None
    interpret: bool = False
    debug: bool = False

    def __post_init__(self) -> None:
        if self.backend not in ("auto", "hip"):
            # One backend only: the reference's "tpu_flash"/"jax_flash" are TPU
            # kernels and its dense "reference" oracle lives in the test oracle.
            raise ValueError(f"unknown attention backend: {self.backend!r}")
        if self.softmax_scale is not None and self.softmax_scale <= 0.0:
            raise ValueError("softmax_scale must be positive")
        if self.interpret:
            raise ValueError("interpret mode does not exist for the HIP backend")


def validate_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """``_validate_qkv`` (``tpu_flash_attention.py:145-168``)."""

    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError(
            f"q, k, and v must use BHSD rank-4 layout; got {tuple(q.shape)}, {tuple(k.shape)}, and {tuple(v.shape)}"
        )
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("dense causal self-attention requires identical q/k/v shapes")
    if not all(q.shape):
        raise ValueError(f"q/k/v dimensions must be nonzero, got {tuple(q.shape)}")
    if q.shape[-1] > 128 or q.shape[-1] % 8:
        raise ValueError(f"the kernel requires head_dim <= 128 and divisible by 8; got {q.shape[-1]}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError(f"q, k, and v dtypes must match; got {q.dtype}, {k.dtype}, {v.dtype}")
    if not q.dtype.is_floating_point:
        raise TypeError(f"q, k, and v must be floating point, got {q.dtype}")


def _kernel_view(t: torch.Tensor) -> torch.Tensor:
    """A BHSD view the kernel accepts: unit last stride, 8-element strides, 16-byte base."""

    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _strides(*ts: torch.Tensor) -> torch.Tensor:
    flat = []
    for t in ts:
        flat.extend(t.stride()[:3])
    return torch.tensor(flat, dtype=torch.int64)


def flash_forward(q, k, v, segment_ids, scale: float):
    """O (bf16, contiguous BHSD) and LSE (f32 [B,H,S]) from the HIP kernel."""

    B, H, S, D = q.shape
    q, k, v = (_kernel_view(t) for t in (q, k, v))
    o = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    st = _strides(q, k, v, o)
    _lib.call("gptrig_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(segment_ids), o.data_ptr(),
              lse.data_ptr(), B, H, S, D, st.data_ptr(), float(scale), _lib.stream())
    return o, lse


def flash_backward(q, k, v, o, lse, do, segment_ids, scale: float):
    B, H, S, D = q.shape
    q, k, v, o, do = (_kernel_view(t) for t in (q, k, v, o, do))
    dq = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    ws = _lib.workspace(_lib.query("gptrig_attn_bwd_workspace_bytes", B, H, S, D), q.device)
    st = _strides(q, k, v, o, do, dq, dk, dv)
    _lib.call("gptrig_attn_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
              lse.data_ptr(), _lib.ptr(segment_ids), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
              ws.numel(), B, H, S, D, st.data_ptr(), float(scale), _lib.stream())
    return dq, dk, dv


class _FlashAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, segment_ids, scale):
        o, lse = flash_forward(q, k, v, segment_ids, scale)
        ctx.save_for_backward(q, k, v, o, lse, segment_ids)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, segment_ids = ctx.saved_tensors
        dq, dk, dv = flash_backward(q, k, v, o, lse, do, segment_ids, ctx.scale)
        # No cotangent for the segment index: it is data (tpu_flash_attention.py:1159).
        return dq, dk, dv, None, None


def _pad_head_dim(t: torch.Tensor, width: int) -> torch.Tensor:
    return torch.nn.functional.pad(t, (0, width - t.shape[-1]))


def make_causal_attention(config: AttentionConfig = AttentionConfig()) -> Callable:
    """``make_causal_attention`` (``tpu_flash_attention.py:962-1164``)."""

    def attention(q, k, v, segment_ids=None):
        validate_qkv(q, k, v)
        if config.tiles is not None and config.tiles != kernel_tiles(q.shape[-1]):
            raise ValueError(f"the HIP kernels run one fixed tile plan per head dim "
                             f"({kernel_tiles(q.shape[-1])}); got {config.tiles}")
        scale = float(q.shape[-1] ** -0.5 if config.softmax_scale is None else config.softmax_scale)
        if q.dtype != torch.bfloat16:
            raise TypeError(f"the HIP flash kernel supports bfloat16 q/k/v; got {q.dtype}")
        _lib.require_device(q, k, v, segment_ids)
        if segment_ids is not None:
            if tuple(segment_ids.shape) != (q.shape[0], q.shape[2]):
                raise ValueError(f"segment_ids must be [batch, sequence]; got {tuple(segment_ids.shape)}")
            segment_ids = segment_ids.to(torch.int32).contiguous()
        D = q.shape[-1]
        width = next(w for w in _KERNEL_DIMS if w >= D)
        if width != D:
            q, k, v = (_pad_head_dim(t, width) for t in (q, k, v))
            return _FlashAttention.apply(q, k, v, segment_ids, scale)[..., :D]
        return _FlashAttention.apply(q, k, v, segment_ids, scale)

    return attention


def causal_attention(q, k, v, *, config: AttentionConfig = AttentionConfig()):
    """Convenience wrapper around :func:`make_causal_attention`."""

    return make_causal_attention(config)(q, k, v)
