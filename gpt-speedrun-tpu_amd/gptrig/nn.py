"""Model primitives on gfx950, mirroring ``rig/nn.py``.

``rms_norm``, ``apply_rotary`` and ``gelu`` run the HIP kernels of
``csrc/elementwise.hip`` with hand-written backward passes; ``linear`` is a
plain library GEMM (hipBLASLt through torch) with the reference's bf16
rounding points.
"""

from __future__ import annotations

from typing import Any, Mapping

import numpy as np
import torch

from . import _lib

BF16 = torch.bfloat16


def normal(rng: np.random.Generator, shape: tuple[int, ...], scale: float) -> np.ndarray:
    """``rig/nn.py:20-23``: float32 standard normal times a float32 scale."""

    return rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)


def _rows(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1]).contiguous()


def rmsnorm_forward(x2: torch.Tensor, scale_bf16: torch.Tensor, out: torch.Tensor | None = None):
    rows, d = x2.shape
    y = torch.empty_like(x2) if out is None else out
    rstd = torch.empty(rows, dtype=torch.float32, device=x2.device)
    _lib.call("gptrig_rmsnorm_fwd", x2.data_ptr(), scale_bf16.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, d,
              _lib.stream())
    return y, rstd


def add_rmsnorm_forward(x2: torch.Tensor, branch: torch.Tensor, branch_scale: float, scale_bf16: torch.Tensor,
                        sum_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
                        branch_bias: torch.Tensor | None = None):
    """``s = x + bf16(branch * branch_scale)`` then ``rms_norm(s)``: the block's
    residual add and the norm after it in one pass.  Returns ``(s, y, rstd)``.

    ``branch_bias`` (bf16 ``[d]``): ``branch`` is a linear's bf16 GEMM output
    without its bias, which is added here with its own rounding
    (``rig/nn.py:55-56``) before the residual add."""

    rows, d = x2.shape
    s = torch.empty_like(x2) if sum_out is None else sum_out
    y = torch.empty_like(x2) if out is None else out
    rstd = torch.empty(rows, dtype=torch.float32, device=x2.device)
    _lib.call("gptrig_add_bias_rmsnorm_fwd", x2.data_ptr(), branch.data_ptr(), _lib.ptr(branch_bias),
              float(branch_scale), scale_bf16.data_ptr(), s.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, d,
              _lib.stream())
    return s, y, rstd


def rmsnorm_backward(dy2, x2, scale_bf16, rstd, dscale: torch.Tensor | None = None, accumulate: bool = False,
                     dresidual: torch.Tensor | None = None, out: torch.Tensor | None = None):
    rows, d = x2.shape
    dx = torch.empty_like(x2) if out is None else out
    if dscale is None:
        dscale = torch.empty(d, dtype=torch.float32, device=x2.device)
        accumulate = False
    ws = _lib.workspace(_lib.query("gptrig_rmsnorm_bwd_workspace_bytes", rows, d), x2.device)
    _lib.call("gptrig_rmsnorm_bwd", dy2.data_ptr(), x2.data_ptr(), scale_bf16.data_ptr(), rstd.data_ptr(),
              _lib.ptr(dresidual), dx.data_ptr(), dscale.data_ptr(), int(accumulate), ws.data_ptr(), ws.numel(),
              rows, d, _lib.stream())
    return dx, dscale


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scale):
        x2 = _rows(x)
        s = scale.to(BF16).contiguous()
        y, rstd = rmsnorm_forward(x2, s)
        ctx.save_for_backward(x2, s, rstd)
        ctx.meta = (x.shape, scale.dtype)
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, s, rstd = ctx.saved_tensors
        shape, sdtype = ctx.meta
        dx, dscale = rmsnorm_backward(_rows(dy.to(BF16)), x2, s, rstd)
        return dx.reshape(shape), dscale.to(sdtype)


def rms_norm(x: torch.Tensor, scale: torch.Tensor, dtype: Any = BF16) -> torch.Tensor:
    """``rig/nn.py:26-33``: ``bf16(bf16(x*rsqrt(mean(x^2)+1e-5)) * bf16(scale))``."""

    if dtype != BF16 or x.dtype != BF16:
        raise TypeError("the HIP rms_norm computes bfloat16 activations")
    _lib.require_device(x, scale)
    return _RMSNorm.apply(x, scale)


_ROPE_TABLES: dict = {}


def rope_tables(seq: int, head_dim: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 cos/sin ``[seq, head_dim/2]`` built on the device (``rig/nn.py:43-47``)."""

    key = (seq, head_dim, str(device))
    if key not in _ROPE_TABLES:
        c = torch.empty((seq, head_dim // 2), dtype=BF16, device=device)
        s = torch.empty_like(c)
        _lib.call("gptrig_rope_table", c.data_ptr(), s.data_ptr(), seq, head_dim, _lib.stream())
        _ROPE_TABLES[key] = (c, s)
    return _ROPE_TABLES[key]


def rope_inplace(buf: torch.Tensor, row_stride: int, rows: int, seq: int, heads: int, head_dim: int,
                 backward: bool = False) -> None:
    c, s = rope_tables(seq, head_dim, buf.device)
    _lib.call("gptrig_rope_bwd" if backward else "gptrig_rope_fwd", buf.data_ptr(), int(row_stride), rows, seq,
              heads, head_dim, c.data_ptr(), s.data_ptr(), _lib.stream())


def bias_rope_inplace(buf: torch.Tensor, bias: torch.Tensor, seq: int, heads: int, head_dim: int) -> None:
    """In place on a ``[rows, cols]`` bf16 projection output without its bias:
    every column gets ``bf16(x + bias)`` (``rig/nn.py:55-56``), then the first
    ``heads * head_dim`` columns are rotated (``rig/nn.py:36-52``)."""

    rows, cols = buf.shape
    c, s = rope_tables(seq, head_dim, buf.device)
    _lib.call("gptrig_bias_rope_fwd", buf.data_ptr(), int(buf.stride(0)), rows, cols, bias.data_ptr(), seq, heads,
              head_dim, c.data_ptr(), s.data_ptr(), _lib.stream())


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        B, S, H, D = x.shape
        y = x.contiguous().clone()
        rope_inplace(y, H * D, B * S, S, H, D)
        return y

    @staticmethod
    def backward(ctx, dy):
        B, S, H, D = dy.shape
        g = dy.to(BF16).contiguous().clone()
        rope_inplace(g, H * D, B * S, S, H, D, backward=True)
        return g


def apply_rotary(x: torch.Tensor) -> torch.Tensor:
    """``rig/nn.py:36-52``: interleaved base-10,000 RoPE on a BTHD tensor."""

    if x.shape[-1] % 2:
        raise ValueError("rotary attention requires an even head dimension")
    if x.dtype != BF16:
        raise TypeError("the HIP rotary kernel takes bfloat16")
    if x.shape[-1] % 8:
        raise ValueError("the HIP rotary kernel needs head_dim % 8 == 0")
    _lib.require_device(x)
    return _Rotary.apply(x)


class _Gelu(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        xc = x.contiguous()
        y = torch.empty_like(xc)
        _lib.call("gptrig_gelu_fwd", xc.data_ptr(), y.data_ptr(), xc.numel(), _lib.stream())
        ctx.save_for_backward(xc)
        return y

    @staticmethod
    def backward(ctx, dy):
        (xc,) = ctx.saved_tensors
        g = dy.to(BF16).contiguous()
        dx = torch.empty_like(xc)
        _lib.call("gptrig_gelu_bwd", g.data_ptr(), xc.data_ptr(), dx.data_ptr(), xc.numel(), _lib.stream())
        return dx


def gelu(x: torch.Tensor) -> torch.Tensor:
    """``jax.nn.gelu(approximate=True)`` (``recipes/reference/train.py:1171``)."""

    if x.dtype != BF16:
        raise TypeError("the HIP gelu kernel takes bfloat16")
    _lib.require_device(x)
    return _Gelu.apply(x)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, dtype: Any = BF16) -> torch.Tensor:
    """``rig/nn.py:55-56``: ``x @ W.astype(dtype) + b.astype(dtype)`` (a plain
    library GEMM; bf16 product rounded, then the bf16 bias add)."""

    return torch.matmul(x.to(dtype), weight.to(dtype)) + bias.to(dtype)


def parameter_count(params: Any) -> int:
    """``rig/nn.py:59-60``."""

    if isinstance(params, Mapping):
        return sum(parameter_count(v) for v in params.values())
    if isinstance(params, (list, tuple)):
        return sum(parameter_count(v) for v in params)
    return int(params.numel() if isinstance(params, torch.Tensor) else np.asarray(params).size)
