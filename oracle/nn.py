"""Model primitives restated from ``rig/nn.py`` and ``recipes/reference/train.py``.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math

import numpy as np
import torch

BF16 = torch.bfloat16
F32 = torch.float32


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """Round to bfloat16 (round-to-nearest-even) and return float32."""

    return x.to(BF16).to(F32)


def normal(rng: np.random.Generator, shape: tuple[int, ...], scale: float) -> np.ndarray:
    """``rig/nn.py:20-23``: float32 standard normal times a float32 scale."""

    return rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)


def rms_norm(x: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``rig/nn.py:26-33``.

    The statistic is float32 mean of squares plus 1e-5; the normalised value is
    cast to ``dtype`` *before* the multiply by ``scale.astype(dtype)`` (so in
    bfloat16 there are two roundings: the normalised value and the product).
    """

    x32 = x.to(F32)
    normalized = x32 * torch.rsqrt((x32 * x32).mean(dim=-1, keepdim=True) + 1.0e-5)
    return normalized.to(dtype) * scale.to(dtype)


def rotary_tables(length: int, head_dim: int, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Cosine/sine tables of ``rig/nn.py:43-47`` cast to ``dtype``: ``[S, D/2]``."""

    if head_dim % 2:
        raise ValueError("rotary attention requires an even head dimension")
    fraction = torch.arange(0, head_dim, 2, dtype=F32) / float(head_dim)
    inverse_frequency = torch.pow(torch.tensor(10000.0, dtype=F32), -fraction)
    angle = torch.arange(length, dtype=F32)[:, None] * inverse_frequency[None, :]
    return torch.cos(angle).to(dtype), torch.sin(angle).to(dtype)


def apply_rotary(x: torch.Tensor) -> torch.Tensor:
    """``rig/nn.py:36-52``: interleaved base-10,000 RoPE on a BTHD tensor.

    Pairs are (even, odd) lanes of the head dimension; the result is
    ``(e*c - o*s, e*s + o*c)`` re-interleaved.  cos/sin are rounded to
    ``x.dtype``.  The pair arithmetic is evaluated in float32 and rounded once
    (XLA-CPU's default excess precision inside one fusion); whether XLA rounds
    the two products individually is not pinnable without jax.
    """

    length, head_dim = x.shape[1], x.shape[-1]
    cosine, sine = rotary_tables(length, head_dim, x.dtype)
    c = cosine.to(F32)[None, :, None, :]
    s = sine.to(F32)[None, :, None, :]
    x32 = x.to(F32)
    even, odd = x32[..., 0::2], x32[..., 1::2]
    out = torch.stack((even * c - odd * s, even * s + odd * c), dim=-1)
    return out.reshape(x.shape).to(x.dtype)


def apply_rotary_backward(dy: torch.Tensor) -> torch.Tensor:
    """Transpose of :func:`apply_rotary` (rotation by the negative angle)."""

    length, head_dim = dy.shape[1], dy.shape[-1]
    cosine, sine = rotary_tables(length, head_dim, dy.dtype)
    c = cosine.to(F32)[None, :, None, :]
    s = sine.to(F32)[None, :, None, :]
    g = dy.to(F32)
    ge, go = g[..., 0::2], g[..., 1::2]
    out = torch.stack((ge * c + go * s, -ge * s + go * c), dim=-1)
    return out.reshape(dy.shape).to(dy.dtype)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``rig/nn.py:55-56``: ``einsum(x, W.astype(dtype)) + b.astype(dtype)``.

    With bfloat16 operands the product is accumulated in float32 and rounded to
    bfloat16, then the bias add rounds again.
    """

    y = torch.matmul(x.to(F32), weight.to(dtype).to(F32)).to(dtype)
    return y + bias.to(dtype)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """``jax.nn.gelu(approximate=True)`` as used at ``train.py:1171``.

    0.5*x*(1 + tanh(sqrt(2/pi)*(x + 0.044715*x^3))) in float32, rounded once
    to the input dtype.
    """

    x32 = x.to(F32)
    inner = math.sqrt(2.0 / math.pi) * (x32 + 0.044715 * x32 * x32 * x32)
    return (0.5 * x32 * (1.0 + torch.tanh(inner))).to(x.dtype)


def gelu_tanh_grad(x: torch.Tensor) -> torch.Tensor:
    """d/dx of :func:`gelu_tanh` in float32 (closed form)."""

    x32 = x.to(F32)
    k = math.sqrt(2.0 / math.pi)
    inner = k * (x32 + 0.044715 * x32 ** 3)
    t = torch.tanh(inner)
    return 0.5 * (1.0 + t) + 0.5 * x32 * (1.0 - t * t) * k * (1.0 + 3.0 * 0.044715 * x32 * x32)


def parameter_count(params) -> int:
    """``rig/nn.py:59-60``."""

    total = 0
    stack = [params]
    while stack:
        item = stack.pop()
        if isinstance(item, dict):
            stack.extend(item.values())
        elif isinstance(item, (list, tuple)):
            stack.extend(item)
        else:
            total += int(np.asarray(item).size) if not isinstance(item, torch.Tensor) else item.numel()
    return total
