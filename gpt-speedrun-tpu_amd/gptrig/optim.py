"""Optimizer schedule and per-tensor AdamW hyper-parameters, mirroring
``recipes/reference/train.py:1219-1345``.

The update itself is the fused ``gptrig_adamw`` kernel; this module resolves
the host-side scalars (learning rate per step, bias corrections) and the
per-tensor table ``{lr_mult, epsilon, decay}`` the kernel reads.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class OptimizerConfig:
    """``run.optimizer`` of ``recipes/reference/config.yaml:98-108``."""

    learning_rate: float = 2.0 ** -8
    min_lr_ratio: float = 0.1
    warmup_steps: int = 0
    steps: int = 1
    weight_decay: float = 0.1
    adam_epsilon: float = 1.0e-8
    beta1: float = 0.9
    beta2: float = 0.95
    grad_clip: float = 0.0
    batch_multiplier: float = 1.0
    data_multiplier: float = 1.0


def _f32(x: float) -> float:
    return float(np.float32(x))


def learning_rate(step: int, cfg: OptimizerConfig) -> float:
    """``learning_rate`` (``train.py:1219-1236``) with float32 arithmetic."""

    s = _f32(step)
    warmup = min(1.0, _f32(s / float(cfg.warmup_steps))) if cfg.warmup_steps else 1.0
    span = max(1, cfg.steps - cfg.warmup_steps)
    progress = min(max(_f32((s - float(cfg.warmup_steps)) / float(span)), 0.0), 1.0)
    cosine = _f32(0.5 * (1.0 + _f32(math.cos(_f32(math.pi * progress)))))
    mult = _f32(cfg.min_lr_ratio + (1.0 - cfg.min_lr_ratio) * cosine)
    horizon = math.sqrt(cfg.batch_multiplier / cfg.data_multiplier)
    return _f32(_f32(_f32(cfg.learning_rate * horizon) * warmup) * mult)


def effective_adam_betas(cfg: OptimizerConfig) -> tuple[float, float]:
    """``effective_adam_betas`` (``train.py:1336-1345``)."""

    ratio = cfg.batch_multiplier / cfg.data_multiplier
    beta1 = 1.0 - (1.0 - cfg.beta1) * ratio
    beta2 = 1.0 - (1.0 - cfg.beta2) * ratio
    if not 0.0 <= beta1 < 1.0 or not 0.0 <= beta2 < 1.0:
        raise ValueError("fixed-TPP batch/data scaling produced invalid Adam momenta; use a closer transfer base")
    return beta1, beta2


def decays(path: str) -> bool:
    """``weight_decay_mask`` (``train.py:1252-1271``): decided by role name."""

    name = path.rsplit("/", 1)[-1]
    if name in {"token_embedding", "output_embedding"} or name.endswith("_w"):
        return True
    if name.endswith(("_b", "_bias", "_scale")):
        return False
    raise ValueError(f"weight-decay policy has no rule for parameter {name!r}")


def multipliers(path: str, parameterization: str, width: float, depth: float, alpha: float):
    """(lr, epsilon, decay) multipliers of ``optimizer_hyperparameter_trees``
    (``train.py:1274-1333``)."""

    if parameterization != "completep_fixed_tpp_v1":
        return 1.0, 1.0, 1.0
    name = path.rsplit("/", 1)[-1]
    if path.startswith("blocks/"):
        is_w = name.endswith("_w")
        lr = width ** -1 * depth ** (alpha - 1.0) if is_w else depth ** (alpha - 1.0)
        return lr, width ** -1 * depth ** -alpha, (width if is_w else 1.0)
    if name == "token_embedding":
        return 1.0, width ** -1, 1.0
    if name == "output_embedding":
        return width ** -1, 1.0, width
    if name == "final_ln_scale":
        return 1.0, 1.0, 1.0
    raise ValueError(f"no multiplier rule for {path!r}")


def tensor_hparams(paths, cfg: OptimizerConfig, parameterization: str, width: float, depth: float,
                   alpha: float) -> np.ndarray:
    """``[T, 3]`` float32 table of (lr_mult, epsilon, decay) per tensor
    (``train.py:1420-1435``)."""

    eps_h = math.sqrt(cfg.data_multiplier / cfg.batch_multiplier)
    dec_h = math.sqrt(cfg.batch_multiplier / cfg.data_multiplier)
    rows = []
    for path in paths:
        lr_m, eps_m, dec_m = multipliers(path, parameterization, width, depth, alpha)
        eps = cfg.adam_epsilon * eps_h * eps_m
        decay = cfg.weight_decay * dec_h * dec_m if decays(path) else 0.0
        rows.append((lr_m, eps, decay))
    return np.asarray(rows, dtype=np.float32)
