"""AdamW, learning-rate schedule and per-tensor multipliers restated from
``recipes/reference/train.py:1219-1457``.

Test infrastructure only (see ``oracle/__init__.py``).  Parameters are a flat
``{path: float32 tensor}`` mapping whose keys end in the reference leaf names
(``token_embedding``, ``blocks/3/qkv_w``, ...).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .nn import F32


@dataclass(frozen=True)
class OptimizerConfig:
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


def learning_rate(step: int, cfg: OptimizerConfig) -> float:
    """``learning_rate`` (``train.py:1219-1236``), evaluated in float32."""

    f = lambda value: float(torch.tensor(value, dtype=F32))  # noqa: E731
    step_float = f(step)
    warmup = min(1.0, f(step_float / float(cfg.warmup_steps))) if cfg.warmup_steps else 1.0
    decay_span = max(1, cfg.steps - cfg.warmup_steps)
    progress = min(max(f((step_float - float(cfg.warmup_steps)) / float(decay_span)), 0.0), 1.0)
    cosine = f(0.5 * (1.0 + f(math.cos(f(math.pi * progress)))))
    multiplier = f(cfg.min_lr_ratio + (1.0 - cfg.min_lr_ratio) * cosine)
    horizon = math.sqrt(cfg.batch_multiplier / cfg.data_multiplier)
    return f(f(f(cfg.learning_rate * horizon) * warmup) * multiplier)


def leaf_name(path: str) -> str:
    return path.rsplit("/", 1)[-1]


def decays(path: str) -> bool:
    """``weight_decay_mask`` (``train.py:1252-1271``): by role, never by rank."""

    name = leaf_name(path)
    if name in {"token_embedding", "output_embedding"} or name.endswith("_w"):
        return True
    if name.endswith(("_b", "_bias", "_scale")):
        return False
    raise ValueError(f"weight-decay policy has no rule for parameter {name!r}")


def multipliers(path: str, parameterization: str, width: float = 1.0, depth: float = 1.0,
                alpha: float = 0.0) -> tuple[float, float, float]:
    """(lr, epsilon, decay) multipliers of ``optimizer_hyperparameter_trees``
    (``train.py:1274-1333``)."""

    if parameterization != "completep_fixed_tpp_v1":
        return 1.0, 1.0, 1.0
    name = leaf_name(path)
    if path.startswith("blocks/"):
        lr = width ** -1 * depth ** (alpha - 1.0) if name.endswith("_w") else depth ** (alpha - 1.0)
        eps = width ** -1 * depth ** -alpha
        dec = width if name.endswith("_w") else 1.0
        return lr, eps, dec
    if name == "token_embedding":
        return 1.0, width ** -1, 1.0
    if name == "output_embedding":
        return width ** -1, 1.0, width
    if name == "final_ln_scale":
        return 1.0, 1.0, 1.0
    raise ValueError(f"no multiplier rule for {path!r}")


def effective_adam_betas(cfg: OptimizerConfig) -> tuple[float, float]:
    """``effective_adam_betas`` (``train.py:1336-1345``)."""

    ratio = cfg.batch_multiplier / cfg.data_multiplier
    beta1 = 1.0 - (1.0 - cfg.beta1) * ratio
    beta2 = 1.0 - (1.0 - cfg.beta2) * ratio
    if not 0.0 <= beta1 < 1.0 or not 0.0 <= beta2 < 1.0:
        raise ValueError("fixed-TPP batch/data scaling produced invalid Adam momenta")
    return beta1, beta2


def adamw_step(params: dict, grads: dict, m: dict, v: dict, step: int, cfg: OptimizerConfig,
               parameterization: str = "standard", width: float = 1.0, depth: float = 1.0,
               alpha: float = 0.0) -> tuple[float, float]:
    """One update, in place (``_apply_training_update``, ``train.py:1386-1445``).

    ``step`` is the new (1-based) step.  Returns ``(lr, grad_norm)``.
    """

    beta1, beta2 = effective_adam_betas(cfg)
    grad_norm = math.sqrt(sum(float((g.to(torch.float64) ** 2).sum()) for g in grads.values()))
    clip = min(1.0, cfg.grad_clip / (grad_norm + 1.0e-6)) if cfg.grad_clip > 0.0 else 1.0
    lr = learning_rate(step, cfg)
    bc1 = 1.0 - beta1 ** float(step)
    bc2 = 1.0 - beta2 ** float(step)
    eps_h = math.sqrt(cfg.data_multiplier / cfg.batch_multiplier)
    dec_h = math.sqrt(cfg.batch_multiplier / cfg.data_multiplier)
    for path, p in params.items():
        g = grads[path].to(F32) * clip
        m[path].mul_(beta1).add_((1.0 - beta1) * g)
        v[path].mul_(beta2).add_((1.0 - beta2) * g * g)
        lr_mult, eps_mult, dec_mult = multipliers(path, parameterization, width, depth, alpha)
        eps = cfg.adam_epsilon * eps_h * eps_mult
        adam = (m[path] / bc1) / (torch.sqrt(v[path] / bc2) + eps)
        decay = cfg.weight_decay * dec_h * dec_mult * p if decays(path) else 0.0
        p.sub_(lr * lr_mult * (adam + decay))
    return lr, grad_norm
