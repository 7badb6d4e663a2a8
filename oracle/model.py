"""GPT training step restated from ``recipes/reference/train.py``.

Test infrastructure only (see ``oracle/__init__.py``).

torch-CPU autograd stands in for ``jax.value_and_grad``; attention and the
tiled loss use the reference's custom-VJP formulas (``oracle.attention``,
``oracle.flce``).  Parameters are float32 and cast to the compute dtype at
use (``train.py:1107``, ``rig/nn.py:55-56``), so their gradients are float32
conversions of compute-dtype cotangents, as in the reference.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import numpy as np
import torch

from . import attention as oattn
from . import flce as oflce
from . import moe as omoe
from . import optim as ooptim
from .nn import F32, apply_rotary, gelu_tanh, linear, normal, rms_norm

BLOCK_LEAVES = (
    "ln1_scale", "qkv_w", "qkv_b", "attn_w", "attn_b",
    "ln2_scale", "mlp_up_w", "mlp_up_b", "mlp_down_w", "mlp_down_b",
)
# Routed blocks (recipes/reference_moe/train.py:914-944): the MLP leaves are
# replaced by the router and the stacked experts.
MOE_BLOCK_LEAVES = (
    "ln1_scale", "qkv_w", "qkv_b", "attn_w", "attn_b",
    "ln2_scale", "router_w", "expert_up_w", "expert_up_b", "expert_down_w", "expert_down_b",
)


@dataclass(frozen=True)
class Config:
    """The fields of the reference ``Config`` (``train.py:176-282``) the step reads."""

    layers: int = 2
    heads: int = 2
    d_model: int = 64
    mlp_mult: int = 4
    vocab_size: int = 256
    semantic_vocab_size: int = 256
    seq_len: int = 32
    batch_size: int = 4
    parameterization: str = "standard"
    base_width: int = 64
    base_depth: int = 2
    depth_alpha: float = 0.0
    init_std: float = 0.02
    attention_scale: str = "inverse_sqrt_head_dim"
    embeddings: str = "tied"
    dtype: torch.dtype = torch.bfloat16
    attention_backend: str = "flash"   # "flash" (kernel semantics) or "dense" (train.py:1151-1162)
    loss_backend: str = "tiled"
    vocab_tile_size: int = 2048
    document_masking: bool = False
    document_boundary_token: int = 50256
    experts: int = 0                   # reference_moe/train.py:242-245
    expert_top_k: int = 2
    expert_mult: int = 2
    router_aux_coefficient: float = 0.01
    optimizer: ooptim.OptimizerConfig = field(default_factory=ooptim.OptimizerConfig)

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads

    @property
    def width_multiplier(self) -> float:
        return self.d_model / float(self.base_width)

    @property
    def depth_multiplier(self) -> float:
        return self.layers / float(self.base_depth)

    @property
    def softmax_scale(self) -> float:
        return oattn.attention_softmax_scale(self.attention_scale, self.head_dim)


def tpp_parameters(layers: int, d_model: int, vocab_size: int) -> int:
    """``TierDefinition.tpp_parameters`` (``train.py:354-365``)."""

    return 2 * vocab_size * d_model + layers * (12 * d_model * d_model + 11 * d_model) + d_model


def warmup_steps(steps: int, warmup_ratio: float) -> int:
    """Warmup resolution of ``resolve_config`` (``train.py:807-811``)."""

    warm = int(math.floor(steps * warmup_ratio + 0.5))
    return min(warm, steps - 1) if steps > 1 else 0


def smoke_config() -> Config:
    """``recipes/reference/smoke.yaml`` with the bf16 kernel dtype."""

    return Config(optimizer=ooptim.OptimizerConfig(learning_rate=3e-4, steps=2, warmup_steps=0))


def baseline_config(name: str, steps: int = 20) -> Config:
    """Model/optimizer fields of the benchmark configurations: "A" (8L d512, CPU-runnable) and "D" (12L d768, 125M)."""

    opt = ooptim.OptimizerConfig(learning_rate=2.0 ** -8, steps=steps, warmup_steps=warmup_steps(steps, 0.1))
    if name == "A":
        return Config(layers=8, heads=8, d_model=512, vocab_size=50304, semantic_vocab_size=50304,
                      seq_len=1024, batch_size=8, base_width=512, base_depth=8,
                      attention_scale="inverse_sqrt_head_dim", embeddings="untied", optimizer=opt)
    if name == "D":
        return Config(layers=12, heads=12, d_model=768, vocab_size=50304, semantic_vocab_size=50304,
                      seq_len=1024, batch_size=128, base_width=768, base_depth=12,
                      attention_scale="inverse_sqrt_head_dim", embeddings="untied", optimizer=opt)
    raise ValueError(name)


def init_params(config: Config, seed: int) -> dict:
    """``init_params`` (``train.py:865-901``): numpy PCG64, fixed leaf order."""

    rng = np.random.default_rng(seed)
    d = config.d_model
    hidden = config.mlp_mult * d
    hidden_scale = (config.init_std / math.sqrt(config.width_multiplier)
                    if config.parameterization == "completep_fixed_tpp_v1" else 0.02)
    blocks = []
    for _ in range(config.layers):
        block = {
            "ln1_scale": np.ones((d,), np.float32),
            "qkv_w": normal(rng, (d, 3 * d), hidden_scale),
            "qkv_b": np.zeros((3 * d,), np.float32),
            "attn_w": normal(rng, (d, d), hidden_scale),
            "attn_b": np.zeros((d,), np.float32),
            "ln2_scale": np.ones((d,), np.float32),
        }
        if config.experts:
            # reference_moe/train.py:894-944: router, then the stacked experts.
            E, eh = config.experts, config.expert_mult * d
            block["router_w"] = normal(rng, (d, E), hidden_scale)
            block["expert_up_w"] = normal(rng, (E, d, eh), hidden_scale)
            block["expert_up_b"] = np.zeros((E, eh), np.float32)
            block["expert_down_w"] = normal(rng, (E, eh, d), hidden_scale)
            block["expert_down_b"] = np.zeros((E, d), np.float32)
        else:
            block["mlp_up_w"] = normal(rng, (d, hidden), hidden_scale)
            block["mlp_up_b"] = np.zeros((hidden,), np.float32)
            block["mlp_down_w"] = normal(rng, (hidden, d), hidden_scale)
            block["mlp_down_b"] = np.zeros((d,), np.float32)
        blocks.append(block)
    result = {
        "token_embedding": normal(rng, (config.vocab_size, d), config.init_std),
        "blocks": blocks,
        "final_ln_scale": np.ones((d,), np.float32),
    }
    if config.embeddings == "untied":
        result["output_embedding"] = normal(rng, (config.vocab_size, d), config.init_std / config.width_multiplier)
    return result


def flatten(params: dict) -> dict:
    """``{path: array}`` with paths like ``blocks/0/qkv_w`` (reference leaf names)."""

    flat = {}
    for key, value in params.items():
        if key == "blocks":
            for i, block in enumerate(value):
                for name in block:  # the reference's leaf order
                    flat[f"blocks/{i}/{name}"] = block[name]
        else:
            flat[key] = value
    return flat


def gpt_hidden(p: dict, tokens: torch.Tensor, config: Config) -> torch.Tensor:
    """``gpt_hidden`` (``train.py:1096-1176``) over flat float32 params."""

    return gpt_hidden_and_router(p, tokens, config)[0]


def gpt_hidden_and_router(p: dict, tokens: torch.Tensor, config: Config):
    """``gpt_hidden`` (``train.py:1096-1176``; routed blocks:
    ``reference_moe/train.py:1374-1491``) over flat float32 params.

    Returns ``(hidden, balance_loss, loads)``: for a routed model the mean over
    layers of ``load_balance_loss`` and the per-layer ``[layers, experts]``
    load; ``(hidden, None, None)`` for a dense one.
    """

    dtype = config.dtype
    batch, length = tokens.shape
    hd = config.head_dim
    x = p["token_embedding"][tokens.to(torch.int64)].to(dtype)
    segments = (oattn.document_segments(tokens, config.document_boundary_token)
                if config.document_masking else None)
    residual_scale = config.depth_multiplier ** (-config.depth_alpha)
    scale = config.softmax_scale
    balance, loads = [], []
    for i in range(config.layers):
        b = lambda name: p[f"blocks/{i}/{name}"]  # noqa: E731
        residual = x
        xn = rms_norm(x, b("ln1_scale"), dtype)
        qkv = linear(xn, b("qkv_w"), b("qkv_b"), dtype)
        q, k, v = torch.split(qkv, config.d_model, dim=-1)
        q = apply_rotary(q.reshape(batch, length, config.heads, hd))
        k = apply_rotary(k.reshape(batch, length, config.heads, hd))
        v = v.reshape(batch, length, config.heads, hd)
        qt, kt, vt = (t.permute(0, 2, 1, 3) for t in (q, k, v))
        if config.attention_backend == "dense":
            scores = torch.matmul(qt.to(F32), kt.to(F32).transpose(-1, -2)).to(dtype).to(F32) * scale
            visible = oattn.visibility(length, segments)
            scores = torch.where(visible, scores, torch.tensor(torch.finfo(F32).min))
            probs = torch.softmax(scores, dim=-1).to(dtype)
            att = torch.matmul(probs.to(F32), vt.to(F32)).to(dtype)
        else:
            att = oattn.DenseAttention.apply(qt, kt, vt, scale, segments)
        att = att.permute(0, 2, 1, 3).reshape(batch, length, config.d_model)
        out = linear(att, b("attn_w"), b("attn_b"), dtype)
        x = residual + (out if residual_scale == 1.0 else (residual_scale * out).to(dtype))
        residual = x
        xn = rms_norm(x, b("ln2_scale"), dtype)
        if config.experts:
            out, mean_probability, load, _, _, _ = omoe.routed_mlp_local(
                xn, b("router_w"), b("expert_up_w"), b("expert_up_b"), b("expert_down_w"), b("expert_down_b"),
                experts=config.experts, top_k_count=config.expert_top_k, dtype=dtype)
            balance.append(omoe.load_balance_loss(mean_probability, load))
            loads.append(load)
        else:
            h = gelu_tanh(linear(xn, b("mlp_up_w"), b("mlp_up_b"), dtype))
            out = linear(h, b("mlp_down_w"), b("mlp_down_b"), dtype)
        x = residual + (out if residual_scale == 1.0 else (residual_scale * out).to(dtype))
    hidden = rms_norm(x, p["final_ln_scale"], dtype)
    if not config.experts:
        return hidden, None, None
    return hidden, torch.stack(balance).mean(), torch.stack(loads)


def cross_entropy(p: dict, x: torch.Tensor, y: torch.Tensor, config: Config) -> torch.Tensor:
    """``cross_entropy`` (``train.py:1194-1216``), tiled loss backend; for a
    routed model plus ``router_aux_coefficient`` times the layers' mean balance
    loss (``reference_moe/train.py:1524-1560``)."""

    hidden, balance, _ = gpt_hidden_and_router(p, x, config)
    head = p.get("output_embedding", p["token_embedding"])
    loss = oflce.tiled_tied_cross_entropy(hidden, head, y, semantic_vocab_size=config.semantic_vocab_size,
                                          vocab_tile_size=config.vocab_tile_size, compute_dtype=config.dtype)
    if balance is not None and config.router_aux_coefficient:
        loss = loss + config.router_aux_coefficient * balance
    return loss


def eval_step(p: dict, x: torch.Tensor, y: torch.Tensor, mask: torch.Tensor,
              config: Config) -> tuple[torch.Tensor, torch.Tensor]:
    """``eval_step`` (``train.py:1493-1525``), tiled loss backend: the masked
    loss sum and the target count, both float32."""

    hidden = gpt_hidden(p, x, config)
    head = p.get("output_embedding", p["token_embedding"])
    losses = oflce.tiled_tied_cross_entropy_losses(hidden, head, y, semantic_vocab_size=config.semantic_vocab_size,
                                                   vocab_tile_size=config.vocab_tile_size,
                                                   compute_dtype=config.dtype)
    weights = mask.to(F32)
    return (losses * weights).sum(dtype=F32), weights.sum(dtype=F32)


@dataclass
class TrainState:
    params: dict
    m: dict
    v: dict
    step: int = 0
    history: list = field(default_factory=list)


def init_state(config: Config, seed: int) -> TrainState:
    flat = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in flatten(init_params(config, seed)).items()}
    zeros = lambda: {k: torch.zeros_like(v) for k, v in flat.items()}  # noqa: E731
    return TrainState(flat, zeros(), zeros())


def train_step(state: TrainState, x: torch.Tensor, y: torch.Tensor, config: Config,
               grads_out: dict | None = None) -> dict:
    """``train_step`` / ``_apply_training_update`` (``train.py:1362-1472``).

    ``grads_out`` (optional) receives the raw float32 gradients (before any
    clipping), keyed by parameter path."""

    leaves = {k: v.detach().requires_grad_(True) for k, v in state.params.items()}
    loss = cross_entropy(leaves, x, y, config)
    grads_t = torch.autograd.grad(loss, list(leaves.values()))
    grads = {k: g.to(F32) for k, g in zip(leaves.keys(), grads_t)}
    if grads_out is not None:
        grads_out.update({k: g.detach().clone() for k, g in grads.items()})
    state.step += 1
    lr, gnorm = ooptim.adamw_step(state.params, grads, state.m, state.v, state.step, config.optimizer,
                                  config.parameterization, config.width_multiplier, config.depth_multiplier,
                                  config.depth_alpha)
    record = {"loss": float(loss.detach()), "learning_rate": lr, "grad_norm": gnorm}
    state.history.append((record["loss"], lr, gnorm))
    return record


def synthetic_windows(seed: int, steps: int, batch: int, seq_len: int, vocab: int) -> np.ndarray:
    """Uniform int32 token windows ``[steps, batch, seq_len + 1]`` from numpy PCG64."""

    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, size=(steps, batch, seq_len + 1), dtype=np.int32)


def with_optimizer(config: Config, **kwargs) -> Config:
    return replace(config, optimizer=replace(config.optimizer, **kwargs))
