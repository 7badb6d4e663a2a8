"""Top-k routed MLP restated from ``recipes/reference_moe/train.py:1230-1371``.

Test infrastructure only (see ``oracle/__init__.py``).

``megablox.gmm`` (jax 0.11.0, not vendored) is restated as a per-expert dense
matmul over contiguous row groups, which is its published contract; its
internal accumulation order is not pinnable here.
"""

from __future__ import annotations

import torch

from .nn import F32, gelu_tanh


def top_k(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``jax.lax.top_k`` over the last axis: descending values, and on equal
    values the lower index first."""

    order = torch.sort(-logits, dim=-1, stable=True).indices[..., :k]
    return torch.gather(logits, -1, order), order.to(torch.int32)


def route(logits: torch.Tensor, experts: int, top_k_count: int):
    """Routing part of ``routed_mlp_local`` (``:1259-1273``).

    Returns ``(probabilities, chosen, gate, order, sorted_assignments, counts, rows)``.
    """

    probabilities = torch.softmax(logits, dim=-1)
    chosen_logits, chosen = top_k(logits, top_k_count)
    gate = torch.softmax(chosen_logits, dim=-1)
    assignments = chosen.reshape(-1).to(torch.int64)
    order = torch.sort(assignments, stable=True).indices
    sorted_assignments = assignments[order]
    counts = torch.bincount(assignments, minlength=experts).to(torch.int32)
    rows = torch.arange(logits.shape[0]).repeat_interleave(top_k_count)[order]
    return probabilities, chosen, gate, order, sorted_assignments, counts, rows


def grouped_matmul(lhs: torch.Tensor, rhs: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
    """``megablox.gmm`` contract: rows grouped by expert, ``lhs[g] @ rhs[e]``."""

    out = torch.zeros((lhs.shape[0], rhs.shape[-1]), dtype=F32)
    start = 0
    for e, c in enumerate(counts.tolist()):
        out[start:start + c] = lhs[start:start + c].to(F32) @ rhs[e].to(F32)
        start += c
    return out.to(lhs.dtype)


def routed_mlp_local(x, router_w, up_w, up_b, down_w, down_b, *, experts: int, top_k_count: int, dtype):
    """``routed_mlp_local`` (``reference_moe/train.py:1230-1307``) on one device."""

    batch, length, width = x.shape
    flat = x.reshape(batch * length, width)
    logits = flat.to(F32) @ router_w.to(F32)
    probabilities, chosen, gate, order, sorted_assignments, counts, rows = route(logits, experts, top_k_count)
    grouped = flat[rows].to(dtype)
    hidden = grouped_matmul(grouped, up_w.to(dtype), counts)
    hidden = hidden + up_b[sorted_assignments].to(hidden.dtype)
    hidden = gelu_tanh(hidden)
    out = grouped_matmul(hidden.to(dtype), down_w.to(dtype), counts)
    out = out + down_b[sorted_assignments].to(out.dtype)
    weighted = out * gate.reshape(-1)[order][:, None].to(out.dtype)
    combined = torch.zeros((batch * length, width), dtype=out.dtype).index_add_(0, rows, weighted)
    mean_probability = probabilities.mean(0)
    load = counts.to(F32) / float(batch * length * top_k_count)
    entropy = -(probabilities * torch.log(probabilities + 1.0e-9)).sum(-1).mean()
    top1_gate = gate.max(-1).values.mean()
    logit_rms = torch.sqrt((logits * logits).mean())
    summary = torch.stack((entropy, top1_gate, logit_rms))
    return combined.reshape(batch, length, width), mean_probability, load, summary, chosen, gate


def load_balance_loss(mean_probability: torch.Tensor, load: torch.Tensor) -> torch.Tensor:
    """``load_balance_loss`` (``:1347-1371``): ``E * sum(load * P)``."""

    if mean_probability.ndim != 1 or load.ndim != 1:
        raise ValueError("load_balance_loss takes per-expert vectors already reduced over tokens")
    return float(load.shape[0]) * (load * mean_probability).sum()
