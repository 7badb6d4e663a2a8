"""Top-k routed MLP on the gfx950 kernels.

Mirrors ``routed_mlp_local`` and ``load_balance_loss`` of
``recipes/reference_moe/train.py:1230-1307,1347-1371`` on one device (the
``axis_name`` reductions collapse): fp32 router logits, ``jax.lax.top_k``
routing with a stable bucket sort, two grouped expert GEMMs (``megablox.gmm``)
with bias / GELU epilogues, and the gated scatter-add.  Forward and backward
run entirely in ``libgptrig.so``; torch only allocates.
"""

from __future__ import annotations

import torch

from . import _lib

BF16 = torch.bfloat16
F32 = torch.float32


def _route(flat: torch.Tensor, router_w: torch.Tensor, experts: int, top_k: int):
    tokens, width = flat.shape
    dev = flat.device
    s = _lib.stream()
    logits = torch.empty((tokens, experts), dtype=F32, device=dev)
    _lib.call("gptrig_moe_router_logits", flat.data_ptr(), router_w.data_ptr(), logits.data_ptr(), tokens, width,
              experts, s)
    probs = torch.empty((tokens, experts), dtype=F32, device=dev)
    chosen = torch.empty((tokens, top_k), dtype=torch.int32, device=dev)
    gate = torch.empty((tokens, top_k), dtype=F32, device=dev)
    counts = torch.empty(experts, dtype=torch.int32, device=dev)
    order = torch.empty(tokens * top_k, dtype=torch.int32, device=dev)
    rows = torch.empty(tokens * top_k, dtype=torch.int32, device=dev)
    position = torch.empty(tokens * top_k, dtype=torch.int32, device=dev)
    ws = _lib.workspace(_lib.query("gptrig_moe_route_workspace_bytes", tokens, experts, top_k), dev)
    _lib.call("gptrig_moe_route", logits.data_ptr(), probs.data_ptr(), chosen.data_ptr(), gate.data_ptr(),
              counts.data_ptr(), order.data_ptr(), rows.data_ptr(), position.data_ptr(), ws.data_ptr(), ws.numel(),
              tokens, experts, top_k, s)
    return logits, probs, chosen, gate, counts, rows, position


def _gmm(lhs, rhs, transposed: bool, counts, bias, mode: int, pre, rows: int, k: int, n: int,
         experts: int) -> torch.Tensor:
    out = torch.empty((rows, n), dtype=BF16, device=lhs.device)
    _lib.call("gptrig_moe_gmm", lhs.data_ptr(), lhs.stride(0), rhs.data_ptr(), int(transposed), counts.data_ptr(),
              None if bias is None else bias.data_ptr(), mode, out.data_ptr(), None if pre is None else pre.data_ptr(),
              n, rows, k, n, experts, _lib.stream())
    return out


class _RoutedMLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, router_w, up_w, up_b, down_w, down_b, experts: int, top_k: int):
        batch, length, width = x.shape
        tokens = batch * length
        hidden_width = up_w.shape[-1]
        R = tokens * top_k
        flat = x.reshape(tokens, width).to(BF16).contiguous()
        rw = router_w.to(F32).contiguous()
        logits, probs, chosen, gate, counts, rows, position = _route(flat, rw, experts, top_k)
        upw, upb = up_w.to(BF16).contiguous(), up_b.to(BF16).contiguous()
        dnw, dnb = down_w.to(BF16).contiguous(), down_b.to(BF16).contiguous()
        grouped = torch.empty((R, width), dtype=BF16, device=x.device)
        _lib.call("gptrig_moe_gather_rows", flat.data_ptr(), rows.data_ptr(), grouped.data_ptr(), R, width,
                  _lib.stream())
        pre = torch.empty((R, hidden_width), dtype=BF16, device=x.device)
        hidden = _gmm(grouped, upw, False, counts, upb, 1, pre, R, width, hidden_width, experts)
        out = _gmm(hidden, dnw, False, counts, dnb, 0, None, R, hidden_width, width, experts)
        combined = torch.empty((tokens, width), dtype=BF16, device=x.device)
        s = _lib.stream()
        _lib.call("gptrig_moe_combine", out.data_ptr(), position.data_ptr(), gate.data_ptr(), combined.data_ptr(),
                  tokens, width, top_k, s)
        mean_probability = torch.empty(experts, dtype=F32, device=x.device)
        load = torch.empty(experts, dtype=F32, device=x.device)
        summary = torch.empty(3, dtype=F32, device=x.device)
        _lib.call("gptrig_moe_stats", logits.data_ptr(), probs.data_ptr(), gate.data_ptr(), counts.data_ptr(), tokens,
                  experts, top_k, mean_probability.data_ptr(), load.data_ptr(), summary.data_ptr(), s)
        ctx.save_for_backward(flat, grouped, rw, upw, dnw, probs, chosen, gate, counts, position, pre, hidden, out)
        ctx.meta = (batch, length, width, hidden_width, experts, top_k, x.dtype, router_w.dtype, up_w.dtype,
                    up_b.dtype, down_w.dtype, down_b.dtype)
        ctx.mark_non_differentiable(load, summary)
        return combined.reshape(batch, length, width).to(x.dtype), mean_probability, load, summary

    @staticmethod
    def backward(ctx, dcombined, dmean_probability, _dload, _dsummary):
        flat, grouped, rw, upw, dnw, probs, chosen, gate, counts, position, pre, hidden, out = ctx.saved_tensors
        batch, length, width, hidden_width, experts, top_k, xdt, rdt, uwdt, ubdt, dwdt, dbdt = ctx.meta
        tokens = batch * length
        R = tokens * top_k
        dev = flat.device
        s = _lib.stream()
        if dcombined is None:
            dcombined = torch.zeros((tokens, width), dtype=BF16, device=dev)
        dc = dcombined.reshape(tokens, width).to(BF16).contiguous()
        dout = torch.empty((R, width), dtype=BF16, device=dev)
        dgate = torch.empty(R, dtype=F32, device=dev)
        _lib.call("gptrig_moe_combine_bwd", dc.data_ptr(), out.data_ptr(), position.data_ptr(), gate.data_ptr(),
                  dout.data_ptr(), dgate.data_ptr(), tokens, width, top_k, s)
        d_up_w = torch.zeros((experts, width, hidden_width), dtype=F32, device=dev)
        d_up_b = torch.zeros((experts, hidden_width), dtype=F32, device=dev)
        d_down_w = torch.zeros((experts, hidden_width, width), dtype=F32, device=dev)
        d_down_b = torch.zeros((experts, width), dtype=F32, device=dev)
        d_router = torch.zeros((width, experts), dtype=F32, device=dev)
        # Down projection: dW, db from (hidden, dout); d(pre) = (dout W^T) * gelu'(pre).
        _lib.call("gptrig_moe_gmm_dw", hidden.data_ptr(), hidden_width, dout.data_ptr(), width, counts.data_ptr(),
                  d_down_w.data_ptr(), d_down_b.data_ptr(), R, hidden_width, width, experts, s)
        dpre = _gmm(dout, dnw, True, counts, None, 2, pre, R, width, hidden_width, experts)
        # Up projection: dW, db from (grouped, dpre); d(grouped) = dpre W^T.
        _lib.call("gptrig_moe_gmm_dw", grouped.data_ptr(), width, dpre.data_ptr(), hidden_width, counts.data_ptr(),
                  d_up_w.data_ptr(), d_up_b.data_ptr(), R, width, hidden_width, experts, s)
        dgrouped = _gmm(dpre, upw, True, counts, None, 0, None, R, hidden_width, width, experts)
        dx = torch.empty((tokens, width), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gather_bwd", dgrouped.data_ptr(), position.data_ptr(), dx.data_ptr(), tokens, width,
                  top_k, s)
        dmp = None if dmean_probability is None else dmean_probability.to(F32).contiguous()
        _lib.call("gptrig_moe_router_bwd", flat.data_ptr(), rw.data_ptr(), probs.data_ptr(), chosen.data_ptr(),
                  gate.data_ptr(), dgate.data_ptr(), None if dmp is None else dmp.data_ptr(), dx.data_ptr(),
                  d_router.data_ptr(), tokens, width, experts, top_k, s)
        return (dx.reshape(batch, length, width).to(xdt), d_router.to(rdt), d_up_w.to(uwdt), d_up_b.to(ubdt),
                d_down_w.to(dwdt), d_down_b.to(dbdt), None, None)


def routed_mlp_local(x: torch.Tensor, router_w: torch.Tensor, up_w: torch.Tensor, up_b: torch.Tensor,
                     down_w: torch.Tensor, down_b: torch.Tensor, *, experts: int, top_k: int,
                     dtype=torch.bfloat16, axis_name=None):
    """``routed_mlp_local`` (``reference_moe/train.py:1230-1307``) on one device.

    ``x`` [batch, length, width]; ``router_w`` [width, experts] (fp32 math);
    ``up_w`` [experts, width, hidden], ``up_b`` [experts, hidden], ``down_w``
    [experts, hidden, width], ``down_b`` [experts, width].  Returns
    ``(combined, mean_probability, load, summary)``; ``load`` and ``summary``
    carry no gradient (``load`` is a count ratio, as in the reference).
    """

    if dtype != torch.bfloat16:
        raise TypeError("the routed MLP kernels compute in bfloat16")
    if axis_name is not None:
        raise ValueError("one device: the data-axis reductions collapse; pass axis_name=None")
    if x.ndim != 3:
        raise ValueError(f"x must be [batch, length, width], got {tuple(x.shape)}")
    width = x.shape[-1]
    hidden = up_w.shape[-1]
    if router_w.shape != (width, experts):
        raise ValueError(f"router_w must be [{width}, {experts}], got {tuple(router_w.shape)}")
    if up_w.shape != (experts, width, hidden) or up_b.shape != (experts, hidden):
        raise ValueError("up_w / up_b must be [experts, width, hidden] / [experts, hidden]")
    if down_w.shape != (experts, hidden, width) or down_b.shape != (experts, width):
        raise ValueError("down_w / down_b must be [experts, hidden, width] / [experts, width]")
    if not 0 < top_k <= experts:
        raise ValueError(f"top_k must be in [1, experts], got {top_k}")
    _lib.require_device(x, router_w, up_w, up_b, down_w, down_b)
    return _RoutedMLP.apply(x, router_w, up_w, up_b, down_w, down_b, int(experts), int(top_k))


def load_balance_loss(mean_probability: torch.Tensor, load: torch.Tensor) -> torch.Tensor:
    """``load_balance_loss`` (``reference_moe/train.py:1347-1371``): ``E * sum(load * P)``."""

    if mean_probability.ndim != 1 or load.ndim != 1:
        raise ValueError("load_balance_loss takes per-expert vectors already reduced over tokens, got shapes "
                         f"{tuple(mean_probability.shape)} and {tuple(load.shape)}")
    return float(load.shape[0]) * (load * mean_probability).sum()
