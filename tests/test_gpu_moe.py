"""GPU parity of the routed MLP (``gptrig.moe``) against the CPU oracle.

The oracle (``oracle/moe.py``) restates ``routed_mlp_local`` /
``load_balance_loss`` of ``recipes/reference_moe/train.py:1230-1371``.  Inputs
are drawn so that no token has two router logits within 1e-4 of each other
around the top-k boundary: the GPU's fp32 logits (a different summation
order) then route every token exactly as the oracle does, and the routing
indices are compared bit-exactly.  Tolerances: combined output and every
gradient max-abs <= 3e-2 of the reference's largest magnitude (bf16 chain of
two GEMMs, GELU and the bf16 scatter-add); mean probability <= 1e-5; load
exact; summary <= 1e-4 relative.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def draw(batch, length, width, hidden, experts, seed):
    rng = np.random.default_rng(seed)

    def n(shape, std):
        return torch.from_numpy((rng.standard_normal(shape) * std).astype(np.float32))

    x = n((batch, length, width), 1.0).to(torch.bfloat16)
    router_w = n((width, experts), 0.1)
    up_w, up_b = n((experts, width, hidden), 0.05), n((experts, hidden), 0.05)
    down_w, down_b = n((experts, hidden, width), 0.05), n((experts, width), 0.05)
    return x, router_w, up_w, up_b, down_w, down_b


def routing_margin(x, router_w, top_k):
    logits = x.reshape(-1, x.shape[-1]).float() @ router_w
    srt = torch.sort(logits, dim=-1, descending=True).values
    return float((srt[:, : top_k] - srt[:, 1: top_k + 1]).min())


def maxabs(a, b):
    return float((a.detach().float().cpu() - b.detach().float().cpu()).abs().max())


def scale(t):
    return max(float(t.detach().float().abs().max()), 1e-6)


@pytest.mark.parametrize("batch,length,width,hidden,experts,top_k", [(4, 128, 256, 512, 8, 2), (2, 96, 128, 256, 4, 1),
                                                                     (2, 64, 128, 128, 6, 3)])
def test_routed_mlp_forward_backward_matches_oracle(batch, length, width, hidden, experts, top_k):
    from gptrig import moe

    print(f"moe case B={batch} L={length} D={width} F={hidden} E={experts} k={top_k}", flush=True)
    x, router_w, up_w, up_b, down_w, down_b = draw(batch, length, width, hidden, experts, 5)
    assert routing_margin(x, router_w, top_k) > 1e-4
    g = torch.from_numpy(np.random.default_rng(6).standard_normal((batch, length, width)).astype(np.float32))
    g = g.to(torch.bfloat16).float()
    aux = 0.01

    # Oracle: forward + autograd gradients.
    leaves = [t.clone().requires_grad_(True) for t in (x, router_w, up_w, up_b, down_w, down_b)]
    comb_r, mp_r, load_r, summ_r, chosen_r, gate_r = omoe.routed_mlp_local(
        *leaves, experts=experts, top_k_count=top_k, dtype=torch.bfloat16)
    loss_r = (comb_r.float() * g).sum() + aux * omoe.load_balance_loss(mp_r, load_r)
    grads_r = torch.autograd.grad(loss_r, leaves)

    # GPU.
    dev_leaves = [t.to(DEV).requires_grad_(True) for t in (x, router_w, up_w, up_b, down_w, down_b)]
    comb, mp, load, summ = moe.routed_mlp_local(*dev_leaves, experts=experts, top_k=top_k)
    loss = (comb.float() * g.to(DEV)).sum() + aux * moe.load_balance_loss(mp, load)
    grads = torch.autograd.grad(loss, dev_leaves)
    torch.cuda.synchronize()

    assert torch.equal(load.cpu(), load_r.detach())
    assert maxabs(mp, mp_r) <= 1e-5
    assert float(((summ.cpu() - summ_r.detach()).abs() / summ_r.detach().abs()).max()) <= 1e-4
    assert maxabs(comb, comb_r) <= 3e-2 * scale(comb_r)
    names = ("x", "router_w", "up_w", "up_b", "down_w", "down_b")
    for name, got, want in zip(names, grads, grads_r):
        err = maxabs(got, want)
        print(f"  d{name}: max-abs {err:.3e} (scale {scale(want):.3e})", flush=True)
        assert err <= 3e-2 * scale(want), name


def test_routing_indices_bit_exact_through_the_front_end():
    from gptrig import _lib
    from gptrig.moe import _route

    x, router_w, *_ = draw(2, 256, 256, 128, 8, 11)
    flat = x.reshape(-1, 256)
    logits_g, probs, chosen, gate, counts, rows, position = _route(flat.to(DEV).contiguous(), router_w.to(DEV), 8, 2)
    torch.cuda.synchronize()
    # Logits within fp32 summation-order noise; routing from the GPU's own logits bit-exact.
    logits_r = flat.float() @ router_w
    assert maxabs(logits_g, logits_r) <= 1e-5 * scale(logits_r) + 1e-6
    _, chosen_r, gate_r, order_r, _, counts_r, rows_r = omoe.route(logits_g.cpu(), 8, 2)
    assert torch.equal(chosen.cpu(), chosen_r)
    assert torch.equal(counts.cpu(), counts_r)
    assert torch.equal(rows.cpu().long(), rows_r)
    assert _lib.version()


def test_config_e_layer_shape_token_subset():
    """Config E's routed layer (32 x 1024 tokens, width 768, 8 experts of width
    3072, top-2) on the GPU; each token's output depends only on that token, so
    64 sampled tokens are checked against the oracle run on those tokens alone,
    and the input gradient of the same tokens likewise (no balance term)."""

    from gptrig import moe

    B, L, D, F, E, k = 32, 1024, 768, 3072, 8, 2
    rng = np.random.default_rng(21)

    def n(shape, std):
        return torch.from_numpy((rng.standard_normal(shape) * std).astype(np.float32))

    x = n((B, L, D), 1.0).to(torch.bfloat16)
    router_w = n((D, E), 0.02)
    up_w, up_b = n((E, D, F), 0.02), n((E, F), 0.02)
    down_w, down_b = n((E, F, D), 0.02), n((E, D), 0.02)
    g = n((B, L, D), 1.0).to(torch.bfloat16)
    xg = x.to(DEV).requires_grad_(True)
    params = [t.to(DEV) for t in (router_w, up_w, up_b, down_w, down_b)]
    comb, mp, load, summ = moe.routed_mlp_local(xg, *params, experts=E, top_k=k)
    (dx,) = torch.autograd.grad((comb.float() * g.to(DEV).float()).sum(), [xg])
    torch.cuda.synchronize()
    assert int(load.sum().mul(B * L * k).round()) == B * L * k
    flat_idx = torch.from_numpy(np.random.default_rng(22).choice(B * L, 64, replace=False))
    xs = x.reshape(B * L, D)[flat_idx].reshape(1, 64, D)
    assert routing_margin(xs, router_w, k) > 1e-5
    xs_leaf = xs.clone().requires_grad_(True)
    comb_r, *_ = omoe.routed_mlp_local(xs_leaf, router_w, up_w, up_b, down_w, down_b, experts=E, top_k_count=k,
                                       dtype=torch.bfloat16)
    gs = g.reshape(B * L, D)[flat_idx].reshape(1, 64, D).float()
    (dx_r,) = torch.autograd.grad((comb_r.float() * gs).sum(), [xs_leaf])
    got = comb.reshape(B * L, D)[flat_idx.to(DEV)]
    assert maxabs(got, comb_r.reshape(64, D)) <= 3e-2 * scale(comb_r)
    got_dx = dx.reshape(B * L, D)[flat_idx.to(DEV)]
    assert maxabs(got_dx, dx_r.reshape(64, D)) <= 3e-2 * scale(dx_r)


def test_config_e_routing_bit_exact_on_all_tokens():
    """Config E's routing at its full size (32 x 1024 = 32,768 tokens, width
    768, 8 experts, top-2, router ~ N(0, 0.02) as initialised): every token's
    expert indices, the per-expert counts, the stable bucket order (one
    1024-thread workgroup sorts all 65,536 assignments) and its inverse are
    bit-exact against the oracle's route of the GPU's own fp32 logits, the
    gates and probabilities within 1e-6.  A second pass plants integer logits
    (ties) in every 16th token to exercise the lower-index rule at this size."""
    from gptrig import _lib
    from gptrig.moe import _route

    T, D, E, k = 32 * 1024, 768, 8, 2
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(torch.bfloat16)
    router_w = torch.from_numpy((rng.standard_normal((D, E)) * 0.02).astype(np.float32))
    print(f"config E routing, {T} tokens", flush=True)
    logits, probs, chosen, gate, counts, rows, position = _route(x.to(DEV), router_w.to(DEV), E, k)
    torch.cuda.synchronize()
    probs_r, chosen_r, gate_r, order_r, _, counts_r, rows_r = omoe.route(logits.cpu(), E, k)
    assert torch.equal(chosen.cpu(), chosen_r)
    assert torch.equal(counts.cpu(), counts_r)
    assert torch.equal(rows.cpu().long(), rows_r)
    inv = torch.empty_like(order_r)
    inv[order_r] = torch.arange(T * k)
    assert torch.equal(position.cpu().long(), inv)
    assert maxabs(gate, gate_r) <= 1e-6 and maxabs(probs, probs_r) <= 1e-6

    tied = logits.cpu().clone()
    tied[::16] = torch.from_numpy(rng.integers(-2, 3, size=(T // 16, E)).astype(np.float32))
    probs_r, chosen_r, gate_r, order_r, _, counts_r, rows_r = omoe.route(tied, E, k)
    lg = tied.to(DEV)
    order = torch.empty(T * k, dtype=torch.int32, device=DEV)
    ws = _lib.workspace(_lib.query("gptrig_moe_route_workspace_bytes", T, E, k), lg.device)
    _lib.call("gptrig_moe_route", lg.data_ptr(), probs.data_ptr(), chosen.data_ptr(), gate.data_ptr(),
              counts.data_ptr(), order.data_ptr(), rows.data_ptr(), position.data_ptr(), ws.data_ptr(), ws.numel(),
              T, E, k, _lib.stream())
    torch.cuda.synchronize()
    assert torch.equal(chosen.cpu(), chosen_r)
    assert torch.equal(counts.cpu(), counts_r)
    assert torch.equal(order.cpu().long(), order_r)
    assert torch.equal(rows.cpu().long(), rows_r)
