"""Pins the rest of the oracle (CPU only): RoPE, RMSNorm, GELU, AdamW/LR,
init_params counts, top-k routing and the routed MLP."""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import moe as omoe
from oracle import nn as onn
from oracle import optim as oopt


# --- RoPE ---------------------------------------------------------------------

def test_rope_reference_invariants():
    # tests/test_trainer_static.py:173-181: position 0 unchanged, norms preserved.
    values = torch.arange(24, dtype=torch.float32).reshape(1, 3, 2, 4)
    rotated = onn.apply_rotary(values)
    np.testing.assert_allclose(rotated[:, 0].numpy(), values[:, 0].numpy(), atol=1e-6)
    np.testing.assert_allclose((rotated ** 2).sum(-1).numpy(), (values ** 2).sum(-1).numpy(), rtol=1e-6, atol=1e-5)


def test_rope_closed_form():
    x = torch.randn(2, 5, 3, 8, generator=torch.Generator().manual_seed(0))
    got = onn.apply_rotary(x).double()
    for b, s, h, i in itertools.product(range(2), range(5), range(3), range(4)):
        theta = s * 10000.0 ** (-(2 * i) / 8)
        e, o = float(x[b, s, h, 2 * i]), float(x[b, s, h, 2 * i + 1])
        assert abs(float(got[b, s, h, 2 * i]) - (e * math.cos(theta) - o * math.sin(theta))) < 1e-5
        assert abs(float(got[b, s, h, 2 * i + 1]) - (e * math.sin(theta) + o * math.cos(theta))) < 1e-5


def test_rope_backward_is_transpose():
    x = torch.randn(1, 7, 2, 16, dtype=torch.float32, generator=torch.Generator().manual_seed(1)).requires_grad_(True)
    dy = torch.randn(1, 7, 2, 16, generator=torch.Generator().manual_seed(2))
    (g,) = torch.autograd.grad(onn.apply_rotary(x), x, dy)
    np.testing.assert_allclose(onn.apply_rotary_backward(dy).numpy(), g.numpy(), rtol=1e-6, atol=1e-6)


def test_rope_odd_head_dim_rejected():
    with pytest.raises(ValueError):
        onn.apply_rotary(torch.zeros(1, 2, 1, 3))


# --- RMSNorm / GELU / linear ---------------------------------------------------

def test_rms_norm_closed_form():
    x = torch.randn(3, 10, generator=torch.Generator().manual_seed(3))
    scale = torch.linspace(0.5, 1.5, 10)
    got = onn.rms_norm(x, scale, torch.float32)
    for r in range(3):
        row = [float(v) for v in x[r]]
        inv = 1.0 / math.sqrt(sum(v * v for v in row) / 10 + 1e-5)
        for c in range(10):
            assert abs(float(got[r, c]) - row[c] * inv * float(scale[c])) < 1e-5


def test_rms_norm_bf16_rounds_before_scale():
    x = torch.randn(4, 64, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    scale = torch.full((64,), 1.7)
    got = onn.rms_norm(x, scale, torch.bfloat16)
    x32 = x.float()
    normalized = (x32 * torch.rsqrt((x32 ** 2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16)
    want = (normalized.float() * torch.tensor(1.7).to(torch.bfloat16).float()).to(torch.bfloat16)
    assert torch.equal(got, want)


def test_gelu_tanh_known_values_and_grad():
    # 0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715x^3))) at x=1 is 0.8411919906082768.
    assert abs(float(onn.gelu_tanh(torch.tensor([1.0]))) - 0.8411919906082768) < 1e-6
    x = torch.linspace(-6, 6, 101, dtype=torch.float64)
    ref = torch.nn.functional.gelu(x, approximate="tanh")
    np.testing.assert_allclose(onn.gelu_tanh(x.float()).double().numpy(), ref.numpy(), atol=1e-6)
    xg = x.clone().requires_grad_(True)
    (g,) = torch.autograd.grad(torch.nn.functional.gelu(xg, approximate="tanh").sum(), xg)
    np.testing.assert_allclose(onn.gelu_tanh_grad(x.float()).double().numpy(), g.numpy(), atol=1e-6)


def test_linear_rounds_product_then_bias():
    x = torch.randn(3, 8, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    w = torch.randn(8, 4, generator=torch.Generator().manual_seed(6))
    b = torch.randn(4, generator=torch.Generator().manual_seed(7))
    got = onn.linear(x, w, b, torch.bfloat16)
    prod = (x.double() @ w.to(torch.bfloat16).double()).to(torch.bfloat16)
    want = (prod.double() + b.to(torch.bfloat16).double()).to(torch.bfloat16)
    assert torch.equal(got, want)


# --- AdamW / LR -------------------------------------------------------------------

def test_learning_rate_schedule_endpoints():
    cfg = oopt.OptimizerConfig(learning_rate=0.01, min_lr_ratio=0.1, warmup_steps=10, steps=110)
    assert abs(oopt.learning_rate(5, cfg) - 0.005) < 1e-9
    assert abs(oopt.learning_rate(10, cfg) - 0.01) < 1e-9
    assert abs(oopt.learning_rate(60, cfg) - 0.01 * (0.1 + 0.9 * 0.5)) < 1e-8
    assert abs(oopt.learning_rate(110, cfg) - 0.001) < 1e-9
    assert abs(oopt.learning_rate(500, cfg) - 0.001) < 1e-9


def test_adamw_first_two_steps_by_hand():
    cfg = oopt.OptimizerConfig(learning_rate=0.01, warmup_steps=0, steps=1000, weight_decay=0.1)
    p = {"blocks/0/qkv_w": torch.tensor([1.0, -2.0]), "blocks/0/qkv_b": torch.tensor([0.5])}
    m = {k: torch.zeros_like(v) for k, v in p.items()}
    v = {k: torch.zeros_like(v) for k, v in p.items()}
    g = {"blocks/0/qkv_w": torch.tensor([0.3, -0.1]), "blocks/0/qkv_b": torch.tensor([2.0])}
    lr1, gn = oopt.adamw_step(p, g, m, v, 1, cfg)
    assert abs(gn - math.sqrt(0.09 + 0.01 + 4.0)) < 1e-6
    # step 1: m_hat = g, v_hat = g^2, so adam = sign(g) (eps negligible).
    lr_expected = 0.01 * (0.1 + 0.9 * 0.5 * (1 + math.cos(math.pi * 1 / 1000)))
    assert abs(lr1 - lr_expected) < 1e-9
    np.testing.assert_allclose(p["blocks/0/qkv_w"].numpy(),
                               [1.0 - lr1 * (1.0 + 0.1 * 1.0), -2.0 - lr1 * (-1.0 + 0.1 * -2.0)], rtol=1e-6)
    np.testing.assert_allclose(p["blocks/0/qkv_b"].numpy(), [0.5 - lr1 * 1.0], rtol=1e-6)  # no decay on biases
    # step 2 with the same gradient: m = 0.19 g, v = 0.0975 g^2 (before bias correction).
    w1 = p["blocks/0/qkv_w"].clone()
    lr2, _ = oopt.adamw_step(p, g, m, v, 2, cfg)
    mh = 0.19 * 0.3 / (1 - 0.81)
    vh = 0.0975 * 0.09 / (1 - 0.95 ** 2)
    assert abs(float(p["blocks/0/qkv_w"][0]) - (float(w1[0]) - lr2 * (mh / (math.sqrt(vh) + 1e-8) + 0.1 * float(w1[0])))) < 1e-6


def ratio_four(module, **kw):
    """batch_multiplier / data_multiplier = 2 / 0.5 = 4 (train.py:792-800: batch / anchor and
    tpp / base tpp); epsilon 0.2 so that its horizon factor shows in the update."""
    base = dict(learning_rate=0.01, warmup_steps=0, steps=1000, weight_decay=0.1, adam_epsilon=0.2,
                batch_multiplier=2.0, data_multiplier=0.5)
    base.update(kw)
    return module.OptimizerConfig(**base)


def test_batch_data_ratio_four_betas_and_learning_rate_by_hand():
    """train.py:1336-1345 and :1231 at ratio 4: beta1 = 1 - 0.1 * 4 = 0.6,
    beta2 = 1 - 0.05 * 4 = 0.8, and the learning rate doubles (sqrt 4).  The
    plausible slips give other numbers: betas 1 - (1 - beta) / 4 = 0.975 /
    0.9875, or the horizon sqrt(data / batch) = 1/2 (a factor 4 off)."""
    cfg = ratio_four(oopt)
    b1, b2 = oopt.effective_adam_betas(cfg)
    assert abs(b1 - 0.6) < 1e-12 and abs(b2 - 0.8) < 1e-12
    # Constant learning rate after a 10-step warmup over 10 + 1000 steps at step 10: base x 2.
    flat = ratio_four(oopt, warmup_steps=10, steps=1010, min_lr_ratio=1.0)
    assert abs(oopt.learning_rate(10, flat) - 0.02) < 1e-9
    assert abs(oopt.learning_rate(5, flat) - 0.01) < 1e-9  # half-way through the warmup
    # The same ratio from other multipliers gives the same numbers (only batch / data enters).
    other = ratio_four(oopt, batch_multiplier=4.0, data_multiplier=1.0, warmup_steps=10, steps=1010, min_lr_ratio=1.0)
    assert oopt.effective_adam_betas(other) == pytest.approx((0.6, 0.8), abs=1e-12)
    assert abs(oopt.learning_rate(10, other) - 0.02) < 1e-9


def test_batch_data_ratio_four_adamw_two_steps_by_hand():
    """Two AdamW updates at ratio 4 (train.py:1386-1445) worked by hand:
    epsilon 0.2 x sqrt(1/4) = 0.1, weight decay 0.1 x sqrt(4) = 0.2, betas
    0.6 / 0.8, learning rate 0.01 x 2 x cosine(step)."""
    cfg = ratio_four(oopt)
    p = {"blocks/0/qkv_w": torch.tensor([1.0, -2.0]), "blocks/0/qkv_b": torch.tensor([0.5])}
    m = {k: torch.zeros_like(v) for k, v in p.items()}
    v = {k: torch.zeros_like(v) for k, v in p.items()}
    g1 = {"blocks/0/qkv_w": torch.tensor([0.3, -0.1]), "blocks/0/qkv_b": torch.tensor([2.0])}
    lr1, _ = oopt.adamw_step(p, g1, m, v, 1, cfg)
    assert abs(lr1 - 0.02 * (0.1 + 0.45 * (1 + math.cos(math.pi / 1000)))) < 1e-8
    # Step 1: m = 0.4 g, v = 0.2 g^2; bias corrections 0.4 and 0.2 give m^ = g, v^ = g^2,
    # so adam = g / (|g| + 0.1): 0.3 / 0.4 = 0.75, -0.1 / 0.2 = -0.5, 2 / 2.1.
    np.testing.assert_allclose(p["blocks/0/qkv_w"].numpy(),
                               [1.0 - lr1 * (0.75 + 0.2 * 1.0), -2.0 - lr1 * (-0.5 + 0.2 * -2.0)], rtol=1e-6)
    np.testing.assert_allclose(p["blocks/0/qkv_b"].numpy(), [0.5 - lr1 * (2.0 / 2.1)], rtol=1e-6)
    np.testing.assert_allclose(m["blocks/0/qkv_w"].numpy(), [0.12, -0.04], rtol=1e-6)
    np.testing.assert_allclose(v["blocks/0/qkv_w"].numpy(), [0.018, 0.002], rtol=1e-6)
    # Step 2 with g2 = (-0.1, 0.2): m = 0.6 * (0.12, -0.04) + 0.4 * (-0.1, 0.2) = (0.032, 0.056),
    # v = 0.8 * (0.018, 0.002) + 0.2 * (0.01, 0.04) = (0.0164, 0.0096); corrections 1 - 0.36 = 0.64
    # and 1 - 0.64 = 0.36.
    w1 = p["blocks/0/qkv_w"].clone().double()
    g2 = {"blocks/0/qkv_w": torch.tensor([-0.1, 0.2]), "blocks/0/qkv_b": torch.tensor([-1.0])}
    lr2, _ = oopt.adamw_step(p, g2, m, v, 2, cfg)
    np.testing.assert_allclose(m["blocks/0/qkv_w"].numpy(), [0.032, 0.056], rtol=1e-6)
    np.testing.assert_allclose(v["blocks/0/qkv_w"].numpy(), [0.0164, 0.0096], rtol=1e-6)
    adam = [(0.032 / 0.64) / (math.sqrt(0.0164 / 0.36) + 0.1), (0.056 / 0.64) / (math.sqrt(0.0096 / 0.36) + 0.1)]
    want = [float(w1[i]) - lr2 * (adam[i] + 0.2 * float(w1[i])) for i in range(2)]
    np.testing.assert_allclose(p["blocks/0/qkv_w"].double().numpy(), want, rtol=1e-6)
    # A slip in any horizon factor moves these updates by far more than the tolerance.
    assert abs(adam[0] - (0.032 / 0.64) / (math.sqrt(0.0164 / 0.36) + 0.4)) > 0.05


def test_batch_data_ratio_rejects_invalid_momenta():
    """train.py:1340-1344: beta1 = 1 - 0.1 * ratio leaves [0, 1) above ratio 10,
    and ratio 0 gives beta = 1."""
    for module in (oopt,):
        assert module.effective_adam_betas(ratio_four(module, batch_multiplier=10.0, data_multiplier=1.0))[0] < 1e-12
        with pytest.raises(ValueError):
            module.effective_adam_betas(ratio_four(module, batch_multiplier=10.5, data_multiplier=1.0))
        with pytest.raises(ValueError):
            module.effective_adam_betas(ratio_four(module, batch_multiplier=0.0, data_multiplier=1.0))


def test_router_statistics_closed_forms():
    """routed_mlp_local's summary (reference_moe/train.py:1290-1306): the
    mean over tokens of the softmax entropy (with its +1e-9), the mean top-1
    gate, and the root of the mean squared logit.
      * Rows of equal logits c_r: entropy -log(1/E + 1e-9), top-1 gate 1/k,
        RMS sqrt(mean c_r^2) (c = 1 and 3: sqrt 5, where a mean |logit| would
        give 2).
      * Rows (ln 7, 0, ..., 0) with E = 8: probabilities 1/2 and 1/14, entropy
        (1/2) ln 2 + (1/2) ln 14, top-2 gate (7/8, 1/8).
      * Half of each: the entropy is the mean of the two (the entropy of the
        mean probability would be larger)."""
    E, k = 8, 2

    def summary(logits: torch.Tensor) -> torch.Tensor:
        # The router sees the given logits: identity token rows times router_w = logits.
        t = logits.shape[0]
        xs = torch.eye(t).reshape(1, t, t)
        out = omoe.routed_mlp_local(xs, logits, torch.zeros(E, t, 3), torch.zeros(E, 3), torch.zeros(E, 3, t),
                                    torch.zeros(E, t), experts=E, top_k_count=k, dtype=torch.float32)
        return out[3].double()

    uniform = torch.tensor([[1.0] * E, [3.0] * E])
    s = summary(uniform)
    assert abs(float(s[0]) + math.log(1 / E + 1e-9)) < 1e-6
    assert abs(float(s[1]) - 0.5) < 1e-7
    assert abs(float(s[2]) - math.sqrt(5.0)) < 1e-6
    peaked = torch.tensor([[math.log(7.0)] + [0.0] * (E - 1)] * 2)
    s = summary(peaked)
    h_peak = -(0.5 * math.log(0.5 + 1e-9) + 7 * (1 / 14) * math.log(1 / 14 + 1e-9))
    assert abs(h_peak - (0.5 * math.log(2) + 0.5 * math.log(14))) < 1e-7
    assert abs(float(s[0]) - h_peak) < 1e-6
    assert abs(float(s[1]) - 7 / 8) < 1e-6
    assert abs(float(s[2]) - math.log(7.0) / math.sqrt(E)) < 1e-6
    mixed = torch.cat([uniform[:1], peaked[:1]])
    s = summary(mixed)
    h_uniform = -math.log(1 / E + 1e-9)
    assert abs(float(s[0]) - (h_uniform + h_peak) / 2) < 1e-6
    pbar = torch.tensor([1 / E] * E) / 2 + torch.tensor([0.5] + [1 / 14] * (E - 1)) / 2
    assert float(-(pbar * torch.log(pbar)).sum()) - float(s[0]) > 0.05
    assert abs(float(s[1]) - (0.5 + 7 / 8) / 2) < 1e-6
    assert abs(float(s[2]) - math.sqrt((E * 1.0 + math.log(7.0) ** 2) / (2 * E))) < 1e-6


def test_weight_decay_mask_roles():
    assert oopt.decays("token_embedding") and oopt.decays("blocks/0/mlp_up_w")
    assert not oopt.decays("blocks/0/mlp_up_b") and not oopt.decays("final_ln_scale")
    with pytest.raises(ValueError):
        oopt.decays("blocks/0/mystery")


# --- init_params --------------------------------------------------------------

def test_smoke_parameter_count():
    # tests/test_trainer_static.py:161 of the reference.
    assert onn.parameter_count(om.init_params(om.smoke_config(), 7)) == 116_160


def test_tier_tpp_parameters_known_answers():
    # tests/test_trainer_static.py:185-191 of the reference.
    expected = {(12, 384): 59_918_208, (12, 640): 123_456_640, (16, 896): 244_444_032,
                (19, 1280): 502_602_240, (21, 1792): 989_943_808}
    for (layers, width), count in expected.items():
        assert om.tpp_parameters(layers, width, 50304) == count


def test_untied_125m_parameter_count():
    cfg = om.baseline_config("D")
    counts = om.flatten(om.init_params(om.Config(**{**cfg.__dict__, "vocab_size": 64,
                                                      "semantic_vocab_size": 64}), 0))
    per_layer = 12 * 768 * 768 + 11 * 768
    assert sum(v.size for v in counts.values()) == 12 * per_layer + 2 * 64 * 768 + 768
    assert 12 * per_layer + 2 * 50304 * 768 + 768 == 162_303_744


def test_smoke_train_step_starts_near_uniform_loss():
    cfg = om.smoke_config()
    state = om.init_state(cfg, 0)
    w = om.synthetic_windows(0, 1, cfg.batch_size, cfg.seq_len, cfg.vocab_size)[0]
    x, y = torch.from_numpy(w[:, :-1]), torch.from_numpy(w[:, 1:])
    rec = om.train_step(state, x, y, cfg)
    assert abs(rec["loss"] - math.log(256)) < 0.05
    assert rec["grad_norm"] > 0 and state.step == 1


# --- routing ------------------------------------------------------------------

def test_eval_step_masked_sum():
    """eval_step (train.py:1493-1525): with an all-ones mask the loss sum over
    the count is the training loss (cross_entropy's mean, a separate path
    through the tiled losses); a zero mask gives (0, 0); the masked sum is
    linear in the mask."""
    cfg = om.smoke_config()
    p = om.flatten(om.init_params(cfg, 5))
    p = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in p.items()}
    w = torch.from_numpy(om.synthetic_windows(3, 1, 2, 32, cfg.semantic_vocab_size)[0])
    x, y = w[:, :-1], w[:, 1:]
    total, count = om.eval_step(p, x, y, torch.ones(x.shape), cfg)
    mean = om.cross_entropy(p, x, y, cfg)
    assert float(count) == x.numel()
    assert abs(float(total) / float(count) - float(mean)) <= 1e-6 * abs(float(mean))
    zero = om.eval_step(p, x, y, torch.zeros(x.shape), cfg)
    assert float(zero[0]) == 0.0 and float(zero[1]) == 0.0
    g = torch.Generator().manual_seed(9)
    m1 = (torch.rand(x.shape, generator=g) < 0.5).float()
    m2 = torch.rand(x.shape, generator=g) * (1 - m1)
    a, b, ab = (om.eval_step(p, x, y, m, cfg) for m in (m1, m2, m1 + m2))
    assert abs(float(ab[0]) - float(a[0]) - float(b[0])) <= 1e-5 * abs(float(ab[0]))
    assert abs(float(ab[1]) - float(a[1]) - float(b[1])) <= 1e-5 * float(ab[1])


def test_top_k_brute_force_with_ties():
    rng = np.random.default_rng(0)
    logits = torch.from_numpy(rng.integers(-2, 3, size=(200, 6)).astype(np.float32))
    vals, idx = omoe.top_k(logits, 2)
    for r in range(200):
        row = logits[r].tolist()
        best = max(itertools.permutations(range(6), 2), key=lambda ab: (row[ab[0]], row[ab[1]], -ab[0], -ab[1]))
        assert tuple(idx[r].tolist()) == best
        assert vals[r].tolist() == [row[best[0]], row[best[1]]]


def test_route_load_and_balance_loss():
    logits = torch.randn(64, 8, generator=torch.Generator().manual_seed(1))
    probs, chosen, gate, order, sorted_a, counts, rows = omoe.route(logits, 8, 2)
    assert int(counts.sum()) == 128
    assert torch.all(sorted_a[1:] >= sorted_a[:-1])
    assert abs(float(counts.float().sum() / 128) - 1.0) < 1e-7
    uniform = torch.full((8,), 1 / 8)
    assert abs(float(omoe.load_balance_loss(uniform, uniform)) - 1.0) < 1e-6
    np.testing.assert_allclose(gate.sum(-1).numpy(), 1.0, rtol=1e-6)


def test_routed_mlp_matches_per_token_dense():
    g = torch.Generator().manual_seed(2)
    B, S, d, E, f = 2, 5, 8, 4, 12
    x = torch.randn(B, S, d, generator=g)
    rw = torch.randn(d, E, generator=g)
    up_w, up_b = torch.randn(E, d, f, generator=g) * 0.3, torch.randn(E, f, generator=g) * 0.1
    dn_w, dn_b = torch.randn(E, f, d, generator=g) * 0.3, torch.randn(E, d, generator=g) * 0.1
    out, *_ , chosen, gate = omoe.routed_mlp_local(x, rw, up_w, up_b, dn_w, dn_b, experts=E, top_k_count=2,
                                                   dtype=torch.float32)
    flat = x.reshape(-1, d)
    for t in range(B * S):
        want = torch.zeros(d)
        for j in range(2):
            e = int(chosen[t, j])
            h = onn.gelu_tanh(flat[t] @ up_w[e] + up_b[e])
            want += gate[t, j] * (h @ dn_w[e] + dn_b[e])
        np.testing.assert_allclose(out.reshape(-1, d)[t].numpy(), want.numpy(), rtol=1e-5, atol=1e-5)
