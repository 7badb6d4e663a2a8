"""Pins of the oracle's step composition (``oracle/model.py``) by cases the
mathematics fixes (CPU).

``gpt_hidden`` / ``cross_entropy`` restate ``recipes/reference/train.py:
1096-1216``; the optimizer multipliers restate ``:1274-1345``.  Each test
below builds a parameter set for which the reference's forward reduces to a
closed form that is evaluated here independently, in float64 numpy with
bfloat16 rounding (torch's round-to-nearest-even cast) at the points where
the reference casts:

* every block weight zero            -> ``rms_norm(embedding[x])``;
* q/k projections zero               -> uniform causal attention, i.e. the
                                        prefix mean of v (no rotation of v);
* attention branch zero              -> a per-token MLP formula;
* no layers, sign-vector embeddings  -> a closed-form cross entropy;
* completep at width = depth = 2     -> a hand-computed multiplier table.

Each closed-form test also checks that a plausible wiring mistake (dropped
final norm, rotated v, non-causal mask, wrong residual, wrong norm scale,
missing GELU, residual scale ignored, tied/untied head swapped) moves the
result far outside the tolerance, so the test would catch it.
"""

from __future__ import annotations

import math
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import optim as oopt

D_MODEL, HEADS, SEQ, BATCH, VOCAB = 64, 2, 12, 2, 96


def bf(a) -> np.ndarray:
    """float64 values rounded to bfloat16 (via float32, as the fp32 compute rounds)."""

    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def rms64(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """rig/nn.py:26-33 evaluated in float64: normalised value rounded, then times bf16(scale), rounded."""

    normalized = bf(x / np.sqrt((x * x).mean(-1, keepdims=True) + 1.0e-5))
    return bf(normalized * bf(scale))


def lin64(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """rig/nn.py:55-56: bf16 product (fp32 accumulation) then the bf16 bias add."""

    return bf(bf(x @ bf(w)) + bf(b))


def gelu64(x: np.ndarray) -> np.ndarray:
    return bf(0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3))))


def rope64(x: np.ndarray) -> np.ndarray:
    """Interleaved base-10000 rotation of [B, S, H, Dh] (used only for a mistake model)."""

    S, Dh = x.shape[1], x.shape[-1]
    inv = 10000.0 ** (-np.arange(0, Dh, 2) / Dh)
    ang = np.arange(S)[:, None] * inv[None, :]
    c, s = np.cos(ang)[None, :, None, :], np.sin(ang)[None, :, None, :]
    e, o = x[..., 0::2], x[..., 1::2]
    return np.stack((e * c - o * s, e * s + o * c), -1).reshape(x.shape)


def close(got: np.ndarray, want: np.ndarray, floor: float = 0.1) -> float:
    """Largest difference in units of the tolerance (2^-6 relative, floor 2^-6 * floor):
    a few bf16 ulps of rounding-order slack."""

    tol = 2.0 ** -6 * np.maximum(np.abs(want), floor)
    return float(np.max(np.abs(got - want) / tol))


def params(config: om.Config, seed: int = 0) -> dict:
    return {k: torch.from_numpy(np.ascontiguousarray(v)).clone() for k, v in
            om.flatten(om.init_params(config, seed)).items()}


def tokens(seed: int = 1) -> torch.Tensor:
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.integers(0, VOCAB, size=(BATCH, SEQ), dtype=np.int32))


def config(**kw) -> om.Config:
    base = dict(layers=1, heads=HEADS, d_model=D_MODEL, vocab_size=VOCAB, semantic_vocab_size=VOCAB, seq_len=SEQ,
                batch_size=BATCH, base_width=D_MODEL, base_depth=1, embeddings="untied")
    base.update(kw)
    return om.Config(**base)


def hidden(p: dict, x: torch.Tensor, cfg: om.Config) -> np.ndarray:
    with torch.no_grad():
        return om.gpt_hidden(p, x, cfg).to(torch.float64).numpy()


def zero_blocks(p: dict) -> None:
    for k, v in p.items():
        if k.startswith("blocks/") and not k.endswith("_scale"):
            v.zero_()


def test_zero_blocks_reduce_to_the_normed_embedding():
    """Every block linear zero: attention of v = 0 and GELU(0) = 0 leave the
    residual stream at the embedding, so gpt_hidden = rms_norm(embedding[x])."""
    cfg = config(layers=3)
    p = params(cfg)
    zero_blocks(p)
    gen = torch.Generator().manual_seed(2)
    p["token_embedding"] = torch.randn(VOCAB, D_MODEL, generator=gen)
    p["final_ln_scale"] = 1.0 + 0.25 * torch.randn(D_MODEL, generator=gen)
    x = tokens()
    e = bf(p["token_embedding"].numpy()[x.numpy()])
    want = rms64(e, p["final_ln_scale"].numpy())
    got = hidden(p, x, cfg)
    assert close(got, want) <= 1.0
    assert np.mean(got == want) > 0.98
    # mistakes: no final norm; the final scale not applied.
    assert close(e, want) > 20
    assert close(rms64(e, np.ones(D_MODEL)), want) > 20


def attention_only(p: dict, cfg: om.Config, gen: torch.Generator) -> None:
    """q/k columns of qkv_w zero (uniform causal attention), v and the output
    projection random, the MLP zero."""
    d = D_MODEL
    for i in range(cfg.layers):
        b = f"blocks/{i}/"
        w = torch.randn(d, 3 * d, generator=gen) / math.sqrt(d)
        w[:, :2 * d] = 0.0
        p[b + "qkv_w"] = w
        p[b + "qkv_b"] = torch.cat([torch.zeros(2 * d), 0.1 * torch.randn(d, generator=gen)])
        p[b + "attn_w"] = torch.randn(d, d, generator=gen) / math.sqrt(d)
        p[b + "attn_b"] = 0.1 * torch.randn(d, generator=gen)
        p[b + "ln1_scale"] = 1.0 + 0.25 * torch.randn(d, generator=gen)
        for name in ("mlp_up_w", "mlp_up_b", "mlp_down_w", "mlp_down_b"):
            p[b + name].zero_()
    p["token_embedding"] = torch.randn(VOCAB, d, generator=gen)


def attention_closed_form(p: dict, x: torch.Tensor, cfg: om.Config, *, rotate_v=False, causal=True,
                          residual_on_norm=False, residual_scale=None, normalised=False) -> np.ndarray:
    """Zero scores through the Pallas kernel's numerics: every visible
    unnormalised probability is exp(0 - 0) = 1 (exact in bf16), so the output
    is bf16 of the exact causal prefix mean of v.  normalised=True rounds the
    normalised weights 1/(t+1) to bf16 first, as the kernel's test oracle
    does."""
    d, H = D_MODEL, HEADS
    s = cfg.depth_multiplier ** (-cfg.depth_alpha) if residual_scale is None else residual_scale
    h = bf(p["token_embedding"].numpy()[x.numpy()])
    S = h.shape[1]
    for i in range(cfg.layers):
        b = lambda n: p[f"blocks/{i}/{n}"].numpy()  # noqa: E731
        xn = rms64(h, b("ln1_scale"))
        v = lin64(xn, b("qkv_w")[:, 2 * d:], b("qkv_b")[2 * d:])
        if rotate_v:
            v = bf(rope64(v.reshape(BATCH, S, H, d // H)).reshape(v.shape))
        t = np.arange(S)
        if causal:
            w = 1.0 / (t[:, None] + 1.0)
            weights = np.where(t[None, :] <= t[:, None], bf(w) if normalised else w, 0.0)
        else:
            weights = np.full((S, S), float(bf(1.0 / S)))
        if causal and not normalised:
            # float32 prefix sums times the float32 reciprocal of the count, as
            # the kernel's accumulator (acc * (1 / l)) computes them
            sums = np.cumsum(v.astype(np.float32), axis=1, dtype=np.float32)
            att = bf(sums * (np.float32(1.0) / (t.astype(np.float32) + np.float32(1.0)))[None, :, None])
        else:
            att = bf(np.einsum("ts,bsd->btd", weights, v))
        out = lin64(att, b("attn_w"), b("attn_b"))
        base = xn if residual_on_norm else h
        h = bf(base + (out if s == 1.0 else bf(s * out)))
    return rms64(h, p["final_ln_scale"].numpy())


@pytest.mark.parametrize("layers,base_depth,alpha", [(1, 1, 0.0), (2, 1, 1.0)])
def test_uniform_attention_is_the_prefix_mean_of_v(layers, base_depth, alpha):
    """q = k = 0 makes every visible score 0: the attention output is the
    causal prefix mean of v (unrotated), through the output projection and the
    residual; with depth_alpha = 1 and depth multiplier 2 each branch is
    scaled by 1/2 (train.py:1164-1175)."""
    cfg = config(layers=layers, base_depth=base_depth, depth_alpha=alpha)
    p = params(cfg)
    attention_only(p, cfg, torch.Generator().manual_seed(3))
    x = tokens()
    got = hidden(p, x, cfg)
    want = attention_closed_form(p, x, cfg)
    assert close(got, want) <= 1.0
    for mistake in (dict(rotate_v=True), dict(causal=False), dict(residual_on_norm=True)):
        assert close(attention_closed_form(p, x, cfg, **mistake), want) > 10, mistake
    # The normalised rounding is a bf16-level difference, still far outside the slack.
    assert close(attention_closed_form(p, x, cfg, normalised=True), want) > 2
    if alpha:
        assert close(attention_closed_form(p, x, cfg, residual_scale=1.0), want) > 10


def mlp_closed_form(p: dict, x: torch.Tensor, *, norm_scale="ln2_scale", gelu=True) -> np.ndarray:
    h = bf(p["token_embedding"].numpy()[x.numpy()])
    b = lambda n: p[f"blocks/0/{n}"].numpy()  # noqa: E731
    xn = rms64(h, b(norm_scale))
    up = lin64(xn, b("mlp_up_w"), b("mlp_up_b"))
    out = lin64(gelu64(up) if gelu else up, b("mlp_down_w"), b("mlp_down_b"))
    return rms64(bf(h + out), p["final_ln_scale"].numpy())


def test_mlp_only_block_is_the_per_token_formula():
    """Attention branch zero (its output is 0 + bias 0): each token is
    rms(e + W2 gelu(W1 rms(e; ln2) + b1) + b2; final) on its own."""
    cfg = config(layers=1)
    p = params(cfg)
    zero_blocks(p)
    gen = torch.Generator().manual_seed(4)
    d, f = D_MODEL, 4 * D_MODEL
    p["token_embedding"] = torch.randn(VOCAB, d, generator=gen)
    p["blocks/0/mlp_up_w"] = torch.randn(d, f, generator=gen) / math.sqrt(d)
    p["blocks/0/mlp_up_b"] = 0.5 * torch.randn(f, generator=gen)
    p["blocks/0/mlp_down_w"] = torch.randn(f, d, generator=gen) / math.sqrt(f)
    p["blocks/0/mlp_down_b"] = 0.1 * torch.randn(d, generator=gen)
    for name in ("blocks/0/ln1_scale", "blocks/0/ln2_scale", "final_ln_scale"):
        p[name] = 1.0 + 0.5 * torch.randn(d, generator=gen)
    x = tokens()
    got = hidden(p, x, cfg)
    want = mlp_closed_form(p, x)
    assert close(got, want) <= 1.0
    assert close(mlp_closed_form(p, x, norm_scale="ln1_scale"), want) > 10
    assert close(mlp_closed_form(p, x, gelu=False), want) > 10
    # tokens are independent: permuting the sequence permutes the rows.
    perm = torch.randperm(SEQ, generator=gen)
    np.testing.assert_array_equal(hidden(p, x[:, perm], cfg), got[:, perm.numpy()])


def sign_embeddings(gen, rows, c):
    """Rows c_r * sigma_r with sigma_r in {-1, +1}^d: rms_norm gives sigma_r
    exactly in bf16 (1/sqrt(1 + 1e-5/c^2) rounds to 1)."""
    sigma = torch.where(torch.rand(rows, D_MODEL, generator=gen) < 0.5, -1.0, 1.0)
    return sigma, c[:, None] * sigma


@pytest.mark.parametrize("embeddings,semantic", [("untied", VOCAB), ("tied", VOCAB), ("untied", VOCAB - 7)])
def test_no_layers_closed_form_cross_entropy(embeddings, semantic):
    """layers = 0: hidden = sigma_x exactly, logits = alpha_v * <sigma_x,
    sigma'_v> are exact small integers times bf16 alphas, and the mean loss is
    logsumexp over the semantic rows minus the target logit, in float64."""
    cfg = config(layers=0, embeddings=embeddings, semantic_vocab_size=semantic)
    p = params(cfg)
    gen = torch.Generator().manual_seed(5)
    c = torch.from_numpy(bf(2.0 + 2.0 * torch.rand(VOCAB, generator=gen).numpy())).float()
    sig_in, p["token_embedding"] = sign_embeddings(gen, VOCAB, c)
    if embeddings == "untied":
        alpha = torch.from_numpy(bf(0.05 * torch.rand(VOCAB, generator=gen).numpy() + 0.01)).float()
        sig_out, p["output_embedding"] = sign_embeddings(gen, VOCAB, alpha)
        head, scale = sig_out.double().numpy(), alpha.double().numpy()
    else:
        head, scale = sig_in.double().numpy(), c.double().numpy() / 16.0
        p["token_embedding"] = p["token_embedding"] / 16.0  # keep the logits moderate; rms_norm is scale-free
    x = tokens(6)
    y = tokens(7) % semantic
    h = sig_in.double().numpy()[x.numpy()]  # [B, S, d]
    logits = (h @ head.T) * scale[None, None, :]
    logits = logits[..., :semantic]
    m = logits.max(-1, keepdims=True)
    lse = (m + np.log(np.exp(logits - m).sum(-1, keepdims=True)))[..., 0]
    target = np.take_along_axis(logits, y.numpy()[..., None].astype(np.int64), -1)[..., 0]
    want = float(np.mean(lse - target))
    with torch.no_grad():
        got = float(om.cross_entropy(p, x, y, cfg))
    assert abs(got - want) <= 1e-5 * abs(want)
    # mistake: the other head (tied <-> untied) or the storage rows in the softmax.
    if embeddings == "untied":
        other = (h @ sig_in.double().numpy().T) * c.double().numpy()[None, None, :]
        assert abs(float(np.mean(np.log(np.exp(other[..., :semantic]).sum(-1)))) - want) > 0.1
    if semantic < VOCAB:
        full = (h @ head.T) * scale[None, None, :]
        mf = full.max(-1, keepdims=True)
        lse_f = (mf + np.log(np.exp(full - mf).sum(-1, keepdims=True)))[..., 0]
        assert abs(float(np.mean(lse_f - target)) - want) > 1e-3


def test_completep_multiplier_table_by_hand():
    """optimizer_hyperparameter_trees (train.py:1274-1333) at width = depth = 2,
    alpha = 1: hidden lr = 1/2 * 2^0, vector lr = 2^0, hidden eps = 1/2 * 1/2,
    decay 2 on hidden weights; token embedding eps 1/2; output embedding lr 1/2,
    decay 2; the final norm all ones.  Standard parameterization: all ones."""
    table = {
        "blocks/0/qkv_w": (0.5, 0.25, 2.0), "blocks/1/mlp_down_w": (0.5, 0.25, 2.0),
        "blocks/0/qkv_b": (1.0, 0.25, 1.0), "blocks/1/ln2_scale": (1.0, 0.25, 1.0),
        "token_embedding": (1.0, 0.5, 1.0), "output_embedding": (0.5, 1.0, 2.0),
        "final_ln_scale": (1.0, 1.0, 1.0),
    }
    from gptrig.optim import OptimizerConfig, multipliers, tensor_hparams

    for path, want in table.items():
        assert oopt.multipliers(path, "completep_fixed_tpp_v1", 2.0, 2.0, 1.0) == want, path
        assert multipliers(path, "completep_fixed_tpp_v1", 2.0, 2.0, 1.0) == want, path
        assert oopt.multipliers(path, "standard", 2.0, 2.0, 1.0) == (1.0, 1.0, 1.0)
    # alpha = 0.5 at depth 4: hidden lr = 1/2 * 4^-0.5 = 1/4, eps = 1/2 * 4^-0.5 = 1/4, vector lr = 1/2.
    assert oopt.multipliers("blocks/0/attn_w", "completep_fixed_tpp_v1", 2.0, 4.0, 0.5) == (0.25, 0.25, 2.0)
    assert oopt.multipliers("blocks/0/attn_b", "completep_fixed_tpp_v1", 2.0, 4.0, 0.5) == (0.5, 0.25, 1.0)
    # the kernel's table: (lr_mult, eps * eps_mult, wd * decay_mult if decayed else 0); batch/data multipliers
    # scale eps by sqrt(data/batch) and decay by sqrt(batch/data) (train.py:1416-1417).
    cfg = OptimizerConfig(adam_epsilon=1e-8, weight_decay=0.1, batch_multiplier=4.0, data_multiplier=1.0)
    rows = tensor_hparams(list(table), cfg, "completep_fixed_tpp_v1", 2.0, 2.0, 1.0)
    for (path, (lr_m, eps_m, dec_m)), row in zip(table.items(), rows):
        decayed = path.endswith("_w") or path.endswith("embedding")
        want = (lr_m, 1e-8 * 0.5 * eps_m, 0.1 * 2.0 * dec_m if decayed else 0.0)
        np.testing.assert_allclose(row, np.asarray(want, np.float32), rtol=1e-7, err_msg=path)


def test_completep_init_scales():
    """init_params (train.py:865-901) under completep: hidden weights std
    init_std / sqrt(width), the untied output embedding init_std / width,
    the token embedding init_std."""
    cfg = config(layers=2, d_model=256, heads=4, base_width=64, base_depth=1, vocab_size=512,
                 semantic_vocab_size=512, parameterization="completep_fixed_tpp_v1", depth_alpha=1.0)
    flat = om.flatten(om.init_params(cfg, 0))
    width = 4.0
    assert abs(float(np.std(flat["blocks/0/mlp_up_w"])) / (0.02 / math.sqrt(width)) - 1) < 0.01
    assert abs(float(np.std(flat["output_embedding"])) / (0.02 / width) - 1) < 0.01
    assert abs(float(np.std(flat["token_embedding"])) / 0.02 - 1) < 0.01
    std = om.flatten(om.init_params(replace(cfg, parameterization="standard"), 0))
    assert abs(float(np.std(std["blocks/0/mlp_up_w"])) / 0.02 - 1) < 0.01


def test_completep_adamw_first_steps_by_hand():
    """Two AdamW steps (train.py:1386-1445) with completep multipliers and a
    clip that is active on step 1 only, for one element of each tensor class."""
    cfg = oopt.OptimizerConfig(learning_rate=0.01, steps=10, warmup_steps=0, weight_decay=0.1, adam_epsilon=1e-3,
                               grad_clip=1.0)
    paths = ["blocks/0/qkv_w", "blocks/0/qkv_b", "token_embedding", "output_embedding"]
    p0 = {k: torch.tensor([0.5, -0.25]) for k in paths}
    p = {k: v.clone() for k, v in p0.items()}
    m = {k: torch.zeros(2) for k in paths}
    v = {k: torch.zeros(2) for k in paths}
    g1 = {k: torch.tensor([3.0, 0.0]) for k in paths}          # |g| = sqrt(4 * 9) = 6 -> clip 1/6
    g2 = {k: torch.tensor([0.1, 0.05]) for k in paths}        # |g| < 1 -> no clip
    lr1, n1 = oopt.adamw_step(p, g1, m, v, 1, cfg, "completep_fixed_tpp_v1", 2.0, 2.0, 1.0)
    assert abs(n1 - 6.0) < 1e-6
    lr2, _ = oopt.adamw_step(p, g2, m, v, 2, cfg, "completep_fixed_tpp_v1", 2.0, 2.0, 1.0)
    mult = {"blocks/0/qkv_w": (0.5, 0.25, 2.0), "blocks/0/qkv_b": (1.0, 0.25, 1.0),
            "token_embedding": (1.0, 0.5, 1.0), "output_embedding": (0.5, 1.0, 2.0)}
    for k in paths:
        lr_m, eps_m, dec_m = mult[k]
        eps = 1e-3 * eps_m
        decays = not k.endswith("_b")
        for j in range(2):
            w = float(p0[k][j])
            ga = 3.0 / (6.0 + 1e-6) if j == 0 else 0.0        # clipped step-1 gradient
            mm, vv = 0.1 * ga, 0.05 * ga * ga
            w = w - lr1 * lr_m * ((mm / 0.1) / (math.sqrt(vv / 0.05) + eps) + (0.1 * dec_m * w if decays else 0.0))
            gb = float(g2[k][j])
            mm, vv = 0.9 * mm + 0.1 * gb, 0.95 * vv + 0.05 * gb * gb
            bc1, bc2 = 1 - 0.9 ** 2, 1 - 0.95 ** 2
            w = w - lr2 * lr_m * ((mm / bc1) / (math.sqrt(vv / bc2) + eps) + (0.1 * dec_m * w if decays else 0.0))
            assert abs(float(p[k][j]) - w) <= 1e-6 * max(1.0, abs(w)), (k, j)


# --- routed (MoE) blocks: recipes/reference_moe/train.py:1230-1371,1374-1560 ---

E_MOE, MULT = 4, 2


def moe_config(**kw) -> om.Config:
    return config(layers=1, experts=E_MOE, expert_top_k=2, expert_mult=MULT, mlp_mult=2 * MULT, **kw)


def moe_params(cfg, gen):
    p = params(cfg)
    d, eh = D_MODEL, MULT * D_MODEL
    p["token_embedding"] = torch.randn(VOCAB, d, generator=gen)
    p["blocks/0/expert_up_w"] = torch.randn(E_MOE, d, eh, generator=gen) / math.sqrt(d)
    p["blocks/0/expert_up_b"] = 0.3 * torch.randn(E_MOE, eh, generator=gen)
    p["blocks/0/expert_down_w"] = torch.randn(E_MOE, eh, d, generator=gen) / math.sqrt(eh)
    p["blocks/0/expert_down_b"] = 0.1 * torch.randn(E_MOE, d, generator=gen)
    return p


def test_moe_init_leaf_order_and_draws():
    """init_params (reference_moe/train.py:894-944): the routed block's leaves in
    the reference's order, router N(0, 0.02), expert biases zero."""
    cfg = moe_config()
    flat = om.flatten(om.init_params(cfg, 0))
    names = [k.split("/")[-1] for k in flat if k.startswith("blocks/0/")]
    assert tuple(names) == om.MOE_BLOCK_LEAVES
    assert flat["blocks/0/router_w"].shape == (D_MODEL, E_MOE)
    assert flat["blocks/0/expert_up_w"].shape == (E_MOE, D_MODEL, MULT * D_MODEL)
    assert not np.any(flat["blocks/0/expert_up_b"]) and not np.any(flat["blocks/0/expert_down_b"])


def test_identical_experts_reduce_to_the_dense_block():
    """Every expert the same MLP: the renormalised top-k gates sum to one, so
    the routed block equals a dense block with that MLP (up to the bf16
    rounding of the gates and of the scatter-add)."""
    gen = torch.Generator().manual_seed(8)
    mcfg = moe_config()
    p = moe_params(mcfg, gen)
    p["blocks/0/router_w"] = torch.randn(D_MODEL, E_MOE, generator=gen)
    for name in ("expert_up_w", "expert_up_b", "expert_down_w", "expert_down_b"):
        p[f"blocks/0/{name}"] = p[f"blocks/0/{name}"][:1].expand_as(p[f"blocks/0/{name}"]).clone()
    dcfg = config(layers=1, mlp_mult=MULT)
    dense = {k: v for k, v in p.items() if "expert" not in k and "router" not in k}
    dense["blocks/0/mlp_up_w"] = p["blocks/0/expert_up_w"][0]
    dense["blocks/0/mlp_up_b"] = p["blocks/0/expert_up_b"][0]
    dense["blocks/0/mlp_down_w"] = p["blocks/0/expert_down_w"][0]
    dense["blocks/0/mlp_down_b"] = p["blocks/0/expert_down_b"][0]
    x = tokens()
    got = hidden(p, x, mcfg)
    want = hidden(dense, x, dcfg)
    # (floor 1: the gates' bf16 rounding, about 2^-8 of the branch, shows up in
    # full where the residual and the branch nearly cancel; the outputs are
    # RMS-normalised, so of order 1.)
    assert close(got, want, floor=1.0) <= 1.0
    # mistake: gates taken from the full softmax (not renormalised over the chosen experts)
    scale = 2.0 / E_MOE
    half = {k: v.clone() for k, v in dense.items()}
    half["blocks/0/mlp_down_w"] = half["blocks/0/mlp_down_w"] * scale
    half["blocks/0/mlp_down_b"] = half["blocks/0/mlp_down_b"] * scale
    assert close(hidden(half, x, dcfg), want, floor=1.0) > 10


def test_zero_router_routes_to_the_first_experts_with_unit_balance_loss():
    """Zero router weights: every probability is 1/E and top-2 ties go to the
    lower indices, so each token uses experts 0 and 1 with gates 1/2; the load
    is (1/2, 1/2, 0, ...), the balance loss E * sum(load * P) is exactly 1,
    and the block output is the mean of the two experts' MLPs."""
    gen = torch.Generator().manual_seed(9)
    cfg = moe_config()
    p = moe_params(cfg, gen)
    p["blocks/0/router_w"].zero_()
    x = tokens()
    with torch.no_grad():
        h, balance, loads = om.gpt_hidden_and_router(p, x, cfg)
    assert float(balance) == 1.0
    np.testing.assert_array_equal(loads.numpy(), [[0.5, 0.5, 0.0, 0.0]])
    # The block equals a dense one whose MLP is the two experts side by side
    # with the down projection halved (the mean of the two experts' outputs).
    b = lambda n: p[f"blocks/0/{n}"].numpy()  # noqa: E731
    up = np.concatenate([b("expert_up_w")[0], b("expert_up_w")[1]], axis=1)
    upb = np.concatenate([b("expert_up_b")[0], b("expert_up_b")[1]])
    down = np.concatenate([b("expert_down_w")[0], b("expert_down_w")[1]], axis=0) * 0.5
    downb = 0.5 * (b("expert_down_b")[0] + b("expert_down_b")[1])
    dcfg = config(layers=1, mlp_mult=2 * MULT)
    dense = {k: v for k, v in p.items() if "expert" not in k and "router" not in k}
    dense["blocks/0/mlp_up_w"] = torch.from_numpy(up)
    dense["blocks/0/mlp_up_b"] = torch.from_numpy(upb)
    dense["blocks/0/mlp_down_w"] = torch.from_numpy(down)
    dense["blocks/0/mlp_down_b"] = torch.from_numpy(downb)
    assert close(h.double().numpy(), hidden(dense, x, dcfg), floor=1.0) <= 1.0
    # The training objective adds coefficient x balance (reference_moe/train.py:1557-1558).
    y = tokens(10)
    with torch.no_grad():
        ce = om.cross_entropy(p, x, y, om.replace(cfg, router_aux_coefficient=0.0))
        total = om.cross_entropy(p, x, y, cfg)
    assert abs(float(total) - float(ce) - 0.01) <= 1e-6


def test_balance_loss_router_gradient_closed_form():
    """d/d router_w of E * sum_e load_e * mean_t softmax(x_t W)_e with the load
    a constant (counts carry no gradient, reference_moe/train.py:1272,1296):
    grad[d, k] = E / T * sum_t x_td p_tk (load_k - sum_e load_e p_te)."""
    gen = torch.Generator().manual_seed(10)
    T, d = 40, 16
    xt = torch.randn(T, d, generator=gen)
    w = (0.5 * torch.randn(d, E_MOE, generator=gen)).requires_grad_(True)
    logits = xt @ w
    probs = torch.softmax(logits, -1)
    _, chosen = om.omoe.top_k(logits.detach(), 2)
    load = torch.bincount(chosen.reshape(-1).long(), minlength=E_MOE).float() / (T * 2)
    om.omoe.load_balance_loss(probs.mean(0), load).backward()
    x64, p64, l64 = xt.double().numpy(), probs.detach().double().numpy(), load.double().numpy()
    want = E_MOE / T * x64.T @ (p64 * (l64[None, :] - (p64 * l64[None, :]).sum(-1, keepdims=True)))
    np.testing.assert_allclose(w.grad.double().numpy(), want, rtol=1e-5, atol=1e-7)
