"""Host-side validation of the trainer's configuration (CPU)."""

from __future__ import annotations

from dataclasses import replace

import pytest


def routed(**kw):
    from gptrig.train import GPTConfig

    base = dict(layers=2, heads=2, d_model=128, vocab_size=1000, semantic_vocab_size=997, seq_len=128, batch_size=4,
                micro_batch_size=4, experts=4, expert_top_k=2, expert_mult=2, mlp_mult=4, base_width=128, base_depth=2)
    base.update(kw)
    return GPTConfig(**base)


def test_routed_config_rules():
    """recipes/reference_moe/train.py:362-371: top_k <= experts and
    top_k * expert_mult == mlp_mult; plus this build's one-pass rule (the
    balance loss is a product of two global-batch means) and the router
    kernel's limits."""
    routed().validate()
    with pytest.raises(ValueError):
        routed(expert_top_k=5).validate()
    with pytest.raises(ValueError):
        routed(expert_mult=3).validate()
    with pytest.raises(ValueError):
        routed(micro_batch_size=2).validate()
    with pytest.raises(ValueError):
        routed(experts=32, expert_top_k=2).validate()
    cfg = routed()
    replace(cfg, experts=0, micro_batch_size=2).validate()  # dense: micro-batching allowed


def test_routed_init_leaves_follow_the_reference_order():
    """init_params (reference_moe/train.py:894-944) is bit-identical to the
    oracle's restatement, leaf order included."""
    import numpy as np

    from gptrig.train import init_params
    from oracle import model as om

    cfg = routed()
    ocfg = om.Config(layers=2, heads=2, d_model=128, vocab_size=1000, semantic_vocab_size=997, seq_len=128,
                     batch_size=4, experts=4, expert_top_k=2, expert_mult=2, mlp_mult=4, embeddings="untied",
                     base_width=128, base_depth=2)
    got = init_params(cfg, 5)
    want = om.flatten(om.init_params(ocfg, 5))
    assert list(got) == list(want)
    for k in want:
        np.testing.assert_array_equal(got[k], want[k])


def test_optimizer_host_scalars_at_batch_data_ratio_four():
    """The trainer's host-side optimizer scalars at batch_multiplier /
    data_multiplier = 2 / 0.5 = 4, worked by hand (train.py:1231, :1336-1345,
    :1413-1414): betas 0.6 / 0.8, learning rate x 2, and the kernel's
    per-tensor table with epsilon x 1/2 and weight decay x 2 (0 on biases and
    norm scales); ratio 10.5 and 0 are rejected like the reference's."""
    import numpy as np

    from gptrig.optim import OptimizerConfig, effective_adam_betas, learning_rate, tensor_hparams

    cfg = OptimizerConfig(learning_rate=0.01, warmup_steps=10, steps=1010, min_lr_ratio=1.0, weight_decay=0.1,
                          adam_epsilon=0.2, batch_multiplier=2.0, data_multiplier=0.5)
    b1, b2 = effective_adam_betas(cfg)
    assert abs(b1 - 0.6) < 1e-12 and abs(b2 - 0.8) < 1e-12
    assert abs(learning_rate(10, cfg) - 0.02) < 1e-9 and abs(learning_rate(5, cfg) - 0.01) < 1e-9
    paths = ["token_embedding", "blocks/0/qkv_w", "blocks/0/qkv_b", "blocks/0/ln1_scale", "final_ln_scale",
             "output_embedding"]
    table = tensor_hparams(paths, cfg, "standard", 1.0, 1.0, 0.0)
    want = np.array([[1, 0.1, 0.2], [1, 0.1, 0.2], [1, 0.1, 0.0], [1, 0.1, 0.0], [1, 0.1, 0.0], [1, 0.1, 0.2]],
                    np.float32)
    np.testing.assert_allclose(table, want, rtol=1e-6)
    for bm in (10.5, 0.0):
        with pytest.raises(ValueError):
            effective_adam_betas(replace(cfg, batch_multiplier=bm, data_multiplier=1.0))
