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
