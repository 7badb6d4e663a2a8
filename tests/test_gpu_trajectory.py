"""20-step config-A training trajectory on the GPU vs the CPU oracle's.

The expected rows are the committed fixture ``tests/golden/config_a_trajectory.json``
written by ``tests/golden/make_trajectory.py`` (the oracle's ``train_step`` on
the same seed-0 parameters and token windows).

This run (base LR 2^-8 after a 2-step warmup) is chaotic: Adam's normalised
updates turn last-bit differences of near-zero gradient components into
full-size parameter differences, and the loss jumps (step 4's gradient norm
is 12x step 3's).  Three GPU runs of this very test, differing only in the
order of fp32 atomic additions, differ from each other by up to 1.3% in
single-step loss and by up to 8x in single-step gradient norm (spikes at
different steps).  The gates are therefore:
  * steps 1-5 (before the divergence grows): loss within 0.2% of the oracle,
    gradient norm within 1% over steps 1-3;
  * all 20 steps: mean relative loss difference <= 1% and every step <= 2.5%;
  * learning rate identical (1e-6 relative); median relative gradient-norm
    difference <= 10%.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "config_a_trajectory.json")


def test_config_a_twenty_step_trajectory_matches_oracle():
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    with open(FIXTURE) as f:
        want = np.asarray(json.load(f)["rows"], dtype=np.float64)
    steps = want.shape[0]
    ocfg = om.baseline_config("A", steps=steps)
    cfg = GPTConfig(layers=ocfg.layers, heads=ocfg.heads, d_model=ocfg.d_model, vocab_size=ocfg.vocab_size,
                    semantic_vocab_size=ocfg.semantic_vocab_size, seq_len=ocfg.seq_len,
                    batch_size=ocfg.batch_size, micro_batch_size=ocfg.batch_size, base_width=ocfg.base_width,
                    base_depth=ocfg.base_depth, attention_scale=ocfg.attention_scale, embeddings=ocfg.embeddings,
                    optimizer=OptimizerConfig(learning_rate=ocfg.optimizer.learning_rate, steps=steps,
                                              warmup_steps=ocfg.optimizer.warmup_steps))
    windows = torch.from_numpy(om.synthetic_windows(0, steps, cfg.batch_size, cfg.seq_len, cfg.vocab_size))
    print(f"trajectory case config A, {steps} steps", flush=True)
    trainer = GPTTrainer(cfg, seed=0)
    dev_windows = windows.cuda()
    for i in range(steps):
        trainer.train_step(dev_windows[i, :, :-1], dev_windows[i, :, 1:])
    got = trainer.history_rows()
    print("gpu losses   ", np.round(got[:, 0], 4).tolist(), flush=True)
    print("oracle losses", np.round(want[:, 0], 4).tolist(), flush=True)
    print("gpu grad norms   ", np.round(got[:, 2], 4).tolist(), flush=True)
    print("oracle grad norms", np.round(want[:, 2], 4).tolist(), flush=True)
    loss_rel = np.abs(got[:, 0] - want[:, 0]) / want[:, 0]
    assert np.all(loss_rel[:5] <= 2e-3), loss_rel[:5]
    assert float(loss_rel.mean()) <= 1e-2 and float(loss_rel.max()) <= 2.5e-2, loss_rel
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    rel = np.abs(got[:, 2] - want[:, 2]) / want[:, 2]
    assert np.all(rel[:3] <= 1e-2), rel[:3]
    assert float(np.median(rel)) <= 1e-1, rel
