"""20-step config-A training trajectory on the GPU vs the CPU oracle's.

The expected rows are the committed fixture ``tests/golden/config_a_trajectory.json``
written by ``tests/golden/make_trajectory.py`` (the oracle's ``train_step`` on
the same seed-0 parameters and token windows).

Gates (the north star's "20-step loss trajectory within 1%", on every step):
  * every step's loss within 1% of the oracle's, steps 1-5 within 0.1%;
  * learning rate identical (1e-6 relative);
  * gradient norm within 1% over steps 1-3, median relative difference <= 5%.
For scale: two exact restatements of the same step that the reference itself
treats as equivalent (its dense attention backend instead of the flash
semantics; float64 instead of float32 accumulation in the linears) stay within
0.21% of this fixture on every step (``tests/golden/config_a_trajectory_*.json``,
pinned by ``tests/test_golden_fixture.py``), and this GPU path within 0.15%.
The gradient norm is the noisier figure (Adam turns last-bit gradient
differences into parameter differences): those variants differ by up to 10%
on single steps.
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
    print("loss relative differences", np.round(loss_rel, 5).tolist(), flush=True)
    assert np.all(loss_rel[:5] <= 1e-3), loss_rel[:5]
    assert float(loss_rel.max()) <= 1e-2, loss_rel
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    rel = np.abs(got[:, 2] - want[:, 2]) / want[:, 2]
    assert np.all(rel[:3] <= 1e-2), rel[:3]
    assert float(np.median(rel)) <= 5e-2, rel
