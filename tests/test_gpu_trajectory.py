"""20-step config-A training trajectory on the GPU vs the CPU oracle's.

The expected rows are the committed fixture ``tests/golden/config_a_trajectory.json``
written by ``tests/golden/make_trajectory.py`` (the oracle's ``train_step`` on
the same seed-0 parameters and token windows).

Gates (the north star's "20-step loss trajectory within 1%", on every step):
  * every step's loss within 1% of the oracle's, steps 1-5 within 0.1%;
  * learning rate identical (1e-6 relative);
  * gradient norm within 1% over steps 1-3, median relative difference <= 5%.
For scale (``tests/test_golden_fixture.py``): the oracle redone with a change
the reference treats as the same computation (float64 linears; the kernel's
test-oracle or the dense backend's attention instead of the Pallas kernel's
numerics) stays within 0.15% of this fixture, but the same oracle on 8 CPU
threads instead of 3 departs by 1.2% at step 8: around the loss spike (steps
4-9) the run is chaotic and any change of summation order moves it.  This GPU
path, whose fp32 atomics add in a different order on every run: 0.08-0.48%
over five runs.  The gradient norm is the noisier figure (Adam turns last-bit
gradient differences into parameter differences): the variants differ by up
to 5% on single steps, the 8-thread run by up to 57%.
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
