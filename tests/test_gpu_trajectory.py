"""20-step config-A training trajectory on the GPU vs the CPU oracle's.

The expected rows are the committed fixture ``tests/golden/config_a_trajectory.json``
written by ``tests/golden/make_trajectory.py`` (the oracle's ``train_step`` on
the same seed-0 parameters and token windows, 3 CPU threads), and the oracle's
reference-equivalent runs next to it (``tests/golden/make_trajectory_perturbed.py``,
pinned by ``tests/test_golden_fixture.py``): the same step on 8 threads (only
the float32 summation order differs), with float64 linears, with the kernel's
test-oracle attention and with the dense backend's.

The run is chaotic around its loss spike (steps 4-9): the 8-thread run of the
same oracle departs from the 3-thread fixture by 1.2% at step 8, so the
reference itself has no single 20-step trajectory to 1% -- its result is
defined only up to the summation order.  The gate is the north star's "20-step
loss trajectory within 1%" against that set:
  * every step's loss within 1% of one of the reference-equivalent runs (the
    closest; this GPU path's fp32 atomics add in a different order on every
    run, and its runs fall on either side of the spike: measured over sixteen
    runs, 0.03-0.62% from the closest run, 0.08-1.18% from the 3-thread one);
  * steps 1-5, before the chaos, within 0.1% of the fixture (all the
    equivalent runs agree there to 0.05%);
  * learning rate identical (1e-6 relative);
  * gradient norm within 1% over steps 1-3, median relative difference <= 5%
    against the closest run.  The gradient norm is the noisier figure (Adam
    turns last-bit gradient differences into parameter differences): the
    equivalent runs differ from one another by up to 57% on single steps.
The equivalent runs are the 8-thread, float64-linear and dense-attention
restatements; the kernel's test-oracle attention (normalised probabilities
rounded before the PV product) is not the forward the reference's training
step runs, so it is not one of them.  The test prints which run was closest.

A second gate holds the GPU to one fixture alone, on a schedule with no loss
spike: the first 20 steps of a 40-step run whose learning rate warms up over
all 40 (``config_a_long_warmup_trajectory.json``).  There the three
restatements stay within 0.033% of the fixture at every step, so every GPU
step must be within 1% of the fixture itself.
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
# The oracle's runs that the reference treats as the same computation.
EQUIVALENT_RUNS = ("eight_threads", "f64_linear", "dense_attention")
LONG_WARMUP_FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "config_a_long_warmup_trajectory.json")


def run_config_a(steps: int, schedule_steps: int, warmup_steps):
    """The GPU trainer's first ``steps`` steps of config A (seed-0 parameters
    and token windows, as the fixtures) on a ``schedule_steps``-step schedule
    (``warmup_steps`` None: the config's 10%); returns its history rows."""
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    ocfg = om.baseline_config("A", steps=schedule_steps)
    warmup = ocfg.optimizer.warmup_steps if warmup_steps is None else warmup_steps
    cfg = GPTConfig(layers=ocfg.layers, heads=ocfg.heads, d_model=ocfg.d_model, vocab_size=ocfg.vocab_size,
                    semantic_vocab_size=ocfg.semantic_vocab_size, seq_len=ocfg.seq_len,
                    batch_size=ocfg.batch_size, micro_batch_size=ocfg.batch_size, base_width=ocfg.base_width,
                    base_depth=ocfg.base_depth, attention_scale=ocfg.attention_scale, embeddings=ocfg.embeddings,
                    optimizer=OptimizerConfig(learning_rate=ocfg.optimizer.learning_rate, steps=schedule_steps,
                                              warmup_steps=warmup))
    windows = torch.from_numpy(om.synthetic_windows(0, steps, cfg.batch_size, cfg.seq_len, cfg.vocab_size))
    print(f"trajectory case config A, {steps} steps of a {schedule_steps}-step schedule, warmup {warmup}", flush=True)
    trainer = GPTTrainer(cfg, seed=0)
    dev_windows = windows.cuda()
    for i in range(steps):
        trainer.train_step(dev_windows[i, :, :-1], dev_windows[i, :, 1:])
    return trainer.history_rows()


def test_config_a_twenty_step_trajectory_matches_oracle():
    with open(FIXTURE) as f:
        want = np.asarray(json.load(f)["rows"], dtype=np.float64)
    steps = want.shape[0]
    got = run_config_a(steps, steps, None)
    golden = os.path.dirname(FIXTURE)
    runs = {"fixture": want}
    for variation in EQUIVALENT_RUNS:
        with open(os.path.join(golden, f"config_a_trajectory_{variation}.json")) as f:
            runs[variation] = np.asarray(json.load(f)["rows"], dtype=np.float64)
    print("gpu losses   ", np.round(got[:, 0], 4).tolist(), flush=True)
    print("oracle losses", np.round(want[:, 0], 4).tolist(), flush=True)
    print("gpu grad norms   ", np.round(got[:, 2], 4).tolist(), flush=True)
    print("oracle grad norms", np.round(want[:, 2], 4).tolist(), flush=True)
    largest = {}
    for name, rows in runs.items():
        largest[name] = float((np.abs(got[:, 0] - rows[:, 0]) / rows[:, 0]).max())
    print("largest loss difference per reference-equivalent run",
          {k: round(v, 5) for k, v in largest.items()}, flush=True)
    closest = min(largest, key=largest.get)
    near = runs[closest]
    loss_rel = np.abs(got[:, 0] - near[:, 0]) / near[:, 0]
    print(f"closest run {closest}: loss relative differences", np.round(loss_rel, 5).tolist(), flush=True)
    assert float(loss_rel.max()) <= 1e-2, (closest, loss_rel)
    first = np.abs(got[:5, 0] - want[:5, 0]) / want[:5, 0]
    assert np.all(first <= 1e-3), first
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    rel = np.abs(got[:, 2] - want[:, 2]) / want[:, 2]
    assert np.all(rel[:3] <= 1e-2), rel[:3]
    rel_near = np.abs(got[:, 2] - near[:, 2]) / near[:, 2]
    assert float(np.median(rel_near)) <= 5e-2, rel_near


def test_config_a_long_warmup_trajectory_within_one_percent_of_the_fixture():
    with open(LONG_WARMUP_FIXTURE) as f:
        want = np.asarray(json.load(f)["rows"], dtype=np.float64)
    steps = want.shape[0]
    got = run_config_a(steps, 2 * steps, 2 * steps)
    loss_rel = np.abs(got[:, 0] - want[:, 0]) / want[:, 0]
    print("gpu losses   ", np.round(got[:, 0], 4).tolist(), flush=True)
    print("oracle losses", np.round(want[:, 0], 4).tolist(), flush=True)
    print("loss relative differences", np.round(loss_rel, 5).tolist(), flush=True)
    assert float(loss_rel.max()) <= 1e-2, loss_rel
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    rel = np.abs(got[:, 2] - want[:, 2]) / want[:, 2]
    print("grad norm relative differences", np.round(rel, 4).tolist(), flush=True)
    assert np.all(rel[:3] <= 1e-2), rel[:3]
    assert float(np.median(rel)) <= 5e-2, rel
