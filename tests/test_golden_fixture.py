"""Checks of the committed config-A trajectory fixture (CPU).

The fixture holds the oracle's 20-step (loss, learning rate, grad norm)
history; the GPU trajectory test compares against it.  Here its columns are
checked against what the mathematics fixes independently of the oracle's code:
the learning-rate column against the closed-form warmup + cosine schedule of
``recipes/reference/train.py:1219-1236`` (base 2^-8, 2 warmup steps of 20,
floor 0.1), and the first loss against ln(V) for a near-uniform softmax at
std-0.02 initialisation.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "config_a_trajectory.json")


def closed_form_lr(step: int, steps: int = 20, warmup: int = 2, base: float = 2.0 ** -8, floor: float = 0.1):
    w = min(1.0, step / warmup)
    progress = min(max((step - warmup) / max(1, steps - warmup), 0.0), 1.0)
    return base * w * (floor + (1.0 - floor) * 0.5 * (1.0 + math.cos(math.pi * progress)))


def test_fixture_shape_and_learning_rate_column():
    with open(FIXTURE) as f:
        data = json.load(f)
    rows = np.asarray(data["rows"], dtype=np.float64)
    assert rows.shape == (20, 3)
    want = np.array([closed_form_lr(s) for s in range(1, 21)])
    np.testing.assert_allclose(rows[:, 1], want, rtol=1e-6)
    assert np.all(np.isfinite(rows)) and np.all(rows[:, 2] > 0)


def test_fixture_first_loss_is_near_uniform():
    with open(FIXTURE) as f:
        rows = np.asarray(json.load(f)["rows"], dtype=np.float64)
    assert abs(rows[0, 0] - math.log(50304)) <= 0.02 * math.log(50304)


# Largest per-step loss difference from the fixture that each variation was
# measured at (tests/golden/make_trajectory_perturbed.py), with a margin.
SEMANTIC_BOUNDS = {  # measured 0.10%, 0.14%, 0.15%, all at step 8
    "f64_linear": 3e-3,
    "normalized_attention": 3e-3,
    "dense_attention": 3e-3,
}
THREADS_BOUND = 1.5e-2  # measured 1.22% at step 8


def check_variation(variation, bound, base):
    path = os.path.join(os.path.dirname(__file__), "golden", f"config_a_trajectory_{variation}.json")
    with open(path) as f:
        rows = np.asarray(json.load(f)["rows"], dtype=np.float64)
    loss_rel = np.abs(rows[:, 0] - base[:, 0]) / base[:, 0]
    assert float(loss_rel.max()) <= bound, (variation, loss_rel)
    assert float(loss_rel.max()) > 0.0, variation  # the variation does change the run
    assert float(loss_rel[:5].max()) <= 5e-4, variation  # before the loss spike
    np.testing.assert_allclose(rows[:, 1], base[:, 1], rtol=1e-7)
    assert float(np.abs(rows[0, 2] - base[0, 2]) / base[0, 2]) <= 5e-3, variation
    return float(loss_rel.max())


def test_equivalent_restatements_stay_within_the_trajectory_gate():
    """The basis of the GPU trajectory gate: the oracle's 20-step run redone
    with a change the reference itself treats as the same computation --
    float64 accumulation in the linears, or the attention forward of the
    kernel's test oracle (normalised probabilities rounded) or of the
    reference's dense backend (``recipes/reference/train.py:1151-1162``)
    instead of the Pallas kernel's numerics -- stays within 0.3% of the
    fixture's loss on every step (the gate is 1%), with identical learning
    rates and first-step gradient norms to 0.5%; single-step gradient norms
    differ by up to 5% (and the dense backend's by 4x at step 20)."""
    with open(FIXTURE) as f:
        base = np.asarray(json.load(f)["rows"], dtype=np.float64)
    for variation, bound in SEMANTIC_BOUNDS.items():
        check_variation(variation, bound, base)


def test_summation_order_alone_moves_the_loss_spike():
    """The same oracle on 8 CPU threads instead of the fixture's 3 (only the
    float32 summation order changes) follows the fixture to 0.05% through
    step 5 and then departs by 1.2% at step 8, outside the north star's 1%
    gate: around its loss spike (steps 4-9) this run is chaotic, so the gate
    is tight there for any implementation whose reductions add in another
    order, the reference's own included."""
    with open(FIXTURE) as f:
        base = np.asarray(json.load(f)["rows"], dtype=np.float64)
    assert check_variation("eight_threads", THREADS_BOUND, base) > 1e-2


LONG_WARMUP = os.path.join(os.path.dirname(__file__), "golden", "config_a_long_warmup_trajectory.json")
LONG_WARMUP_RUNS = ("eight_threads", "f64_linear", "dense_attention")


def test_long_warmup_fixture_learning_rate_column():
    """The second schedule: 40 steps warming up over all 40, so the decay span
    is max(1, 0) = 1, the cosine factor stays 1 and the rate is 2^-8 * step / 40
    (``recipes/reference/train.py:1219-1236``) -- at most 2^-9 over the 20
    stored steps."""
    with open(LONG_WARMUP) as f:
        rows = np.asarray(json.load(f)["rows"], dtype=np.float64)
    assert rows.shape == (20, 3)
    np.testing.assert_allclose(rows[:, 1], [2.0 ** -8 * s / 40 for s in range(1, 21)], rtol=1e-6)
    np.testing.assert_allclose(rows[:, 1], [closed_form_lr(s, steps=40, warmup=40) for s in range(1, 21)],
                               rtol=1e-6)
    assert abs(rows[0, 0] - math.log(50304)) <= 0.02 * math.log(50304)
    assert np.all(np.isfinite(rows)) and np.all(rows[:, 2] > 0)


def test_long_warmup_restatements_agree_to_a_tenth_of_a_percent():
    """The basis of the GPU's one-fixture gate: on the long-warmup schedule the
    three reference-equivalent restatements (8 threads, float64 linears, the
    dense attention backend) stay within 0.1% of the fixture's loss at every
    step (measured: 0.028%, 0.030%, 0.033%, all at step 16), ten times inside
    the 1% gate, with identical learning rates."""
    with open(LONG_WARMUP) as f:
        base = np.asarray(json.load(f)["rows"], dtype=np.float64)
    for variation in LONG_WARMUP_RUNS:
        path = os.path.join(os.path.dirname(__file__), "golden",
                            f"config_a_long_warmup_trajectory_{variation}.json")
        with open(path) as f:
            rows = np.asarray(json.load(f)["rows"], dtype=np.float64)
        loss_rel = np.abs(rows[:, 0] - base[:, 0]) / base[:, 0]
        assert float(loss_rel.max()) <= 1e-3, (variation, loss_rel)
        assert float(loss_rel.max()) > 0.0, variation
        np.testing.assert_allclose(rows[:, 1], base[:, 1], rtol=1e-7)
