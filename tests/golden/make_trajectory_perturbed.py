"""Write the config-A 20-step trajectory of the CPU oracle under a variation
that the reference itself treats as the same computation, to measure how far
two correct implementations of the step drift apart on this chaotic run.

Identical to ``make_trajectory.py`` (same config, seed-0 parameters and token
windows) except for one of:

* ``f64_linear``: every dense linear (``rig/nn.py:55-56``) accumulates its
  bf16 products in float64 instead of float32 before the bf16 rounding (the
  reference fixes the result only up to the accumulation order of its dots);
* ``dense_attention``: the reference's own dense attention backend
  (``recipes/reference/train.py:1151-1162``: QK^T rounded to bf16, mask
  ``finfo(f32).min``; the backend its train.py runs off TPU) instead of the
  Pallas kernel's numerics (``rig/kernels/tpu_flash_attention.py:236-349``);
* ``normalized_attention``: the attention forward of the kernel's test
  oracle (``tpu_flash_attention.py:171-207``: the normalised softmax rounded
  to bf16 before the PV product) instead of the kernel's (the unnormalised
  ``exp(s - running max)`` rounded per 256-key chunk).

* ``eight_threads``: nothing but the CPU thread count (8 instead of the
  fixture's 3), which changes torch's float32 summation order.

Usage: ``python tests/golden/make_trajectory_perturbed.py f64_linear|dense_attention|normalized_attention|eight_threads
[spike|long_warmup]`` (10-40 minutes on 8 cores).  Output:
``tests/golden/config_a_trajectory_<variation>.json`` (``config_a_long_warmup_trajectory_<variation>.json``
for the second schedule, see ``make_trajectory.py``).
"""

from __future__ import annotations

import json
import os
import sys
import time
from dataclasses import replace

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, HERE)

import torch  # noqa: E402

from make_trajectory import fixture_name, schedule_config  # noqa: E402
from oracle import attention as oattn  # noqa: E402
from oracle import model as om  # noqa: E402

STEPS = 20
SEED = 0
THREADS = 3  # as make_trajectory.py


def linear_f64(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``rig/nn.py:55-56`` with float64 accumulation; the backward of the
    float64 matmul also accumulates in float64."""

    y = torch.matmul(x.to(torch.float64), weight.to(dtype).to(torch.float64)).to(dtype)
    return y + bias.to(dtype)


def main() -> None:
    variation = sys.argv[1] if len(sys.argv) > 1 else "f64_linear"
    schedule = sys.argv[2] if len(sys.argv) > 2 else "spike"
    torch.set_num_threads(8 if variation == "eight_threads" else THREADS)
    config = schedule_config(schedule)
    if variation == "f64_linear":
        om.linear = linear_f64
        note = "dense linears accumulate in float64 instead of float32"
    elif variation == "dense_attention":
        config = replace(config, attention_backend="dense")
        note = "the reference's dense attention backend (train.py:1151-1162) instead of the flash kernel's numerics"
    elif variation == "eight_threads":
        note = "the same computation on 8 CPU threads instead of 3 (float32 summation order)"
    elif variation == "normalized_attention":
        def normalized(q, k, v, *, softmax_scale=None, segment_ids=None):
            return oattn.attention_forward(q, k, v, softmax_scale=softmax_scale, segment_ids=segment_ids)

        oattn.flash_attention_forward = normalized
        note = ("the kernel's test-oracle attention forward (tpu_flash_attention.py:171-207, normalised "
                "probabilities rounded) instead of the kernel's own (:236-349)")
    else:
        raise SystemExit(f"unknown variation {variation!r}")
    windows = om.synthetic_windows(SEED, STEPS, config.batch_size, config.seq_len, config.vocab_size)
    state = om.init_state(config, SEED)
    rows = []
    for i in range(STEPS):
        t0 = time.time()
        w = torch.from_numpy(windows[i])
        rec = om.train_step(state, w[:, :-1], w[:, 1:], config)
        rows.append([rec["loss"], rec["learning_rate"], rec["grad_norm"]])
        print(f"step {i + 1}: {rows[-1]} ({time.time() - t0:.1f} s)", flush=True)
    out = {
        "config": (f"A: 8L d512 8x64 vocab 50304 seq 1024 batch 8, AdamW lr 2^-8 warmup "
                   f"{config.optimizer.warmup_steps} of {config.optimizer.steps} steps, cosine, first {STEPS} steps"),
        "perturbation": note,
        "seed": SEED,
        "windows": "numpy default_rng(0).integers(0, 50304, (20, 8, 1025), int32)",
        "columns": ["loss", "learning_rate", "grad_norm"],
        "rows": rows,
    }
    with open(os.path.join(HERE, fixture_name(schedule, variation)), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
