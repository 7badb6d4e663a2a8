"""Write two steps of the CPU oracle's config-D training step on two sequences.

Config D's model (the reference GPT 125M step: 12 layers, d_model 768,
12 heads x 64, MLP 3072, vocab 50304, seq 1024, untied head, AdamW base LR
2^-8 with a 2-step warmup of a 20-step cosine schedule), seed-0 parameters,
token windows from numpy ``default_rng(2)`` (``[2, 2, 1025]``: two steps of
two sequences).  Saved: the (loss, learning_rate, grad_norm) rows of both
steps and the float32 norm of every parameter's raw gradient at step 1.

Usage: ``python tests/golden/make_config_d_steps.py`` (a few minutes on 8
cores).  Output: ``tests/golden/config_d_two_steps.json``.
"""

from __future__ import annotations

import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import torch  # noqa: E402

from oracle import model as om  # noqa: E402

STEPS, BATCH, SEED, TOKEN_SEED = 2, 2, 0, 2


def main() -> None:
    torch.set_num_threads(max(1, len(os.sched_getaffinity(0))))
    config = om.replace(om.baseline_config("D", steps=20), batch_size=BATCH)
    windows = om.synthetic_windows(TOKEN_SEED, STEPS, BATCH, config.seq_len, config.vocab_size)
    state = om.init_state(config, SEED)
    rows, norms = [], {}
    for i in range(STEPS):
        t0 = time.time()
        w = torch.from_numpy(windows[i])
        grads = {} if i == 0 else None
        rec = om.train_step(state, w[:, :-1], w[:, 1:], config, grads_out=grads)
        rows.append([rec["loss"], rec["learning_rate"], rec["grad_norm"]])
        if grads is not None:
            norms = {k: float(g.double().norm()) for k, g in grads.items()}
        print(f"step {i + 1}: {rows[-1]} ({time.time() - t0:.1f} s)", flush=True)
    out = {
        "config": "D model: 12L d768 12x64 mlp 3072 vocab 50304 seq 1024 untied; batch 2; AdamW lr 2^-8 warmup 2 of 20",
        "seed": SEED,
        "windows": "numpy default_rng(2).integers(0, 50304, (2, 2, 1025), int32)",
        "columns": ["loss", "learning_rate", "grad_norm"],
        "rows": rows,
        "step1_grad_norms": norms,
    }
    with open(os.path.join(HERE, "config_d_two_steps.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
