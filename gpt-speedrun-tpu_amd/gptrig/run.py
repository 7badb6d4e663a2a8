"""A training run on synthetic tokens that leaves a reference-shaped run directory.

The caller side of the step (``recipes/reference/train.py:run``, artefacts at
``:2194-2366``, result line at ``:2411-2415``), cut down to what one GPU and
synthetic data can honestly fill: ``training.riglog`` (loss / learning rate /
gradient norm of every step), ``validation.csv`` (one canonical row from the
masked eval step on held-out synthetic windows), ``checkpoint.npz`` and
``metrics.json``, then ``RIG_RESULT=<json>`` as the last stdout line.  Every
step and the evaluation run through the HIP library; this module only draws
tokens, times and writes files.

The FLOP count is analytic (causal-exact matmul FLOPs, 3x forward), not the
reference's traced jaxpr count; ``flop_accounting.method`` says so.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import sys
import time
from pathlib import Path
from typing import Any

import torch

from . import runlog
from .optim import OptimizerConfig
from .train import GPTConfig, GPTTrainer

MI355X_BF16_DENSE_TFLOPS = 2500.0


def flops_per_token(config: GPTConfig) -> int:
    """Training FLOPs per token: 3 x (2 x linear weights + LM head, plus QK^T and
    PV over the causal prefix, on average (S+1)/2 keys)."""

    d, L = config.d_model, config.layers
    linear = (4 + 2 * config.mlp_mult) * d * d * L  # qkv 3d^2, out d^2, up + down 2*mult*d^2
    forward = 2 * linear + 2 * d * config.vocab_size + 2 * d * (config.seq_len + 1) * L
    return 3 * forward


def _windows(generator: torch.Generator, config: GPTConfig, rows: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    tokens = torch.randint(0, config.semantic_vocab_size, (rows, config.seq_len + 1), generator=generator,
                           device=device, dtype=torch.int32)
    return tokens[:, :-1].contiguous(), tokens[:, 1:].contiguous()


def model_metadata(config: GPTConfig) -> dict[str, Any]:
    """Architecture fields (``recipes/reference/train.py:904-920``)."""

    return {"layers": config.layers, "heads": config.heads, "d_model": config.d_model, "mlp_mult": config.mlp_mult,
            "normalization": "rmsnorm", "position_encoding": "rope", "mlp_activation": "gelu_tanh",
            "vocab_size": config.vocab_size, "semantic_vocab_size": config.semantic_vocab_size,
            "tied_embeddings": config.embeddings == "tied", "parameterization": config.parameterization}


def run(config: GPTConfig, output_dir, *, seed: int = 0, data_seed: int = 1, stop_after_step: int | None = None,
        validation_batches: int = 1, checkpoint: bool = True, device: str = "cuda:0",
        peak_tflops: float = MI355X_BF16_DENSE_TFLOPS) -> dict[str, Any]:
    """Train ``config.optimizer.steps`` steps (or ``stop_after_step`` of them,
    the schedule unchanged), evaluate, write the run directory; returns the result."""

    schedule_steps = config.optimizer.steps
    final_step = schedule_steps if stop_after_step is None else int(stop_after_step)
    if not 0 < final_step <= schedule_steps:
        raise ValueError(f"stop_after_step {final_step} is past the {schedule_steps}-step schedule")
    if validation_batches <= 0:
        raise ValueError("validation_batches must be positive")
    out = Path(output_dir).expanduser().resolve()
    dev = torch.device(device)
    trainer = GPTTrainer(config, seed=seed, device=device, history_steps=schedule_steps)
    tokens_per_step = config.batch_size * config.seq_len
    train_gen = torch.Generator(device=dev).manual_seed(data_seed)

    torch.cuda.synchronize(dev)
    start = time.perf_counter()
    for _ in range(final_step):
        trainer.train_step(*_windows(train_gen, config, config.batch_size, dev))
    torch.cuda.synchronize(dev)
    train_seconds = runlog.finite_metric("train_seconds", time.perf_counter() - start, positive=True)
    history = trainer.history_rows()
    train_loss = runlog.finite_metric("train_loss", history[-1, 0])

    val_gen = torch.Generator(device=dev).manual_seed(data_seed + 1_000_003)
    total = torch.zeros((), dtype=torch.float64, device=dev)
    count = torch.zeros((), dtype=torch.float64, device=dev)
    torch.cuda.synchronize(dev)
    eval_start = time.perf_counter()
    for _ in range(validation_batches):
        x, y = _windows(val_gen, config, config.batch_size, dev)
        s, c = trainer.eval_step(x, y, torch.ones(x.shape, dtype=torch.float32, device=dev))
        total += s
        count += c
    validation_loss = runlog.finite_metric("validation_loss", float(total) / float(count))
    validation_seconds = runlog.finite_metric("validation_seconds", time.perf_counter() - eval_start, positive=True)
    validation_tokens = int(round(float(count)))

    tokens_processed = final_step * tokens_per_step
    fpt = flops_per_token(config)
    total_flops = fpt * tokens_processed
    achieved = runlog.finite_metric("achieved_tflops", total_flops / train_seconds / 1e12)
    params_total = trainer.arena.numel()

    runlog.write_training_log(out, history, tokens_per_step=tokens_per_step, final_step=final_step,
                              flops_per_token=fpt)
    perplexity = runlog.finite_metric("perplexity", math.exp(validation_loss), positive=True)
    runlog.write_validation_csv(out, [runlog.ValidationRow(final_step, tokens_processed, "fineweb", "fineweb",
                                                           validation_tokens, validation_loss, perplexity,
                                                           validation_seconds, True)])
    artifacts = {"training_curve": runlog.TRAINING_LOG_NAME, "validation_curve": runlog.VALIDATION_CSV_NAME}
    model = model_metadata(config)
    if checkpoint:
        params = {path: trainer.arena.param(path).detach().cpu().numpy() for path in trainer.arena.paths}
        runlog.save_checkpoint(out, params, {"schema_version": runlog.SCHEMA_VERSION, "seed": seed,
                                             "model": {**model, "seq_len": config.seq_len, "dtype": "bfloat16"}})
    props = torch.cuda.get_device_properties(dev)
    result: dict[str, Any] = {
        "schema_version": runlog.SCHEMA_VERSION,
        "status": "ok",
        "track": "open",
        "seed": int(seed),
        "checkpoint": runlog.CHECKPOINT_NAME if checkpoint else None,
        "artifacts": artifacts,
        "system": {"python_version": ".".join(map(str, sys.version_info[:3])), "torch_version": torch.__version__,
                   "platform": "rocm", "device_count": 1, "device_kinds": [props.name],
                   "gcn_arch": getattr(props, "gcnArchName", None)},
        "contract": {"model_id": "reference-gpt-v3-family", "dataset_id": "synthetic-uniform",
                     "tokenizer_id": "none", "sequence_length": config.seq_len, "model": model},
        "implementation": {"framework": "gptrig", "attention_backend": "flash", "loss_backend": "tiled",
                           "vocab_tile_size": config.vocab_tile_size, "document_masking": config.document_masking,
                           "micro_batch_size": config.micro_batch_size},
        "metrics": {
            "train_seconds": train_seconds,
            "tokens_processed": int(tokens_processed),
            "training_token_budget": int(tokens_processed),
            "training_steps": int(final_step),
            "schedule_steps": int(schedule_steps),
            "stop_after_step": None if stop_after_step is None else int(stop_after_step),
            "parameter_count": int(params_total),
            "parameters": int(params_total),
            "base_learning_rate": float(config.optimizer.learning_rate),
            "validation_loss": validation_loss,
            "validation_tokens": validation_tokens,
            "final_validation_seconds": validation_seconds,
            "train_loss": train_loss,
            "flops_per_token": int(fpt),
            "estimated_total_flops": int(total_flops),
            "flop_accounting": {"method": "analytic-causal-exact", "warnings": []},
            "tokens_per_second": runlog.finite_metric("tokens_per_second", tokens_processed / train_seconds,
                                                      positive=True),
            "achieved_tflops": achieved,
            "mfu_estimate": runlog.finite_metric("mfu_estimate", achieved / peak_tflops),
        },
    }
    runlog.write_result(out, result)
    return result


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--output-dir", required=True)
    p.add_argument("--config", default="{}", help="JSON of GPTConfig fields (optimizer fields under 'optimizer')")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--data-seed", type=int, default=1)
    p.add_argument("--stop-after-step", type=int, default=None)
    p.add_argument("--validation-batches", type=int, default=1)
    p.add_argument("--omit-checkpoint", action="store_true")
    return p


def config_from_json(text: str) -> GPTConfig:
    fields = json.loads(text)
    opt = OptimizerConfig(**fields.pop("optimizer", {}))
    known = {f.name for f in dataclasses.fields(GPTConfig)}
    unknown = set(fields) - known
    if unknown:
        raise ValueError(f"unknown config fields: {sorted(unknown)}")
    return GPTConfig(**fields, optimizer=opt)


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)
    try:
        result = run(config_from_json(args.config), args.output_dir, seed=args.seed, data_seed=args.data_seed,
                     stop_after_step=args.stop_after_step, validation_batches=args.validation_batches,
                     checkpoint=not args.omit_checkpoint)
    except Exception as error:  # the reference prints a one-line error and exits 1 (train.py:2402-2409)
        print(f"\nerror: {error}", file=sys.stderr)
        return 1
    print(runlog.result_line(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
