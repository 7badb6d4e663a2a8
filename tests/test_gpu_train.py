"""GPU training step vs the CPU oracle's step (``oracle.model.train_step``).

Same seed-0 numpy PCG64 initialisation on both sides (bit-identical
parameters), same synthetic token windows; the loss / learning-rate /
gradient-norm history of a few steps must agree: first-step loss to 1e-3
relative, later losses within 1%, gradient norms within 2%.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import optim as oopt

pytestmark = pytest.mark.gpu


def configs(steps: int, micro: int, embeddings: str = "untied", masking: bool = False):
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig

    common = dict(layers=2, heads=2, d_model=128, vocab_size=1000, semantic_vocab_size=997, seq_len=128,
                  batch_size=4, base_width=128, base_depth=2, attention_scale="inverse_sqrt_head_dim",
                  embeddings=embeddings, document_masking=masking, document_boundary_token=7)
    ocfg = om.Config(**common, attention_backend="flash",
                     optimizer=oopt.OptimizerConfig(learning_rate=2.0 ** -8, steps=steps, warmup_steps=1))
    gcfg = GPTConfig(**common, micro_batch_size=micro,
                     optimizer=OptimizerConfig(learning_rate=2.0 ** -8, steps=steps, warmup_steps=1))
    return ocfg, gcfg


@pytest.mark.parametrize("micro,embeddings,masking", [(2, "untied", False), (4, "tied", False),
                                                      (2, "untied", True)])
def test_train_step_history_matches_oracle(micro, embeddings, masking):
    from gptrig.train import GPTTrainer

    print(f"train case micro={micro} embeddings={embeddings} masking={masking}", flush=True)
    steps = 4
    ocfg, gcfg = configs(steps, micro, embeddings, masking)
    windows = om.synthetic_windows(0, steps, 4, 128, 997)
    if masking:
        windows[:, :, ::37] = 7  # document boundaries
    state = om.init_state(ocfg, 0)
    trainer = GPTTrainer(gcfg, seed=0)
    for i in range(steps):
        w = torch.from_numpy(windows[i])
        om.train_step(state, w[:, :-1], w[:, 1:], ocfg)
        trainer.train_step(w[:, :-1].cuda(), w[:, 1:].cuda())
    got = trainer.history_rows()
    want = np.asarray(state.history)
    print("gpu   ", got.tolist(), flush=True)
    print("oracle", want.tolist(), flush=True)
    assert abs(got[0, 0] - want[0, 0]) <= 1e-3 * want[0, 0]
    assert np.all(np.abs(got[:, 0] - want[:, 0]) <= 1e-2 * want[:, 0])
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    assert np.all(np.abs(got[:, 2] - want[:, 2]) <= 2e-2 * want[:, 2])


@pytest.mark.parametrize("label,model,trainer_only", [
    ("kept softmax in 2 token chunks per micro-batch", dict(vocab_tile_size=256), {}),
    ("kept softmax in one chunk", {}, dict(flce_whole_vocab=True)),
    ("d_model 192: recompute over vocabulary chunks", dict(d_model=192, heads=3, vocab_tile_size=256), {}),
])
def test_train_step_flce_paths_match_oracle(label, model, trainer_only):
    """The trainer's three FLCE wirings against the oracle's step: the
    default kept softmax cut into token chunks by vocab_tile_size (256 here:
    128-token chunks of the 256-token micro-batch), one chunk over all tokens
    (flce_whole_vocab), and, for d_model not a multiple of 128, the forward
    plus recompute backward over vocabulary chunks of vocab_tile_size."""
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer, flce_token_chunk

    steps = 3
    common = dict(layers=2, heads=2, d_model=128, vocab_size=1000, semantic_vocab_size=997, seq_len=128,
                  batch_size=4, base_width=128, base_depth=2, attention_scale="inverse_sqrt_head_dim",
                  embeddings="untied")
    common.update(model)
    opt = dict(learning_rate=2.0 ** -8, steps=steps, warmup_steps=1)
    ocfg = om.Config(**common, attention_backend="flash", optimizer=oopt.OptimizerConfig(**opt))
    gcfg = GPTConfig(**common, **trainer_only, micro_batch_size=2, optimizer=OptimizerConfig(**opt))
    chunk = flce_token_chunk(256, 1000, gcfg.vocab_tile_size, gcfg.flce_whole_vocab)
    print(f"train case {label}: token chunk {chunk}", flush=True)
    if "token chunks" in label:
        assert chunk == 128
    windows = om.synthetic_windows(7, steps, 4, 128, 997)
    state = om.init_state(ocfg, 0)
    trainer = GPTTrainer(gcfg, seed=0)
    for i in range(steps):
        w = torch.from_numpy(windows[i])
        om.train_step(state, w[:, :-1], w[:, 1:], ocfg)
        trainer.train_step(w[:, :-1].cuda(), w[:, 1:].cuda())
    got = trainer.history_rows()
    want = np.asarray(state.history)
    print("gpu   ", got.tolist(), flush=True)
    print("oracle", want.tolist(), flush=True)
    assert abs(got[0, 0] - want[0, 0]) <= 1e-3 * want[0, 0]
    assert np.all(np.abs(got[:, 0] - want[:, 0]) <= 1e-2 * want[:, 0])
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    assert np.all(np.abs(got[:, 2] - want[:, 2]) <= 2e-2 * want[:, 2])
    # The head's update carries the FLCE gradient directly.
    init = om.flatten(om.init_params(ocfg, 0))
    p0 = torch.from_numpy(np.asarray(init["output_embedding"]))
    du = (trainer.arena.param("output_embedding").cpu() - p0).double().reshape(-1)
    dw = (state.params["output_embedding"] - p0).double().reshape(-1)
    ratio, cos = float(du.norm() / dw.norm()), float(du @ dw / (du.norm() * dw.norm()))
    print(f"output_embedding update norm ratio {ratio:.4f}, cosine {cos:.4f}", flush=True)
    assert abs(ratio - 1) <= 0.1 and cos >= 0.9


@pytest.mark.parametrize("masking", [False, True])
def test_train_step_head_dim_128_matches_oracle(masking):
    """A 2-layer model with 2 heads of 128 (d_model 256): the trainer's
    attention runs the head_dim-128 kernels on the interleaved qkv rows, with
    the RoPE VJP fused into the backward (and, with document masking, the
    segment-id path); history against the oracle's step."""
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    steps = 3
    common = dict(layers=2, heads=2, d_model=256, vocab_size=1000, semantic_vocab_size=997, seq_len=128,
                  batch_size=4, base_width=256, base_depth=2, attention_scale="inverse_sqrt_head_dim",
                  embeddings="untied", document_masking=masking, document_boundary_token=7)
    opt = dict(learning_rate=2.0 ** -8, steps=steps, warmup_steps=1)
    ocfg = om.Config(**common, attention_backend="flash", optimizer=oopt.OptimizerConfig(**opt))
    gcfg = GPTConfig(**common, micro_batch_size=2, optimizer=OptimizerConfig(**opt))
    assert gcfg.head_dim == 128
    print(f"train case head_dim 128, document masking {masking}", flush=True)
    windows = om.synthetic_windows(11, steps, 4, 128, 997)
    if masking:
        windows[:, :, ::29] = 7  # document boundaries
    state = om.init_state(ocfg, 0)
    trainer = GPTTrainer(gcfg, seed=0)
    for i in range(steps):
        w = torch.from_numpy(windows[i])
        om.train_step(state, w[:, :-1], w[:, 1:], ocfg)
        trainer.train_step(w[:, :-1].cuda(), w[:, 1:].cuda())
    got = trainer.history_rows()
    want = np.asarray(state.history)
    print("gpu   ", got.tolist(), flush=True)
    print("oracle", want.tolist(), flush=True)
    assert abs(got[0, 0] - want[0, 0]) <= 1e-3 * want[0, 0]
    assert np.all(np.abs(got[:, 0] - want[:, 0]) <= 1e-2 * want[:, 0])
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    assert np.all(np.abs(got[:, 2] - want[:, 2]) <= 2e-2 * want[:, 2])


def test_train_step_completep_clip_and_residual_scale_match_oracle():
    """The official parameterization (completep_fixed_tpp_v1, recipes/reference/
    config.yaml:22-30) at width multiplier 2 and depth multiplier 2 with
    depth_alpha 1: per-tensor LR / epsilon / decay multipliers
    (train.py:1274-1333), init scales, residual branches scaled by 1/2
    (train.py:1164-1175), plus an active gradient clip (train.py:1390-1395);
    history against the oracle's step as above."""
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    steps = 4
    common = dict(layers=2, heads=2, d_model=128, vocab_size=1000, semantic_vocab_size=997, seq_len=128,
                  batch_size=4, base_width=64, base_depth=1, depth_alpha=1.0,
                  parameterization="completep_fixed_tpp_v1", attention_scale="inverse_head_dim", embeddings="untied")
    opt = dict(learning_rate=2.0 ** -8, steps=steps, warmup_steps=1, grad_clip=0.1)
    ocfg = om.Config(**common, attention_backend="flash", optimizer=oopt.OptimizerConfig(**opt))
    gcfg = GPTConfig(**common, micro_batch_size=2, optimizer=OptimizerConfig(**opt))
    print("train case completep width 2 depth 2 alpha 1, clip 0.1", flush=True)
    windows = om.synthetic_windows(1, steps, 4, 128, 997)
    state = om.init_state(ocfg, 0)
    trainer = GPTTrainer(gcfg, seed=0)
    assert trainer.residual_scale == 0.5
    for i in range(steps):
        w = torch.from_numpy(windows[i])
        om.train_step(state, w[:, :-1], w[:, 1:], ocfg)
        trainer.train_step(w[:, :-1].cuda(), w[:, 1:].cuda())
    got = trainer.history_rows()
    want = np.asarray(state.history)
    print("gpu   ", got.tolist(), flush=True)
    print("oracle", want.tolist(), flush=True)
    assert np.all(want[:, 2] > 0.1), "the clip must be active"
    assert abs(got[0, 0] - want[0, 0]) <= 1e-3 * want[0, 0]
    assert np.all(np.abs(got[:, 0] - want[:, 0]) <= 1e-2 * want[:, 0])
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    assert np.all(np.abs(got[:, 2] - want[:, 2]) <= 2e-2 * want[:, 2])
    # The clipped, multiplier-scaled updates, tensor by tensor: Adam turns
    # last-bit differences of near-zero gradient elements into full-size
    # element updates, so the update is compared as a whole (its norm, and its
    # direction by the cosine), which a wrong per-tensor multiplier (a factor
    # of 2 here) would fail.
    init = om.flatten(om.init_params(ocfg, 0))
    for path in ("blocks/0/qkv_w", "blocks/1/attn_w", "blocks/1/mlp_down_b", "blocks/0/ln2_scale", "token_embedding",
                 "output_embedding", "final_ln_scale"):
        p0 = torch.from_numpy(np.asarray(init[path]))
        du = (trainer.arena.param(path).cpu() - p0).double().reshape(-1)
        dw = (state.params[path] - p0).double().reshape(-1)
        ratio = float(du.norm() / dw.norm())
        cos = float(du @ dw / (du.norm() * dw.norm()))
        print(f"{path}: update norm ratio {ratio:.4f}, cosine {cos:.4f}", flush=True)
        assert abs(ratio - 1) <= 0.1 and cos >= 0.9, path


def test_train_step_batch_data_ratio_matches_oracle():
    """The fixed-TPP transfer rule away from ratio 1: batch_multiplier 2 over
    data_multiplier 0.5 (train.py:792-800) gives betas 0.6 / 0.8
    (:1336-1345), the learning rate x 2 (:1231), epsilon x 1/2 and weight
    decay x 2 (:1413-1414).  Weight decay 20 and epsilon 1e-3 make the decay
    and epsilon terms a visible part of every update: on the CPU, the oracle
    with the decay horizon inverted moves the weight updates' norms by a
    factor 0.44-0.57, with the epsilon horizon inverted the norm-scale
    update by 0.48, and with the LR horizon inverted every update by 0.25;
    a slip in the betas (1 - (1 - beta) / ratio) shows in the Adam moments,
    compared tensor by tensor as well."""
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    steps = 4
    common = dict(layers=2, heads=2, d_model=128, vocab_size=1000, semantic_vocab_size=997, seq_len=128,
                  batch_size=4, base_width=128, base_depth=2, attention_scale="inverse_sqrt_head_dim",
                  embeddings="untied")
    opt = dict(learning_rate=2.0 ** -9, steps=steps, warmup_steps=1, weight_decay=20.0, adam_epsilon=1.0e-3,
               batch_multiplier=2.0, data_multiplier=0.5)
    ocfg = om.Config(**common, attention_backend="flash", optimizer=oopt.OptimizerConfig(**opt))
    gcfg = GPTConfig(**common, micro_batch_size=2, optimizer=OptimizerConfig(**opt))
    print("train case batch_multiplier 2, data_multiplier 0.5", flush=True)
    assert oopt.effective_adam_betas(ocfg.optimizer) == pytest.approx((0.6, 0.8), abs=1e-12)
    windows = om.synthetic_windows(6, steps, 4, 128, 997)
    state = om.init_state(ocfg, 0)
    trainer = GPTTrainer(gcfg, seed=0)
    assert (trainer.beta1, trainer.beta2) == pytest.approx((0.6, 0.8), abs=1e-12)
    for i in range(steps):
        w = torch.from_numpy(windows[i])
        om.train_step(state, w[:, :-1], w[:, 1:], ocfg)
        trainer.train_step(w[:, :-1].cuda(), w[:, 1:].cuda())
    got = trainer.history_rows()
    want = np.asarray(state.history)
    print("gpu   ", got.tolist(), flush=True)
    print("oracle", want.tolist(), flush=True)
    # Step 2 (one step into the cosine over 3): base 2^-9 x 2 x (0.1 + 0.9 x 0.75).
    assert abs(want[1, 1] - 2.0 ** -9 * 2 * (0.1 + 0.9 * 0.75)) < 1e-9
    assert abs(got[0, 0] - want[0, 0]) <= 1e-3 * want[0, 0]
    assert np.all(np.abs(got[:, 0] - want[:, 0]) <= 1e-2 * want[:, 0])
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-6)
    assert np.all(np.abs(got[:, 2] - want[:, 2]) <= 2e-2 * want[:, 2])
    init = om.flatten(om.init_params(ocfg, 0))
    for path in ("blocks/0/qkv_w", "blocks/1/mlp_up_w", "blocks/1/mlp_down_b", "blocks/0/ln2_scale",
                 "token_embedding", "output_embedding"):
        p0 = torch.from_numpy(np.asarray(init[path]))
        du = (trainer.arena.param(path).cpu() - p0).double().reshape(-1)
        dw = (state.params[path] - p0).double().reshape(-1)
        ratio = float(du.norm() / dw.norm())
        cos = float(du @ dw / (du.norm() * dw.norm()))
        print(f"{path}: update norm ratio {ratio:.4f}, cosine {cos:.4f}", flush=True)
        assert abs(ratio - 1) <= 0.1 and cos >= 0.9, path
        for name, arena, ref in (("m", trainer.arena.m, state.m), ("v", trainer.arena.v, state.v)):
            got_mom = trainer.arena._view(arena, path).cpu().double().reshape(-1)
            want_mom = ref[path].double().reshape(-1)
            r = float(got_mom.norm() / want_mom.norm())
            c = float(got_mom @ want_mom / (got_mom.norm() * want_mom.norm()))
            print(f"  {name}: norm ratio {r:.4f}, cosine {c:.4f}", flush=True)
            assert abs(r - 1) <= 0.1 and c >= 0.9, (path, name)


def test_initial_parameters_are_bit_identical_to_the_reference_draws():
    from gptrig.train import GPTTrainer

    _, gcfg = configs(1, 2)
    ocfg, _ = configs(1, 2)
    trainer = GPTTrainer(gcfg, seed=3)
    flat = om.flatten(om.init_params(ocfg, 3))
    for path, value in flat.items():
        assert torch.equal(trainer.arena.param(path).cpu(), torch.from_numpy(np.asarray(value))), path


def test_eval_step_matches_oracle():
    """eval_step (train.py:1493-1525) against the oracle's, from bit-identical
    initial parameters: masked loss sum to 1e-3 relative, target count to fp32
    summation order; one or two micro-batches; bad shapes raise."""
    from gptrig.train import GPTTrainer

    ocfg, gcfg = configs(1, 2)
    trainer = GPTTrainer(gcfg, seed=0)
    state = om.init_state(ocfg, 0)
    w = torch.from_numpy(om.synthetic_windows(4, 1, 4, 128, 997)[0])
    x, y = w[:, :-1], w[:, 1:]
    g = torch.Generator().manual_seed(11)
    mask = (torch.rand(x.shape, generator=g) < 0.7).float() * torch.rand(x.shape, generator=g)
    for rows in (4, 2):
        total, count = trainer.eval_step(x[:rows].cuda(), y[:rows].cuda(), mask[:rows].cuda())
        want_total, want_count = om.eval_step(state.params, x[:rows], y[:rows], mask[:rows], ocfg)
        print(f"eval rows={rows}: gpu {float(total):.6f} / {float(count):.3f}, "
              f"oracle {float(want_total):.6f} / {float(want_count):.3f}", flush=True)
        assert abs(float(total) - float(want_total)) <= 1e-3 * abs(float(want_total))
        assert abs(float(count) - float(want_count)) <= 1e-5 * float(want_count)
    with pytest.raises(ValueError):
        trainer.eval_step(x[:3].cuda(), y[:3].cuda(), mask[:3].cuda())


def test_training_log_round_trips_the_device_history(tmp_path):
    """An early-stopped run (3 of 6 steps) writes ``training.riglog`` with one
    record per step taken, bit-equal to the on-device history (rig/runlog.py:257-302)."""
    from gptrig import runlog
    from gptrig.train import GPTTrainer

    _, gcfg = configs(6, 2)
    trainer = GPTTrainer(gcfg, seed=0)
    windows = om.synthetic_windows(5, 3, 4, 128, 997)
    for i in range(3):
        w = torch.from_numpy(windows[i])
        trainer.train_step(w[:, :-1].cuda(), w[:, 1:].cuda())
    path = trainer.write_training_log(tmp_path, flops_per_token=1.0e6)
    log = runlog.read_log(path)
    rows = trainer.history_rows()
    print("history", rows.tolist(), flush=True)
    assert rows.shape == (3, 3) and np.all(rows[:, 0] > 0)
    np.testing.assert_array_equal(log.steps, [1, 2, 3])
    np.testing.assert_array_equal(log.values, rows)
    np.testing.assert_array_equal(log.axis("tokens_processed"), np.arange(1, 4) * 4 * 128)
    np.testing.assert_array_equal(log.axis("cumulative_flops"), np.arange(1, 4) * 4 * 128 * 1.0e6)


def test_run_directory_is_what_the_harness_reads(tmp_path, capsys):
    """``gptrig.run`` (train.py:run's artefacts and result line) on a tiny
    config stopped at step 3 of 5: every artefact re-read and cross-checked."""
    import json
    import math

    from test_runlog import harness_accepts

    from gptrig import run as grun
    from gptrig import runlog

    config = ('{"layers": 2, "heads": 2, "d_model": 128, "vocab_size": 1000, "semantic_vocab_size": 997, '
              '"seq_len": 128, "batch_size": 4, "micro_batch_size": 2, "base_width": 128, "base_depth": 2, '
              '"optimizer": {"learning_rate": 0.00390625, "steps": 5, "warmup_steps": 1}}')
    assert grun.main(["--output-dir", str(tmp_path), "--config", config, "--stop-after-step", "3"]) == 0
    last = capsys.readouterr().out.strip().splitlines()[-1]
    assert last.startswith(runlog.RESULT_PREFIX)
    result = json.loads(last[len(runlog.RESULT_PREFIX):])
    assert json.loads((tmp_path / "metrics.json").read_text()) == result
    assert harness_accepts(result, tmp_path)
    m = result["metrics"]
    print({k: m[k] for k in ("train_seconds", "tokens_per_second", "validation_loss", "train_loss")}, flush=True)
    assert m["training_steps"] == 3 and m["schedule_steps"] == 5 and m["tokens_processed"] == 3 * 4 * 128
    assert m["validation_tokens"] == 4 * 128
    assert abs(m["validation_loss"] - math.log(997)) < 0.5  # random init on uniform tokens

    log = runlog.read_log(tmp_path / "training.riglog")
    np.testing.assert_array_equal(log.steps, [1, 2, 3])
    assert log.values[-1, 0] == np.float32(m["train_loss"])
    assert log.flops_per_token == m["flops_per_token"] and log.tokens_per_step == 4 * 128
    rows = (tmp_path / "validation.csv").read_text().splitlines()
    assert rows[1].split(",")[:5] == ["3", str(3 * 512), "fineweb", "fineweb", "512"] and rows[1].endswith("true")
    assert float(rows[1].split(",")[5]) == m["validation_loss"]

    with np.load(tmp_path / "checkpoint.npz", allow_pickle=False) as z:
        meta = json.loads(z["metadata.json"].tobytes().decode())
        assert meta["model"]["layers"] == 2 and meta["seed"] == 0
        names = [k for k in z.files if k.startswith("params/")]
        assert sum(int(z[k].size) for k in names) == m["parameter_count"]
        assert all(np.isfinite(z[k]).all() for k in names)
