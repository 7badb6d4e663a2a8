"""Benchmark: one-GPU training step of the reference 125M GPT (12 layers, d_model 768).

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

Workload: 12 layers, d_model 768, 12 heads x 64, GELU MLP 3072, vocab 50304,
seq 1024, global batch 128 sequences (by default as 2 micro-batches of 64), AdamW
(base LR 2^-8, betas 0.9/0.95, wd 0.1), bf16 compute with float32 master
weights, synthetic uniform tokens from numpy seed 2, random-normal init
(std 0.02) — the full step (forward, backward, AdamW) every iteration.
All token batches are resident in HBM before the timed region.

``value`` is training tokens/s.  ``roofline`` describes the fused linear
cross-entropy (the largest hand-written MFMA kernel of the step), timed live
with HIP events on the launch stream; ``roofline_attn_bwd`` does the same for
the flash-attention backward.  ``cpu_baseline`` times the CPU restatement of
the reference step (``oracle/``) on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import replace

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpt-speedrun-tpu_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "train tokens/s at 125M S=1024; attn-bwd + FLCE TFLOP/s as % of bf16 MFMA peak"
MFMA_BF16_PEAK_TFLOPS = 2500.0
# HBM bytes of one FLCE fwd+bwd launch sequence (the trainer's kept-softmax
# pairs), by (micro-batch tokens N, tokens per chunk) (d 768, V 50304): FETCH_SIZE (x 2.0, the factor the counter
# reads for a 256 MiB copy) + WRITE_SIZE (x 1.0) summed over its launches, from
# `rocprofv3 --pmc` runs of `bench.py --traffic-pass`; the per-launch table and
# commands are in profiles/flce_traffic_config_d.md.  Re-measure after kernel
# changes; a shape without a measurement reports null.
FLCE_TRAFFIC_BYTES = {(65536, 5056): (37537 + 15518) * 2 ** 20, (65536, 65536): (32550 + 13751) * 2 ** 20}


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--micro-batch", type=int, default=64,
                    help="sequences per forward/backward pass (the global batch of 128 is accumulated over 128 / micro-batch passes; 64 measured fastest: at 128 the attention working set outgrows the L2 + MALL)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-isolated", action="store_true", help="skip the isolated attention (B) and FLCE (C) configs")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the 4x32 micro-batch split and the config-E (MoE) step lines")
    ap.add_argument("--config-e", action="store_true",
                    help="run only the config-E (MoE) step lines, as one JSON object (the program profiled for the "
                         "MoE kernel table)")
    ap.add_argument("--traffic-pass", action="store_true",
                    help="run one 256 MiB calibration copy, one FLCE forward+backward and one attention "
                         "forward+backward at the bench's micro-batch shapes, and exit (the program profiled by "
                         "the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs)")
    return ap.parse_args()


def traffic_pass(micro_batch: int) -> None:
    """One launch sequence of each hand-written hot path at the bench's
    micro-batch shape, for HBM-counter runs."""

    from gptrig.kernels import flash_attention as fa
    from gptrig.kernels import linear_cross_entropy as lce
    dev = "cuda:0"
    torch.manual_seed(0)
    src = torch.randn(64 * 1024 * 1024, device=dev)  # 256 MiB: calibrates the counters
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    n, d, vocab = micro_batch * 1024, 768, 50304
    h = torch.randn(n, d, device=dev).bfloat16()
    w = (torch.randn(vocab, d, device=dev) * 0.02).bfloat16()
    t = torch.randint(0, vocab, (n,), device=dev, dtype=torch.int32)
    # The trainer's FLCE sequence: kept-softmax forward and backward per token
    # chunk (bounded by the default vocab_tile_size), then the same over one
    # chunk of all tokens (flce_whole_vocab).
    from gptrig.train import flce_token_chunk

    dw = torch.empty(vocab, d, device=dev)
    for chunk in (flce_token_chunk(n, vocab, 2048, False), n):
        keep = None
        for c0 in range(0, n, chunk):
            c1 = min(n, c0 + chunk)
            _, lse, keep = lce.flce_forward_keep(h[c0:c1], w, t[c0:c1], vocab, keep)
            lce.flce_backward_keep(h[c0:c1], w, t[c0:c1], lse, keep, None, 1.0 / n, vocab, dweight=dw,
                                   accumulate=c0 > 0)
        torch.cuda.synchronize()
        del keep
        print(f"flce sequence with token chunks of {chunk} done", flush=True)
    del dw
    q, k, v, do = (torch.randn(micro_batch, 12, 1024, 64, device=dev).bfloat16() for _ in range(4))
    o, lse2 = fa.flash_forward(q, k, v, None, 0.125)
    fa.flash_backward(q, k, v, o, lse2, do, None, 0.125)
    torch.cuda.synchronize()
    del q, k, v, do, o, lse2, h, w, t
    # One full config-D step (every kernel of the product step, for the counter tables).
    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    cfg = GPTConfig(layers=12, heads=12, d_model=768, vocab_size=50304, semantic_vocab_size=50304, seq_len=1024,
                    batch_size=128, micro_batch_size=micro_batch,
                    optimizer=OptimizerConfig(learning_rate=2.0 ** -8, steps=1000, warmup_steps=100))
    trainer = GPTTrainer(cfg, seed=0, history_steps=1)
    rng = np.random.default_rng(2)
    win = torch.from_numpy(rng.integers(0, cfg.vocab_size, size=(128, 1025), dtype=np.int32)).to(dev)
    trainer.train_step(win[:, :-1].contiguous(), win[:, 1:].contiguous())
    torch.cuda.synchronize()
    print("traffic pass done", flush=True)


def isolated_configs(reps: int = 20) -> dict:
    """The reference metric's isolated kernel configs, measured alone after the
    step: B = causal attention fwd+bwd at B16 H12 S1024 D64 (q, k, v, dO ~ N(0,1)
    from numpy seed 1, RoPE on q and k, scale 1/8) and C = FLCE fwd+bwd at
    N16384 d768 V50304 (h ~ N(0,1), W ~ N(0,0.02), uniform targets).  Each
    launch sequence is timed with HIP events on the stream it runs on,
    averaged over ``reps`` after one untimed call."""

    from gptrig import _lib
    from gptrig.kernels import flash_attention as fa
    from gptrig.kernels import linear_cross_entropy as lce
    from gptrig.nn import apply_rotary

    dev = "cuda:0"

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps

    assert _lib.stream() == torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(1)
    B, H, S, D = 16, 12, 1024, 64
    q, k, v, do = (torch.from_numpy(rng.standard_normal((B, H, S, D), dtype=np.float32)).to(dev).bfloat16()
                   for _ in range(4))
    q, k = (apply_rotary(t.transpose(1, 2).contiguous()).transpose(1, 2).contiguous() for t in (q, k))
    o, lse = fa.flash_forward(q, k, v, None, 0.125)
    fwd_ms = timed(lambda: fa.flash_forward(q, k, v, None, 0.125))
    bwd_ms = timed(lambda: fa.flash_backward(q, k, v, o, lse, do, None, 0.125))
    visible = S * (S + 1) // 2
    fwd_tf = 4 * B * H * D * visible / (fwd_ms / 1e3) / 1e12
    bwd_tf = attn_bwd_flops(B, H, S, D) / (bwd_ms / 1e3) / 1e12
    del q, k, v, do, o, lse
    # head_dim 128 at the same model width (6 heads x 128; no BASELINE config
    # uses it): the kernels the reference's D <= 128 range reaches.
    H2, D2 = 6, 128
    q, k, v, do = (torch.from_numpy(rng.standard_normal((B, H2, S, D2), dtype=np.float32)).to(dev).bfloat16()
                   for _ in range(4))
    sc2 = D2 ** -0.5
    o, lse = fa.flash_forward(q, k, v, None, sc2)
    fwd128_ms = timed(lambda: fa.flash_forward(q, k, v, None, sc2))
    bwd128_ms = timed(lambda: fa.flash_backward(q, k, v, o, lse, do, None, sc2))
    fwd128_tf = 4 * B * H2 * D2 * visible / (fwd128_ms / 1e3) / 1e12
    bwd128_tf = attn_bwd_flops(B, H2, S, D2) / (bwd128_ms / 1e3) / 1e12
    del q, k, v, do, o, lse

    n, d, vocab = 16384, 768, 50304
    h = torch.from_numpy(rng.standard_normal((n, d), dtype=np.float32)).to(dev).bfloat16()
    w = torch.from_numpy(rng.standard_normal((vocab, d), dtype=np.float32) * 0.02).to(dev).bfloat16()
    t = torch.from_numpy(rng.integers(0, vocab, size=n, dtype=np.int32)).to(dev)
    def flce_with(chunk):
        def run():
            _, lse_c = lce.flce_forward(h, w, t, vocab)
            lce.flce_backward(h, w, t, lse_c, None, 1.0 / n, vocab, chunk)
        return run

    from gptrig.train import flce_token_chunk

    keep_buf = []
    dw = torch.empty(vocab, d, device=dev)

    def flce_keep(chunk):
        def run():
            for c0 in range(0, n, chunk):
                c1 = min(n, c0 + chunk)
                _, lse_c, kb = lce.flce_forward_keep(h[c0:c1], w, t[c0:c1], vocab, keep_buf[0] if keep_buf else None)
                keep_buf[:] = [kb]
                lce.flce_backward_keep(h[c0:c1], w, t[c0:c1], lse_c, kb, None, 1.0 / n, vocab, dweight=dw,
                                       accumulate=c0 > 0)
        return run

    # The trainer's path (kept softmax over token chunks bounded by the default
    # vocab_tile_size), the same over one chunk of all tokens, the whole
    # vocabulary with the logits recomputed, and the public API's default
    # vocab_tile_size (2048: the reference's bounded [tokens, tile] working set).
    chunk = flce_token_chunk(n, vocab, lce.DEFAULT_VOCAB_TILE_SIZE, False)
    flce_ms = timed(flce_keep(chunk))
    flce_tf = flce_flops(n, d, vocab) / (flce_ms / 1e3) / 1e12
    keep_bytes = keep_buf[0].numel()
    keep_buf.clear()
    one_ms = timed(flce_keep(n))
    one_tf = flce_flops(n, d, vocab) / (one_ms / 1e3) / 1e12
    keep_buf.clear()
    del dw
    whole_ms = timed(flce_with(lce.grad_chunk(n, vocab)))
    whole_tf = flce_flops(n, d, vocab) / (whole_ms / 1e3) / 1e12
    tile_ms = timed(flce_with(lce.chunk_for(lce.DEFAULT_VOCAB_TILE_SIZE)))
    tile_tf = flce_flops(n, d, vocab) / (tile_ms / 1e3) / 1e12
    peak = MFMA_BF16_PEAK_TFLOPS
    return {
        "attention_B16_H12_S1024_D64": {
            "fwd_ms": round(fwd_ms, 4), "fwd_tflops": round(fwd_tf, 1), "fwd_frac": round(fwd_tf / peak, 4),
            "bwd_ms": round(bwd_ms, 4), "bwd_tflops": round(bwd_tf, 1), "bwd_frac": round(bwd_tf / peak, 4),
            "bwd_algorithmic_flops": attn_bwd_flops(B, H, S, D)},
        "attention_B16_H6_S1024_D128": {
            "fwd_ms": round(fwd128_ms, 4), "fwd_tflops": round(fwd128_tf, 1),
            "fwd_frac": round(fwd128_tf / peak, 4), "bwd_ms": round(bwd128_ms, 4),
            "bwd_tflops": round(bwd128_tf, 1), "bwd_frac": round(bwd128_tf / peak, 4)},
        "flce_N16384_d768_V50304": {"ms": round(flce_ms, 4), "tflops": round(flce_tf, 1),
                                    "frac": round(flce_tf / peak, 4), "algorithmic_flops": flce_flops(n, d, vocab),
                                    "path": f"kept softmax over token chunks of {chunk} (the trainer's default: "
                                            f"{keep_bytes} kept bytes <= tokens x 2048 x 4)",
                                    "one_chunk_kept": {"ms": round(one_ms, 4), "tflops": round(one_tf, 1),
                                                       "frac": round(one_tf / peak, 4)},
                                    "whole_vocabulary_recompute": {"ms": round(whole_ms, 4),
                                                                   "tflops": round(whole_tf, 1),
                                                                   "frac": round(whole_tf / peak, 4)},
                                    "default_tile_2048": {"ms": round(tile_ms, 4), "tflops": round(tile_tf, 1),
                                                          "frac": round(tile_tf / peak, 4),
                                                          "workspace_bytes": lce.workspace_bytes(n, d, vocab)}},
    }


def flce_whole_vocab(n: int, d: int, vocab: int, reps: int = 5) -> dict:
    """The FLCE of one micro-batch (n tokens) as one chunk over all tokens
    (``GPTConfig.flce_whole_vocab``: fp16 [vocab, n] kept probabilities, not
    bounded by vocab_tile_size), timed with HIP events on its stream over
    ``reps`` launch sequences after one untimed."""

    from gptrig.kernels import linear_cross_entropy as lce

    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(n, d, device=dev, generator=g).bfloat16()
    w = (torch.randn(vocab, d, device=dev, generator=g) * 0.02).bfloat16()
    t = torch.randint(0, vocab, (n,), device=dev, dtype=torch.int32, generator=g)
    dw = torch.empty(vocab, d, device=dev)
    keep = []

    def run():
        _, lse, kb = lce.flce_forward_keep(h, w, t, vocab, keep[0] if keep else None)
        keep[:] = [kb]
        lce.flce_backward_keep(h, w, t, lse, kb, None, 1.0 / n, vocab, dweight=dw)

    run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    tf = flce_flops(n, d, vocab) / (ms / 1e3) / 1e12
    traffic = FLCE_TRAFFIC_BYTES.get((n, n))
    out = {"kernel": f"flce fwd+bwd, one kept-softmax chunk over all {n} tokens ([vocab, tokens] fp16, "
                     "GPTConfig.flce_whole_vocab)", "bound": "mfma", "achieved": round(tf, 1),
           "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
           "traffic": traffic, "ms": round(ms, 3), "kept_bytes": int(keep[0].numel())}
    del h, w, t, dw, keep
    torch.cuda.empty_cache()
    return out


def attn_bwd_flops(batch, heads, seq, head_dim):
    """Causal-exact algorithmic FLOPs of one attention backward (dV, dP, dK, dQ)."""
    visible = seq * (seq + 1) // 2
    return 8 * batch * heads * head_dim * visible


def flce_flops(n, d, vocab):
    """Forward + backward algorithmic FLOPs of the LM-head cross-entropy (6 N d V)."""
    return 6 * n * d * vocab


def step_flops(layers, d, seq, tokens, vocab, mlp=4):
    """Causal-exact training FLOPs of one step (3x forward)."""
    per_token = 2 * (12 * d * d if mlp == 4 else (4 + 2 * mlp) * d * d) * layers  # qkv, out, up, down
    per_token += 2 * d * vocab  # LM head
    attn = 4 * d * (seq + 1) / 2 * layers  # QK^T and PV over the causal prefix, per token
    return 3 * (per_token + attn) * tokens


def cpu_baseline() -> dict:
    """The CPU restatement of the reference's semantics (``oracle/``, torch-CPU
    fp32 math with bf16 rounding at the reference's cast points) on the host
    cores of this box, as planned in BASELINE.md: config A's full train step
    (forward, backward, AdamW; median of 5 after 2 warm-ups), the isolated
    attention (B) and FLCE (C) configs (one timed call after a warm-up), and a
    config-D figure extrapolated from a measured per-sequence forward+backward
    (median of 3 after 1 warm-up) plus one AdamW update."""

    import statistics

    from oracle import attention as oattn
    from oracle import flce as oflce
    from oracle import model as om
    from oracle import optim as oopt

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def clock(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    # Config A: the full step, medians of 5 after 2 warm-ups.
    cfg_a = om.baseline_config("A", steps=1000)
    state = om.init_state(cfg_a, 0)
    win = om.synthetic_windows(0, 7, cfg_a.batch_size, cfg_a.seq_len, cfg_a.vocab_size)
    times = []
    for i in range(7):
        w = torch.from_numpy(win[i])
        t = clock(lambda: om.train_step(state, w[:, :-1], w[:, 1:], cfg_a))
        if i >= 2:
            times.append(t)
    a_step = statistics.median(times)
    del state
    # Config B: attention fwd + bwd at B16 H12 S1024 D64 (scale 1/8).
    g = torch.Generator().manual_seed(1)
    q, k, v, do = (torch.randn(16, 12, 1024, 64, generator=g).to(torch.bfloat16) for _ in range(4))

    def attn():
        o, lse = oattn.attention_forward(q, k, v, softmax_scale=0.125)
        oattn.attention_backward(q, k, v, o, lse, do, softmax_scale=0.125)

    attn()
    b_s = clock(attn)
    del q, k, v, do
    # Config C: FLCE fwd + bwd at N16384 d768 V50304 (tile 2048).
    hc = torch.randn(16384, 768, generator=g).to(torch.bfloat16)
    wc = torch.randn(50304, 768, generator=g) * 0.02
    tc = torch.randint(0, 50304, (16384,), generator=g, dtype=torch.int32)
    ct = torch.full((16384,), 1.0 / 16384)

    def flce():
        _, lse = oflce.losses_and_lse(hc, wc, tc, semantic_vocab_size=50304)
        oflce.losses_backward(hc, wc, tc, lse, ct, semantic_vocab_size=50304)

    flce()
    c_s = clock(flce)
    del hc, wc, tc
    # Config D: per-sequence forward + backward and one AdamW update, extrapolated.
    cfg_d = om.baseline_config("D", steps=1000)
    state = om.init_state(cfg_d, 0)
    wd = om.synthetic_windows(2, 1, 1, cfg_d.seq_len, cfg_d.vocab_size)[0]
    x, y = torch.from_numpy(wd[:, :-1]), torch.from_numpy(wd[:, 1:])
    leaves = {k: v.detach().requires_grad_(True) for k, v in state.params.items()}

    def fwd_bwd():
        loss = om.cross_entropy(leaves, x, y, cfg_d)
        return torch.autograd.grad(loss, list(leaves.values()))

    grads = fwd_bwd()
    t_fb = statistics.median(clock(fwd_bwd) for _ in range(3))
    gd = {k: gr.float() for k, gr in zip(leaves.keys(), grads)}
    t_adam = clock(lambda: oopt.adamw_step(state.params, gd, state.m, state.v, 1, cfg_d.optimizer))
    d_step = 128 * t_fb + t_adam
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {
        "value": round(cfg_a.batch_size * cfg_a.seq_len / a_step, 1),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"CPU restatement of reference semantics (oracle/, torch-CPU fp32 math with bf16 rounding), "
                   f"{threads} threads on {cpu}.  value: config A (8L d512, the reference's CPU-runnable step: "
                   f"8 x 1024 tokens) full train step, median of 5 steps after 2 warm-ups ({a_step:.2f} s/step)"),
        "config_D_extrapolated": {"tokens_per_s": round(128 * 1024 / d_step, 1), "extrapolated": True,
                                  "from": f"a measured per-sequence forward+backward ({t_fb:.2f} s, median of 3 "
                                          f"after a warm-up) x 128 sequences + one AdamW update ({t_adam:.2f} s)"},
        "config_B_attention_fwd_bwd_s": round(b_s, 3),
        "config_C_flce_fwd_bwd_s": round(c_s, 3),
    }


def timed_steps(trainer, xs, ys, warmup: int, steps: int) -> float:
    """ms per step of ``trainer`` over ``steps`` steps after ``warmup`` (device
    clock, bracketed by synchronisations)."""

    for i in range(warmup):
        trainer.train_step(xs[i % len(xs)], ys[i % len(ys)])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        trainer.train_step(xs[(warmup + i) % len(xs)], ys[(warmup + i) % len(ys)])
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def moe_step(expert_mult: int, warmup: int = 2, steps: int = 3) -> dict:
    """Config E: the MoE recipe's train step (12x768 backbone, 8 experts top-2,
    seq 1024, batch 32 in one pass, synthetic tokens from numpy seed 2)."""

    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer

    cfg = GPTConfig(layers=12, heads=12, d_model=768, vocab_size=50304, semantic_vocab_size=50304, seq_len=1024,
                    batch_size=32, micro_batch_size=32, experts=8, expert_top_k=2, expert_mult=expert_mult,
                    mlp_mult=2 * expert_mult, optimizer=OptimizerConfig(learning_rate=2.0 ** -8, steps=1000,
                                                                        warmup_steps=100))
    trainer = GPTTrainer(cfg, seed=0, history_steps=warmup + steps)
    rng = np.random.default_rng(2)
    win = torch.from_numpy(rng.integers(0, cfg.vocab_size, size=(warmup + steps, 32, 1025), dtype=np.int32)).cuda()
    xs = [win[i, :, :-1].contiguous() for i in range(warmup + steps)]
    ys = [win[i, :, 1:].contiguous() for i in range(warmup + steps)]
    ms = timed_steps(trainer, xs, ys, warmup, steps)
    tokens = cfg.batch_size * cfg.seq_len
    loss = float(trainer.history_rows()[-1, 0])
    del trainer, win, xs, ys
    torch.cuda.empty_cache()
    return {"expert_width": expert_mult * 768, "ms_per_step": round(ms, 3),
            "tokens_per_s": round(tokens / (ms / 1e3), 1), "last_loss": round(loss, 4)}


def main():
    args = parse_args()
    if args.traffic_pass:
        traffic_pass(args.micro_batch)
        return
    if args.config_e:
        print(json.dumps({"config_E_moe_step": {"reference_valid_width": moe_step(2, args.warmup, args.steps),
                                                "baseline_width": moe_step(4, args.warmup, args.steps)}}), flush=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU (--gpus > 1) is not implemented",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    from gptrig.optim import OptimizerConfig
    from gptrig.train import GPTConfig, GPTTrainer, flce_token_chunk

    cfg = GPTConfig(layers=12, heads=12, d_model=768, mlp_mult=4, vocab_size=50304, semantic_vocab_size=50304,
                    seq_len=1024, batch_size=128, micro_batch_size=args.micro_batch,
                    optimizer=OptimizerConfig(learning_rate=2.0 ** -8, steps=1000, warmup_steps=100))
    total = args.warmup + args.steps
    trainer = GPTTrainer(cfg, seed=0, history_steps=total)
    rng = np.random.default_rng(2)
    windows = torch.from_numpy(rng.integers(0, cfg.vocab_size, size=(total, cfg.batch_size, cfg.seq_len + 1),
                                            dtype=np.int32)).cuda()
    xs = [windows[i, :, :-1].contiguous() for i in range(total)]
    ys = [windows[i, :, 1:].contiguous() for i in range(total)]
    torch.cuda.synchronize()

    for i in range(args.warmup):
        trainer.train_step(xs[i], ys[i])
    torch.cuda.synchronize()

    trainer.timers = {}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(args.warmup, total):
        trainer.train_step(xs[i], ys[i])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end)
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps
    tokens_per_step = cfg.batch_size * cfg.seq_len
    value = tokens_per_step / (ms_per_step / 1e3)

    def avg_ms(name):
        ev = trainer.timers.get(name, [])
        return sum(s.elapsed_time(e) for s, e in ev) / max(len(ev), 1), len(ev)

    n_micro = cfg.batch_size // cfg.micro_batch_size
    mb_tokens = cfg.micro_batch_size * cfg.seq_len
    chunk = flce_token_chunk(mb_tokens, cfg.vocab_size, cfg.vocab_tile_size, cfg.flce_whole_vocab)
    traffic = FLCE_TRAFFIC_BYTES.get((mb_tokens, chunk))  # measured per shape; None for an unmeasured one
    # FLCE: every timed launch sequence of the step, per micro-batch (fwd + bwd of all its token chunks).
    flce_ms_launch, flce_n = avg_ms("flce")
    flce_ms = flce_ms_launch * flce_n / (n_micro * args.steps)
    flce_tf = flce_flops(mb_tokens, cfg.d_model, cfg.vocab_size) / (flce_ms / 1e3) / 1e12
    ab_ms, _ = avg_ms("attn_bwd")
    ab_tf = attn_bwd_flops(cfg.micro_batch_size, cfg.heads, cfg.seq_len, cfg.head_dim) / (ab_ms / 1e3) / 1e12
    af_ms, _ = avg_ms("attn_fwd")
    adam_ms, _ = avg_ms("adamw")
    adam_gbs = 28 * trainer.arena.numel() / (adam_ms / 1e3) / 1e9
    hist = trainer.history_rows()
    total_flops = step_flops(cfg.layers, cfg.d_model, cfg.seq_len, tokens_per_step, cfg.vocab_size)

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config D: reference GPT 125M (12x768, 12 heads x 64, mlp 3072, vocab 50304) "
                               f"full train step, S=1024, global batch 128 as {n_micro} micro-batches of "
                               f"{cfg.micro_batch_size}, AdamW",
                   "global_batch": cfg.batch_size, "micro_batch": cfg.micro_batch_size, "seq_len": cfg.seq_len,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": f"flce (fused LM-head cross-entropy fwd+bwd per {cfg.micro_batch_size}x1024-token "
                               f"micro-batch: kept softmax over token chunks of {chunk}, bounded by vocab_tile_size "
                               f"{cfg.vocab_tile_size} like the reference's tiled loss)",
                     "bound": "mfma", "achieved": round(flce_tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flce_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": traffic, "traffic_GBps": None if traffic is None else round(traffic / flce_ms / 1e6, 1),
                     "ms": round(flce_ms, 3), "algorithmic_flops": flce_flops(mb_tokens, cfg.d_model,
                                                                              cfg.vocab_size)},
        "roofline_attn_bwd": {"kernel": f"attn_bwd (B{cfg.micro_batch_size} H12 S1024 D64 causal)", "bound": "mfma",
                              "achieved": round(ab_tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(ab_tf / MFMA_BF16_PEAK_TFLOPS, 4), "ms": round(ab_ms, 3)},
        "step_tflops": round(total_flops / (ms_per_step / 1e3) / 1e12, 1),
        "step_mfu": round(total_flops / (ms_per_step / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "attn_fwd_ms": round(af_ms, 3),
        "adamw": {"ms": round(adam_ms, 3), "achieved_GBps": round(adam_gbs, 1), "peak_GBps": 8000},
        "loss_first_last": [float(hist[0, 0]), float(hist[-1, 0])],
    }
    del trainer
    torch.cuda.empty_cache()
    result["roofline_flce_whole_vocab"] = flce_whole_vocab(mb_tokens, cfg.d_model, cfg.vocab_size)
    if not args.no_extra and args.micro_batch != 32:
        # BASELINE.json's split of the same step: 4 micro-batches of 32.
        split = GPTTrainer(replace(cfg, micro_batch_size=32), seed=0, history_steps=7)
        ms = timed_steps(split, xs, ys, 2, 5)
        result["split_4x32"] = {"ms_per_step": round(ms, 3), "tokens_per_s": round(tokens_per_step / (ms / 1e3), 1),
                                "steps": 5, "warmup": 2}
        del split
        torch.cuda.empty_cache()
    del windows, xs, ys
    torch.cuda.empty_cache()
    if not args.no_extra:
        result["config_E_moe_step"] = {"workload": "MoE recipe train step: 12x768 backbone, 8 experts top-2, "
                                                   "seq 1024, batch 32 (one pass), AdamW",
                                       "reference_valid_width": moe_step(2), "baseline_width": moe_step(4)}
    if not args.no_isolated:
        result["isolated"] = isolated_configs()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
