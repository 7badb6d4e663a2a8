"""GPU parity of the FLCE backward's paths, through the C ABI (ctypes).

* the chunked backward (several vocabulary chunks: the public API's default
  ``vocab_tile_size`` = 2048, pipelined launches over two halves of the
  ``[tokens, chunk]`` buffer), the one-chunk launches and the kept-softmax
  pair (the trainer's whole-vocabulary opt-in: the forward keeps its fp16
  probabilities, the backward rescales them instead of recomputing the
  logits) against the CPU oracle (``oracle.flce``, restating
  ``rig/kernels/linear_cross_entropy.py``), at config C's full size (16384
  tokens x 768 x 50304) and at small ragged shapes;
* the reference's width-5 bfloat16 fixture (``tests/test_linear_cross_entropy.py:
  73-80,129-152``), through the zero-padded public API.

Tolerances: mean loss relative error <= 1e-3 (north star), per-token loss
``1e-3 |loss| + 2e-4``, dh and dW max-abs <= 2% of their largest magnitude
(bf16 operands of the reference's own tiled matmuls).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import flce as oflce

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def maxabs(a, b):
    return float((a.float().cpu() - b.float().cpu()).abs().max())


def inputs(n, d, V, sv, seed, h_scale=1.0, w_scale=0.02):
    g = torch.Generator().manual_seed(seed)
    h = (torch.randn((n, d), generator=g) * h_scale).to(torch.bfloat16)
    w = torch.randn((V, d), generator=g) * w_scale
    t = torch.randint(0, sv, (n,), generator=g, dtype=torch.int32)
    return h, w, t


def run_backward(h, w, t, sv, chunk, ct=None, scale=0.0, dweight=None, accumulate=False):
    from gptrig.kernels import linear_cross_entropy as lce

    hg, wg, tg = h.to(DEV), w.to(torch.bfloat16).to(DEV), t.to(DEV)
    losses, lse = lce.flce_forward(hg, wg, tg, sv)
    dh, dw = lce.flce_backward(hg, wg, tg, lse, None if ct is None else ct.to(DEV), scale, sv, chunk,
                               dweight=dweight, accumulate=accumulate)
    torch.cuda.synchronize()
    return losses.cpu(), lse.cpu(), dh.cpu(), dw.cpu()


@pytest.mark.skip(reason="ran the in-kernel work-queue FLCE backward (cross-workgroup dependency counters), which "
                         "went silent for 180 s on its first GPU run with no cause found by reading; that kernel is "
                         "removed, and the chunked path (pipelined launches, no waits inside a launch) is covered by "
                         "test_config_c_pipelined_default_tile_matches_oracle")
def test_config_c_default_tile_and_whole_vocabulary_match_oracle():
    """Config C (16384 x 768 x 50304) through the removed work-queue kernel."""


def test_config_c_pipelined_default_tile_matches_oracle():
    """Config C (16384 x 768 x 50304, W ~ N(0, 0.02), mean loss): the public
    API's default tile (2048: 50 chunks of 1024 rows, 51 pipelined launches)
    and the trainer's single chunk against the oracle's tiled reference."""
    import time

    from gptrig.kernels import linear_cross_entropy as lce

    n, d, V = 16384, 768, 50304
    print(f"flce config C n={n} d={d} V={V}: oracle on the CPU", flush=True)
    h, w, t = inputs(n, d, V, V, 51)
    torch.set_num_threads(16)
    t0 = time.time()
    losses_ref, lse_ref = oflce.losses_and_lse(h, w, t, semantic_vocab_size=V, vocab_tile_size=2048)
    print(f"oracle forward {time.time() - t0:.1f} s", flush=True)
    ct = torch.full((n,), 1.0 / n)
    dh_ref, dw_ref = oflce.losses_backward(h, w, t, lse_ref, ct, semantic_vocab_size=V, vocab_tile_size=2048)
    print(f"oracle backward done {time.time() - t0:.1f} s; GPU public API", flush=True)
    sh, sw = float(dh_ref.float().abs().max()), float(dw_ref.abs().max())
    # Public API, default vocab_tile_size (2048).
    hg = h.to(DEV).requires_grad_(True)
    wg = w.to(DEV).requires_grad_(True)
    loss = lce.tiled_tied_cross_entropy(hg, wg, t.to(DEV), semantic_vocab_size=V)
    loss.backward()
    torch.cuda.synchronize()
    want = float(losses_ref.mean())
    print(f"mean loss gpu {float(loss):.6f} oracle {want:.6f}; dh {maxabs(hg.grad, dh_ref) / sh:.4f}, "
          f"dW {maxabs(wg.grad, dw_ref) / sw:.4f} of max", flush=True)
    assert abs(float(loss) - want) <= 1e-3 * abs(want)
    assert maxabs(hg.grad, dh_ref) <= 2e-2 * sh
    assert maxabs(wg.grad, dw_ref) <= 2e-2 * sw
    # Trainer opt-in: one chunk, scalar cotangent.
    print("GPU one chunk", flush=True)
    _, _, dh1, dw1 = run_backward(h, w, t, V, lce.grad_chunk(n, V), scale=1.0 / n)
    assert maxabs(dh1, dh_ref) <= 2e-2 * sh
    assert maxabs(dw1, dw_ref) <= 2e-2 * sw
    # The two paths sum the same bf16 products in different fp32 orders.
    assert maxabs(dh1, hg.grad) <= 1e-2 * sh
    # Kept-softmax pair (the trainer's path): same losses as the forward, and
    # gradients from the rescaled kept probabilities.
    print("GPU kept softmax", flush=True)
    lk, lsek, dhk, dwk = run_keep(h, w, t, V, scale=1.0 / n)
    assert abs(float(lk.mean()) - want) <= 1e-3 * abs(want)
    assert maxabs(dhk, dh_ref) <= 2e-2 * sh
    assert maxabs(dwk, dw_ref) <= 2e-2 * sw
    assert maxabs(dhk, dh1) <= 1e-2 * sh and maxabs(dwk, dw1) <= 1e-2 * sw


def run_keep(h, w, t, sv, ct=None, scale=0.0, dweight=None, accumulate=False):
    from gptrig.kernels import linear_cross_entropy as lce

    hg, wg, tg = h.to(DEV), w.to(torch.bfloat16).to(DEV), t.to(DEV)
    losses, lse, keep = lce.flce_forward_keep(hg, wg, tg, sv)
    dh, dw = lce.flce_backward_keep(hg, wg, tg, lse, keep, None if ct is None else ct.to(DEV), scale, sv,
                                    dweight=dweight, accumulate=accumulate)
    torch.cuda.synchronize()
    return losses.cpu(), lse.cpu(), dh.cpu(), dw.cpu()


KEEP_CASES = [
    # (n, d, V, semantic V): ragged vocabulary tiles and a partial last token tile; d a multiple of 128
    (2056, 256, 1300, 1297),
    (4096, 768, 5000, 4999),
    (8, 128, 600, 600),
    (1536, 384, 2312, 2000),
]


@pytest.mark.parametrize("n,d,V,sv", KEEP_CASES)
def test_kept_softmax_pair_matches_oracle_and_forward(n, d, V, sv):
    """gptrig_flce_fwd_keep / gptrig_flce_bwd_keep: the forward's losses and
    lse equal gptrig_flce_fwd's bit for bit (same launches plus stores), and
    the gradients from the rescaled kept probabilities match the oracle to the
    tolerances of the recompute path (one more fp16 rounding per probability),
    with invalid targets, per-token cotangents, padding rows and dW
    accumulation."""
    print(f"flce kept case n={n} d={d} V={V} sv={sv}", flush=True)
    h, w, t = inputs(n, d, V, sv, 71, 0.5, 0.5)
    t[::11] = -1
    g = torch.Generator().manual_seed(72)
    ct = torch.rand(n, generator=g)
    losses_ref, lse_ref = oflce.losses_and_lse(h, w, t, semantic_vocab_size=sv, vocab_tile_size=256)
    dh_ref, dw_ref = oflce.losses_backward(h, w, t, lse_ref, ct, semantic_vocab_size=sv, vocab_tile_size=256)
    lo, ls, _, _ = run_backward(h, w, t, sv, 1 << 20, ct=ct)
    lk, lsk, dhk, dwk = run_keep(h, w, t, sv, ct=ct)
    assert torch.equal(torch.isfinite(lk), torch.isfinite(lo))
    fin = torch.isfinite(lo)
    assert torch.equal(lk[fin], lo[fin]) and torch.equal(lsk, ls)
    sh, sw = float(dh_ref.float().abs().max()), float(dw_ref.abs().max())
    print(f"  dh {maxabs(dhk, dh_ref) / sh:.4f}, dW {maxabs(dwk, dw_ref) / sw:.4f} of max", flush=True)
    assert maxabs(dhk, dh_ref) <= 2e-2 * sh
    assert maxabs(dwk, dw_ref) <= 2e-2 * sw
    assert (dwk[sv:] == 0).all()
    base = torch.randn(V, d, generator=g)
    _, _, dh2, dw2 = run_keep(h, w, t, sv, ct=ct, dweight=base.to(DEV), accumulate=True)
    # (The one-chunk dh GEMM adds its K splits with f32 atomics: equal up to
    # the order of those adds, one bf16 step at most.)
    assert maxabs(dh2, dhk) <= 1e-2 * sh
    assert maxabs(dw2 - base, dwk) <= 1e-5 * max(1.0, float(base.abs().max()))


def test_kept_softmax_token_chunks_equal_one_chunk():
    """The trainer's bounded form of the kept-softmax pair: the tokens cut into
    chunks (of 1024 and a ragged 520), each chunk's forward and backward run
    back to back with dW accumulated, against the oracle and against one call
    over all tokens.  Losses and lse are per token, so they are bit-equal; dh
    rows are per token too (equal up to the dh GEMM's split-K order); dW sums
    the chunks in another order (f32)."""
    from gptrig.kernels import linear_cross_entropy as lce

    n, d, V, sv = 3592, 256, 3000, 2998
    print(f"flce kept token chunks n={n} d={d} V={V}", flush=True)
    h, w, t = inputs(n, d, V, sv, 81, 0.5, 0.5)
    t[::13] = -1
    losses_ref, lse_ref = oflce.losses_and_lse(h, w, t, semantic_vocab_size=sv, vocab_tile_size=256)
    ct = torch.full((n,), 1.0 / n)
    dh_ref, dw_ref = oflce.losses_backward(h, w, t, lse_ref, ct, semantic_vocab_size=sv, vocab_tile_size=256)
    l1, ls1, dh1, dw1 = run_keep(h, w, t, sv, scale=1.0 / n)
    hg, wg, tg = h.to(DEV), w.to(torch.bfloat16).to(DEV), t.to(DEV)
    dw = torch.empty(V, d, device=DEV)
    parts_l, parts_s, parts_dh = [], [], []
    keep = None
    for c0 in range(0, n, 1024):
        c1 = min(n, c0 + 1024)
        lc, lsc, keep = lce.flce_forward_keep(hg[c0:c1], wg, tg[c0:c1], sv, keep)
        dhc, _ = lce.flce_backward_keep(hg[c0:c1], wg, tg[c0:c1], lsc, keep, None, 1.0 / n, sv, dweight=dw,
                                        accumulate=c0 > 0)
        parts_l.append(lc.cpu())
        parts_s.append(lsc.cpu())
        parts_dh.append(dhc.cpu())
    torch.cuda.synchronize()
    lk, lsk, dhk, dwk = torch.cat(parts_l), torch.cat(parts_s), torch.cat(parts_dh), dw.cpu()
    fin = torch.isfinite(l1)
    assert torch.equal(torch.isfinite(lk), fin) and torch.equal(lk[fin], l1[fin]) and torch.equal(lsk, ls1)
    sh, sw = float(dh_ref.float().abs().max()), float(dw_ref.abs().max())
    print(f"  dh {maxabs(dhk, dh_ref) / sh:.4f}, dW {maxabs(dwk, dw_ref) / sw:.4f} of max", flush=True)
    assert maxabs(dhk, dh_ref) <= 2e-2 * sh and maxabs(dwk, dw_ref) <= 2e-2 * sw
    assert maxabs(dhk, dh1) <= 1e-2 * sh
    assert maxabs(dwk, dw1) <= 1e-3 * sw
    assert (dwk[sv:] == 0).all()


CHUNKED_CASES = [
    # (n, d, V, semantic V, chunk): ragged token tiles, partial d tiles, ragged last chunks, the
    # alternating (256-row chunk) and pipelined (>= 512) forms
    (2056, 192, 1300, 1297, 512),
    (4096, 768, 5000, 4999, 1024),
    (8, 64, 600, 600, 256),
    (1536, 320, 2311, 2000, 768),
    (296, 128, 1000, 997, 256),
]


@pytest.mark.parametrize("n,d,V,sv,chunk", CHUNKED_CASES)
def test_chunked_backward_matches_oracle(n, d, V, sv, chunk):
    print(f"flce chunked case n={n} d={d} V={V} sv={sv} chunk={chunk}", flush=True)
    h, w, t = inputs(n, d, V, sv, 61, 0.5, 0.5)
    t[::13] = -1  # invalid targets: no gradient
    g = torch.Generator().manual_seed(62)
    ct = torch.rand(n, generator=g)
    losses_ref, lse_ref = oflce.losses_and_lse(h, w, t, semantic_vocab_size=sv, vocab_tile_size=chunk)
    dh_ref, dw_ref = oflce.losses_backward(h, w, t, lse_ref, ct, semantic_vocab_size=sv, vocab_tile_size=chunk)
    losses, lse, dh, dw = run_backward(h, w, t, sv, chunk, ct=ct)
    finite = torch.isfinite(losses_ref)
    assert torch.equal(finite, torch.isfinite(losses))
    assert bool(((losses[finite] - losses_ref[finite]).abs() <= 1e-3 * losses_ref[finite].abs() + 2e-4).all())
    sh, sw = float(dh_ref.float().abs().max()), float(dw_ref.abs().max())
    assert maxabs(dh, dh_ref) <= 2e-2 * sh
    assert maxabs(dw, dw_ref) <= 2e-2 * sw
    assert (dw[sv:] == 0).all()
    # accumulate_dweight: adds into an existing dW; the second call sees the same inputs.
    base = torch.randn(V, d, generator=g)
    _, _, dh2, dw2 = run_backward(h, w, t, sv, chunk, ct=ct, dweight=base.to(DEV), accumulate=True)
    assert torch.equal(dh2, dh)
    assert maxabs(dw2 - base, dw) <= 1e-5 * max(1.0, float(base.abs().max()))


def test_width_five_bfloat16_fixture():
    """tests/test_linear_cross_entropy.py:129-152 of the reference: hidden
    (2, 3, 5) from default_rng(7) as bfloat16, embedding (13, 5) from
    default_rng(11), semantic vocabulary 11, tile 7; the value within
    4e-3 of the dense bf16 oracle, gradients in the input dtypes."""
    from gptrig.kernels import tiled_tied_cross_entropy

    hidden = torch.from_numpy(np.random.default_rng(7).normal(size=(2, 3, 5)).astype(np.float32)).to(torch.bfloat16)
    embedding = torch.from_numpy(np.random.default_rng(11).normal(size=(13, 5)).astype(np.float32))
    targets = torch.tensor([[0, 1, 10], [3, 8, 6]], dtype=torch.int32)
    hg = hidden.to(DEV).requires_grad_(True)
    eg = embedding.to(DEV).requires_grad_(True)
    value = tiled_tied_cross_entropy(hg, eg, targets.to(DEV), semantic_vocab_size=11, vocab_tile_size=7)
    value.backward()
    h2 = hidden.clone().requires_grad_(True)
    e2 = embedding.clone().requires_grad_(True)
    oracle = oflce.dense_losses(h2, e2, targets, 11, torch.bfloat16).mean()
    oracle.backward()
    print(f"width 5: gpu {float(value):.6f} dense {float(oracle):.6f}", flush=True)
    assert abs(float(value) - float(oracle)) <= 4e-3 + 4e-3 * abs(float(oracle))
    assert value.dtype == torch.float32
    assert hg.grad.dtype == torch.bfloat16 and eg.grad.dtype == torch.float32
    assert tuple(hg.grad.shape) == (2, 3, 5) and tuple(eg.grad.shape) == (13, 5)
    assert maxabs(hg.grad, h2.grad) <= 2e-2 * float(h2.grad.float().abs().max())
    assert maxabs(eg.grad, e2.grad) <= 2e-2 * float(e2.grad.abs().max())
    assert (eg.grad[11:] == 0).all()


def test_float32_compute_reference_fixture():
    """compute_dtype=float32 (rig/kernels/linear_cross_entropy.py:38-41) on
    the reference's own float32 cases (tests/test_linear_cross_entropy.py:
    84-127): hidden (2, 3, 5) from default_rng(7), embedding (13, 5) from
    default_rng(11), semantic vocabulary 11, tile 4; per-token losses within
    rtol = atol = 2e-6 of the dense float32 oracle, the mean and both
    gradients within 3e-6, storage-only rows' gradient exactly zero."""
    from gptrig.kernels import tiled_tied_cross_entropy, tiled_tied_cross_entropy_losses

    hidden = torch.from_numpy(np.random.default_rng(7).normal(size=(2, 3, 5)).astype(np.float32))
    embedding = torch.from_numpy(np.random.default_rng(11).normal(size=(13, 5)).astype(np.float32))
    targets = torch.tensor([[0, 1, 10], [3, 8, 6]], dtype=torch.int32)
    print("flce float32 compute, reference fixture", flush=True)
    losses = tiled_tied_cross_entropy_losses(hidden.to(DEV), embedding.to(DEV), targets.to(DEV),
                                             semantic_vocab_size=11, vocab_tile_size=4, compute_dtype=torch.float32)
    want = oflce.dense_losses(hidden, embedding, targets, 11, torch.float32)
    np.testing.assert_allclose(losses.cpu().numpy(), want.numpy(), rtol=2e-6, atol=2e-6)
    hg = hidden.to(DEV).requires_grad_(True)
    eg = embedding.to(DEV).requires_grad_(True)
    value = tiled_tied_cross_entropy(hg, eg, targets.to(DEV), semantic_vocab_size=11, vocab_tile_size=4,
                                     compute_dtype=torch.float32)
    value.backward()
    h2 = hidden.clone().requires_grad_(True)
    e2 = embedding.clone().requires_grad_(True)
    dense = oflce.dense_losses(h2, e2, targets, 11, torch.float32).mean()
    dense.backward()
    print(f"  gpu {float(value):.8f} dense {float(dense):.8f}", flush=True)
    assert abs(float(value) - float(dense)) <= 2e-6 + 2e-6 * abs(float(dense))
    np.testing.assert_allclose(hg.grad.cpu().numpy(), h2.grad.numpy(), rtol=3e-6, atol=3e-6)
    np.testing.assert_allclose(eg.grad.cpu().numpy(), e2.grad.numpy(), rtol=3e-6, atol=3e-6)
    assert hg.grad.dtype == torch.float32 and eg.grad.dtype == torch.float32
    assert (eg.grad[11:] == 0).all()


@pytest.mark.parametrize("n,d,V,sv,tile", [(300, 96, 1000, 997, 256), (1030, 200, 3001, 2900, 2048), (8, 5, 13, 11, 4)])
def test_float32_compute_matches_float64_dense(n, d, V, sv, tile):
    """The float32 path against the float64 dense closed form at larger,
    ragged shapes (tokens, width, vocabulary and chunks not multiples of the
    64 tile), with invalid targets (+inf loss, no gradient) and per-token
    cotangents: losses to 2e-6 relative, gradients to 1e-5 of their scale."""
    from gptrig.kernels import tiled_tied_cross_entropy_losses

    g = torch.Generator().manual_seed(91)
    h = torch.randn((n, d), generator=g)
    w = torch.randn((V, d), generator=g) * 0.3
    t = torch.randint(0, sv, (n,), generator=g, dtype=torch.int32)
    t[::17] = -1
    ct = torch.rand(n, generator=g)
    print(f"flce float32 compute n={n} d={d} V={V} sv={sv} tile={tile}", flush=True)
    hg = h.to(DEV).requires_grad_(True)
    wg = w.to(DEV).requires_grad_(True)
    losses = tiled_tied_cross_entropy_losses(hg, wg, t.to(DEV), semantic_vocab_size=sv, vocab_tile_size=tile,
                                             compute_dtype=torch.float32)
    finite = torch.isfinite(losses)
    (losses[finite] * ct.to(DEV)[finite]).sum().backward()
    h64 = h.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    logits = h64 @ w64[:sv].t()
    valid = t >= 0
    lse = torch.logsumexp(logits, -1)
    ref = torch.full((n,), float("inf"), dtype=torch.float64)
    ref[valid] = lse[valid] - logits[valid].gather(1, t[valid].long()[:, None])[:, 0]
    (ref[valid] * ct.double()[valid]).sum().backward()
    lc = losses.detach().cpu().double()
    assert torch.equal(torch.isfinite(lc), valid)
    rel = ((lc[valid] - ref[valid]).abs() / ref[valid].abs()).max()
    print(f"  loss rel {float(rel):.2e}", flush=True)
    assert float(rel) <= 2e-6
    for got, want in ((hg.grad, h64.grad), (wg.grad, w64.grad)):
        err = float((got.cpu().double() - want).abs().max())
        scale = float(want.abs().max())
        print(f"  grad max-abs {err:.3e} of {scale:.3e}", flush=True)
        assert err <= 1e-5 * scale
    assert (wg.grad[sv:] == 0).all()
