"""Pins ``oracle.attention`` (CPU only).

Forward: brute-force per-row softmax in pure Python; the kernel-numerics
forward against the exact softmax with unrounded probabilities (every tile
shape, padding and block skipping) and, with bf16 probabilities, against the
one-chunk closed form ``sum_j bf16(exp(s_j - m)) v_j / sum_j exp(s_j - m)``.
Backward: float64 autograd of the textbook softmax-attention formula (an
independent derivation).  Invariants mirror ``tests/test_tpu_flash_attention.py``
of the reference (causal prefix ``:34-39``, documents ``:107-136``).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa


def qkv(shape, seed=0, scale=0.15, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(shape, generator=g) * scale).to(dtype) for _ in range(3))


def brute_force(q, k, v, scale, segments=None):
    B, H, S, D = q.shape
    out = np.zeros((B, H, S, D))
    for b in range(B):
        for h in range(H):
            for i in range(S):
                cols = [j for j in range(i + 1) if segments is None or segments[b][j] == segments[b][i]]
                s = [scale * sum(float(q[b, h, i, d]) * float(k[b, h, j, d]) for d in range(D)) for j in cols]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                tot = sum(e)
                for d in range(D):
                    out[b, h, i, d] = sum(e[t] / tot * float(v[b, h, j, d]) for t, j in enumerate(cols))
    return out


def test_forward_matches_brute_force():
    q, k, v = qkv((1, 2, 9, 8), seed=1, scale=0.8)
    scale = 8 ** -0.5
    got = oa.reference_causal_attention(q, k, v)
    np.testing.assert_allclose(got.numpy(), brute_force(q, k, v, scale), rtol=1e-5, atol=1e-6)


def test_forward_with_segments_matches_brute_force():
    q, k, v = qkv((2, 1, 10, 8), seed=2, scale=0.8)
    seg = torch.tensor([[0, 0, 0, 1, 1, 1, 1, 2, 2, 2], [0, 1, 1, 1, 1, 1, 2, 2, 3, 3]], dtype=torch.int32)
    got = oa.reference_causal_attention(q, k, v, softmax_scale=0.3, segment_ids=seg)
    np.testing.assert_allclose(got.numpy(), brute_force(q, k, v, 0.3, seg.tolist()), rtol=1e-5, atol=1e-6)


def test_lse_is_log_of_row_partition_function():
    q, k, v = qkv((1, 1, 6, 8), seed=3, scale=1.0)
    _, lse = oa.attention_forward(q, k, v, softmax_scale=0.5)
    for i in range(6):
        s = [0.5 * float((q[0, 0, i] * k[0, 0, j]).sum()) for j in range(i + 1)]
        assert abs(float(lse[0, 0, i]) - math.log(sum(math.exp(x) for x in s))) < 1e-5


def dense64(q, k, v, scale, segments=None):
    S = q.shape[2]
    s = (q @ k.transpose(-1, -2)) * scale
    vis = oa.visibility(S, segments)
    s = s.masked_fill(~vis, float("-inf"))
    return torch.softmax(s, -1) @ v


@pytest.mark.parametrize("segmented", [False, True])
def test_backward_matches_float64_autograd(segmented):
    q, k, v = qkv((2, 2, 33, 16), seed=4, scale=0.7)
    do = qkv((2, 2, 33, 16), seed=5, scale=1.0)[0]
    seg = None
    if segmented:
        seg = torch.tensor([[0] * 10 + [1] * 13 + [2] * 10, [0] * 33], dtype=torch.int32)
    scale = 0.21
    o, lse = oa.attention_forward(q, k, v, softmax_scale=scale, segment_ids=seg)
    dq, dk, dv = oa.attention_backward(q, k, v, o, lse, do, softmax_scale=scale, segment_ids=seg)
    q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
    out = dense64(q64, k64, v64, scale, seg)
    np.testing.assert_allclose(o.numpy(), out.detach().numpy(), rtol=1e-5, atol=1e-6)
    g = torch.autograd.grad(out, (q64, k64, v64), do.double())
    for got, want in zip((dq, dk, dv), g):
        np.testing.assert_allclose(got.numpy(), want.numpy(), rtol=1e-4, atol=1e-6)


def test_causal_prefix_invariance():
    q, k, v = qkv((1, 2, 16, 8), seed=6)
    changed = v.clone()
    changed[:, :, 9:, :] = 10_000.0
    a = oa.reference_causal_attention(q, k, v)
    b = oa.reference_causal_attention(q, k, changed)
    np.testing.assert_allclose(a[:, :, :9].numpy(), b[:, :, :9].numpy())


def segments_from_cuts(sequence, cuts):
    starts = np.zeros(sequence, np.int32)
    starts[list(cuts)] = 1
    return torch.from_numpy(np.cumsum(starts)[None, :] - 1).to(torch.int32)


def test_document_independence_and_single_segment():
    q, k, v = qkv((1, 2, 256, 8), seed=7)
    seg = segments_from_cuts(256, (0, 61, 130, 131, 200))
    packed = oa.reference_causal_attention(q, k, v, segment_ids=seg)
    alone = oa.reference_causal_attention(q[:, :, 61:130], k[:, :, 61:130], v[:, :, 61:130])
    np.testing.assert_allclose(packed[:, :, 61:130].numpy(), alone.numpy(), rtol=1e-6, atol=1e-6)
    assert not np.allclose(packed.numpy(), oa.reference_causal_attention(q, k, v).numpy(), atol=1e-4)
    single = oa.reference_causal_attention(q, k, v, segment_ids=torch.zeros((1, 256), dtype=torch.int32))
    np.testing.assert_allclose(single.numpy(), oa.reference_causal_attention(q, k, v).numpy(), rtol=1e-6, atol=1e-6)


def test_document_segments_known_answer():
    # rig/attention.py:205-208; expected values from tests/test_attention.py:206-211.
    tokens = torch.tensor([[9, 1, 2, 9, 3], [4, 9, 5, 9, 9]], dtype=torch.int32)
    assert oa.document_segments(tokens, 9).tolist() == [[1, 1, 1, 2, 2], [0, 1, 1, 2, 3]]


def test_softmax_scale_rules():
    # tests/test_attention.py:34-42 of the reference.
    assert oa.attention_softmax_scale("inverse_head_dim", 64) == 1.0 / 64
    assert oa.attention_softmax_scale("inverse_sqrt_head_dim", 64) == 0.125
    with pytest.raises(ValueError):
        oa.attention_softmax_scale("bogus", 64)


def test_validation_errors():
    q, k, v = qkv((1, 1, 8, 8))
    with pytest.raises(ValueError):
        oa.reference_causal_attention(q[0], k[0], v[0])
    with pytest.raises(ValueError):
        oa.reference_causal_attention(q, k[:, :, :4], v)
    with pytest.raises(ValueError):
        oa.reference_causal_attention(*qkv((1, 1, 8, 12)))
    with pytest.raises(TypeError):
        oa.reference_causal_attention(q, k.double(), v)


def test_flash_tiles_follow_the_reference_choice():
    # select_attention_tiles (tpu_flash_attention.py:112-142): 512/512/256 is
    # the preferred shape and legal from S = 512 on; shorter or odd extents fall
    # back to the nearest legal candidate.
    assert oa.flash_tiles(1024) == (512, 512, 256)
    assert oa.flash_tiles(2048) == (512, 512, 256)
    assert oa.flash_tiles(512) == (512, 512, 256)
    assert oa.flash_tiles(256) == (256, 256, 128)
    assert oa.flash_tiles(200) == (256, 256, 128)  # padded to 256
    assert oa.flash_tiles(384) == (128, 128, 128)
    assert oa.flash_tiles(100) == (128, 128, 128)


def bf16_ulps(a, b):
    ai = a.to(torch.bfloat16).view(torch.int16).int()
    bi = b.to(torch.bfloat16).view(torch.int16).int()
    return (ai - bi).abs()


@pytest.mark.parametrize("S,segmented", [(9, False), (200, False), (300, True), (1024, False), (1024, True)])
def test_flash_forward_with_unrounded_probabilities_is_the_exact_softmax(S, segmented):
    # With float32 probabilities the rescaled recurrence is the exact softmax
    # average whatever the tiles: this pins the chunk order, the running max,
    # the corrections, the block skipping, the padding mask and the LSE.
    g = torch.Generator().manual_seed(S)
    q, k, v = ((torch.randn((1, 2, S, 16), generator=g) * 0.9).to(torch.bfloat16) for _ in range(3))
    seg = segments_from_cuts(S, (0, S // 3, S // 3 + 1, (2 * S) // 3)) if segmented else None
    o, lse = oa.flash_attention_forward(q, k, v, softmax_scale=0.4, segment_ids=seg, probability_dtype=torch.float32)
    s = (q.double() @ k.double().transpose(-1, -2)) * 0.4
    s = s.masked_fill(~oa.visibility(S, seg), float("-inf"))
    want = torch.softmax(s, -1) @ v.double()
    ulps = bf16_ulps(o, want)
    assert int(ulps.max()) <= 1 and float((ulps > 0).float().mean()) < 0.02
    np.testing.assert_allclose(lse.double().numpy(), torch.logsumexp(s, -1).numpy(), rtol=2e-6, atol=2e-6)


def test_flash_forward_rounds_the_unnormalised_probabilities():
    # S <= 128 is one chunk: out = sum_j bf16(e_j) v_j / sum_j e_j with
    # e_j = exp(s_j - max_j s_j), the normaliser taken from the unrounded e.
    q, k, v = qkv((1, 1, 40, 8), seed=11, scale=1.5, dtype=torch.bfloat16)
    o, _ = oa.flash_attention_forward(q, k, v, softmax_scale=0.7)
    want = np.zeros((40, 8))
    for i in range(40):
        s = [0.7 * float((q[0, 0, i].double() * k[0, 0, j].double()).sum()) for j in range(i + 1)]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        eb = [float(torch.tensor(x, dtype=torch.float32).to(torch.bfloat16)) for x in e]
        for d in range(8):
            want[i, d] = sum(eb[j] * float(v[0, 0, j, d]) for j in range(i + 1)) / sum(e)
    ulps = bf16_ulps(o[0, 0].float(), torch.from_numpy(want))
    assert int(ulps.max()) <= 1 and float((ulps > 0).float().mean()) < 0.02
    # ... which is not the normalised rounding of the kernel's test oracle.
    assert not torch.equal(o, oa.reference_causal_attention(q, k, v, softmax_scale=0.7))


def test_flash_forward_rows_inside_the_first_chunk_ignore_the_rest():
    # Rows 0..255 of S = 1024 see only the first 256-key chunk: the later
    # chunks of their block are fully masked (p = 0, correction 1), so they get
    # the one-chunk result of the same rows computed alone.
    q, k, v = qkv((1, 2, 1024, 16), seed=12, scale=1.0, dtype=torch.bfloat16)
    full, lse_full = oa.flash_attention_forward(q, k, v)
    alone, lse_alone = oa.flash_attention_forward(q[:, :, :128], k[:, :, :128], v[:, :, :128])
    assert int(bf16_ulps(full[:, :, :128], alone).max()) <= 1
    np.testing.assert_allclose(lse_full[:, :, :128].numpy(), lse_alone.numpy(), rtol=1e-6, atol=1e-6)
