"""Pins ``oracle.flce`` (CPU only) with the reference's own FLCE test cases.

Inputs are regenerated from the numpy seeds of
``tests/test_linear_cross_entropy.py`` (7, 11, 29) and checked against the
dense log-softmax closed form and its autograd gradient, with the reference's
tolerances.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import flce as of


@pytest.fixture
def small():
    hidden = torch.from_numpy(np.random.default_rng(7).normal(size=(2, 3, 5)).astype(np.float32))
    embedding = torch.from_numpy(np.random.default_rng(11).normal(size=(13, 5)).astype(np.float32))
    targets = torch.tensor([[0, 1, 10], [3, 8, 6]], dtype=torch.int32)
    return hidden, embedding, targets


def test_values_match_dense_with_padded_storage(small):
    h, e, t = small
    got = of.tiled_tied_cross_entropy_losses(h, e, t, semantic_vocab_size=11, vocab_tile_size=4,
                                             compute_dtype=torch.float32)
    want = of.dense_losses(h, e, t, 11, torch.float32)
    np.testing.assert_allclose(got.numpy(), want.numpy(), rtol=2e-6, atol=2e-6)


def test_value_and_grads_match_dense(small):
    h, e, t = small
    h1, e1 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    loss = of.tiled_tied_cross_entropy(h1, e1, t, semantic_vocab_size=11, vocab_tile_size=4,
                                       compute_dtype=torch.float32)
    gh, ge = torch.autograd.grad(loss, (h1, e1))
    h2, e2 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    dense = of.dense_losses(h2, e2, t, 11, torch.float32).mean()
    dh, de = torch.autograd.grad(dense, (h2, e2))
    assert abs(float(loss) - float(dense)) < 2e-6
    np.testing.assert_allclose(gh.numpy(), dh.numpy(), rtol=3e-6, atol=3e-6)
    np.testing.assert_allclose(ge.numpy(), de.numpy(), rtol=3e-6, atol=3e-6)
    assert (ge[11:] == 0).all()


def test_bf16_compute_close_and_dtypes(small):
    h, e, t = small
    hb = h.to(torch.bfloat16).requires_grad_(True)
    e1 = e.clone().requires_grad_(True)
    loss = of.tiled_tied_cross_entropy(hb, e1, t, semantic_vocab_size=11, vocab_tile_size=7,
                                       compute_dtype=torch.bfloat16)
    gh, ge = torch.autograd.grad(loss, (hb, e1))
    want = of.dense_losses(hb.detach(), e, t, 11, torch.bfloat16).mean()
    assert abs(float(loss) - float(want)) < 4e-3
    assert loss.dtype == torch.float32 and gh.dtype == torch.bfloat16 and ge.dtype == torch.float32


def test_bf16_wide_target_dot():
    rng = np.random.default_rng(29)
    h = torch.from_numpy(rng.normal(0.0, 0.5, size=(2, 3, 768)).astype(np.float32))
    e = torch.from_numpy(rng.normal(0.0, 0.5, size=(259, 768)).astype(np.float32))
    t = torch.tensor([[0, 127, 256], [7, 128, 42]], dtype=torch.int32)
    h1, e1 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    loss = of.tiled_tied_cross_entropy(h1, e1, t, semantic_vocab_size=257, vocab_tile_size=128,
                                       compute_dtype=torch.bfloat16)
    gh, ge = torch.autograd.grad(loss, (h1, e1))
    h2, e2 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    dense = of.dense_losses(h2, e2, t, 257, torch.bfloat16).mean()
    dh, de = torch.autograd.grad(dense, (h2, e2))
    assert abs(float(loss) - float(dense)) <= 2e-4 + 2e-4 * abs(float(dense))
    np.testing.assert_allclose(gh.numpy(), dh.numpy(), rtol=5e-3, atol=5e-3)
    np.testing.assert_allclose(ge.numpy(), de.numpy(), rtol=5e-3, atol=5e-3)


def test_invalid_targets_infinite_loss_zero_grads(small):
    h, e, _ = small
    bad = torch.tensor([[-1, 1, 99], [3, 8, 6]], dtype=torch.int32)
    h1, e1 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    losses = of.tiled_tied_cross_entropy_losses(h1, e1, bad, semantic_vocab_size=11, vocab_tile_size=4,
                                                compute_dtype=torch.float32)
    assert math.isinf(float(losses.sum()))
    gh, ge = torch.autograd.grad(losses.sum(), (h1, e1))
    w = torch.tensor([[0.0, 1.0, 0.0], [1.0, 1.0, 1.0]])
    h2, e2 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    ref = (of.dense_losses(h2, e2, bad.clamp(0, 10), 11, torch.float32) * w).sum()
    dh, de = torch.autograd.grad(ref, (h2, e2))
    np.testing.assert_allclose(gh.numpy(), dh.numpy(), rtol=3e-6, atol=3e-6)
    np.testing.assert_allclose(ge.numpy(), de.numpy(), rtol=3e-6, atol=3e-6)


def test_per_token_cotangents(small):
    h, e, t = small
    w = torch.tensor([[1.0, 0.0, 0.25], [0.5, 1.0, 0.0]])
    h1, e1 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    got = (of.tiled_tied_cross_entropy_losses(h1, e1, t, semantic_vocab_size=11, vocab_tile_size=4,
                                              compute_dtype=torch.float32) * w).sum()
    gh, ge = torch.autograd.grad(got, (h1, e1))
    h2, e2 = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    want = (of.dense_losses(h2, e2, t, 11, torch.float32) * w).sum()
    dh, de = torch.autograd.grad(want, (h2, e2))
    np.testing.assert_allclose(gh.numpy(), dh.numpy(), rtol=3e-6, atol=3e-6)
    np.testing.assert_allclose(ge.numpy(), de.numpy(), rtol=3e-6, atol=3e-6)


def test_invalid_contracts(small):
    h, e, t = small
    for kwargs in (dict(semantic_vocab_size=0, vocab_tile_size=4), dict(semantic_vocab_size=14, vocab_tile_size=4),
                   dict(semantic_vocab_size=11, vocab_tile_size=0)):
        with pytest.raises(ValueError):
            of.tiled_tied_cross_entropy(h, e, t, **kwargs)
    with pytest.raises(TypeError):
        of.tiled_tied_cross_entropy(h, e, t.float(), semantic_vocab_size=11)
