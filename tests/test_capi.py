"""The C-ABI library loads and exports every symbol ``include/gptrig.h`` declares (CPU only)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from gptrig import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "gptrig.h")


def declared() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:int|size_t|const char\*)\s+(gptrig_\w+)\(", text, re.M)


def test_library_exports_every_declared_symbol():
    names = declared()
    assert len(names) >= 20
    lib = _lib.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_version_and_status_strings():
    assert "gfx950" in _lib.version()
    lib = _lib.lib()
    assert lib.gptrig_status_string(0) == b"ok"
    assert b"workspace" in lib.gptrig_status_string(-6)


def test_host_validation_rejects_bad_arguments_without_launching():
    lib = _lib.lib()
    dummy = ctypes.c_void_p(16)
    # NULL pointers
    assert lib.gptrig_attn_fwd(None, None, None, None, None, None, 1, 1, 8, 64, None, 0.125, None) == -1
    # unsupported head_dim
    assert lib.gptrig_attn_fwd(dummy, dummy, dummy, None, dummy, dummy, 1, 1, 8, 96, None, 0.125, None) == -4
    # non-positive scale
    assert lib.gptrig_attn_fwd(dummy, dummy, dummy, None, dummy, dummy, 1, 1, 8, 64, None, 0.0, None) == -2
    # FLCE: width not a multiple of 64, semantic vocab past storage
    assert lib.gptrig_flce_fwd(dummy, dummy, dummy, dummy, dummy, dummy, 1 << 30, 8, 100, 10, 5, None) == -2
    assert lib.gptrig_flce_fwd(dummy, dummy, dummy, dummy, dummy, dummy, 1 << 30, 8, 128, 10, 11, None) == -2
    # FLCE: workspace too small
    assert lib.gptrig_flce_fwd(dummy, dummy, dummy, dummy, dummy, dummy, 16, 8, 128, 10, 10, None) == -6
    # FLCE kept softmax: width a multiple of 64 but not 128, keep buffer too small, tokens not a multiple of 8
    big = ctypes.c_size_t(1 << 40)
    assert lib.gptrig_flce_fwd_keep(dummy, dummy, dummy, dummy, dummy, dummy, big, dummy, big, 16, 64, 1000, 1000,
                                    None) == -4
    assert lib.gptrig_flce_fwd_keep(dummy, dummy, dummy, dummy, dummy, dummy, 16, dummy, big, 16, 128, 1000, 1000,
                                    None) == -6
    assert lib.gptrig_flce_bwd_keep(dummy, dummy, dummy, dummy, None, ctypes.c_float(1.0), dummy, dummy, 0, dummy,
                                    big, dummy, big, 12, 128, 1000, 1000, None) == -4
    assert lib.gptrig_flce_keep_bytes(16, 1000) >= 2 * 32 * 1000 + 2 * 4 * 16 * 4
    # AdamW: chunk not a multiple of 1024
    assert lib.gptrig_adamw(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 1000, 0.1, 0.9, 0.95, 1, None, None,
                            None) == -2
    # routing: too many experts
    assert lib.gptrig_moe_route(dummy, None, dummy, dummy, dummy, dummy, dummy, None, None, 0, 8, 65, 2, None) == -4
    # bias-fused passes: misaligned bias / data, cols not a multiple of 8, v columns past the row stride
    odd = ctypes.c_void_p(18)
    assert lib.gptrig_bias_gelu_fwd(dummy, odd, dummy, 4, 64, None) == -2
    assert lib.gptrig_bias_gelu_fwd(dummy, dummy, dummy, 4, 60, None) == -2
    assert lib.gptrig_bias_gelu_bwd(dummy, odd, dummy, dummy, 4, 64, None) == -2
    assert lib.gptrig_bias_gelu_fwd(None, dummy, dummy, 4, 64, None) == -1
    assert lib.gptrig_bias_rope_fwd(dummy, 192, 4, 192, odd, 8, 2, 64, dummy, dummy, None) == -2
    assert lib.gptrig_bias_rope_fwd(dummy, 128, 4, 192, dummy, 8, 2, 64, dummy, dummy, None) == -2
    assert lib.gptrig_bias_rope_fwd(dummy, 192, 4, 96, dummy, 8, 2, 64, dummy, dummy, None) == -2
    assert lib.gptrig_add_bias_rmsnorm_fwd(dummy, ctypes.c_void_p(32), ctypes.c_void_p(20), ctypes.c_float(1.0),
                                           dummy, ctypes.c_void_p(48), ctypes.c_void_p(64), None, 4, 64, None) == -2


def test_workspace_queries_are_bounded_by_the_chunk():
    # The FLCE backward workspace depends on the vocab chunk, never on the full vocabulary.
    # (Only the per-launch work counters, 64 bytes per 256 vocabulary rows, grow with it.)
    small = _lib.query("gptrig_flce_bwd_workspace_bytes", 16384, 768, 50304, 4096)
    big = _lib.query("gptrig_flce_bwd_workspace_bytes", 16384, 768, 503040, 4096)
    assert 0 <= big - small <= 64 * 503040 // 256 + 256
    assert small < 16384 * 50304 * 2


def test_backward_workspace_is_bounded_by_the_vocab_tile():
    """The reference keeps at most [tokens, vocab_tile_size] logits live
    (rig/kernels/linear_cross_entropy.py:1-24).  Here the backward's workspace
    is one bf16 [tokens, chunk] logit gradient (chunk = vocab_tile_size rounded
    up to 256; vocab_chunk 0 means the reference's default 2048) plus the f32
    [tokens, width] dh accumulator the reference's loop also carries (:247) and
    a few KB of work-queue counters: it grows with the tile, never with the
    vocabulary."""
    from gptrig.kernels import linear_cross_entropy as lce

    for n, d in ((16384, 768), (65536, 768), (4096, 512), (1000, 64)):
        default = _lib.query("gptrig_flce_bwd_workspace_bytes", n, d, 50304, 0)
        assert default == _lib.query("gptrig_flce_bwd_workspace_bytes", n, d, 50304, 2048)
        for tile in (256, 2048, 4096):
            ws = _lib.query("gptrig_flce_bwd_workspace_bytes", n, d, 50304, tile)
            assert ws <= 2 * n * tile + 4 * n * d + (1 << 20), (n, d, tile)
            assert ws >= 2 * n * tile  # the logit-gradient chunk itself
            big = _lib.query("gptrig_flce_bwd_workspace_bytes", n, d, 10 * 50304, tile)
            assert 0 <= big - ws <= 64 * 10 * 50304 // 256 + 256
        assert lce.workspace_bytes(n, d, 50304) == default
        assert lce.workspace_bytes(n, d, 50304, 2000) == default  # rounded up to 2048
    assert lce.chunk_for(1) == 256 and lce.chunk_for(2048) == 2048 and lce.chunk_for(2049) == 2304


def test_trainer_whole_vocabulary_chunk_opt_in():
    # The trainer's explicit opt-in: one chunk covering the whole vocabulary
    # while its bf16 G^T fits 8 GiB, else the fewest equal 256-row-tile chunks.
    from gptrig.kernels import linear_cross_entropy as lce

    for n in (16384, 65536, 131072, 262144):
        vocab = 50304
        chunk = lce.grad_chunk(n, vocab)
        parts = -(-(2 * n * vocab) // (8 << 30))
        assert chunk == max(256, -(-(-(-vocab // parts)) // 256) * 256), n
        assert 2 * n * chunk <= (8 << 30) or chunk == 256
    assert lce.grad_chunk(65536, 50304) == 50432  # one chunk at the step's 65536 tokens
    assert lce.grad_chunk(262144, 50304) == 12800  # 26.4 GB of G^T: four chunks


def test_product_does_not_import_the_oracle():
    pkg = os.path.join(os.path.dirname(HEADER), "..", "gpt-speedrun-tpu_amd", "gptrig")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                text = open(os.path.join(root, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), f


def test_attention_tile_plan_describes_the_kernels():
    """The tile-plan API (rig/kernels/autotune.py:84-157) reports the
    kernels' fixed plan per head dim and rejects any other plan before a
    launch (CPU tensors: the check runs ahead of the device checks)."""
    import torch

    from gptrig.kernels import AttentionConfig, AttentionTiles, make_causal_attention, select_attention_tiles
    from gptrig.kernels.flash_attention import kernel_tiles

    assert select_attention_tiles(sequence=1024, head_dim=64) == AttentionTiles()
    assert kernel_tiles(64).block_kv_dkv == 256 and kernel_tiles(128).block_kv_dkv == 128
    assert kernel_tiles(48) == kernel_tiles(64) and kernel_tiles(96) == kernel_tiles(128)
    q = torch.zeros((1, 2, 16, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="fixed tile plan"):
        make_causal_attention(AttentionConfig(tiles=AttentionTiles(block_q=64)))(q, q, q)
    with pytest.raises(ValueError, match="fixed tile plan"):
        make_causal_attention(AttentionConfig(tiles=kernel_tiles(128)))(q, q, q)
