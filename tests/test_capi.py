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
    # AdamW: chunk not a multiple of 1024
    assert lib.gptrig_adamw(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 1000, 0.1, 0.9, 0.95, 1, None, None,
                            None) == -2
    # routing: too many experts
    assert lib.gptrig_moe_route(dummy, None, dummy, dummy, dummy, dummy, dummy, None, None, 0, 8, 65, 2, None) == -4


def test_workspace_queries_are_bounded_by_the_chunk():
    # The FLCE backward workspace depends on the vocab chunk, never on the full vocabulary.
    small = _lib.query("gptrig_flce_bwd_workspace_bytes", 16384, 768, 50304, 4096)
    big = _lib.query("gptrig_flce_bwd_workspace_bytes", 16384, 768, 503040, 4096)
    assert small == big
    assert small < 16384 * 50304 * 2


def test_default_chunk_follows_the_workspace_budget():
    # vocab_chunk = 0: the whole vocabulary while the bf16 G^T workspace fits
    # 8 GiB, else the fewest equal 256-row-tile chunks; the same choice as the
    # Python wrapper's grad_chunk.
    from gptrig.kernels import linear_cross_entropy as lce

    for n in (16384, 65536, 131072, 262144):
        vocab = 50304
        default = _lib.query("gptrig_flce_bwd_workspace_bytes", n, 768, vocab, 0)
        chunk = lce.grad_chunk(n, vocab)
        assert default == _lib.query("gptrig_flce_bwd_workspace_bytes", n, 768, vocab, chunk), n
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
