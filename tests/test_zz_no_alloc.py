"""The allocation-free FLCE forward (``gptrig_flce_fwd_noalloc``) against the
workspace entry point (``gptrig_flce_fwd``), through the C ABI.

Both run the same kernels on the same inputs, so losses and LSE must be
bit-identical.  Two calls in a row, the second with a smaller input (the
device scratch array keeps the first call's contents), then a size past the
32 MiB scratch is rejected on the host before any launch.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
E_WORKSPACE = -6


def inputs(n, d, V, sv, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn((n, d), generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn((V, d), generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    t = torch.randint(0, sv, (n,), generator=g, dtype=torch.int32)
    t[::97] = -1  # invalid targets: loss +inf
    return h, w, t.to(DEV)


def noalloc(h, w, t, sv):
    from gptrig import _lib

    n, d = h.shape
    V = w.shape[0]
    losses = torch.empty(n, dtype=torch.float32, device=DEV)
    lse = torch.empty(n, dtype=torch.float32, device=DEV)
    _lib.call("gptrig_flce_fwd_noalloc", h.data_ptr(), w.data_ptr(), t.data_ptr(), losses.data_ptr(), lse.data_ptr(),
              n, d, V, sv, _lib.stream())
    return losses, lse


def test_noalloc_forward_equals_the_workspace_entry_point():
    from gptrig.kernels import linear_cross_entropy as lce

    for n, d, V, sv, seed in ((16384, 768, 50304, 50257, 71), (1000, 256, 50304, 50304, 72)):
        print(f"noalloc flce forward n={n} d={d} V={V}", flush=True)
        h, w, t = inputs(n, d, V, sv, seed)
        losses, lse = noalloc(h, w, t, sv)
        want_losses, want_lse = lce.flce_forward(h, w, t, sv)
        torch.cuda.synchronize()
        assert torch.equal(lse, want_lse)
        assert torch.equal(losses, want_losses)
        assert torch.isinf(losses[::97]).all() and torch.isfinite(losses[1:97]).all()


def test_noalloc_forward_rejects_sizes_past_its_scratch():
    from gptrig import _lib

    n = 24000  # 24000 tokens x 197 tiles x 8 B + 4 B per token > 32 MiB
    # Buffers of the full size, so that a host check that stopped rejecting
    # this call would show as a wrong return code, not as accesses past them.
    h, w, t = inputs(n, 768, 50304, 50304, 73)
    losses = torch.empty(n, dtype=torch.float32, device="cuda")
    lse = torch.empty(n, dtype=torch.float32, device="cuda")
    assert _lib.query("gptrig_flce_fwd_workspace_bytes", n, 768, 50304) > 32 << 20
    rc = _lib.lib().gptrig_flce_fwd_noalloc(h.data_ptr(), w.data_ptr(), t.data_ptr(), losses.data_ptr(),
                                            lse.data_ptr(), n, 768, 50304, 50304, _lib.stream())
    torch.cuda.synchronize()
    assert rc == E_WORKSPACE
