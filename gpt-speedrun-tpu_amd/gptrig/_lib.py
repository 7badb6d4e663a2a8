"""ctypes binding of ``libgptrig.so`` (declared in ``include/gptrig.h``).

The library is loaded lazily from this directory.  There is no fallback: if
the shared object is missing or a call returns a non-zero status, a
``RuntimeError`` is raised.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgptrig.so")

P = c_void_p
I = c_int
L = c_int64
F = c_float
Z = c_size_t

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "gptrig_version": (c_char_p, []),
    "gptrig_status_string": (c_char_p, [I]),
    "gptrig_attn_fwd": (I, [P, P, P, P, P, P, I, I, I, I, P, F, P]),
    "gptrig_attn_bwd_workspace_bytes": (Z, [I, I, I, I]),
    "gptrig_attn_bwd": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, P, F, P]),
    "gptrig_attn_bwd_rope": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, P, F, P, P, P]),
    "gptrig_flce_fwd_workspace_bytes": (Z, [I, I, I]),
    "gptrig_flce_fwd": (I, [P, P, P, P, P, P, Z, I, I, I, I, P]),
    "gptrig_flce_fwd_noalloc": (I, [P, P, P, P, P, I, I, I, I, P]),
    "gptrig_flce_bwd_workspace_bytes": (Z, [I, I, I, I]),
    "gptrig_flce_bwd": (I, [P, P, P, P, P, F, P, P, I, P, Z, I, I, I, I, I, P]),
    "gptrig_flce32_fwd_workspace_bytes": (Z, [I, I, I]),
    "gptrig_flce32_fwd": (I, [P, P, P, P, P, P, Z, I, I, I, I, P]),
    "gptrig_flce32_bwd_workspace_bytes": (Z, [I, I, I, I]),
    "gptrig_flce32_bwd": (I, [P, P, P, P, P, F, P, P, I, P, Z, I, I, I, I, I, P]),
    "gptrig_flce_keep_bytes": (Z, [I, I]),
    "gptrig_flce_fwd_keep": (I, [P, P, P, P, P, P, Z, P, Z, I, I, I, I, P]),
    "gptrig_flce_bwd_keep_workspace_bytes": (Z, [I, I]),
    "gptrig_flce_bwd_keep": (I, [P, P, P, P, P, F, P, P, I, P, Z, P, Z, I, I, I, I, P]),
    "gptrig_rmsnorm_fwd": (I, [P, P, P, P, I, I, P]),
    "gptrig_add_rmsnorm_fwd": (I, [P, P, F, P, P, P, P, I, I, P]),
    "gptrig_add_bias_rmsnorm_fwd": (I, [P, P, P, F, P, P, P, P, I, I, P]),
    "gptrig_rmsnorm_bwd_workspace_bytes": (Z, [I, I]),
    "gptrig_rmsnorm_bwd": (I, [P, P, P, P, P, P, P, I, P, Z, I, I, P]),
    "gptrig_bias_grad": (I, [P, I, I, P, P]),
    "gptrig_weight_grad": (I, [P, P, P, P, I, I, I, P]),
    "gptrig_linear": (I, [P, L, P, L, I, P, P, L, I, I, I, P]),
    "gptrig_linear_gelu": (I, [P, L, P, L, I, P, P, P, L, I, I, I, P]),
    "gptrig_linear_rope": (I, [P, L, P, L, I, P, P, L, I, I, I, P, P, I, I, I, P]),
    "gptrig_linear_dgelu": (I, [P, L, P, L, I, P, L, P, L, I, I, I, P]),
    "gptrig_gelu_fwd": (I, [P, P, L, P]),
    "gptrig_gelu_bwd": (I, [P, P, P, L, P]),
    "gptrig_bias_gelu_fwd": (I, [P, P, P, I, I, P]),
    "gptrig_bias_gelu_bwd": (I, [P, P, P, P, I, I, P]),
    "gptrig_rope_table": (I, [P, P, I, I, P]),
    "gptrig_rope_fwd": (I, [P, L, I, I, I, I, P, P, P]),
    "gptrig_rope_bwd": (I, [P, L, I, I, I, I, P, P, P]),
    "gptrig_bias_rope_fwd": (I, [P, L, I, I, P, I, I, I, P, P, P]),
    "gptrig_embedding_fwd": (I, [P, P, P, I, I, I, P]),
    "gptrig_embedding_bwd": (I, [P, P, P, I, I, I, P]),
    "gptrig_adamw": (I, [P, P, P, P, P, P, P, L, I, F, F, F, I, P, P, P]),
    "gptrig_sq_norm_partials": (I, [P, L, I, P, P]),
    "gptrig_finalize_norm": (I, [P, I, F, P, P, P, F, P, P]),
    "gptrig_transpose_bf16": (I, [P, P, I, I, P]),
    "gptrig_cast_f32_bf16": (I, [P, P, L, P]),
    "gptrig_weighted_sum": (I, [P, L, F, P, P]),
    "gptrig_masked_sum": (I, [P, P, L, P, P]),
    "gptrig_fill_f32": (I, [P, L, F, P]),
    "gptrig_moe_route_workspace_bytes": (Z, [I, I, I]),
    "gptrig_moe_route": (I, [P, P, P, P, P, P, P, P, P, Z, I, I, I, P]),
    "gptrig_moe_router_logits": (I, [P, P, P, I, I, I, P]),
    "gptrig_moe_gather_rows": (I, [P, P, P, I, I, P]),
    "gptrig_moe_gmm": (I, [P, L, P, I, P, P, I, P, P, L, I, I, I, I, P]),
    "gptrig_moe_gmm_dw": (I, [P, L, P, L, P, P, P, I, I, I, I, P]),
    "gptrig_moe_combine": (I, [P, P, P, P, I, I, I, P]),
    "gptrig_moe_combine_bwd": (I, [P, P, P, P, P, P, I, I, I, P]),
    "gptrig_moe_gather_bwd": (I, [P, P, P, I, I, I, P]),
    "gptrig_moe_stats": (I, [P, P, P, P, I, I, I, P, P, P, P]),
    "gptrig_moe_router_bwd": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, P]),
}

_LIB = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""

    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"gptrig HIP library not found at {LIB_PATH}; build it with "
                "`python gpt-speedrun-tpu_amd/build.py` (hipcc, gfx950)"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def call(name: str, *args) -> None:
    """Invoke an entry point; a non-zero status raises ``RuntimeError``."""

    status = getattr(lib(), name)(*args)
    if status != 0:
        text = lib().gptrig_status_string(status).decode()
        raise RuntimeError(f"{name} failed: {text} (status {status})")


def query(name: str, *args) -> int:
    return int(getattr(lib(), name)(*args))


def stream() -> int:
    """Handle of torch's current HIP stream on the current device."""

    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("gptrig kernels run on the GPU; got a CPU tensor")


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def version() -> str:
    return lib().gptrig_version().decode()
