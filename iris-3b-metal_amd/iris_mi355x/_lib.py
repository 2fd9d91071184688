"""ctypes binding of ``libiris_hip.so`` (the C ABI declared in ``include/iris_hip.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch already
loaded (both name ``libamdhip64.so.7``); device pointers and streams come from torch
tensors. There is no fallback: if the library is missing, or no GPU is present, calls raise.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_long, c_void_p
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().with_name("libiris_hip.so")

ABI_VERSION = 3  # iris_abi_version() of the library these signatures describe
F32, BF16 = 0, 1
EPI_NONE, EPI_SILU_MUL, EPI_SILU = 0, 1, 2
ACT_NONE, ACT_SILU = 0, 1
E_INVALID, E_LAUNCH, E_UNSUPPORTED = -1, -2, -3

P = c_void_p
_SIGNATURES: dict[str, list] = {
    "iris_abi_version": [],
    "iris_rms_norm_modulate": [P, c_int, P, c_int, P, P, P, c_long, c_long, c_int, c_long, c_float, P],
    "iris_gated_residual_rms_norm": [P, P, c_int, P, P, c_long, c_long, c_int, c_long, c_float, P],
    "iris_gated_residual_norm_modulate": [P, P, c_int, P, P, c_long, c_long, c_int, c_long, c_float, P, P, P,
                                          c_long, P, c_int, P],
    "iris_gated_residual_grouped": [c_int, P, P, c_int, P, P, P, P, c_int, P, c_float, P, P, P, P, P, c_int, P],
    "iris_qk_norm_rope": [P, c_int, P, c_int, P, P, P, c_long, c_int, c_long, c_long, c_int, c_long, c_long,
                          c_long, c_float, P],
    "iris_v_heads_t": [P, P, c_int, c_long, c_long, c_int, c_long, c_long, c_long, P],
    "iris_qkv_prepare": [P, P, P, P, P, P, P, P, c_long, c_int, c_long, c_long, c_long, c_int, c_int, c_long,
                         c_long, c_long, c_long, c_long, c_float, P],
    "iris_flash_attn": [P, P, P, c_int, c_int, c_int, c_long, c_long, c_long, c_float, P, P, c_long, c_long,
                        c_long, P, P, c_long, c_long, c_long, P],
    "iris_gemm_bf16": [P, P, P, P, c_int, c_int, c_int, c_int, c_long, c_long, c_long, c_int, P],
    "iris_gemm_force_tile": [c_int],
    "iris_flash_attn_force_variant": [c_int],
    "iris_flash_attn_masked": [P, P, P, c_int, c_int, c_int, c_long, c_long, c_float, P, P, c_long, c_long, P],
    "iris_text_key_mask": [P, c_int, c_long, c_int, c_long, c_long, P, P],
    "iris_layer_attention": [P, P, c_long, c_int, c_int, c_int, c_float, P],
    "iris_layer_pool": [P, P, P, P, c_long, c_int, c_int, P, c_int, P],
    "iris_residual_rms_norm": [P, P, c_int, P, P, c_long, c_long, c_int, c_float, P, c_int, P],
    "iris_gemm_bf16_grouped": [c_int, P, P, P, P, P, c_int, c_int, c_int, c_long, c_long, c_long, c_int, P],
    "iris_gemm_bf16_qk_rope": [c_int, P, P, P, P, c_int, c_int, c_long, c_long, c_long, P, P, P, P, P, P, c_long,
                               P, P, c_int, c_int, c_long, P, c_long, c_float, P],
    "iris_gemv_bf16": [P, P, c_int, c_int, c_int, P, P, c_int, P, c_int, c_int, P],
    "iris_timestep_features": [P, P, c_int, c_int, P, P],
    "iris_patchify_embed": [P, c_int, c_int, c_int, c_int, c_int, P, c_long, P, P, P, P, P, c_float, P, c_int, P,
                            P],
    "iris_pixel_rms_norm": [P, c_int, P, P, c_long, c_float, P],
    "iris_pixel_mlp": [P, c_int, P, P, P, P, P, P, P, P, P, c_long, c_float, P],
    "iris_unpatchify_head": [P, P, P, P, c_int, c_int, c_int, c_int, c_int, P],
    "iris_silu_add_rows": [P, P, c_long, c_long, c_int, P, c_int, P],
    "iris_copy_rows": [P, P, c_int, c_long, c_int, c_long, c_long, c_long, c_long, P],
    "iris_flow_euler": [P, P, c_long, c_float, c_float, P, P, P],
    "iris_dpm1_update": [P, P, c_long, c_float, c_float, c_float, P, P],
    "iris_dpm_update": [P, P, P, c_long, c_float, c_float, c_float, c_float, c_float, P, P, P],
    "iris_cfg_combine": [P, P, c_long, c_float, P, P],
    "iris_clamp": [P, c_long, c_float, c_float, P, P],
}

_lib: ctypes.CDLL | None = None


class IrisKernelError(RuntimeError):
    """A kernel launch failed on the device (invalid arguments raise ``ValueError``)."""


def exported_symbols() -> list[str]:
    return ["iris_last_error", *_SIGNATURES]


def load() -> ctypes.CDLL:
    """Load the library (once); raises ``RuntimeError`` if it has not been built."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY.name} is not built; run __graft_entry__.build() first")
        lib = ctypes.CDLL(str(LIBRARY))
        lib.iris_last_error.restype = ctypes.c_char_p
        lib.iris_last_error.argtypes = []
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = c_int
        if lib.iris_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIBRARY.name} has ABI {lib.iris_abi_version()}, these bindings need {ABI_VERSION}: "
                               "rebuild it with __graft_entry__.build()")
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke ``name``; translate a negative status into ``ValueError`` / ``IrisKernelError``."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        message = lib.iris_last_error().decode(errors="replace")
        if rc == E_INVALID:
            raise ValueError(message)
        raise IrisKernelError(f"{name}: {message} (status {rc})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return F32
    if dtype == torch.bfloat16:
        return BF16
    raise ValueError(f"unsupported dtype {dtype}; the HIP kernels take float32 or bfloat16")


def pointer_array(values) -> ctypes.Array:
    return (c_void_p * len(values))(*values)


def int_array(values) -> ctypes.Array:
    return (c_int * len(values))(*values)


def long_array(values) -> ctypes.Array:
    return (c_long * len(values))(*values)
