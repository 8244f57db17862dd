"""The HIP library and the ctypes conventions of its calls (the reference's native.py:43-65, for hipcc/gfx950):
every tensor argument is a raw device pointer, counts are C ints, the stream is the last argument.

hip_library() loads nanochat_amd/libnanochat_amd.so, building it first when it is missing or older than its
sources (build.py). There is no fallback: a missing toolchain or library raises.
"""

from __future__ import annotations

import ctypes
import functools
from typing import TYPE_CHECKING

from nanochat_amd import build as _build

if TYPE_CHECKING:
    import torch

P, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float

# name -> (restype, argtypes); the declarations of include/nanochat_amd.h
SIGNATURES: dict[str, tuple] = {
    "nc_abi_version": (I32, []),
    "nc_last_error": (ctypes.c_char_p, []),
    "qkp_forward": (None, [P, P, P, P, P, P, P, P, I64, I32, I32, P]),
    "nc_kv_append_fp8": (I32, [P, I64, I32, P, P, P, P, P, P, I32, I32, I32, P, P, P, I32, I32, I32, P, P]),
    "nc_kv_store_fp8": (I32, [P, P, I64, I32, P, P, I32, P, P, I32, I32, I32, P]),
    "nc_kv_gather_fp8": (I32, [P, P, I32, I32, P, I32, I32, I32, P, P, P, P, P]),
    "nc_kv_export_fp8": (I32, [P, I64, I32, P, I32, I32, I32, I32, I32, I32, I32, P, P]),
    "nc_kv_import_fp8": (I32, [P, I32, P, I64, P, I32, I32, I32, I32, I32, I32, I32, P]),
    "nc_decode_workspace_bytes": (I64, [I32, I32, I32, I32]),
    "nc_decode_attn_fp8": (I32, [P, P, P, I32, I32, P, I32, I32, I32, I32, I32, F32, P, P, I64, P]),
    "nc_decode_step_fp8": (I32, [P, I64, P, P, P, P, P, P, I32, P, P, I32, I32, I32, I32, I32, I32, I32, F32, P,
                                 P, I64, P]),
    "nc_decode_step_fp8_pieces": (I32, [P, I64, P, P, P, P, P, P, I32, P, P, I32, I32, I32, I32, I32, I32, I32, F32,
                                        I32, P, P, I64, P]),
    "nc_decode_step_fp8_noalloc": (I32, [P, I64, P, P, P, P, P, P, I32, P, P, I32, I32, I32, I32, I32, I32, I32,
                                         F32, P, P]),
    "nc_prefill_attn_fp8": (I32, [P, P, P, I32, P, P, I32, I32, I32, I32, I32, I32, F32, P, P]),
    "nc_argmax_f32": (I32, [P, I32, I32, I64, P, P]),
    "nc_choose_workspace_bytes": (I64, [I32, I32]),
    "nc_choose_tokens": (I32, [P, I32, I32, I64, P, P, P, P, P, P, P, F32, I32, P, P, P, I64, P]),
    "nc_add_rms_norm_bf16": (I32, [P, P, P, P, I32, I32, P]),
    "nc_relu2_bf16": (I32, [P, P, I64, P]),
    "nc_value_embed_bf16": (I32, [P, I64, P, I64, P, P, I64, P, I32, I32, I32, I32, P]),
    "nc_embed_rms_norm": (I32, [P, I32, I64, P, I32, I32, P, P]),
    "nc_mix_bf16": (I32, [P, P, I64, F32, F32, P]),
    "nc_slot_gemm_bf16": (I32, [P, I32, I32, P, I32, I32, P, P, I32, I32, P]),
    "nc_slot_gemm_bf16_prefetch": (I32, [P, I32, I32, P, I32, I32, P, P, I32, I32, P, I64, P]),
    "dec_create": (P, [P, P, P, P, P]),
    "dec_create_v2": (P, [P, I32, P, P, P, P]),
    "dec_destroy": (None, [P]),
    "dec_batch": (I32, [P]),
    "dec_prefill_rows": (I32, [P]),
    "dec_set_prompt": (None, [P, I32, ctypes.c_int32, ctypes.c_int32, F32, F32, ctypes.c_ulonglong]),
    "dec_prefill": (None, [P, I32, P]),
    "dec_save_prompt": (None, [P, I32, I32, I32, I32]),
    "dec_load_prompt": (None, [P, I32, I32, I32, I32]),
    "dec_masks": (P, [P]),
    "dec_set_active": (None, [P, P]),
    "dec_launch_body": (None, [P]),
    "dec_launch_head": (None, [P]),
    "dec_tokens": (None, [P, P]),
    "dec_take_alt": (None, [P, I32]),
}


class HipLibraryError(RuntimeError):
    pass


@functools.cache
def hip_library() -> ctypes.CDLL:
    """The loaded library with every entry point's argtypes set; built in-tree first if missing or stale."""
    if not _build.is_current():
        _build.build()
    lib = ctypes.CDLL(str(_build.LIBRARY))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def check(status: int) -> None:
    """An entry point's status: 0, or raise ValueError with the library's message (host-side argument checks)."""
    if status != 0:
        raise ValueError(hip_library().nc_last_error().decode())


def pointer(t: "torch.Tensor | None") -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream() -> ctypes.c_void_p:
    """The current HIP stream, which the kernels launch on."""
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
