"""ctypes binding of libvllm_apple_amd.so (the C ABI in include/vllm_apple_amd.h).

torch is imported first so its HIP runtime (soname libamdhip64.so.7) is the
one the library binds to: streams and device pointers handed over from torch
then belong to the same runtime instance.

There is no CPU fallback: if the library is missing every op raises
``NativeLibraryError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (binds the HIP runtime before the library loads)

LIB_NAME = "libvllm_apple_amd.so"
_LIB_PATH = Path(os.environ.get("VAA_LIBRARY", Path(__file__).resolve().parent / LIB_NAME))

VAA_OK = 0
VAA_ERR_INVALID_ARG = -1
VAA_ERR_UNSUPPORTED = -2
VAA_ERR_HIP = -3
VAA_ERR_WORKSPACE = -4

VAA_INDEX_I32 = 0
VAA_INDEX_I64 = 1

# partition_size value asking decode to split by the actual lengths on the device.
VAA_PARTITION_BALANCED = -1
VAA_PARTITION_BALANCED_SHARED = -2

# Element types of caches, queries, new K/V and outputs (vaa_attn_params.dtype).
VAA_DTYPE_F16 = 0
VAA_DTYPE_BF16 = 1
ABI_VERSION = 5


class NativeLibraryError(RuntimeError):
    """The HIP library could not be loaded (not built, or wrong platform)."""


class VaaError(RuntimeError):
    """A HIP-side failure reported by the library."""


class VaaAttnParams(ctypes.Structure):
    """Mirror of ``struct vaa_attn_params``."""

    _fields_ = [
        ("scale", ctypes.c_float),
        ("num_seqs", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("num_query_heads", ctypes.c_int32),
        ("queries_per_kv", ctypes.c_int32),
        ("partition_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int64),
        ("k_stride_block", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("k_stride_token", ctypes.c_int64),
        ("v_stride_block", ctypes.c_int64),
        ("v_stride_head", ctypes.c_int64),
        ("v_stride_token", ctypes.c_int64),
        ("q_stride_token", ctypes.c_int64),
        ("q_stride_head", ctypes.c_int64),
        ("o_stride_token", ctypes.c_int64),
        ("o_stride_head", ctypes.c_int64),
        ("new_kv_stride_token", ctypes.c_int64),
        ("new_kv_stride_head", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_PARAMS = ctypes.POINTER(VaaAttnParams)

# name -> (restype, argtypes); must match include/vllm_apple_amd.h
SIGNATURES = {
    "vaa_last_error": (ctypes.c_char_p, []),
    "vaa_abi_version": (_I, []),
    "vaa_write_kv_batch": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I64, _I64, _I64, _I64, _P]),
    "vaa_write_kv_single": (_I, [_P, _P, _P, _P, _I64, _I64, _I, _I, _I64, _I64, _I64, _I64, _P]),
    "vaa_kv_write_slots": (_I, [_PARAMS, _P, _P, _P, _I, _P, _P, _I, _P]),
    "vaa_kv_write_decode": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P, _P]),
    "vaa_paged_attention_decode_workspace_size": (ctypes.c_size_t, [_PARAMS, ctypes.POINTER(ctypes.c_int32)]),
    "vaa_paged_attention_decode": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P]),
    "vaa_paged_attention_prefill": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P, _P, _I, _P]),
    "vaa_paged_attention_prefill_workspace_size": (ctypes.c_size_t, [_PARAMS, _I, _I]),
    "vaa_paged_attention_prefill_split": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P,
                                               ctypes.c_size_t, _P]),
    "vaa_paged_attention_decode_noalloc_max_workspace": (ctypes.c_size_t, []),
    "vaa_paged_attention_decode_noalloc": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "vaa_merge_attn_states": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _I64, _I64, _P, _I, _P]),
    "vaa_build_token_index": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "vaa_build_slot_mapping": (_I, [_P, _I, _I, _P, _P, _I, _I, _P, _P]),
    "vaa_rmsnorm": (_I, [_P, _P, _P, _P, _I, _I, _I64, _I64, _I64, _F, _I, _P]),
    "vaa_add_rmsnorm": (_I, [_P, _P, _P, _P, _I, _I, _I64, _I64, _I64, _F, _I, _P]),
    "vaa_rope_neox": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I64, _I64, _I, _I, _P]),
    "vaa_silu_mul": (_I, [_P, _P, _P, _I64, _I, _P]),
    "vaa_silu_mul_2d": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "vaa_gate_up_silu": (_I, [_P, _I64, _P, _P, _I64, _P, _I64, _I, _I, _I, _I, _P]),
    "vaa_topk_workspace_size": (_I, [_I, _I, _I, _P]),
    "vaa_topk_logits": (_I, [_P, _I, _I, _I64, _I, _P, _P, _I64, _P, ctypes.c_size_t, _P]),
    "vaa_qkv_epilogue": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _I, _P, _P, _I,
                              _P]),
    "vaa_kv_stream_read": (_I, [_PARAMS, _P, _P, _P, _P, _P, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the library, raising NativeLibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise NativeLibraryError(
                f"{_LIB_PATH} is not built; run vllm_apple_amd.build_library() "
                "(hipcc --offload-arch=gfx950)")
        try:
            lib = ctypes.CDLL(str(_LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        except OSError as e:
            raise NativeLibraryError(f"cannot load {_LIB_PATH}: {e}") from e
        # The version first: a library built from other sources may lack
        # symbols this module binds.
        lib.vaa_abi_version.restype = _I
        lib.vaa_abi_version.argtypes = []
        if lib.vaa_abi_version() != ABI_VERSION:
            raise NativeLibraryError(
                f"ABI version mismatch: {_LIB_PATH} has {lib.vaa_abi_version()}, "
                f"this package needs {ABI_VERSION} (rebuild the library)")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().vaa_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    """Map a status code to the exception the reference would raise."""
    if status == VAA_OK:
        return
    msg = f"{what}: {last_error()}"
    if status == VAA_ERR_INVALID_ARG:
        raise ValueError(msg)
    if status == VAA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if status == VAA_ERR_WORKSPACE:
        raise ValueError(msg)
    raise VaaError(msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def stream_handle(stream: "torch.cuda.Stream | None" = None) -> int:
    """Raw hipStream_t of ``stream`` (default: torch's current stream)."""
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)
