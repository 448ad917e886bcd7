"""Attention-backend selection for vLLM on ROCm: the rule of platform.py:100-168.

The reference's ApplePlatform is a whole out-of-tree vLLM platform (device
queries, workers, memory accounting) around one hot-path decision:
get_attn_backend_cls returns the Metal backend's class path when
VLLM_METAL_ATTENTION=1, the head size is one of {32, 64, 96, 128} and the
dtype is float16 or bfloat16, and the torch-SDPA backend otherwise; MLA and
sparse attention raise NotImplementedError.  On ROCm the platform itself is
vLLM's; this module supplies the rule as a mixin for a ROCm platform class,
that class when vLLM is importable, and the plugin entry point
(vllm_apple/__init__.py:14-30, pyproject.toml:45-49).

Differences from the reference's rule: our backend is on unless
VLLM_VAA_ATTENTION=0, and it also steps aside for what its kernels do not
implement: FP8 KV caches (the reference's impl raises for them,
metal_attn.py:387-388) and attention sinks.  Any block size is accepted, as
there.  The fallback is VLLM_VAA_FALLBACK_BACKEND, by default vLLM's Triton
backend on ROCm.
"""
from __future__ import annotations

import logging
import os
from typing import Any, Optional

import torch

logger = logging.getLogger(__name__)

BACKEND_CLS = "vllm_apple_amd.backend.HipAttentionBackend"
ATTENTION_ENV = "VLLM_VAA_ATTENTION"
FALLBACK_ENV = "VLLM_VAA_FALLBACK_BACKEND"
DEFAULT_FALLBACK = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"
SUPPORTED_HEAD_SIZES = (32, 64, 96, 128)
SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)


def _fallback(reason: str) -> str:
    cls = os.environ.get(FALLBACK_ENV, DEFAULT_FALLBACK)
    logger.warning("HIP paged attention not used (%s); falling back to %s", reason, cls)
    return cls


def select_attn_backend(head_size: int, dtype: torch.dtype, kv_cache_dtype: Optional[str],
                        block_size: int, use_mla: bool, has_sink: bool, use_sparse: bool,
                        attn_type: Optional[str] = None,
                        is_attention_free: bool = False) -> str:
    """Class path of the attention backend for these layer properties."""
    if use_mla:
        raise NotImplementedError("MLA is not supported by the HIP paged-attention backend.")
    if use_sparse:
        raise NotImplementedError("Sparse attention is not supported by the HIP backend.")
    if os.environ.get(ATTENTION_ENV, "1") == "0":
        return _fallback(f"{ATTENTION_ENV}=0")
    if head_size not in SUPPORTED_HEAD_SIZES:
        return _fallback(f"head_size={head_size} not in {SUPPORTED_HEAD_SIZES}")
    if dtype not in SUPPORTED_DTYPES:
        return _fallback(f"dtype={dtype}; float16 or bfloat16 needed")
    if kv_cache_dtype is not None and str(kv_cache_dtype).startswith("fp8"):
        return _fallback(f"kv_cache_dtype={kv_cache_dtype}")
    if has_sink:
        return _fallback("attention sinks")
    logger.info("Using the HIP paged-attention backend (head_size=%d, block_size=%d, %s)",
                head_size, block_size, dtype)
    return BACKEND_CLS


class HipAttentionPlatformMixin:
    """get_attn_backend_cls with the reference's signature (platform.py:100-112),
    for a class that also derives from vLLM's ROCm platform."""

    @classmethod
    def get_attn_backend_cls(cls, selected_backend: Any, head_size: int, dtype: torch.dtype,
                             kv_cache_dtype: Optional[str], block_size: int, use_mla: bool,
                             has_sink: bool, use_sparse: bool, attn_type: Optional[str] = None,
                             is_attention_free: bool = False) -> str:
        return select_attn_backend(head_size, dtype, kv_cache_dtype, block_size, use_mla,
                                   has_sink, use_sparse, attn_type, is_attention_free)


try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.platforms.rocm import RocmPlatform

    class HipPlatform(HipAttentionPlatformMixin, RocmPlatform):
        """vLLM's ROCm platform with this backend selected for attention."""

except Exception:  # noqa: BLE001
    HipPlatform = None


def register() -> Optional[str]:
    """vllm.platform_plugins entry point: the platform's class path on a ROCm
    GPU with vLLM present, else None (vLLM then keeps its own platform)."""
    if getattr(torch.version, "hip", None) is None or HipPlatform is None:
        return None
    if torch.cuda.device_count() == 0:
        return None
    return "vllm_apple_amd.platform.HipPlatform"
