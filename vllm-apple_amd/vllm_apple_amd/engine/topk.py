"""EngineTopK: mirror of vllm_apple/engine/ops/topk.py on HIP.

encode (topk.py:324-401) selects, per logits row, the k largest values and
their columns (value-descending, ties by lower column) into int32 indices and
16-bit values, so a step reads back k * 6 bytes per token instead of the whole
row.  k defaults to 50 and VLLM_METAL_TOPK_K overrides it (topk.py:30,296-303);
the kernel takes k up to 256 (the reference's two Metal kernels stop at 50).
reconstruct_logits restates the runner's readback (runner.py:1256-1298): a
full [T, V] row of -inf with the top-k values scattered back.
"""
from __future__ import annotations

import logging
import os
from typing import Any, Dict, Optional

import torch

from .. import kernels
from .step import resolve_stream, view

logger = logging.getLogger(__name__)

TOPK_K_ENV = "VLLM_METAL_TOPK_K"


class EngineTopK:
    def __init__(self, context: Any, k: int = 50):
        self._context = context
        self._k = k
        env_k = os.environ.get(TOPK_K_ENV)
        if env_k:
            try:
                self._k = int(env_k)
            except ValueError:
                logger.warning("Invalid %s value: %s, ignoring", TOPK_K_ENV, env_k)
        if not 1 <= self._k <= kernels.TOPK_MAX_K:
            raise ValueError(f"k={self._k} must be in 1..{kernels.TOPK_MAX_K}")

    @staticmethod
    def _buf(x: Any):
        """Accept a tensor or an (tensor, byte_offset) pair."""
        if isinstance(x, tuple):
            return x
        return x, 0

    def encode(self, step_ctx: Any, logits: Any, indices_out: Any, values_out: Any,
               num_tokens: int, vocab_size: int, k: Optional[int] = None) -> None:
        stream = resolve_stream(step_ctx)
        k = k or self._k
        lb, lo = self._buf(logits)
        ib, io = self._buf(indices_out)
        vb, vo = self._buf(values_out)
        x = view(lb, lo, (num_tokens, vocab_size), dtype=lb.dtype)
        idx = view(ib, io, (num_tokens, k), dtype=torch.int32)
        vals = view(vb, vo, (num_tokens, k), dtype=lb.dtype)
        kernels.topk_logits(x, k, indices=idx, values=vals, stream=stream)

    @property
    def k(self) -> int:
        return self._k

    def get_stats(self) -> Dict[str, Any]:
        return {"k": self._k}


def reconstruct_logits(indices: torch.Tensor, values: torch.Tensor,
                       vocab_size: int) -> torch.Tensor:
    """[T, vocab_size] logits: -inf everywhere but the top-k columns, which hold
    their values (the reconstruction in runner.py:1288-1292)."""
    T = indices.shape[0]
    out = torch.full((T, vocab_size), float("-inf"), dtype=values.dtype, device=values.device)
    out.scatter_(1, indices.long(), values)
    return out
