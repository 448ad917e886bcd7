"""EngineRMSNorm: mirror of vllm_apple/engine/ops/rmsnorm.py on HIP.

encode (rmsnorm.py:226-321): out = x * rsqrt(mean(x^2) + eps) * w, plus the
residual added after the norm when residual_buffer is given (the reference's
rmsnorm_residual_kernel, :128-173).  One wave per row, row kept in registers.
encode_residual_add_norm fuses the residual add and copy that precede the
norm in the reference's layer (runner.py:1107-1130) into the same pass.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional

import torch

from .. import kernels
from .step import resolve_stream, view


@dataclass
class RMSNormConfig:
    hidden_size: int
    eps: float = 1e-6
    dtype: torch.dtype = torch.float16


class EngineRMSNorm:
    def __init__(self, context: Any, hidden_size: int, eps: float = 1e-6,
                 weight_buffer: Optional[torch.Tensor] = None):
        self._context = context
        self.config = RMSNormConfig(hidden_size=hidden_size, eps=eps)
        self._weight_buffer = weight_buffer

    def set_weights(self, weight_buffer: torch.Tensor) -> None:
        self._weight_buffer = weight_buffer

    @staticmethod
    def _buf(x: Any):
        """Accept a tensor or an (tensor, byte_offset) pair."""
        if isinstance(x, tuple):
            return x
        return x, 0

    def encode(self, step_ctx: Any, input_buffer: Any, output_buffer: Any, num_tokens: int,
               residual_buffer: Optional[Any] = None) -> None:
        if self._weight_buffer is None:
            raise RuntimeError("Weights not set - call set_weights() first")
        stream = resolve_stream(step_ctx)
        H = self.config.hidden_size
        ib, io = self._buf(input_buffer)
        ob, oo = self._buf(output_buffer)
        x = view(ib, io, (num_tokens, H), dtype=ib.dtype)
        out = view(ob, oo, (num_tokens, H), dtype=ob.dtype)
        res = None
        if residual_buffer is not None:
            rb, ro = self._buf(residual_buffer)
            res = view(rb, ro, (num_tokens, H), dtype=rb.dtype)
        w = self._weight_buffer.reshape(-1)[:H]
        kernels.rms_norm(x, w, self.config.eps, residual=res, out=out, stream=stream)

    def encode_residual_add_norm(self, step_ctx: Any, input_buffer: Any, residual_buffer: Any,
                                 output_buffer: Any, num_tokens: int) -> None:
        """The layer's residual add, copy into the residual buffer and norm in
        place (runner.py:1107-1130) as one kernel: residual <- input +
        residual, output <- norm(residual).  output may be input."""
        if self._weight_buffer is None:
            raise RuntimeError("Weights not set - call set_weights() first")
        stream = resolve_stream(step_ctx)
        H = self.config.hidden_size
        ib, io = self._buf(input_buffer)
        rb, ro = self._buf(residual_buffer)
        ob, oo = self._buf(output_buffer)
        x = view(ib, io, (num_tokens, H), dtype=ib.dtype)
        res = view(rb, ro, (num_tokens, H), dtype=rb.dtype)
        out = view(ob, oo, (num_tokens, H), dtype=ob.dtype)
        w = self._weight_buffer.reshape(-1)[:H]
        kernels.add_rms_norm(x, res, w, self.config.eps, out=out, stream=stream)

    def get_output_size(self, num_tokens: int) -> int:
        return num_tokens * self.config.hidden_size * 2

    def get_params_dict(self) -> Dict[str, Any]:
        return {"hidden_size": self.config.hidden_size, "eps": self.config.eps}
