"""EngineRoPE and EngineElementwiseOps.encode_silu_mul on HIP.

EngineRoPE (elementwise.py:610-766): NeoX (split-half) rotation in place on
Q [T, H, D] and K [T, KV, D] with an fp32 cos/sin table built exactly as the
reference builds it (numpy float32, :680-697), uploaded once.  GPT-J
interleaved RoPE (is_neox_style=False) is outside this build's scope.
encode_silu_mul (elementwise.py:496-532): out = silu(gate) * up.
"""
from __future__ import annotations

from typing import Any, Optional

import torch

from .. import kernels
from .step import resolve_stream, view


def _as_view(x: Any, shape, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Typed view of a tensor or (tensor, byte offset); dtype None keeps the
    buffer's own 16-bit type (fp16 or bf16)."""
    if isinstance(x, tuple):
        buf, off = x
        return view(buf, off, shape, dtype or buf.dtype)
    if tuple(x.shape) == tuple(shape):
        return x
    return view(x, 0, shape, dtype or x.dtype)


class EngineElementwiseOps:
    def __init__(self, context: Any = None):
        self._context = context

    def encode_silu_mul(self, step_ctx: Any, gate: Any, up: Any, output: Any,
                        num_elements: int) -> None:
        stream = resolve_stream(step_ctx)
        g = _as_view(gate, (num_elements,))
        u = _as_view(up, (num_elements,))
        o = _as_view(output, (num_elements,))
        kernels.silu_mul(g, u, out=o, stream=stream)


class EngineRoPE:
    def __init__(self, context: Any, head_size: int, num_heads: int, num_kv_heads: int,
                 rotary_dim: Optional[int] = None, max_position: int = 8192,
                 base: float = 10000.0, is_neox_style: bool = True,
                 device: Optional[torch.device] = None):
        if not is_neox_style:
            raise NotImplementedError("only NeoX (split-half) RoPE is built for gfx950")
        self._context = context
        self.head_size = head_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.rotary_dim = rotary_dim or head_size
        self.max_position = max_position
        self.base = base
        self.is_neox_style = is_neox_style
        self._device = device or torch.device("cuda")
        self._cos_cache, self._sin_cache = kernels.rope_cos_sin_cache(
            self.rotary_dim, max_position, base, device=self._device)

    def encode(self, step_ctx: Any, query: Any, key: Any, positions: Any, num_tokens: int,
               max_position_in_batch: Optional[int] = None) -> None:
        if max_position_in_batch is not None and max_position_in_batch >= self.max_position:
            raise ValueError(
                f"Position ID {max_position_in_batch} exceeds max_position {self.max_position}. "
                f"Increase max_position in EngineRoPE constructor.")
        stream = resolve_stream(step_ctx)
        q = _as_view(query, (num_tokens, self.num_heads, self.head_size))
        k = None
        if key is not None:
            k = _as_view(key, (num_tokens, self.num_kv_heads, self.head_size))
        pos = _as_view(positions, (num_tokens,), torch.int32)
        kernels.rope_neox_(q, k, self._cos_cache, self._sin_cache, pos,
                           rotary_dim=self.rotary_dim, stream=stream)
