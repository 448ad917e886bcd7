"""Step context: which HIP stream the encode_* calls enqueue on.

The reference's EngineStepContext (vllm_apple/engine/step.py:58-618) owns a
Metal command buffer with ENCODE -> SUBMIT -> READBACK phases and the ops
raise RuntimeError outside ENCODE.  On HIP the stream is the command buffer:
work is ordered and asynchronous by construction, so the context only carries
the stream and the same phase rule.
"""
from __future__ import annotations

from typing import Any, Optional

import torch


class EngineStepContext:
    def __init__(self, stream: Optional[torch.cuda.Stream] = None, step_id: int = 0,
                 step_kind: str = "decode", num_tokens: int = 0):
        self.stream = stream
        self.step_id = step_id
        self.step_kind = step_kind
        self.num_tokens = num_tokens
        self._encoding = False
        self.dispatch_count = 0

    @property
    def is_encoding(self) -> bool:
        return self._encoding

    def __enter__(self):
        self._encoding = True
        return self

    def __exit__(self, *exc):
        self._encoding = False
        return False

    def end_encoding(self) -> None:
        self._encoding = False

    def submit(self) -> None:
        """Nothing to do: HIP launches are already queued on the stream."""

    def wait_until_completed(self) -> None:
        (self.stream or torch.cuda.current_stream()).synchronize()


def resolve_stream(step_ctx: Any):
    """step_ctx -> torch stream (None = torch's current stream)."""
    if step_ctx is None:
        return None
    if isinstance(step_ctx, torch.cuda.Stream):
        return step_ctx
    if isinstance(step_ctx, EngineStepContext):
        if not step_ctx.is_encoding:
            raise RuntimeError("encode called outside ENCODE phase")
        step_ctx.dispatch_count += 1
        return step_ctx.stream
    return getattr(step_ctx, "stream", None)


def view(buffer: torch.Tensor, byte_offset: int, shape, dtype=torch.float16) -> torch.Tensor:
    """A typed view of `shape` starting `byte_offset` bytes into `buffer`
    (the reference's (MTLBuffer, offset) binding)."""
    if buffer.dtype != dtype:
        raise ValueError(f"buffer dtype {buffer.dtype} != {dtype}")
    if not buffer.is_contiguous():
        raise ValueError("engine buffers must be contiguous")
    esz = buffer.element_size()
    if byte_offset % esz:
        raise ValueError(f"byte offset {byte_offset} not a multiple of {esz}")
    n = 1
    for s in shape:
        n *= int(s)
    flat = buffer.reshape(-1)
    start = byte_offset // esz
    if start + n > flat.numel():
        raise ValueError(f"view of {n} elements at offset {start} exceeds buffer ({flat.numel()})")
    return flat[start:start + n].view(*shape)
