"""KVWriteOp: mirror of vllm_apple/engine/ops/kv_write.py on HIP.

encode_decode  (kv_write.py:261-334): each sequence's new token at position
               seq_len-1 through block_table (guards of :86-99).
encode_prefill (kv_write.py:336-402): every token to slot_mapping[t];
               negative slots skipped (:137-138).
Bit-exact 16-byte copies (kv_write.hip).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Any, Dict

import torch

from .. import kernels
from .step import resolve_stream, view


@dataclass
class KVWriteParams:
    """kv_write.py:158-189 (9 uint32)."""

    num_seqs: int
    head_size: int
    block_size: int
    num_kv_heads: int
    k_stride_block: int
    k_stride_head: int
    k_stride_token: int
    new_kv_stride_token: int
    new_kv_stride_head: int

    def to_bytes(self) -> bytes:
        return struct.pack("IIIIIIIII", self.num_seqs, self.head_size, self.block_size,
                           self.num_kv_heads, self.k_stride_block, self.k_stride_head,
                           self.k_stride_token, self.new_kv_stride_token,
                           self.new_kv_stride_head)


class KVWriteOp:
    def __init__(self, context: Any, num_kv_heads: int, head_size: int, block_size: int):
        self._context = context
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.block_size = block_size
        self.kv_stride_block = num_kv_heads * block_size * head_size
        self.kv_stride_head = block_size * head_size
        self.kv_stride_token = head_size
        self.new_kv_stride_token = num_kv_heads * head_size
        self.new_kv_stride_head = head_size

    def _cache(self, buf: torch.Tensor) -> torch.Tensor:
        if buf.dim() == 4:
            return buf
        return buf.reshape(-1, self.num_kv_heads, self.block_size, self.head_size)

    def encode_decode(self, step_ctx: Any, new_keys_buffer: torch.Tensor,
                      new_values_buffer: torch.Tensor, key_buffer: torch.Tensor,
                      value_buffer: torch.Tensor, block_table_buffer: torch.Tensor,
                      seq_lens_buffer: torch.Tensor, num_seqs: int, new_keys_offset: int = 0,
                      new_values_offset: int = 0, max_blocks_per_seq: int = 128) -> None:
        stream = resolve_stream(step_ctx)
        KV, D = self.num_kv_heads, self.head_size
        nk = view(new_keys_buffer, new_keys_offset, (num_seqs, KV, D))
        nv = view(new_values_buffer, new_values_offset, (num_seqs, KV, D))
        bt = view(block_table_buffer, 0, (num_seqs, max_blocks_per_seq), torch.int32)
        sl = view(seq_lens_buffer, 0, (num_seqs,), torch.int32)
        kernels.kv_write_decode(nk, nv, self._cache(key_buffer), self._cache(value_buffer), bt,
                                sl, layout="kernel", stream=stream)

    def encode_prefill(self, step_ctx: Any, new_keys_buffer: torch.Tensor,
                       new_values_buffer: torch.Tensor, key_buffer: torch.Tensor,
                       value_buffer: torch.Tensor, slot_mapping_buffer: torch.Tensor,
                       num_tokens: int, new_keys_offset: int = 0,
                       new_values_offset: int = 0) -> None:
        stream = resolve_stream(step_ctx)
        KV, D = self.num_kv_heads, self.head_size
        nk = view(new_keys_buffer, new_keys_offset, (num_tokens, KV, D))
        nv = view(new_values_buffer, new_values_offset, (num_tokens, KV, D))
        sm = slot_mapping_buffer.reshape(-1)[:num_tokens]
        kernels.kv_write_slots(nk, nv, self._cache(key_buffer), self._cache(value_buffer), sm,
                               layout="kernel", stream=stream)

    def get_params_dict(self) -> Dict[str, Any]:
        return {
            "num_kv_heads": self.num_kv_heads,
            "head_size": self.head_size,
            "block_size": self.block_size,
            "decode_kernel": "kv_copy_kernel<DecodeResolver>",
            "prefill_kernel": "kv_copy_kernel<SlotResolver>",
        }
