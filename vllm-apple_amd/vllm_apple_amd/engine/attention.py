"""PagedAttentionOp: mirror of vllm_apple/engine/ops/attention.py on HIP.

encode_decode_fused  (attention.py:369-537): fused KV write of each
    sequence's new token at seq_len-1 + paged GQA decode, one launch of
    paged_decode_kernel (plus the split-K merge when a sequence is split).
encode_prefill       (attention.py:290-367): token-parallel semantics of
    paged_attention_v2_prefill -- token t attends to [0, positions[t]] of
    sequence token_to_seq[t] -- on the MFMA prefill kernel.  The tokens' K/V
    must already be in the cache (KVWriteOp.encode_prefill).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Any, Dict, Optional

import torch

from .. import kernels
from .step import resolve_stream, view


@dataclass
class FusedAttentionParams:
    """Fields of FusedAttentionParams (paged_attention_fused.metal:24-49)."""

    scale: float
    num_seqs: int
    max_seq_len: int
    max_blocks_per_seq: int
    head_size: int
    block_size: int
    num_kv_heads: int
    num_query_heads: int
    queries_per_kv: int
    k_stride_block: int
    k_stride_head: int
    k_stride_token: int
    v_stride_block: int
    v_stride_head: int
    v_stride_token: int
    q_stride_token: int
    q_stride_head: int
    o_stride_token: int
    o_stride_head: int
    new_kv_stride_token: int
    new_kv_stride_head: int

    def to_bytes(self) -> bytes:
        """Same packing as the reference (1 float + 20 uint32)."""
        return struct.pack("f" + "I" * 20, self.scale, self.num_seqs, self.max_seq_len,
                           self.max_blocks_per_seq, self.head_size, self.block_size,
                           self.num_kv_heads, self.num_query_heads, self.queries_per_kv,
                           self.k_stride_block, self.k_stride_head, self.k_stride_token,
                           self.v_stride_block, self.v_stride_head, self.v_stride_token,
                           self.q_stride_token, self.q_stride_head, self.o_stride_token,
                           self.o_stride_head, self.new_kv_stride_token,
                           self.new_kv_stride_head)


@dataclass
class PagedAttentionParams:
    """Fields of PagedAttentionParams (paged_attention_v2.metal:20-40)."""

    scale: float
    num_seqs: int
    max_seq_len: int
    max_blocks_per_seq: int
    head_size: int
    block_size: int
    num_kv_heads: int
    num_query_heads: int
    queries_per_kv: int
    k_stride_block: int
    k_stride_head: int
    k_stride_token: int
    v_stride_block: int
    v_stride_head: int
    v_stride_token: int
    q_stride_token: int
    q_stride_head: int
    o_stride_token: int
    o_stride_head: int

    def to_bytes(self) -> bytes:
        """Same packing as the reference (1 float + 18 uint32)."""
        return struct.pack("f" + "I" * 18, self.scale, self.num_seqs, self.max_seq_len,
                           self.max_blocks_per_seq, self.head_size, self.block_size,
                           self.num_kv_heads, self.num_query_heads, self.queries_per_kv,
                           self.k_stride_block, self.k_stride_head, self.k_stride_token,
                           self.v_stride_block, self.v_stride_head, self.v_stride_token,
                           self.q_stride_token, self.q_stride_head, self.o_stride_token,
                           self.o_stride_head)


class PagedAttentionOp:
    """Encode-only paged attention (decode with fused KV write, chunked prefill)."""

    def __init__(self, context: Any, num_kv_heads: int, num_query_heads: int, head_size: int,
                 block_size: int, scale: Optional[float] = None):
        # The reference's h128 kernel takes 128 and its generic kernels any
        # head size up to 128 (engine/ops/attention.py:268-290); the HIP
        # kernels take any multiple of 8 up to 128 (16-byte rows).
        if not (8 <= head_size <= 128 and head_size % 8 == 0):
            raise ValueError(f"head_size must be a multiple of 8 up to 128, got {head_size}")
        if num_query_heads % num_kv_heads != 0:
            raise ValueError("num_query_heads must be a multiple of num_kv_heads")
        self._context = context
        self.num_kv_heads = num_kv_heads
        self.num_query_heads = num_query_heads
        self.head_size = head_size
        self.block_size = block_size
        self.scale = scale if scale is not None else 1.0 / (head_size ** 0.5)
        self.queries_per_kv = num_query_heads // num_kv_heads
        # Engine layouts (attention.py:207-220).
        self.kv_stride_block = num_kv_heads * block_size * head_size
        self.kv_stride_head = block_size * head_size
        self.kv_stride_token = head_size
        self.q_stride_token = num_query_heads * head_size
        self.q_stride_head = head_size
        self.o_stride_token = num_query_heads * head_size
        self.o_stride_head = head_size
        self.new_kv_stride_token = num_kv_heads * head_size
        self.new_kv_stride_head = head_size
        self._kernel_name = "paged_decode_kernel"

    # -- helpers --------------------------------------------------------------
    def _cache(self, buf: torch.Tensor) -> torch.Tensor:
        """A K or V cache buffer as [num_blocks, KV, bs, D] (engine layout)."""
        if buf.dim() == 4:
            return buf
        per_block = self.kv_stride_block
        if buf.numel() % per_block:
            raise ValueError("cache buffer size is not a whole number of blocks")
        return buf.reshape(-1, self.num_kv_heads, self.block_size, self.head_size)

    def fused_params(self, num_seqs: int, max_seq_len: int,
                     max_blocks_per_seq: int) -> FusedAttentionParams:
        return FusedAttentionParams(
            self.scale, num_seqs, max_seq_len, max_blocks_per_seq, self.head_size,
            self.block_size, self.num_kv_heads, self.num_query_heads, self.queries_per_kv,
            self.kv_stride_block, self.kv_stride_head, self.kv_stride_token,
            self.kv_stride_block, self.kv_stride_head, self.kv_stride_token,
            self.q_stride_token, self.q_stride_head, self.o_stride_token, self.o_stride_head,
            self.new_kv_stride_token, self.new_kv_stride_head)

    # -- encode ---------------------------------------------------------------
    def encode_prefill(self, step_ctx: Any, query_buffer: torch.Tensor,
                       key_buffer: torch.Tensor, value_buffer: torch.Tensor,
                       block_table_buffer: torch.Tensor, token_to_seq_buffer: torch.Tensor,
                       positions_buffer: torch.Tensor, output_buffer: torch.Tensor,
                       num_tokens: int, num_seqs: int, max_seq_len: int,
                       max_blocks_per_seq: int, query_offset: int = 0,
                       output_offset: int = 0) -> None:
        stream = resolve_stream(step_ctx)
        H, D = self.num_query_heads, self.head_size
        q = view(query_buffer, query_offset, (num_tokens, H, D))
        out = view(output_buffer, output_offset, (num_tokens, H, D))
        bt = view(block_table_buffer, 0, (num_seqs, max_blocks_per_seq), torch.int32)
        tok = view(token_to_seq_buffer, 0, (num_tokens,), torch.int32)
        pos = view(positions_buffer, 0, (num_tokens,), torch.int32)
        kernels.paged_prefill(q, self._cache(key_buffer), self._cache(value_buffer), bt, tok,
                              pos, scale=self.scale, layout="kernel", output=out,
                              stream=stream)

    def encode_decode_fused(self, step_ctx: Any, query_buffer: torch.Tensor,
                            new_keys_buffer: torch.Tensor, new_values_buffer: torch.Tensor,
                            key_buffer: torch.Tensor, value_buffer: torch.Tensor,
                            block_table_buffer: torch.Tensor, seq_lens_buffer: torch.Tensor,
                            output_buffer: torch.Tensor, num_seqs: int, max_seq_len: int,
                            max_blocks_per_seq: int = 0, query_offset: int = 0,
                            new_keys_offset: int = 0, new_values_offset: int = 0,
                            output_offset: int = 0, partition_size: int = 0) -> None:
        stream = resolve_stream(step_ctx)
        if max_blocks_per_seq == 0:
            max_blocks_per_seq = (max_seq_len + self.block_size - 1) // self.block_size
        H, KV, D = self.num_query_heads, self.num_kv_heads, self.head_size
        q = view(query_buffer, query_offset, (num_seqs, H, D))
        nk = view(new_keys_buffer, new_keys_offset, (num_seqs, KV, D))
        nv = view(new_values_buffer, new_values_offset, (num_seqs, KV, D))
        out = view(output_buffer, output_offset, (num_seqs, H, D))
        bt = view(block_table_buffer, 0, (num_seqs, max_blocks_per_seq), torch.int32)
        sl = view(seq_lens_buffer, 0, (num_seqs,), torch.int32)
        kernels.paged_decode(q, self._cache(key_buffer), self._cache(value_buffer), bt, sl,
                             scale=self.scale, max_seq_len=max_seq_len, layout="kernel",
                             output=out, new_keys=nk, new_values=nv,
                             partition_size=partition_size, stream=stream)

    def encode_decode(self, step_ctx: Any, query_buffer: torch.Tensor,
                      key_buffer: torch.Tensor, value_buffer: torch.Tensor,
                      block_table_buffer: torch.Tensor, seq_lens_buffer: torch.Tensor,
                      output_buffer: torch.Tensor, num_seqs: int, max_seq_len: int,
                      max_blocks_per_seq: int = 0, query_offset: int = 0,
                      output_offset: int = 0, partition_size: int = 0) -> None:
        """Decode over a cache that already holds the new tokens (no fused write)."""
        stream = resolve_stream(step_ctx)
        if max_blocks_per_seq == 0:
            max_blocks_per_seq = (max_seq_len + self.block_size - 1) // self.block_size
        H, D = self.num_query_heads, self.head_size
        q = view(query_buffer, query_offset, (num_seqs, H, D))
        out = view(output_buffer, output_offset, (num_seqs, H, D))
        bt = view(block_table_buffer, 0, (num_seqs, max_blocks_per_seq), torch.int32)
        sl = view(seq_lens_buffer, 0, (num_seqs,), torch.int32)
        kernels.paged_decode(q, self._cache(key_buffer), self._cache(value_buffer), bt, sl,
                             scale=self.scale, max_seq_len=max_seq_len, layout="kernel",
                             output=out, partition_size=partition_size, stream=stream)

    def encode_with_kv_write(self, step_ctx: Any, query_buffer, new_keys_buffer,
                             new_values_buffer, key_buffer, value_buffer, block_table_buffer,
                             seq_lens_buffer, output_buffer, num_seqs: int, max_seq_len: int,
                             max_blocks_per_seq: int = 0) -> None:
        """attention.py:539-584: the decode fused path."""
        self.encode_decode_fused(step_ctx=step_ctx, query_buffer=query_buffer,
                                 new_keys_buffer=new_keys_buffer,
                                 new_values_buffer=new_values_buffer, key_buffer=key_buffer,
                                 value_buffer=value_buffer,
                                 block_table_buffer=block_table_buffer,
                                 seq_lens_buffer=seq_lens_buffer, output_buffer=output_buffer,
                                 num_seqs=num_seqs, max_seq_len=max_seq_len,
                                 max_blocks_per_seq=max_blocks_per_seq)

    def get_params_dict(self) -> Dict[str, Any]:
        return {
            "num_kv_heads": self.num_kv_heads,
            "num_query_heads": self.num_query_heads,
            "head_size": self.head_size,
            "block_size": self.block_size,
            "scale": self.scale,
            "kernel": self._kernel_name,
            "prefill_kernel": "paged_prefill_kernel",
        }
