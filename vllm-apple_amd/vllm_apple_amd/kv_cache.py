"""HBM-resident paged K/V cache with the reference's layout, strides and checks.

Mirrors vllm_apple/engine/kv_cache.py (EngineKVCache, KVCacheDescriptor in
engine/descriptors.py:265-316) and vllm_apple/metal/kv_cache.py (MetalKVCache):
per layer, K and V are each [num_blocks, num_kv_heads, block_size, head_size]
fp16 with strides block = KV*bs*D, head = bs*D, token = D.  Instead of one
MTLBuffer per layer the cache is a torch tensor on the GPU; a layer's K/V are
views of it.

The validation methods keep the reference's rules and messages
(engine/kv_cache.py:300-420): block ids may be -1 (unused) but not < -1 or
>= num_blocks; slots may be -1 (padding) but not < -1 or > the last slot.  They
run on host (CPU) tensors/arrays, before a step is enqueued, exactly as the
reference validates at its step boundary; device tensors are copied to the
host first (one synchronisation, the caller's choice).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple, Union

import numpy as np
import torch

from . import kernels

SUPPORTED_HEAD_SIZES = (32, 64, 96, 128)


@dataclass
class KVCacheDescriptor:
    """engine/descriptors.py:265-316."""

    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int
    num_layers: int
    dtype: torch.dtype = torch.float16
    device: str = "cuda"

    def __post_init__(self):
        if self.num_blocks < 1:
            raise ValueError(f"num_blocks must be >= 1, got {self.num_blocks}")
        if self.block_size < 1:
            raise ValueError(f"block_size must be >= 1, got {self.block_size}")
        if self.num_kv_heads < 1:
            raise ValueError(f"num_kv_heads must be >= 1, got {self.num_kv_heads}")
        if self.head_size not in SUPPORTED_HEAD_SIZES:
            raise ValueError(f"head_size must be 32/64/96/128, got {self.head_size}")

    @property
    def block_size_bytes(self) -> int:
        """Bytes of one block of one layer, K and V together: two
        [KV, bs, D] tiles of the cache's element type (2 bytes for fp16 and
        bf16 alike)."""
        elems = self.num_kv_heads * self.block_size * self.head_size
        return 2 * elems * torch.empty((), dtype=self.dtype).element_size()

    @property
    def total_cache_bytes(self) -> int:
        """Bytes of the whole cache: every block of every layer."""
        return self.num_layers * self.num_blocks * self.block_size_bytes

    @property
    def total_cache_mb(self) -> float:
        return self.total_cache_bytes / float(1 << 20)


def _to_host(x: Union[np.ndarray, torch.Tensor]) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy()
    return np.asarray(x)


class HipKVCache:
    """Engine-owned paged KV cache in HBM (one K and one V tensor per layer)."""

    def __init__(self, descriptor: KVCacheDescriptor, device: Union[str, torch.device, None] = None,
                 zero: bool = True):
        descriptor.__post_init__()
        self._desc = descriptor
        dev = torch.device(device or descriptor.device)
        shape = (descriptor.num_layers, 2, descriptor.num_blocks, descriptor.num_kv_heads,
                 descriptor.block_size, descriptor.head_size)
        alloc = torch.zeros if zero else torch.empty
        self._storage = alloc(shape, dtype=descriptor.dtype, device=dev)
        self._strides = {
            "block": descriptor.num_kv_heads * descriptor.block_size * descriptor.head_size,
            "head": descriptor.block_size * descriptor.head_size,
            "token": descriptor.head_size,
            "element": 1,
        }
        self._bytes_per_block = self._strides["block"] * self._storage.element_size()

    # -- layout ---------------------------------------------------------------
    @property
    def descriptor(self) -> KVCacheDescriptor:
        return self._desc

    @property
    def num_blocks(self) -> int:
        return self._desc.num_blocks

    @property
    def block_size(self) -> int:
        return self._desc.block_size

    @property
    def strides(self) -> dict:
        return dict(self._strides)

    def get_buffers(self, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """(key, value) views of one layer, each [nb, KV, bs, D]."""
        return self._storage[layer_idx, 0], self._storage[layer_idx, 1]

    def get_key_buffer(self, layer_idx: int) -> torch.Tensor:
        return self._storage[layer_idx, 0]

    def get_value_buffer(self, layer_idx: int) -> torch.Tensor:
        return self._storage[layer_idx, 1]

    def get_block_offset(self, block_id: int) -> int:
        """Byte offset of a block inside one layer's K (or V) buffer."""
        return block_id * self._bytes_per_block

    def get_slot_offset(self, slot_idx: int) -> Tuple[int, int]:
        """Absolute slot -> (block_id, token_offset) (engine/kv_cache.py:433-444)."""
        return slot_idx // self._desc.block_size, slot_idx % self._desc.block_size

    def get_element_offset(self, block_id: int, head_idx: int, token_offset: int) -> int:
        return (block_id * self._strides["block"] + head_idx * self._strides["head"]
                + token_offset * self._strides["token"])

    def to_params_dict(self) -> dict:
        return {
            "num_blocks": self._desc.num_blocks,
            "block_size": self._desc.block_size,
            "num_kv_heads": self._desc.num_kv_heads,
            "head_size": self._desc.head_size,
            "stride_block": self._strides["block"],
            "stride_head": self._strides["head"],
            "stride_token": self._strides["token"],
        }

    # -- validation (engine/kv_cache.py:300-420) ------------------------------
    def validate_block_table(self, block_table, context: str = "") -> None:
        bt = _to_host(block_table)
        if bt.size == 0:
            return
        max_idx = bt.max()
        if max_idx >= self._desc.num_blocks:
            raise ValueError(
                f"Block table contains index {max_idx} >= num_blocks {self._desc.num_blocks}"
                f"{' (' + context + ')' if context else ''}")
        invalid = bt < -1
        if invalid.any():
            raise ValueError(
                f"Block table contains invalid index {bt[invalid].min()}"
                f"{' (' + context + ')' if context else ''}")

    def validate_slot_mapping(self, slot_mapping, context: str = "") -> None:
        sm = _to_host(slot_mapping)
        max_valid_slot = self._desc.num_blocks * self._desc.block_size - 1
        valid = sm >= 0
        if valid.any():
            max_slot = sm[valid].max()
            if max_slot > max_valid_slot:
                raise ValueError(
                    f"Slot mapping contains index {max_slot} > max valid slot {max_valid_slot} "
                    f"(num_blocks={self._desc.num_blocks}, block_size={self._desc.block_size})"
                    f"{' (' + context + ')' if context else ''}")
        invalid = sm < -1
        if invalid.any():
            raise ValueError(
                f"Slot mapping contains invalid index {sm[invalid].min()}"
                f"{' (' + context + ')' if context else ''}")

    # -- writes ---------------------------------------------------------------
    def write_kv(self, layer_idx: int, block_id: int, token_offset: int,
                 key: torch.Tensor, value: torch.Tensor) -> None:
        """One token's [KV, D] key/value at (block_id, token_offset)
        (metal/kv_cache.py:282-334), through the device single-token write."""
        if token_offset >= self._desc.block_size:
            raise ValueError(f"token_offset {token_offset} >= block_size {self._desc.block_size}")
        k, v = self.get_buffers(layer_idx)
        dev = k.device
        key = torch.as_tensor(key).to(device=dev, dtype=k.dtype).contiguous()
        value = torch.as_tensor(value).to(device=dev, dtype=k.dtype).contiguous()
        kernels.write_kv_single(k, v, key, value, block_id, token_offset, self._strides["block"],
                                self._strides["head"], self._strides["token"],
                                self._desc.num_blocks)

    def write_kv_token(self, layer_idx: int, slot: int, key: torch.Tensor,
                       value: torch.Tensor) -> None:
        """By absolute slot (metal/kv_cache.py:453-481)."""
        block_id, off = self.get_slot_offset(slot)
        self.write_kv(layer_idx, block_id, off, key, value)

    def reset(self) -> None:
        self._storage.zero_()
