"""ORACLE (test infrastructure): top-k logits selection, numpy.

Follows topk_select (vllm_apple/engine/ops/topk.py:40-412): per row, the k
largest logits and their column indices, largest first.  The reference's
insertion merge leaves the order of equal values to its thread layout; here
ties go to the lower column, which the HIP kernel implements.  Values are
compared through an order-preserving map of the 16-bit float bit patterns
(fp16 or bf16), so -0 sorts below +0 and NaNs sit at the ends by sign.

Pinning (tests/test_oracle_topk.py): the key map orders all 65536 fp16 bit
patterns exactly as their float values for every finite or infinite,
non-zero value; the selection equals torch.topk on rows without ties (values
and indices), and a brute-force check of the (value desc, column asc) order
on rows with many ties.
"""
from __future__ import annotations

import numpy as np


def sort_keys(bits: np.ndarray) -> np.ndarray:
    """uint16 bit patterns -> uint32 keys, larger float -> larger key."""
    b = bits.astype(np.uint32)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def topk(bits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """bits [T, V] uint16 -> (indices int32 [T, k], value bits uint16 [T, k])."""
    T, V = bits.shape
    keys = sort_keys(bits)
    cols = np.arange(V)
    idx = np.empty((T, k), dtype=np.int32)
    for t in range(T):
        order = np.lexsort((cols, -keys[t].astype(np.int64)))
        idx[t] = order[:k]
    vals = np.take_along_axis(bits, idx.astype(np.int64), axis=1)
    return idx, vals
