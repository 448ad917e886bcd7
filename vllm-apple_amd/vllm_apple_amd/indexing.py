"""Host-side index rules of the reference runner (CPU tensors, before a step).

derive_token_to_seq   vllm_apple/engine/runner.py:526-546 and the checks of
                      _execute_slice (:642-683): query_start_locs must have
                      num_seqs+1 entries, start at 0, end at num_tokens and be
                      non-decreasing.
check_block_capacity  runner.py:618-628: max(seq_lens) must fit the block table.
slot_mapping_from_blocks
                      apple_model_runner.py:1202-1249: slot = block_ids[pos//bs]*bs
                      + pos%bs, or pos itself when the block list is too short.
The device versions used inside a step are kernels.build_token_index and
kernels.build_slot_mapping (index_ops.hip); they compute the same integers.
"""
from __future__ import annotations

from typing import Sequence

import torch


def derive_token_to_seq(query_start_locs: torch.Tensor, num_seqs: int,
                        num_tokens: int) -> torch.Tensor:
    if query_start_locs is None:
        raise ValueError("Prefill step requires query_start_locs")
    qsl = query_start_locs.to(torch.int32).cpu()
    if qsl.numel() != num_seqs + 1:
        raise ValueError(
            f"query_start_locs has {qsl.numel()} elements, expected {num_seqs + 1} "
            f"(num_seqs_active={num_seqs}).")
    if int(qsl[0].item()) != 0:
        raise ValueError(f"query_start_locs[0] must be 0, got {int(qsl[0].item())}")
    if int(qsl[-1].item()) != num_tokens:
        raise ValueError(
            f"query_start_locs[-1] must equal num_tokens ({num_tokens}), "
            f"got {int(qsl[-1].item())}.")
    lens = (qsl[1:] - qsl[:-1]).to(torch.int64)
    if (lens < 0).any():
        raise ValueError("query_start_locs must be non-decreasing")
    tok = torch.repeat_interleave(torch.arange(num_seqs, dtype=torch.int32), lens)
    if tok.numel() != num_tokens:
        raise ValueError(
            f"token_to_seq has {tok.numel()} elements, expected num_tokens={num_tokens}.")
    return tok


def positions_from_lengths(query_start_locs: torch.Tensor,
                           seq_lens: torch.Tensor) -> torch.Tensor:
    """Absolute positions: the last query_len tokens of each full-length sequence."""
    qsl = query_start_locs.to(torch.int64).cpu()
    sl = seq_lens.to(torch.int64).cpu()
    out = []
    for s in range(qsl.numel() - 1):
        n = int(qsl[s + 1] - qsl[s])
        out.append(torch.arange(int(sl[s]) - n, int(sl[s]), dtype=torch.int32))
    return torch.cat(out) if out else torch.zeros(0, dtype=torch.int32)


def check_block_capacity(seq_lens: torch.Tensor, block_table: torch.Tensor,
                         block_size: int) -> int:
    """max_seq_len, raising if it exceeds the table's capacity (runner.py:612-628)."""
    max_seq_len = int(seq_lens.max().item()) if seq_lens.numel() > 0 else 0
    if block_table.dim() == 2 and block_table.shape[1] > 0:
        max_blocks_per_seq = block_table.shape[1]
        if max_seq_len > max_blocks_per_seq * block_size:
            raise ValueError(
                f"seq_lens max ({max_seq_len}) exceeds block_table capacity "
                f"({max_blocks_per_seq * block_size}). max_blocks_per_seq={max_blocks_per_seq}, "
                f"block_size={block_size}.")
    return max_seq_len


def slot_mapping_from_blocks(block_ids_per_req: Sequence[Sequence[int]],
                             positions_per_req: Sequence[Sequence[int]],
                             block_size: int) -> torch.Tensor:
    slots = []
    for block_ids, positions in zip(block_ids_per_req, positions_per_req):
        for p in positions:
            bi = p // block_size
            slots.append(block_ids[bi] * block_size + p % block_size
                         if bi < len(block_ids) else p)
    return torch.tensor(slots, dtype=torch.int64)


def block_table_from_lists(block_ids_per_req: Sequence[Sequence[int]]) -> torch.Tensor:
    """-1 padded int32 block table (apple_model_runner.py:1251-1278)."""
    max_blocks = max((len(b) for b in block_ids_per_req), default=0)
    if max_blocks == 0:
        return torch.zeros((len(block_ids_per_req), 1), dtype=torch.int32)
    bt = torch.full((len(block_ids_per_req), max_blocks), -1, dtype=torch.int32)
    for i, b in enumerate(block_ids_per_req):
        if b:
            bt[i, :len(b)] = torch.tensor(list(b), dtype=torch.int32)
    return bt
