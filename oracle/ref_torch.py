"""ORACLE (test infrastructure): the reference's CPU torch path, restated.

This is what bench.py times as the CPU baseline ("port") and what the parity
tests use as "the reference's own PyTorch path".  fp16 storage as in the
reference; torch does the arithmetic.

update_kv_cache_scatter  base_attn.py:308-342 (vLLM layout [nb, bs, KV, D],
                         flat view + scatter_).  Negative (padding) slots are
                         dropped first: the torch path cannot take -1 and the
                         Metal kernel skips them (kv_write.py:137-138).
decode_sdpa              mps_attn.py:284-357: per sequence, gather the blocks
                         through block_table, view [L, KV, D], repeat_interleave
                         the KV heads over the GQA group, one SDPA call.
prefill_sdpa_prefix      the prefill semantics of paged_attention_v2.metal:375-478
                         (prefix + causal chunk) with the same gather and an
                         explicit causal mask for SDPA; the reference's own SDPA
                         prefill (base_attn.py:223-306) ignores the prefix.
rms_norm                 F.rms_norm, as the worker patches vLLM's RMSNorm
                         (apple_worker.py:567-603).
rope_neox                runner.py:1500-1524 formula (cos/sin cast to fp16 first).
silu_mul                 F.silu(gate) * up.

Pinned against oracle.attention / oracle.layer_ops (fp64) in
tests/test_oracle_attention.py and tests/test_oracle_layer_ops.py.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def update_kv_cache_scatter(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                            value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    keep = slot_mapping >= 0
    key, value, slot_mapping = key[keep], value[keep], slot_mapping[keep]
    num_tokens, kvh, d = key.shape
    _, _, nkv, hd = key_cache.shape
    kf = key_cache.view(-1, nkv, hd)
    vf = value_cache.view(-1, nkv, hd)
    idx = slot_mapping.to(torch.int64).view(-1, 1, 1).expand(num_tokens, kvh, d)
    kf.scatter_(0, idx, key)
    vf.scatter_(0, idx, value)


def decode_sdpa(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                block_table: torch.Tensor, seq_lens: list[int], scale: float,
                num_kv_heads: int, output: torch.Tensor | None = None) -> torch.Tensor:
    """query [S, H, D]; caches in the vLLM layout [nb, bs, KV, D]."""
    S, H, _ = query.shape
    _, bs, nkv, hd = key_cache.shape
    g = H // num_kv_heads
    if output is None:
        output = torch.zeros_like(query)
    for s in range(S):
        L = int(seq_lens[s])
        if L <= 0:
            continue
        nblk = (L + bs - 1) // bs
        blocks = block_table[s, :nblk].to(torch.int64)
        k = key_cache[blocks].view(-1, nkv, hd)[:L]
        v = value_cache[blocks].view(-1, nkv, hd)[:L]
        q_t = query[s:s + 1].transpose(0, 1)
        k_t = k.transpose(0, 1)
        v_t = v.transpose(0, 1)
        if g != 1:
            k_t = k_t.repeat_interleave(g, dim=0)
            v_t = v_t.repeat_interleave(g, dim=0)
        o = F.scaled_dot_product_attention(q_t.unsqueeze(0), k_t.unsqueeze(0), v_t.unsqueeze(0),
                                           attn_mask=None, dropout_p=0.0, is_causal=False,
                                           scale=scale)
        output[s] = o.squeeze(0).transpose(0, 1).squeeze(0)
    return output


def prefill_sdpa_prefix(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                        block_table: torch.Tensor, query_start_loc: list[int],
                        seq_lens: list[int], scale: float, num_kv_heads: int) -> torch.Tensor:
    """Chunked prefill with the cached prefix; caches in the vLLM layout."""
    T, H, _ = query.shape
    _, bs, nkv, hd = key_cache.shape
    g = H // num_kv_heads
    out = torch.zeros_like(query)
    for s in range(len(query_start_loc) - 1):
        q0, q1 = int(query_start_loc[s]), int(query_start_loc[s + 1])
        n = q1 - q0
        if n == 0:
            continue
        L = int(seq_lens[s])
        nblk = (L + bs - 1) // bs
        blocks = block_table[s, :nblk].to(torch.int64)
        k = key_cache[blocks].view(-1, nkv, hd)[:L].transpose(0, 1)
        v = value_cache[blocks].view(-1, nkv, hd)[:L].transpose(0, 1)
        if g != 1:
            k = k.repeat_interleave(g, dim=0)
            v = v.repeat_interleave(g, dim=0)
        qpos = torch.arange(L - n, L)
        mask = torch.arange(L)[None, :] <= qpos[:, None]
        o = F.scaled_dot_product_attention(query[q0:q1].transpose(0, 1).unsqueeze(0),
                                           k.unsqueeze(0), v.unsqueeze(0), attn_mask=mask,
                                           scale=scale)
        out[q0:q1] = o.squeeze(0).transpose(0, 1)
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return F.rms_norm(x, (x.shape[-1],), weight, eps)


def rope_neox(x: torch.Tensor, positions: torch.Tensor, cos_table: torch.Tensor,
              sin_table: torch.Tensor) -> torch.Tensor:
    """x [T, heads, D]; tables fp32 [max_pos, D/2] -> rotated copy (fp16 cos/sin)."""
    d = x.shape[-1]
    cos = torch.cat([cos_table, cos_table], dim=-1)[positions.long()].to(x.dtype).unsqueeze(1)
    sin = torch.cat([sin_table, sin_table], dim=-1)[positions.long()].to(x.dtype).unsqueeze(1)
    x1, x2 = x[..., :d // 2], x[..., d // 2:]
    rotated = torch.cat((-x2, x1), dim=-1)
    return x * cos + rotated * sin


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return F.silu(gate) * up


def kernel_to_vllm_layout(cache: torch.Tensor) -> torch.Tensor:
    """[nb, KV, bs, D] -> [nb, bs, KV, D] (engine <-> vLLM permute, engine/kv_cache.py:669-674)."""
    return cache.permute(0, 2, 1, 3).contiguous()
