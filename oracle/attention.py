"""ORACLE (test infrastructure): paged attention restated on the CPU.

decode            numpy fp64.  Follows paged_attention_fused.metal:107-201 /
                  paged_attention_v2.metal:49-261: for sequence s, query head h,
                  kv head h // (H/KV), softmax(scale * q.K_j) over cache
                  positions j < seq_lens[s] gathered through block_table; a zero
                  row when seq_len <= 0 (the bridge pre-zeros its output,
                  metal_paged_attention_fused.py:300).  Tokens of an invalid
                  block (<0 or >= num_blocks) are masked out (the reference reads
                  out of bounds there; the library defines them as absent).
prefill           numpy fp64.  Follows paged_attention_v2.metal:375-478: token t
                  of sequence token_to_seq[t] attends to cache positions
                  [0, positions[t]]; rows with an invalid sequence, negative
                  position, context past the block table (:401) or an invalid
                  block inside the context (:428) are not written.
decode_partials   numpy fp64: the decode restricted to key partitions
                  [P*p, P*(p+1)) of each sequence, as (normalised partial
                  output, natural-log softmax denominator); the input of a
                  split-K merge.  No reference counterpart (the reference
                  never splits a context).
merge_states      numpy fp64 log-sum-exp merge of such partials:
                  out = sum_p e^(lse_p - LSE) o_p, LSE = log sum_p e^(lse_p).
                  Pinned by: merging decode_partials gives `decode` for any
                  partition size (the split is exact in real arithmetic); one
                  partition returns its o_p unchanged; a hand-computed
                  two-partition case (weights 1/4, 3/4); empty partitions
                  (lse -inf) are ignored.
decode_loop_fp32  pure-Python fp32 loop with the exact structure of the Metal
                  kernel's online softmax (paged_attention_fused.metal:141-200);
                  small cases only.  Used to pin `decode`.

Pinning (tests/test_oracle_attention.py): decode/prefill against torch SDPA
on gathered K/V (the library routine the reference's PyTorch path calls,
mps_attn.py:344-352), against decode_loop_fp32, against the known-answer test
tests/metal/test_metal_kernels.py:380-438 (seq_len 1 -> V exactly), and
against closed forms (equal keys -> mean of V; one dominant key -> its V;
prefill without a prefix == within-chunk causal attention).
"""
from __future__ import annotations

import numpy as np


def _layout_dims(cache: np.ndarray, layout: str) -> tuple[int, int, int, int]:
    if layout == "kernel":
        nb, kv, bs, d = cache.shape
    elif layout == "vllm":
        nb, bs, kv, d = cache.shape
    else:
        raise ValueError(layout)
    return nb, kv, bs, d


def gather(cache: np.ndarray, bt_row: np.ndarray, length: int,
           layout: str) -> tuple[np.ndarray, np.ndarray]:
    """Cache rows of positions [0, length) -> ([length, KV, D] fp64, valid[length])."""
    nb, kv, bs, d = _layout_dims(cache, layout)
    nblk = (length + bs - 1) // bs
    blocks = np.asarray(bt_row[:nblk], dtype=np.int64)
    valid_blk = (blocks >= 0) & (blocks < nb)
    safe = np.where(valid_blk, blocks, 0)
    g = cache[safe]
    if layout == "kernel":
        g = g.transpose(0, 2, 1, 3)               # [nblk, bs, KV, D]
    rows = g.reshape(nblk * bs, kv, d)[:length].astype(np.float64)
    valid = np.repeat(valid_blk, bs)[:length]
    return rows, valid


def _attend(q: np.ndarray, K: np.ndarray, V: np.ndarray, valid: np.ndarray, scale: float,
            G: int, mask: np.ndarray | None = None) -> np.ndarray:
    """q [M, H, D] against K/V [L, KV, D]; mask [M, L] (True = attend)."""
    M, H, Dq = q.shape
    KV = K.shape[1]
    # Batched fp64 matrix products per kv head over its G query heads (BLAS;
    # the same sums as an einsum, in another order).
    qg = q.astype(np.float64).reshape(M, KV, G, Dq).transpose(1, 2, 0, 3)  # [KV, G, M, D]
    Kt = np.ascontiguousarray(K.transpose(1, 2, 0))                         # [KV, D, L]
    s = np.matmul(qg, Kt[:, None]) * scale                                  # [KV, G, M, L]
    s = s.reshape(H, M, -1)
    allow = np.broadcast_to(valid[None, None, :], s.shape)
    if mask is not None:
        allow = allow & mask[None, :, :]
    s = np.where(allow, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    Vt = np.ascontiguousarray(V.transpose(1, 0, 2))                         # [KV, L, D]
    o = np.matmul(p.reshape(KV, G, M, -1), Vt[:, None]).reshape(H, M, -1)   # [H, M, D]
    o = o.transpose(1, 0, 2)
    l = l.transpose(1, 0, 2)                       # [M, H, 1]
    return np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0)


def decode(query: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
           block_table: np.ndarray, seq_lens: np.ndarray, scale: float,
           layout: str = "kernel") -> np.ndarray:
    """fp64 decode attention; query [S, H, D] -> out [S, H, D] (float64)."""
    nb, kv, bs, d = _layout_dims(k_cache, layout)
    S, H, _ = query.shape
    G = H // kv
    cap = block_table.shape[1] * bs
    out = np.zeros((S, H, d), dtype=np.float64)
    for s in range(S):
        L = min(int(seq_lens[s]), cap)
        if L <= 0:
            continue
        K, valid = gather(k_cache, block_table[s], L, layout)
        V, _ = gather(v_cache, block_table[s], L, layout)
        V = np.where(valid[:, None, None], V, 0.0)
        out[s] = _attend(query[s:s + 1], K, V, valid, scale, G)[0]
    return out


def decode_partials(query: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                    block_table: np.ndarray, seq_lens: np.ndarray, scale: float,
                    part_tokens: int, layout: str = "kernel") -> tuple:
    """(partial_out [S, H, P, D], lse [S, H, P], num_parts [S]) in fp64 for
    partitions of part_tokens keys; P = the most partitions of any sequence.
    Partitions past a sequence's length hold lse = -inf and zeros."""
    nb, kv, bs, d = _layout_dims(k_cache, layout)
    S, H, _ = query.shape
    G = H // kv
    cap = block_table.shape[1] * bs
    lens = [max(0, min(int(x), cap)) for x in seq_lens]
    nparts = [(L + part_tokens - 1) // part_tokens for L in lens]
    P = max(max(nparts, default=0), 1)
    out = np.zeros((S, H, P, d))
    lse = np.full((S, H, P), -np.inf)
    kvh = np.arange(H) // G
    for s in range(S):
        L = lens[s]
        if L <= 0:
            continue
        K, valid = gather(k_cache, block_table[s], L, layout)
        V, _ = gather(v_cache, block_table[s], L, layout)
        V = np.where(valid[:, None, None], V, 0.0)
        sc = np.einsum("hd,lhd->hl", query[s].astype(np.float64), K[:, kvh, :]) * scale
        sc = np.where(valid[None, :], sc, -np.inf)
        for p in range(nparts[s]):
            lo, hi = p * part_tokens, min(L, (p + 1) * part_tokens)
            x = sc[:, lo:hi]
            m = x.max(axis=1, keepdims=True)
            ok = np.isfinite(m[:, 0])
            e = np.exp(x - np.where(np.isfinite(m), m, 0.0))
            l = e.sum(axis=1)
            o = np.einsum("hl,lhd->hd", e, V[lo:hi][:, kvh, :])
            out[s, :, p] = np.where(ok[:, None], o / np.where(l > 0, l, 1.0)[:, None], 0.0)
            lse[s, :, p] = np.where(ok, m[:, 0] + np.log(np.where(l > 0, l, 1.0)), -np.inf)
    return out, lse, np.asarray(nparts, dtype=np.int32)


def merge_states(partial_out: np.ndarray, lse: np.ndarray,
                 num_parts: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """fp64 (out [S, H, D], LSE [S, H]) of partial states [S, H, P, D] / [S, H, P]."""
    S, H, P, _ = partial_out.shape
    use = np.ones((S, H, P), dtype=bool)
    if num_parts is not None:
        use &= (np.arange(P)[None, None, :] < np.asarray(num_parts)[:, None, None])
    x = np.where(use & np.isfinite(lse), lse.astype(np.float64), -np.inf)
    M = x.max(axis=2, keepdims=True)
    has = np.isfinite(M)
    w = np.where(has, np.exp(x - np.where(has, M, 0.0)), 0.0)
    den = w.sum(axis=2)
    out = np.einsum("shp,shpd->shd", w, partial_out.astype(np.float64))
    out = np.where(den[..., None] > 0, out / np.where(den > 0, den, 1.0)[..., None], 0.0)
    LSE = np.where(den > 0, M[..., 0] + np.log(np.where(den > 0, den, 1.0)), -np.inf)
    return out, LSE


def prefill(query: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
            block_table: np.ndarray, token_to_seq: np.ndarray, positions: np.ndarray,
            scale: float, layout: str = "kernel",
            rows: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """fp64 chunked-prefill attention.

    Returns (out [T, H, D] float64, written [T] bool).  ``rows`` restricts the
    computation to a subset of token indices (others are reported unwritten).
    """
    nb, kv, bs, d = _layout_dims(k_cache, layout)
    T, H, _ = query.shape
    G = H // kv
    S, maxb = block_table.shape
    out = np.zeros((T, H, d), dtype=np.float64)
    written = np.zeros(T, dtype=bool)
    sel = np.arange(T) if rows is None else np.asarray(rows)
    ok = []
    for t in sel:
        s, pos = int(token_to_seq[t]), int(positions[t])
        if s < 0 or s >= S or pos < 0:
            continue
        ctx = pos + 1
        nblk = (ctx + bs - 1) // bs
        if nblk > maxb:
            continue
        blocks = block_table[s, :nblk]
        if np.any((blocks < 0) | (blocks >= nb)):
            continue
        ok.append(t)
    ok = np.asarray(ok, dtype=np.int64)
    for s in np.unique(token_to_seq[ok]) if ok.size else []:
        toks = ok[token_to_seq[ok] == s]
        ctx_max = int(positions[toks].max()) + 1
        K, valid = gather(k_cache, block_table[s], ctx_max, layout)
        V, _ = gather(v_cache, block_table[s], ctx_max, layout)
        mask = np.arange(ctx_max)[None, :] <= positions[toks][:, None]
        out[toks] = _attend(query[toks], K, V, valid, scale, G, mask)
        written[toks] = True
    return out, written


def decode_loop_fp32(query: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     block_table: np.ndarray, seq_lens: np.ndarray, scale: float,
                     layout: str = "kernel") -> np.ndarray:
    """Token-serial fp32 online softmax exactly as paged_attention_fused.metal:141-200."""
    nb, kv, bs, d = _layout_dims(k_cache, layout)
    S, H, _ = query.shape
    G = H // kv
    f32 = np.float32
    out = np.zeros((S, H, d), dtype=f32)
    for s in range(S):
        L = int(seq_lens[s])
        if L <= 0:
            continue
        for h in range(H):
            kvh = h // G
            q = query[s, h].astype(f32)
            m_prev, l_prev = f32(-np.inf), f32(0.0)
            acc = np.zeros(d, dtype=f32)
            for bi in range((L + bs - 1) // bs):
                phys = int(block_table[s, bi])
                for off in range(min(bs, L - bi * bs)):
                    if layout == "kernel":
                        k = k_cache[phys, kvh, off].astype(f32)
                        v = v_cache[phys, kvh, off].astype(f32)
                    else:
                        k = k_cache[phys, off, kvh].astype(f32)
                        v = v_cache[phys, off, kvh].astype(f32)
                    score = f32(np.dot(q, k)) * f32(scale)
                    m_new = max(m_prev, score)
                    e_prev = f32(np.exp(m_prev - m_new))
                    e_cur = f32(np.exp(score - m_new))
                    acc = acc * e_prev + e_cur * v
                    l_prev = l_prev * e_prev + e_cur
                    m_prev = m_new
            inv_l = f32(1.0) / l_prev if l_prev > 0 else f32(0.0)
            out[s, h] = acc * inv_l
    return out
