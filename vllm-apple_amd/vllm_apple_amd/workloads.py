"""Seeded synthetic inputs for the five BASELINE configurations.

C1  Qwen2-0.5B-shaped decode: 14q/2kv, D64, B4, ctx U{16..512}, 256-block pool
C2  Mistral-Small-22B-shaped decode: 32q/8kv, D128, B32, ctx U{1024..8192}
    (headline: every ctx = 8192), pool sized for 300k tokens, shuffled
C3  chunked prefill: 4 sequences x (2048 cached + 512 new), 32q/8kv, D128
C4  long decode with split-K: B64, ctx log-uniform [4096, 32768], 1% of the
    valid key rows scaled x8
C5  mixed step: 56 decodes (ctx U{256..16384}) + 8 prefill chunks of 256;
    RMSNorm H=5120, NeoX RoPE base 1e6, SwiGLU I=32768

Every tensor comes from one torch.Generator seeded per configuration (C1..C5
-> 1001..1005) on the target device, so a run is reproducible.  All caches use
the kernel layout [num_blocks, num_kv_heads, block_size, head_size], fp16.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

SEEDS = {"C1": 1001, "C2": 1002, "C3": 1003, "C4": 1004, "C5": 1005}
BLOCK_SIZE = 16


@dataclass
class PagedBatch:
    """A paged KV cache plus one step's attention inputs."""

    num_q_heads: int
    num_kv_heads: int
    head_size: int
    block_size: int
    scale: float
    k_cache: torch.Tensor            # [nb, KV, bs, D]
    v_cache: torch.Tensor
    block_table: torch.Tensor        # [S, max_blocks] int32, -1 padded
    seq_lens: torch.Tensor           # [S] int32, full lengths incl. new tokens
    query: torch.Tensor              # [T, H, D]
    new_k: torch.Tensor              # [T, KV, D]
    new_v: torch.Tensor
    slot_mapping: torch.Tensor       # [T] int64
    query_start_loc: torch.Tensor    # [S + 1] int32
    token_to_seq: torch.Tensor       # [T] int32
    positions: torch.Tensor          # [T] int32
    num_decode_tokens: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return self.seq_lens.numel()

    @property
    def max_seq_len(self) -> int:
        return int(self.extra.get("max_seq_len", 0))

    def decode_kv_bytes(self) -> int:
        """K+V bytes a decode step must read (each row once, GQA-independent)."""
        lens = self.extra["seq_lens_host"]
        return int(sum(lens)) * self.num_kv_heads * self.head_size * 2 * 2

    def decode_algorithmic_bytes(self) -> int:
        """Algorithmic HBM bytes of one fused decode step (KV write + attention).

        sum_s L_s*KV*D*2*2 (cache rows read once; the new token's row comes from
        new K/V instead) + q read + out write + new K/V read + new K/V written +
        block-table entries used + seq_lens.
        """
        lens = self.extra["seq_lens_host"]
        B, H, KV, D = len(lens), self.num_q_heads, self.num_kv_heads, self.head_size
        bt = sum((L + self.block_size - 1) // self.block_size for L in lens) * 4
        return (self.decode_kv_bytes() + 2 * B * H * D * 2 + 2 * 2 * B * KV * D * 2
                + bt + B * 4)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, g, device, std: float = 1.0, mean: float = 0.0,
           dtype: torch.dtype = torch.float16) -> torch.Tensor:
    t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0 or mean != 0.0:
        t = t * std + mean
    return t.to(dtype)


def _paged_batch(*, device, g, H, KV, D, ctx_lens, new_per_seq, pool_blocks,
                 max_blocks=None, scale=None, bs=BLOCK_SIZE,
                 dtype: torch.dtype = torch.float16) -> PagedBatch:
    """Caches + block tables for sequences of total lengths ctx_lens, whose last
    new_per_seq[s] tokens are this step's queries (positions L-n .. L-1)."""
    S = len(ctx_lens)
    nblk = [(L + bs - 1) // bs for L in ctx_lens]
    if max_blocks is None:
        max_blocks = max(nblk) if nblk else 1
    need = sum(nblk)
    if pool_blocks < need:
        raise ValueError(f"pool of {pool_blocks} blocks < {need} needed")
    perm = torch.randperm(pool_blocks, generator=g, device=device).to(torch.int32)
    bt = torch.full((S, max_blocks), -1, dtype=torch.int32, device=device)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    k_cache = _randn((pool_blocks, KV, bs, D), g, device, dtype=dtype)
    v_cache = _randn((pool_blocks, KV, bs, D), g, device, dtype=dtype)
    T = sum(new_per_seq)
    query = _randn((T, H, D), g, device, dtype=dtype)
    new_k = _randn((T, KV, D), g, device, dtype=dtype)
    new_v = _randn((T, KV, D), g, device, dtype=dtype)
    qsl = [0]
    tok, pos = [], []
    for s, (L, n) in enumerate(zip(ctx_lens, new_per_seq)):
        qsl.append(qsl[-1] + n)
        tok += [s] * n
        pos += list(range(L - n, L))
    bt_host = bt.cpu()
    slots = [int(bt_host[s, p // bs]) * bs + p % bs for s, p in zip(tok, pos)]
    batch = PagedBatch(
        num_q_heads=H, num_kv_heads=KV, head_size=D, block_size=bs,
        scale=scale if scale is not None else 1.0 / math.sqrt(D),
        k_cache=k_cache, v_cache=v_cache, block_table=bt,
        seq_lens=torch.tensor(ctx_lens, dtype=torch.int32, device=device),
        query=query, new_k=new_k, new_v=new_v,
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=device),
        token_to_seq=torch.tensor(tok, dtype=torch.int32, device=device),
        positions=torch.tensor(pos, dtype=torch.int32, device=device),
    )
    batch.extra["seq_lens_host"] = list(ctx_lens)
    batch.extra["max_seq_len"] = max(ctx_lens) if ctx_lens else 0
    return batch


def _uniform_int(g, lo: int, hi: int, n: int, device) -> list[int]:
    return torch.randint(lo, hi + 1, (n,), generator=g, device=device).tolist()


def c1_decode(device="cpu", seed: int | None = None) -> PagedBatch:
    g = _gen(device, seed or SEEDS["C1"])
    lens = _uniform_int(g, 16, 512, 4, device)
    return _paged_batch(device=device, g=g, H=14, KV=2, D=64, ctx_lens=lens,
                        new_per_seq=[1] * 4, pool_blocks=256, max_blocks=32, scale=1.0 / 8)


def c2_decode(device="cpu", seed: int | None = None, fixed_len: int | None = None,
              batch: int = 32, dtype: torch.dtype = torch.float16) -> PagedBatch:
    g = _gen(device, seed or SEEDS["C2"])
    lens = [fixed_len] * batch if fixed_len else _uniform_int(g, 1024, 8192, batch, device)
    pool = math.ceil(300_000 / BLOCK_SIZE)
    return _paged_batch(device=device, g=g, H=32, KV=8, D=128, ctx_lens=lens,
                        new_per_seq=[1] * batch, pool_blocks=pool, max_blocks=8192 // BLOCK_SIZE,
                        dtype=dtype)


def c3_prefill(device="cpu", seed: int | None = None, cached: int = 2048, chunk: int = 512,
               num_seqs: int = 4, dtype: torch.dtype = torch.float16) -> PagedBatch:
    g = _gen(device, seed or SEEDS["C3"])
    L = cached + chunk
    nblk = (L + BLOCK_SIZE - 1) // BLOCK_SIZE
    return _paged_batch(device=device, g=g, H=32, KV=8, D=128, ctx_lens=[L] * num_seqs,
                        new_per_seq=[chunk] * num_seqs, pool_blocks=2 * nblk * num_seqs,
                        dtype=dtype)


def c4_long_decode(device="cpu", seed: int | None = None, batch: int = 64) -> PagedBatch:
    g = _gen(device, seed or SEEDS["C4"])
    u = torch.rand(batch, generator=g, device=device, dtype=torch.float64)
    lens = [int(round(math.exp(math.log(4096) + float(x) * (math.log(32768) - math.log(4096)))))
            for x in u.tolist()]
    nblk = sum((L + BLOCK_SIZE - 1) // BLOCK_SIZE for L in lens)
    b = _paged_batch(device=device, g=g, H=32, KV=8, D=128, ctx_lens=lens,
                     new_per_seq=[1] * batch, pool_blocks=nblk + 64,
                     max_blocks=32768 // BLOCK_SIZE)
    # 1% of the valid (token, kv-head) key rows scaled x8 (softmax max-tracking).
    bt = b.block_table.cpu()
    rows = []
    for s, L in enumerate(lens):
        for h in range(b.num_kv_heads):
            n = max(1, L // 100)
            picks = torch.randint(0, L, (n,), generator=g, device=device).cpu()
            for p in picks.tolist():
                rows.append((int(bt[s, p // BLOCK_SIZE]), h, p % BLOCK_SIZE))
    idx = torch.tensor(rows, dtype=torch.int64, device=device)
    sel = b.k_cache[idx[:, 0], idx[:, 1], idx[:, 2]]
    b.k_cache[idx[:, 0], idx[:, 1], idx[:, 2]] = (sel.float() * 8).to(torch.float16)
    b.extra["scaled_rows"] = len(rows)
    return b


def c5_mixed(device="cpu", seed: int | None = None) -> PagedBatch:
    g = _gen(device, seed or SEEDS["C5"])
    dec = _uniform_int(g, 256, 16384, 56, device)
    pre = _uniform_int(g, 256, 16384, 8, device)
    lens = dec + pre
    new = [1] * 56 + [256] * 8
    nblk = sum((L + BLOCK_SIZE - 1) // BLOCK_SIZE for L in lens)
    b = _paged_batch(device=device, g=g, H=32, KV=8, D=128, ctx_lens=lens, new_per_seq=new,
                     pool_blocks=nblk + 64, max_blocks=16384 // BLOCK_SIZE)
    b.num_decode_tokens = 56
    T = sum(new)
    b.extra["hidden"] = _randn((T, 5120), g, device)
    b.extra["norm_weight"] = _randn((5120,), g, device, std=0.1, mean=1.0)
    b.extra["gate"] = _randn((T, 32768), g, device)
    b.extra["up"] = _randn((T, 32768), g, device)
    b.extra["rope_base"] = 1e6
    b.extra["eps"] = 1e-5
    return b


CONFIGS = {"C1": c1_decode, "C2": c2_decode, "C3": c3_prefill, "C4": c4_long_decode,
           "C5": c5_mixed}
