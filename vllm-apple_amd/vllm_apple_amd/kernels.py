"""Functional wrappers over the HIP C ABI, taking torch tensors on the GPU.

Every function enqueues work on torch's current HIP stream (or ``stream``) and
returns without synchronising.  Arguments are checked on the host; tensors
must live on a ROCm device -- there is no CPU fallback.

KV caches are described by a layout name:
  "kernel": K, V each [num_blocks, num_kv_heads, block_size, head_size]
            (vllm_apple/metal/kv_cache.py:213-219)
  "vllm":   K = kv_cache[0], V = kv_cache[1], each [num_blocks, block_size,
            num_kv_heads, head_size] (metal_attn.py:171-185)
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib

LAYOUTS = ("kernel", "vllm")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(
                f"tensor on {t.device}: the HIP path needs ROCm device tensors "
                "(there is no CPU fallback)")


def _require_dtype(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")


# 16-bit element types the attention entry points take (vaa_attn_params.dtype).
ATTN_DTYPES = {torch.float16: _lib.VAA_DTYPE_F16, torch.bfloat16: _lib.VAA_DTYPE_BF16}


def _attn_dtype(**named: torch.Tensor | None) -> torch.dtype:
    """The one element type (fp16 or bf16) shared by all the given tensors."""
    dtypes = {n: t.dtype for n, t in named.items() if t is not None}
    kinds = set(dtypes.values())
    if len(kinds) != 1 or next(iter(kinds)) not in ATTN_DTYPES:
        raise ValueError(f"tensors must all be float16 or all bfloat16, got {dtypes}")
    return next(iter(kinds))


@dataclass(frozen=True)
class CacheStrides:
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int
    stride_block: int
    stride_head: int
    stride_token: int


def cache_strides(cache: torch.Tensor, layout: str) -> CacheStrides:
    """Element strides of one K or V cache tensor in the given layout."""
    if cache.dim() != 4:
        raise ValueError(f"cache must be 4-D, got shape {tuple(cache.shape)}")
    if cache.stride(3) != 1:
        raise ValueError("cache head_size dimension must be contiguous")
    if layout == "kernel":
        nb, kv, bs, d = cache.shape
        sb, sh, st = cache.stride(0), cache.stride(1), cache.stride(2)
    elif layout == "vllm":
        nb, bs, kv, d = cache.shape
        sb, st, sh = cache.stride(0), cache.stride(1), cache.stride(2)
    else:
        raise ValueError(f"layout must be one of {LAYOUTS}, got {layout!r}")
    return CacheStrides(nb, bs, kv, d, sb, sh, st)


def make_params(*, key_cache: torch.Tensor, value_cache: torch.Tensor, layout: str,
                num_query_heads: int, scale: float, num_seqs: int = 0,
                max_seq_len: int = 0, max_blocks_per_seq: int = 0,
                query: torch.Tensor | None = None, output: torch.Tensor | None = None,
                new_kv: torch.Tensor | None = None,
                partition_size: int = 0) -> _lib.VaaAttnParams:
    ks = cache_strides(key_cache, layout)
    vs = cache_strides(value_cache, layout)
    if (ks.num_blocks, ks.block_size, ks.num_kv_heads, ks.head_size) != (
            vs.num_blocks, vs.block_size, vs.num_kv_heads, vs.head_size):
        raise ValueError("key and value caches differ in shape")
    if num_query_heads % ks.num_kv_heads != 0:
        raise ValueError(
            f"num_query_heads={num_query_heads} not a multiple of num_kv_heads={ks.num_kv_heads}")
    if key_cache.dtype != value_cache.dtype or key_cache.dtype not in ATTN_DTYPES:
        raise ValueError(f"caches must both be float16 or bfloat16, got "
                         f"{key_cache.dtype}/{value_cache.dtype}")
    p = _lib.VaaAttnParams()
    p.dtype = ATTN_DTYPES[key_cache.dtype]
    p.scale = float(scale)
    p.num_seqs = int(num_seqs)
    p.max_seq_len = int(max_seq_len)
    p.max_blocks_per_seq = int(max_blocks_per_seq)
    p.head_size = ks.head_size
    p.block_size = ks.block_size
    p.num_kv_heads = ks.num_kv_heads
    p.num_query_heads = int(num_query_heads)
    p.queries_per_kv = int(num_query_heads) // ks.num_kv_heads
    p.partition_size = int(partition_size)
    p.num_blocks = ks.num_blocks
    p.k_stride_block, p.k_stride_head, p.k_stride_token = ks.stride_block, ks.stride_head, ks.stride_token
    p.v_stride_block, p.v_stride_head, p.v_stride_token = vs.stride_block, vs.stride_head, vs.stride_token
    for t, pre in ((query, "q"), (output, "o"), (new_kv, "new_kv")):
        if t is None:
            continue
        if t.dim() != 3 or t.stride(2) != 1:
            raise ValueError(f"{pre} tensor must be [tokens, heads, head_size] with contiguous last dim")
        setattr(p, f"{pre}_stride_token", t.stride(0))
        setattr(p, f"{pre}_stride_head", t.stride(1))
    return p


# ------------------------------------------------------------------ KV write


def kv_write_slots(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                   value_cache: torch.Tensor, slot_mapping: torch.Tensor, *,
                   layout: str = "kernel", stream=None) -> None:
    """cache[slot // bs, :, slot % bs] = key/value[t] for every slot >= 0.

    key/value: [num_tokens, num_kv_heads, head_size] fp16 or bf16 (any token/head
    strides with a contiguous last dim); slot_mapping: int32 or int64
    [num_tokens].  Mirrors kv_write.py:118-156 and base_attn.py:308-342.
    """
    _require_gpu(key, value, key_cache, value_cache, slot_mapping)
    _attn_dtype(key=key, value=value, key_cache=key_cache, value_cache=value_cache)
    if key.stride() != value.stride() or key.shape != value.shape:
        raise ValueError("key and value must have identical shapes and strides")
    if slot_mapping.dtype not in (torch.int32, torch.int64) or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be a contiguous int32/int64 tensor")
    n = key.shape[0]
    if slot_mapping.numel() < n:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries < {n} tokens")
    p = make_params(key_cache=key_cache, value_cache=value_cache, layout=layout,
                    num_query_heads=key.shape[1], scale=1.0, new_kv=key)
    if key.shape[1:] != (p.num_kv_heads, p.head_size):
        raise ValueError(f"key shape {tuple(key.shape)} does not match the cache")
    itype = _lib.VAA_INDEX_I64 if slot_mapping.dtype == torch.int64 else _lib.VAA_INDEX_I32
    _lib.call("vaa_kv_write_slots", ctypes.byref(p), key_cache.data_ptr(), value_cache.data_ptr(),
              slot_mapping.data_ptr(), itype, key.data_ptr(), value.data_ptr(), n,
              _lib.stream_handle(stream))


def kv_write_decode(new_keys: torch.Tensor, new_values: torch.Tensor, key_cache: torch.Tensor,
                    value_cache: torch.Tensor, block_table: torch.Tensor,
                    seq_lens: torch.Tensor, *, layout: str = "kernel", stream=None) -> None:
    """Write each sequence's new token at position seq_lens[s]-1 (kv_write.py:66-114)."""
    _require_gpu(new_keys, new_values, key_cache, value_cache, block_table, seq_lens)
    _attn_dtype(new_keys=new_keys, new_values=new_values, key_cache=key_cache,
                value_cache=value_cache)
    _check_tables(block_table, seq_lens)
    if new_keys.stride() != new_values.stride() or new_keys.shape != new_values.shape:
        raise ValueError("new_keys and new_values must have identical shapes and strides")
    num_seqs = seq_lens.numel()
    p = make_params(key_cache=key_cache, value_cache=value_cache, layout=layout,
                    num_query_heads=new_keys.shape[1], scale=1.0, num_seqs=num_seqs,
                    max_blocks_per_seq=block_table.shape[1], new_kv=new_keys)
    if new_keys.shape[0] < num_seqs:
        raise ValueError("new_keys has fewer rows than sequences")
    _lib.call("vaa_kv_write_decode", ctypes.byref(p), key_cache.data_ptr(), value_cache.data_ptr(),
              block_table.data_ptr(), seq_lens.data_ptr(), new_keys.data_ptr(),
              new_values.data_ptr(), _lib.stream_handle(stream))


def write_kv_batch(key_dst: torch.Tensor, value_dst: torch.Tensor, key_src: torch.Tensor,
                   value_src: torch.Tensor, block_ids: torch.Tensor,
                   token_offsets: torch.Tensor, stride_block: int, stride_head: int,
                   stride_token: int, num_blocks: int, stream=None) -> None:
    """Device counterpart of metal_write_kv_batch (kv_write.c:33-78)."""
    _require_gpu(key_dst, value_dst, key_src, value_src, block_ids, token_offsets)
    if not (key_src.is_contiguous() and value_src.is_contiguous()):
        raise ValueError("key_src/value_src must be contiguous [T, KV, D]")
    if block_ids.dtype != torch.int64 or token_offsets.dtype != torch.int64:
        raise ValueError("block_ids and token_offsets must be int64")
    t, kv, d = key_src.shape
    _lib.call("vaa_write_kv_batch", key_dst.data_ptr(), value_dst.data_ptr(), key_src.data_ptr(),
              value_src.data_ptr(), block_ids.data_ptr(), token_offsets.data_ptr(), t, kv, d,
              stride_block, stride_head, stride_token, num_blocks, _lib.stream_handle(stream))


def write_kv_single(key_dst: torch.Tensor, value_dst: torch.Tensor, key_src: torch.Tensor,
                    value_src: torch.Tensor, block_id: int, token_offset: int,
                    stride_block: int, stride_head: int, stride_token: int,
                    num_blocks: int, stream=None) -> None:
    """Device counterpart of metal_write_kv_single (kv_write.c:84-107)."""
    _require_gpu(key_dst, value_dst, key_src, value_src)
    kv, d = key_src.shape[-2:]
    _lib.call("vaa_write_kv_single", key_dst.data_ptr(), value_dst.data_ptr(), key_src.data_ptr(),
              value_src.data_ptr(), int(block_id), int(token_offset), kv, d, stride_block,
              stride_head, stride_token, num_blocks, _lib.stream_handle(stream))


# ----------------------------------------------------------------- attention


def _check_tables(block_table: torch.Tensor, seq_lens: torch.Tensor) -> None:
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous int32 [num_seqs, max_blocks] tensor")
    if seq_lens.dtype != torch.int32 or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 tensor")
    if block_table.shape[0] < seq_lens.numel():
        raise ValueError("block_table has fewer rows than seq_lens")


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


class _GrowOnlyScratch:
    """One grow-only byte buffer per device, shared by calls ordered on one
    stream.  A buffer that is outgrown is kept alive, never freed: a HIP
    graph captured while it was current holds its address, and replaying
    that graph must not write into memory the caching allocator has handed to
    another tensor.  Sizes grow at least 2x, so the kept buffers sum to less
    than the current one."""

    def __init__(self, min_bytes: int = 1 << 20):
        self._cur: dict[int, torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []
        self._min = min_bytes

    def get(self, nbytes: int, device: torch.device) -> torch.Tensor:
        idx = _dev_index(device)
        ws = self._cur.get(idx)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, self._min)
            if ws is not None:
                self._retired.append(ws)
                size = max(size, 2 * ws.numel())
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            self._cur[idx] = ws
        return ws


_decode_ws = _GrowOnlyScratch()


def decode_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Grow-only split-K scratch (partials) per device, reused across calls
    that are ordered on one stream (torch's current stream by default);
    outgrown buffers stay allocated (graph replays may still use them)."""
    return _decode_ws.get(nbytes, device)


_side_streams: dict[int, torch.cuda.Stream] = {}


def overlap(first_fn, second_fn, device: torch.device | None = None) -> None:
    """Run first_fn on the current stream and second_fn on a side stream at the
    same time.  Both start after the work already on the current stream;
    first_fn is enqueued first on the stream that is already running, so its
    kernels dispatch first whether the step runs eagerly or from a captured
    graph.  The current stream waits for the side stream before returning
    (callers, the caching allocator and graph capture see one ordered step).
    Used for the prefill (MFMA-bound, first) and decode (HBM-bound, second,
    with the shared balanced split) halves of a mixed step: C5 attention step
    about 0.80 -> 0.61 ms on MI355X, eager or replayed.  The side stream keeps
    the default priority."""
    main = torch.cuda.current_stream(device)
    idx = main.device.index if main.device.index is not None else torch.cuda.current_device()
    side = _side_streams.get(idx)
    if side is None:
        side = torch.cuda.Stream(device=main.device)
        _side_streams[idx] = side
    side.wait_stream(main)
    first_fn()
    with torch.cuda.stream(side):
        second_fn()
    main.wait_stream(side)


def decode_workspace_size(p: _lib.VaaAttnParams) -> tuple[int, int]:
    part = ctypes.c_int32(0)
    n = _lib.load().vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part))
    return int(n), int(part.value)


# Decode launch geometry (paged_decode.hip): partitions in multiples of 128
# tokens; partitions up to 1024 tokens run 4-wave workgroups, two per CU (one's
# start-up overlaps the other's streaming), longer ones one 8-wave workgroup
# per CU.  The balanced split runs 4-wave workgroups, two per CU's worth (four
# for the shared split), gives each workgroup at least 32 tiles (512 tokens)
# and takes at most 8192 sequences.
_DECODE_QUANTUM = 128
_SHORT_PART_TOKENS = 1024
# How much faster than its share of HBM a decode workgroup streams when the
# launch leaves slots idle (8-wave: one slot per CU; 4-wave: two, each half a
# CU's share), and the start-up of a 4-wave workgroup relative to an 8-wave
# one.  Fitted on MI355X (32q/8kv D128; us per step, measured best in
# brackets): the model picks B=1 x 8192 -> 256 (20.6 [19.6 at 512]),
# B=2 x 4096 -> 256 (16.7), B=8 x 2048 -> 512 (19.3), B=4 x 1024 -> 128
# (10.8), B=16 x 4096 -> 1024 (47.4; unsplit 54.1), B=1 x 32768 -> 1024
# (37.5 [33.4 at 2048]); C1 and the headline stay unsplit.
_LONE_WG_SPEEDUP = 1.7
_SHORT_WG_SPEEDUP = 2.0
_SHORT_START = 0.5
_BALANCED_MIN_TOKENS = 512
_BALANCED_MAX_SEQS = 8192
PARTITION_BALANCED = _lib.VAA_PARTITION_BALANCED
PARTITION_BALANCED_SHARED = _lib.VAA_PARTITION_BALANCED_SHARED
_num_cus: dict[int, int] = {}


def device_cus(device: torch.device | None = None) -> int:
    idx = _dev_index(device) if device is not None else torch.cuda.current_device()
    if idx not in _num_cus:
        _num_cus[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _num_cus[idx]


def choose_partition_size(seq_lens_host, num_kv_heads: int, num_cus: int,
                          merge_tokens: int = 256, wg_tokens: int = 96) -> int:
    """Split-K mode for known sequence lengths: a partition size in tokens, or
    PARTITION_BALANCED.

    Estimates the step time in "tokens of one kv head streamed by one CU".
    Fixed partitions of P tokens: the list-scheduling makespan
    max(total/m, largest piece) plus half a piece of tail when there is more
    than one wave of workgroups, a start-up cost per workgroup and, when any
    sequence is split, the merge launch.  With fewer workgroups than slots a
    workgroup streams faster than its share of HBM: the largest piece is
    scaled by 1/min(speed-up cap, slots/workgroups).  Short partitions (at
    most _SHORT_PART_TOKENS) run two 4-wave workgroups per CU, each with half
    a CU's share and a cheaper start-up (for tiny batches a merge launch
    costs more than the split saves).  Balanced split: total/m plus one
    start-up per sequence piece a workgroup meets and the merge launch, which
    it always has.  Equal lengths that already cover the CUs stay unsplit;
    the balanced split must win by 3 % to be chosen.  Memoised per length
    tuple (the same step is decoded by every layer).
    """
    key = (tuple(int(x) for x in seq_lens_host), int(num_kv_heads), int(num_cus),
           merge_tokens, wg_tokens)
    hit = _partition_cache.get(key)
    if hit is not None:
        return hit
    import numpy as np

    lens = np.maximum(np.asarray(key[0], dtype=np.int64), 0)
    if lens.size == 0 or lens.max() == 0:
        return 0
    m = max(1, num_cus)
    q = _DECODE_QUANTUM
    longest = int(lens.max())
    total = float(lens.sum()) * num_kv_heads
    cands = {((longest + k - 1) // k + q - 1) // q * q for k in range(1, 65)}
    cands |= {q << i for i in range(0, 10)}
    P = np.array(sorted(cands), dtype=np.int64)
    pieces = ((lens[None, :] + P[:, None] - 1) // P[:, None]).sum(axis=1)
    wgs = pieces * num_kv_heads
    big = np.minimum(P, longest).astype(np.float64)
    # Split into short partitions: 4-wave workgroups, two slots per CU.
    short = (P <= _SHORT_PART_TOKENS) & (longest > P)
    slots = np.where(short, 2 * m, m)
    cap = np.where(short, _SHORT_WG_SPEEDUP, _LONE_WG_SPEEDUP)
    speed = np.clip(slots / np.maximum(wgs, 1), 1.0, cap) / np.where(short, 2.0, 1.0)
    start = wg_tokens * np.where(short, _SHORT_START, 1.0) * wgs / m
    t = np.maximum(total / m, big / speed) + np.where(wgs > slots, big / 2, 0.0) + start
    t = t + np.where(longest > P, merge_tokens, 0)
    i = int(np.argmin(t))
    best, t_fix = int(P[i]), float(t[i])
    if lens.size <= _BALANCED_MAX_SEQS:
        # Two workgroups per CU's worth share the CU: each streams half its
        # share while the other's start-up overlaps it.
        c = 2 * ((m + num_kv_heads - 1) // num_kv_heads)
        per = max(total / (c * num_kv_heads), float(_BALANCED_MIN_TOKENS))
        t_bal = 2 * per + wg_tokens * (1.0 + lens.size / c) + merge_tokens
        if t_bal < 0.97 * t_fix:
            best = PARTITION_BALANCED
    if len(_partition_cache) > 4096:
        _partition_cache.clear()
    _partition_cache[key] = best
    return best


_partition_cache: dict = {}


def paged_decode(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                 block_table: torch.Tensor, seq_lens: torch.Tensor, *, scale: float,
                 max_seq_len: int, layout: str = "kernel", output: torch.Tensor | None = None,
                 new_keys: torch.Tensor | None = None, new_values: torch.Tensor | None = None,
                 partition_size: int = 0, workspace: torch.Tensor | None = None,
                 seq_lens_host=None, shared: bool = False, stream=None) -> torch.Tensor:
    """Paged GQA decode attention, one query token per sequence.

    query [num_seqs, H, D] fp16 or bf16 (the caches', new K/V's and output's
    type too); returns/fills output [num_seqs, H, D].  With
    new_keys/new_values ([num_seqs, KV, D]) the token at position
    seq_lens[s]-1 is written to the cache by the same launch (fused KV write).
    max_seq_len must bound seq_lens (it sizes the split-K grid).  With
    seq_lens_host (host copies of the lengths, no device sync needed) and
    partition_size 0 the split-K mode is chosen from the actual lengths;
    partition_size PARTITION_BALANCED splits by the lengths on the device.
    shared=True says the launch runs concurrently with another kernel (see
    overlap): an automatic balanced split then uses PARTITION_BALANCED_SHARED,
    half-size workgroups, four per CU's worth of the split, that share CUs
    with the other kernel.
    """
    _require_gpu(query, key_cache, value_cache, block_table, seq_lens, output, new_keys, new_values)
    dt = _attn_dtype(query=query, key_cache=key_cache, value_cache=value_cache, output=output,
                     new_keys=new_keys, new_values=new_values)
    _check_tables(block_table, seq_lens)
    num_seqs = seq_lens.numel()
    if output is None:
        output = torch.empty(query.shape, dtype=dt, device=query.device)
    if query.shape[0] < num_seqs or output.shape[0] < num_seqs:
        raise ValueError("query/output have fewer rows than sequences")
    if (new_keys is None) != (new_values is None):
        raise ValueError("new_keys and new_values go together")
    if new_keys is not None and new_keys.stride() != new_values.stride():
        raise ValueError("new_keys and new_values must share strides")
    if partition_size == 0 and seq_lens_host is not None:
        kvh = key_cache.shape[1] if layout == "kernel" else key_cache.shape[2]
        # Groups of more than 16 query heads run one workgroup per chunk of
        # at most 16 heads: the cost model counts those chunks as kv heads.
        chunks = -(-(query.shape[1] // kvh) // 16)
        partition_size = choose_partition_size(seq_lens_host, kvh * chunks,
                                               device_cus(query.device))
        if shared and partition_size == PARTITION_BALANCED:
            partition_size = PARTITION_BALANCED_SHARED
    p = make_params(key_cache=key_cache, value_cache=value_cache, layout=layout,
                    num_query_heads=query.shape[1], scale=scale, num_seqs=num_seqs,
                    max_seq_len=max_seq_len, max_blocks_per_seq=block_table.shape[1],
                    query=query, output=output, new_kv=new_keys, partition_size=partition_size)
    if query.shape[2] != p.head_size:
        raise ValueError(f"query head_size {query.shape[2]} != cache head_size {p.head_size}")
    nbytes, _ = decode_workspace_size(p)
    ws_ptr, ws_len = None, 0
    if nbytes:
        if workspace is None:
            workspace = decode_workspace(nbytes, query.device)
        if workspace.numel() * workspace.element_size() < nbytes:
            raise ValueError(f"workspace smaller than {nbytes} bytes")
        ws_ptr, ws_len = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _lib.call("vaa_paged_attention_decode", ctypes.byref(p), query.data_ptr(),
              key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
              seq_lens.data_ptr(), output.data_ptr(), _ptr(new_keys), _ptr(new_values),
              ws_ptr, ws_len, _lib.stream_handle(stream))
    return output


def merge_attn_states(partial_out: torch.Tensor, partial_lse: torch.Tensor, *,
                      num_parts: torch.Tensor | None = None, output: torch.Tensor | None = None,
                      output_lse: torch.Tensor | None = None, dtype: torch.dtype = torch.float16,
                      stream=None) -> torch.Tensor:
    """Log-sum-exp merge of attention states (vaa_merge_attn_states):
    out[s, h] = sum_p e^(lse_p - LSE) o_p, LSE = log sum_p e^(lse_p).

    partial_out fp32 [S, H, P, D] (normalised partial outputs), partial_lse
    fp32 [S, H, P] (natural-log softmax denominators, -inf for an empty
    partition), num_parts int32 [S] (the first num_parts[s] partitions count)
    or None.  Returns output [S, H, D] in `dtype` (fp16 or bf16, or output's
    type); output_lse fp32 [S, H] receives LSE when given."""
    _require_gpu(partial_out, partial_lse, num_parts, output, output_lse)
    if partial_out.dtype != torch.float32 or partial_out.dim() != 4 \
            or not partial_out.is_contiguous():
        raise ValueError("partial_out must be a contiguous fp32 [S, H, P, D] tensor")
    S, H, P, D = partial_out.shape
    if partial_lse.dtype != torch.float32 or tuple(partial_lse.shape) != (S, H, P) \
            or not partial_lse.is_contiguous():
        raise ValueError(f"partial_lse must be a contiguous fp32 [{S}, {H}, {P}] tensor")
    if num_parts is not None and (num_parts.dtype != torch.int32 or num_parts.numel() < S
                                  or not num_parts.is_contiguous()):
        raise ValueError("num_parts must be a contiguous int32 [S] tensor")
    if output is None:
        output = torch.empty((S, H, D), dtype=dtype, device=partial_out.device)
    if output.dim() != 3 or tuple(output.shape) != (S, H, D) or output.stride(2) != 1:
        raise ValueError("output must be [S, H, D] with a contiguous last dim")
    if output_lse is not None and (output_lse.dtype != torch.float32
                                   or tuple(output_lse.shape) != (S, H)
                                   or not output_lse.is_contiguous()):
        raise ValueError("output_lse must be a contiguous fp32 [S, H] tensor")
    _lib.call("vaa_merge_attn_states", partial_out.data_ptr(), partial_lse.data_ptr(),
              _ptr(num_parts), S, H, P, D, output.data_ptr(), output.stride(0), output.stride(1),
              _ptr(output_lse), ATTN_DTYPES[_attn_dtype(output=output)],
              _lib.stream_handle(stream))
    return output


_prefill_ws = _GrowOnlyScratch()
_PREFILL_KEY_TILE = 64      # keys per prefill tile (paged_prefill.hip)
_PREFILL_SPLIT_QUANTUM = 1024  # split sizes in multiples of 16 key tiles
_prefill_split_cache: dict = {}
# Largest split-K prefill workspace choose_prefill_split plans for: the
# partials take num_tokens * H * pieces * (D + 2) * 4 bytes, so a long
# context beside many short prefill tokens gets fewer, longer pieces (or no
# split) instead of a large allocation in the middle of serving.
PREFILL_SPLIT_MAX_WORKSPACE = 256 << 20


def choose_prefill_split(ctx_lens_host, query_lens_host, num_kv_heads: int,
                         num_query_heads: int, num_cus: int, head_size: int = 128,
                         max_workspace_bytes: int = PREFILL_SPLIT_MAX_WORKSPACE) -> int:
    """Key split for a prefill batch (0: none), from the host lengths.

    The prefill kernel gives each workgroup a query tile (32 tokens of 4
    heads, or the same rows over fewer heads) and streams that sequence's
    whole context, so one long context next to short ones makes the longest
    workgroups the critical path while the others leave CUs idle.  Work is
    counted in 64-key tiles per workgroup; with two workgroups per CU the
    per-slot share is total / (2 * CUs).  A split is chosen when the longest
    workgroup exceeds 1.5x that share, with pieces of about half the share
    (rounded up to 1024 keys) so the dispatcher can balance the pieces.
    The pieces are counted over the longest prefill context (pass that as
    paged_prefill's max_seq_len), and the partials of all prefill tokens
    (sum of the query lengths) must fit max_workspace_bytes: otherwise the
    pieces grow until they do, or the split is dropped.
    Memoised per length tuple (every layer of a step sees the same batch).
    """
    key = (tuple(int(x) for x in ctx_lens_host), tuple(int(x) for x in query_lens_host),
           int(num_kv_heads), int(num_query_heads), int(num_cus), int(head_size),
           int(max_workspace_bytes))
    hit = _prefill_split_cache.get(key)
    if hit is not None:
        return hit
    g = max(1, num_query_heads // max(1, num_kv_heads))
    heads_per_wg = 4 if g >= 4 else (3 if g == 3 else g)
    tokens_per_wg = 32 * (1 if g >= 3 else 4 // g)
    chunks = -(-g // heads_per_wg)
    total, longest = 0, 0
    for ctx, q in zip(key[0], key[1]):
        if q <= 0 or ctx <= 0:
            continue
        tiles = -(-ctx // _PREFILL_KEY_TILE)
        total += -(-q // tokens_per_wg) * tiles
        longest = max(longest, tiles)
    total *= num_kv_heads * chunks
    share = total / max(1, 2 * num_cus)
    split = 0
    if longest > 32 and longest > 1.5 * share:
        piece = max(_PREFILL_SPLIT_QUANTUM, int(share / 2) * _PREFILL_KEY_TILE)
        split = -(-piece // _PREFILL_SPLIT_QUANTUM) * _PREFILL_SPLIT_QUANTUM
        if split >= longest * _PREFILL_KEY_TILE:
            split = 0
    if split:
        tokens = sum(max(0, q) for q in key[1])
        # Partial rows are computed at the head size rounded up to 32.
        row_bytes = num_query_heads * (-(-head_size // 32) * 32 + 2) * 4
        max_pieces = max_workspace_bytes // max(1, tokens * row_bytes)
        keys = longest * _PREFILL_KEY_TILE
        if -(-keys // split) > max_pieces:
            split = 0
            if max_pieces >= 2:
                split = -(-keys // max_pieces)
                split = -(-split // _PREFILL_SPLIT_QUANTUM) * _PREFILL_SPLIT_QUANTUM
                if split >= keys:
                    split = 0
    if len(_prefill_split_cache) > 4096:
        _prefill_split_cache.clear()
    _prefill_split_cache[key] = split
    return split


def prefill_workspace_size(p: _lib.VaaAttnParams, num_tokens: int, split_keys: int) -> int:
    return int(_lib.load().vaa_paged_attention_prefill_workspace_size(
        ctypes.byref(p), int(num_tokens), int(split_keys)))


def paged_prefill(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                  block_table: torch.Tensor, token_to_seq: torch.Tensor,
                  positions: torch.Tensor, *, scale: float, layout: str = "kernel",
                  output: torch.Tensor | None = None, split_keys: int = 0,
                  max_seq_len: int = 0, workspace: torch.Tensor | None = None,
                  stream=None) -> torch.Tensor:
    """Chunked-prefill attention: token t attends to cache positions [0, positions[t]].

    query [num_tokens, H, D] fp16 or bf16, as the caches and output; the
    tokens' own K/V must already be cached.
    Rows the reference kernel leaves unwritten (invalid sequence, negative
    position, context past the block table, invalid block) stay untouched.
    split_keys > 0 cuts each context into pieces of that many keys (a
    multiple of 64; see choose_prefill_split) merged by log-sum-exp;
    max_seq_len bounds the contexts (default: the block table's capacity) and
    sizes the partials' workspace (grow-only scratch unless given).
    """
    _require_gpu(query, key_cache, value_cache, block_table, token_to_seq, positions, output)
    dt = _attn_dtype(query=query, key_cache=key_cache, value_cache=value_cache, output=output)
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous int32 2-D tensor")
    for t, n in ((token_to_seq, "token_to_seq"), (positions, "positions")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous int32 tensor")
    num_tokens = query.shape[0]
    if token_to_seq.numel() < num_tokens or positions.numel() < num_tokens:
        raise ValueError("token_to_seq/positions shorter than query")
    if output is None:
        output = torch.zeros(query.shape, dtype=dt, device=query.device)
    p = make_params(key_cache=key_cache, value_cache=value_cache, layout=layout,
                    num_query_heads=query.shape[1], scale=scale, num_seqs=block_table.shape[0],
                    max_blocks_per_seq=block_table.shape[1], query=query, output=output)
    if not split_keys:
        _lib.call("vaa_paged_attention_prefill", ctypes.byref(p), query.data_ptr(),
                  key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
                  token_to_seq.data_ptr(), positions.data_ptr(), output.data_ptr(), num_tokens,
                  _lib.stream_handle(stream))
        return output
    p.max_seq_len = int(max_seq_len) if max_seq_len else block_table.shape[1] * p.block_size
    nbytes = prefill_workspace_size(p, num_tokens, split_keys)
    ws_ptr = None
    if nbytes:
        if workspace is None:
            workspace = _prefill_ws.get(nbytes, query.device)
        if workspace.numel() * workspace.element_size() < nbytes:
            raise ValueError(f"workspace smaller than {nbytes} bytes")
        ws_ptr = workspace.data_ptr()
    _lib.call("vaa_paged_attention_prefill_split", ctypes.byref(p), query.data_ptr(),
              key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
              token_to_seq.data_ptr(), positions.data_ptr(), output.data_ptr(), num_tokens,
              int(split_keys), ws_ptr, nbytes, _lib.stream_handle(stream))
    return output


def build_token_index(query_start_loc: torch.Tensor, seq_lens: torch.Tensor, num_tokens: int,
                      stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(token_to_seq, positions) int32 [num_tokens] computed on the device."""
    _require_gpu(query_start_loc, seq_lens)
    for t, n in ((query_start_loc, "query_start_loc"), (seq_lens, "seq_lens")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous int32 tensor")
    num_seqs = query_start_loc.numel() - 1
    if num_seqs < 0 or seq_lens.numel() < num_seqs:
        raise ValueError("query_start_loc must have num_seqs + 1 entries")
    tok = torch.empty(num_tokens, dtype=torch.int32, device=query_start_loc.device)
    pos = torch.empty(num_tokens, dtype=torch.int32, device=query_start_loc.device)
    _lib.call("vaa_build_token_index", query_start_loc.data_ptr(), seq_lens.data_ptr(), num_seqs,
              num_tokens, tok.data_ptr(), pos.data_ptr(), _lib.stream_handle(stream))
    return tok, pos


def build_slot_mapping(block_table: torch.Tensor, block_size: int, token_to_seq: torch.Tensor,
                       positions: torch.Tensor, stream=None) -> torch.Tensor:
    """int64 slot_mapping for (token_to_seq, positions) through block_table."""
    _require_gpu(block_table, token_to_seq, positions)
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous int32 2-D tensor")
    n = token_to_seq.numel()
    out = torch.empty(n, dtype=torch.int64, device=token_to_seq.device)
    _lib.call("vaa_build_slot_mapping", block_table.data_ptr(), block_table.shape[1], block_size,
              token_to_seq.data_ptr(), positions.data_ptr(), block_table.shape[0], n,
              out.data_ptr(), _lib.stream_handle(stream))
    return out


# ----------------------------------------------------------------- layer ops


def _layer_dtype(**named: torch.Tensor | None) -> int:
    """VAA_DTYPE_* code of a layer op's 16-bit tensors: all fp16 (the
    reference's type) or all bf16."""
    return ATTN_DTYPES[_attn_dtype(**named)]


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, *,
             residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
    """round16(x * rsqrt(mean(x^2) + eps) * w) [+ residual], rows of a 2-D view;
    fp16 or bf16."""
    _require_gpu(x, weight, residual, out)
    dt = _layer_dtype(x=x, weight=weight, residual=residual, out=out)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [num_tokens, hidden] with contiguous rows")
    t, h = x.shape
    if weight.numel() != h or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [hidden] tensor")
    if out is None:
        out = torch.empty_like(x)
    for r, n in ((out, "out"), (residual, "residual")):
        if r is not None and (r.shape != x.shape or r.stride(1) != 1 or r.dtype != x.dtype):
            raise ValueError(f"{n} must match x ([T, H], x's type, contiguous rows)")
    _lib.call("vaa_rmsnorm", x.data_ptr(), out.data_ptr(), weight.data_ptr(), _ptr(residual), t, h,
              x.stride(0), out.stride(0), residual.stride(0) if residual is not None else 0,
              float(eps), dt, _lib.stream_handle(stream))
    return out


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float, *,
                 out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """residual <- half(x + residual); out = rms_norm(residual) (vaa_add_rmsnorm).
    One pass for the reference layer's residual add, copy and norm
    (runner.py:1107-1130).  out may be x itself (the reference's in-place
    hidden buffer) but not residual.  fp16 or bf16."""
    _require_gpu(x, residual, weight, out)
    dt = _layer_dtype(x=x, residual=residual, weight=weight, out=out)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [num_tokens, hidden] with contiguous rows")
    t, h = x.shape
    if weight.numel() != h or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [hidden] tensor")
    if out is None:
        out = torch.empty_like(x)
    for r, n in ((out, "out"), (residual, "residual")):
        if r.shape != x.shape or r.stride(1) != 1 or r.dtype != x.dtype:
            raise ValueError(f"{n} must match x ([T, H], x's type, contiguous rows)")
    _lib.call("vaa_add_rmsnorm", x.data_ptr(), residual.data_ptr(), weight.data_ptr(),
              out.data_ptr(), t, h, x.stride(0), residual.stride(0), out.stride(0), float(eps),
              dt, _lib.stream_handle(stream))
    return out


def rope_cos_sin_cache(rotary_dim: int, max_position: int, base: float,
                       device: torch.device | str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables [max_position, rotary_dim // 2].

    Same construction as EngineRoPE._precompute_cache (elementwise.py:680-697):
    float32 numpy, inv_freq = 1 / base ** (arange(half) / half).
    """
    import numpy as np

    half = rotary_dim // 2
    inv_freq = 1.0 / (base ** (np.arange(0, half, dtype=np.float32) / half))
    positions = np.arange(max_position, dtype=np.float32)
    freqs = np.outer(positions, inv_freq)
    cos = torch.from_numpy(np.cos(freqs).astype(np.float32))
    sin = torch.from_numpy(np.sin(freqs).astype(np.float32))
    return cos.to(device), sin.to(device)


def rope_neox_(query: torch.Tensor, key: torch.Tensor | None, cos_cache: torch.Tensor,
               sin_cache: torch.Tensor, positions: torch.Tensor, *,
               rotary_dim: int | None = None, stream=None) -> None:
    """In-place NeoX rotation of query [T, H, D] and key [T, KV, D]; fp16 or bf16."""
    _require_gpu(query, key, cos_cache, sin_cache, positions)
    dt = _layer_dtype(query=query, key=key)
    if query.dim() != 3 or query.stride(2) != 1 or query.stride(1) != query.shape[2]:
        raise ValueError("query must be [T, H, D] with heads packed at stride D")
    if key is not None and (key.dim() != 3 or key.stride(2) != 1 or key.stride(1) != key.shape[2]
                            or key.shape[0] != query.shape[0]):
        raise ValueError("key must be [T, KV, D] with heads packed at stride D")
    if positions.dtype != torch.int32 or not positions.is_contiguous():
        raise ValueError("positions must be a contiguous int32 tensor")
    t, h, d = query.shape
    rot = rotary_dim or d
    if cos_cache.dtype != torch.float32 or cos_cache.dim() != 2 or cos_cache.shape[1] != rot // 2:
        raise ValueError("cos/sin caches must be fp32 [max_position, rotary_dim/2]")
    if not (cos_cache.is_contiguous() and sin_cache.is_contiguous()):
        raise ValueError("cos/sin caches must be contiguous")
    kv = key.shape[1] if key is not None else 0
    _lib.call("vaa_rope_neox", query.data_ptr(), _ptr(key), cos_cache.data_ptr(),
              sin_cache.data_ptr(), positions.data_ptr(), t, h, kv, d, rot, query.stride(0),
              key.stride(0) if key is not None else 0, cos_cache.shape[0], dt,
              _lib.stream_handle(stream))


def qkv_epilogue(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                 positions: torch.Tensor, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                 slot_mapping: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                 *, bias: torch.Tensor | None = None, rotary_dim: int | None = None,
                 layout: str = "kernel", stream=None) -> None:
    """Bias add + NeoX RoPE + KV write in one launch (vaa_qkv_epilogue).

    query [T, H, D], key/value [T, KV, D] (views into the planar QKV buffer
    are fine: heads packed at stride D, key and value sharing strides), all
    fp16 or all bf16 with the caches.  In place: q <- rope(q + b_q),
    k <- rope(k + b_k), v <- v + b_v; K and V also go to their cache slot
    (slot_mapping int32/int64, negative = padding).  bias: [H*D + 2*KV*D] in
    the same type, or None.  Equals bias add, rope_neox_ and kv_write_slots
    run in turn (engine/ops/qkv.py:391-416, elementwise.py:185-239,
    kv_write.py:118-156).
    """
    _require_gpu(query, key, value, positions, cos_cache, sin_cache, slot_mapping, key_cache,
                 value_cache, bias)
    _attn_dtype(query=query, key=key, value=value, key_cache=key_cache,
                value_cache=value_cache, bias=bias)
    for t, n in ((query, "query"), (key, "key"), (value, "value")):
        if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
            raise ValueError(f"{n} must be [tokens, heads, head_size] with heads packed")
    if key.shape != value.shape or key.stride() != value.stride():
        raise ValueError("key and value must have identical shapes and strides")
    T, H, D = query.shape
    if key.shape[0] != T or key.shape[2] != D:
        raise ValueError("query/key token count or head_size differ")
    if positions.dtype != torch.int32 or not positions.is_contiguous() or positions.numel() < T:
        raise ValueError("positions must be a contiguous int32 tensor with one entry per token")
    if slot_mapping.dtype not in (torch.int32, torch.int64) or not slot_mapping.is_contiguous() \
            or slot_mapping.numel() < T:
        raise ValueError("slot_mapping must be a contiguous int32/int64 tensor, one per token")
    rot = rotary_dim or D
    if cos_cache.dtype != torch.float32 or cos_cache.dim() != 2 or cos_cache.shape[1] != rot // 2 \
            or sin_cache.shape != cos_cache.shape or not cos_cache.is_contiguous() \
            or not sin_cache.is_contiguous():
        raise ValueError("cos/sin caches must be contiguous fp32 [max_position, rotary_dim/2]")
    KV = key.shape[1]
    if bias is not None and (bias.dim() != 1 or bias.numel() != (H + 2 * KV) * D
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous [{(H + 2 * KV) * D}] vector")
    p = make_params(key_cache=key_cache, value_cache=value_cache, layout=layout,
                    num_query_heads=H, scale=1.0, query=query, new_kv=key)
    if KV != p.num_kv_heads or D != p.head_size:
        raise ValueError(f"key shape {tuple(key.shape)} does not match the cache")
    itype = _lib.VAA_INDEX_I64 if slot_mapping.dtype == torch.int64 else _lib.VAA_INDEX_I32
    _lib.call("vaa_qkv_epilogue", ctypes.byref(p), query.data_ptr(), key.data_ptr(),
              value.data_ptr(), _ptr(bias), cos_cache.data_ptr(), sin_cache.data_ptr(), rot,
              cos_cache.shape[0], positions.data_ptr(), slot_mapping.data_ptr(), itype,
              key_cache.data_ptr(), value_cache.data_ptr(), T, _lib.stream_handle(stream))


TOPK_MAX_K = 256


_topk_ws = _GrowOnlyScratch()


def topk_workspace_size(num_tokens: int, vocab_size: int, k: int) -> int:
    """Bytes of workspace vaa_topk_logits needs (0 when a row fits one workgroup)."""
    n = ctypes.c_size_t(0)
    _lib.call("vaa_topk_workspace_size", num_tokens, vocab_size, k, ctypes.byref(n))
    return int(n.value)


def topk_logits(logits: torch.Tensor, k: int, *, indices: torch.Tensor | None = None,
                values: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                stream=None) -> tuple:
    """(indices int32 [T, k], values [T, k]): the k largest logits of each row,
    value-descending, ties by lower column (vaa_topk_logits; the reference's
    EngineTopK, engine/ops/topk.py:40-412).  logits: [T, V] fp16 or bf16 with
    a contiguous last dim.  Without `workspace` a grow-only per-device buffer
    is used, safe for calls ordered on one stream."""
    _require_gpu(logits, indices, values, workspace)
    if logits.dtype not in ATTN_DTYPES:
        raise ValueError(f"logits must be float16 or bfloat16, got {logits.dtype}")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [tokens, vocab] with a contiguous last dim")
    T, V = logits.shape
    if not 1 <= k <= min(TOPK_MAX_K, V):
        raise ValueError(f"k={k} must be in 1..{min(TOPK_MAX_K, V)}")
    if indices is None:
        indices = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    if values is None:
        values = torch.empty((T, k), dtype=logits.dtype, device=logits.device)
    if indices.dtype != torch.int32 or indices.shape != (T, k) or values.shape != (T, k) \
            or values.dtype != logits.dtype or indices.stride() != values.stride() \
            or indices.stride(1) != 1:
        raise ValueError("indices/values must be [T, k] (int32 / the logits' type), same strides")
    nbytes = topk_workspace_size(T, V, k)
    if workspace is None and nbytes > 0:
        workspace = _topk_ws.get(nbytes, logits.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _lib.call("vaa_topk_logits", logits.data_ptr(), T, V, logits.stride(0), k,
              indices.data_ptr(), values.data_ptr(), indices.stride(0), ws_ptr, ws_bytes,
              _lib.stream_handle(stream))
    return indices, values


def kv_stream_read(key_cache: torch.Tensor, value_cache: torch.Tensor,
                   block_table: torch.Tensor, seq_lens: torch.Tensor, *, layout: str = "kernel",
                   partition_size: int = 0, max_seq_len: int = 0,
                   sink: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Read-only stream of the K and V rows a paged decode of these tables
    reads (vaa_kv_stream_read): the measured ceiling beside the decode's HBM
    roofline.  With partition_size P > 0 (a multiple of 16; max_seq_len
    bounds seq_lens) each sequence is read in pieces of P tokens, one
    workgroup per piece, as the decode's fixed partitions cut it.  Returns
    sink, int32 [num_seqs, parts, num_kv_heads] (parts = ceil(max_seq_len / P),
    or 1): the XOR of every 32-bit word of the piece's K and V rows, read
    through block_table (rows in an invalid table entry skipped)."""
    _require_gpu(key_cache, value_cache, block_table, seq_lens, sink)
    _check_tables(block_table, seq_lens)
    num_seqs = seq_lens.numel()
    p = make_params(key_cache=key_cache, value_cache=value_cache, layout=layout,
                    num_query_heads=cache_strides(key_cache, layout).num_kv_heads, scale=1.0,
                    num_seqs=num_seqs, max_seq_len=max_seq_len,
                    max_blocks_per_seq=block_table.shape[1], partition_size=partition_size)
    parts = -(-max_seq_len // partition_size) if partition_size > 0 else 1
    if partition_size > 0 and max_seq_len <= 0:
        raise ValueError("partition_size needs max_seq_len > 0")
    if sink is None:
        sink = torch.empty((num_seqs, parts, p.num_kv_heads), dtype=torch.int32,
                           device=key_cache.device)
    if sink.dtype != torch.int32 or not sink.is_contiguous() \
            or sink.numel() < num_seqs * parts * p.num_kv_heads:
        raise ValueError("sink must be a contiguous int32 tensor of "
                         "num_seqs * parts * num_kv_heads entries")
    _lib.call("vaa_kv_stream_read", ctypes.byref(p), key_cache.data_ptr(), value_cache.data_ptr(),
              block_table.data_ptr(), seq_lens.data_ptr(), sink.data_ptr(),
              _lib.stream_handle(stream))
    return sink


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
    """out = round16(silu(float(gate)) * float(up)); 1-D or row-strided 2-D views;
    fp16 or bf16."""
    _require_gpu(gate, up, out)
    dt = _layer_dtype(gate=gate, up=up, out=out)
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    if out is None:
        out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    if out.shape != gate.shape:
        raise ValueError("out must match gate")
    if gate.is_contiguous() and up.is_contiguous() and out.is_contiguous():
        _lib.call("vaa_silu_mul", gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
                  dt, _lib.stream_handle(stream))
        return out
    if gate.dim() != 2:
        raise ValueError("non-contiguous gate/up/out must be 2-D row-strided views")
    g2, u2, o2 = gate, up, out
    for x in (g2, u2, o2):
        if x.stride(-1) != 1:
            raise ValueError("last dimension must be contiguous")
    _lib.call("vaa_silu_mul_2d", g2.data_ptr(), u2.data_ptr(), o2.data_ptr(), g2.shape[0],
              g2.shape[1], g2.stride(0), u2.stride(0), o2.stride(0), dt, _lib.stream_handle(stream))
    return out


def gate_up_silu(x: torch.Tensor, gate_weight: torch.Tensor,
                 up_weight: torch.Tensor | None = None, *, out: torch.Tensor | None = None,
                 stream=None) -> torch.Tensor:
    """SwiGLU of the gated-MLP up projection in one MFMA pass:
    out = round16(silu(x @ gate_weight.T) * (x @ up_weight.T)), both products
    accumulated in fp32 and never rounded before the epilogue.

    x is [T, H] with contiguous rows.  The weights are [I, H] (vLLM's
    gate_proj / up_proj layout, the reference's transpose_B GEMMs in
    engine/ops/mlp.py:300-330), or, with up_weight None, gate_weight is the
    fused gate_up_proj [2I, H] (gate rows first, mlp.py:267-296).  H must be a
    multiple of 64 and I of 128.  fp16 or bf16."""
    _require_gpu(x, gate_weight, up_weight, out)
    if up_weight is None:
        if gate_weight.dim() != 2 or gate_weight.shape[0] % 2:
            raise ValueError("a fused gate_up weight must be [2I, H]")
        i2 = gate_weight.shape[0] // 2
        gate_weight, up_weight = gate_weight[:i2], gate_weight[i2:]
    dt = _layer_dtype(x=x, gate_weight=gate_weight, up_weight=up_weight, out=out)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [num_tokens, hidden] with contiguous rows")
    t, h = x.shape
    if (gate_weight.dim() != 2 or gate_weight.shape != up_weight.shape
            or gate_weight.shape[1] != h):
        raise ValueError("gate and up weights must both be [I, H] with x's H")
    if (gate_weight.stride(1) != 1 or up_weight.stride(1) != 1
            or gate_weight.stride(0) != up_weight.stride(0)):
        raise ValueError("gate and up weights need contiguous rows at one row stride")
    inter = gate_weight.shape[0]
    if out is None:
        out = torch.empty((t, inter), dtype=x.dtype, device=x.device)
    if out.shape != (t, inter) or out.stride(1) != 1:
        raise ValueError("out must be [num_tokens, intermediate] with contiguous rows")
    _lib.call("vaa_gate_up_silu", x.data_ptr(), x.stride(0), gate_weight.data_ptr(),
              up_weight.data_ptr(), gate_weight.stride(0), out.data_ptr(), out.stride(0), t, h,
              inter, dt, _lib.stream_handle(stream))
    return out


def default_scale(head_size: int) -> float:
    return 1.0 / math.sqrt(head_size)
