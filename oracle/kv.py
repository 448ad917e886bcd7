"""ORACLE (test infrastructure): ctypes access to kv_oracle.c and to the
reference's kv_write.c compiled from /root/reference into oracle/_ref.

Functions and the reference lines they follow
  kv_write_slots     vllm_apple/engine/ops/kv_write.py:118-156 (slot<0 skipped)
  kv_write_decode    paged_attention_fused.metal:55-101, kv_write.py:86-99 guards
  token_index        vllm_apple/engine/runner.py:526-546, apple_model_runner.py:1188-1200
  slot_mapping       vllm_apple/v1/worker/apple_model_runner.py:1202-1249
  write_kv_batch     kv_write.c:33-78 with the library's index guard (block id
                     outside the pool, offset whose write leaves the block:
                     skipped)
  ref_write_kv_batch the reference's metal_write_kv_batch itself (kv_write.c:33-78)
Pinned by tests/test_oracle_kv.py.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "liboracle.so"
REF_SO = HERE / "_ref" / "libkv_write_ref.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64

_oracle = None
_ref = None


def build(force: bool = False) -> None:
    """make -C oracle (C restatement, plus _ref when /root/reference exists)."""
    if force or not ORACLE_SO.exists() or not REF_SO.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def lib() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_SO.exists():
            build()
        l = ctypes.CDLL(str(ORACLE_SO))
        l.oracle_kv_write_slots.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I64, _I64, _I64, _I64, _I64, _I64]
        l.oracle_kv_write_decode.argtypes = [_P, _P, _P, _I, _P, _I, _P, _P, _I, _I, _I, _I64, _I64, _I64, _I64, _I64, _I64]
        l.oracle_token_index.argtypes = [_P, _P, _I, _I, _P, _P]
        l.oracle_slot_mapping.argtypes = [_P, _I, _I, _P, _P, _I, _I, _P]
        l.oracle_write_kv_batch.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I64, _I64,
                                            _I64, _I64]
        for f in (l.oracle_kv_write_slots, l.oracle_kv_write_decode, l.oracle_token_index,
                  l.oracle_slot_mapping, l.oracle_write_kv_batch):
            f.restype = None
        _oracle = l
    return _oracle


def ref_lib() -> ctypes.CDLL | None:
    """The reference's kv_write.c built by oracle/Makefile, or None if absent."""
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            try:
                build()
            except Exception:
                return None
        if not REF_SO.exists():
            return None
        l = ctypes.CDLL(str(REF_SO))
        l.metal_write_kv_batch.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]
        l.metal_write_kv_batch.restype = None
        l.metal_write_kv_single.argtypes = [_P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I]
        l.metal_write_kv_single.restype = None
        _ref = l
    return _ref


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"] or a.ndim == 0
    return a.ctypes.data


def _u16(a: np.ndarray) -> np.ndarray:
    return a.view(np.uint16)


def cache_strides(cache: np.ndarray, layout: str) -> tuple[int, int, int]:
    """Element strides (block, head, token) of a contiguous cache array."""
    s = [x // cache.itemsize for x in cache.strides]
    if layout == "kernel":   # [nb, KV, bs, D]
        return s[0], s[1], s[2]
    if layout == "vllm":     # [nb, bs, KV, D]
        return s[0], s[2], s[1]
    raise ValueError(layout)


def kv_write_slots(k_cache: np.ndarray, v_cache: np.ndarray, key: np.ndarray,
                   value: np.ndarray, slots: np.ndarray, layout: str = "kernel") -> None:
    """In-place scatter of key/value [T, KV, D] fp16 into the caches."""
    assert k_cache.dtype == np.float16 and key.dtype == np.float16
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    T, KV, D = key.shape
    sb, sh, st = cache_strides(k_cache, layout)
    bs = k_cache.shape[2] if layout == "kernel" else k_cache.shape[1]
    lib().oracle_kv_write_slots(_p(k_cache), _p(v_cache), _p(slots), _p(key), _p(value), T, KV,
                                D, bs, k_cache.shape[0], sb, sh, st, KV * D, D)


def kv_write_decode(k_cache: np.ndarray, v_cache: np.ndarray, key: np.ndarray,
                    value: np.ndarray, block_table: np.ndarray, seq_lens: np.ndarray,
                    layout: str = "kernel") -> None:
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    S = sl.shape[0]
    _, KV, D = key.shape
    sb, sh, st = cache_strides(k_cache, layout)
    bs = k_cache.shape[2] if layout == "kernel" else k_cache.shape[1]
    lib().oracle_kv_write_decode(_p(k_cache), _p(v_cache), _p(bt), bt.shape[1], _p(sl), S,
                                 _p(key), _p(value), KV, D, bs, k_cache.shape[0], sb, sh, st,
                                 KV * D, D)


def token_index(query_start_loc: np.ndarray, seq_lens: np.ndarray,
                num_tokens: int) -> tuple[np.ndarray, np.ndarray]:
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    tok = np.empty(num_tokens, dtype=np.int32)
    pos = np.empty(num_tokens, dtype=np.int32)
    lib().oracle_token_index(_p(qsl), _p(sl), qsl.shape[0] - 1, num_tokens, _p(tok), _p(pos))
    return tok, pos


def slot_mapping(block_table: np.ndarray, block_size: int, token_to_seq: np.ndarray,
                 positions: np.ndarray) -> np.ndarray:
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    tok = np.ascontiguousarray(token_to_seq, dtype=np.int32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.empty(tok.shape[0], dtype=np.int64)
    lib().oracle_slot_mapping(_p(bt), bt.shape[1], block_size, _p(tok), _p(pos), bt.shape[0],
                              tok.shape[0], _p(out))
    return out


def write_kv_batch(k_cache: np.ndarray, v_cache: np.ndarray, key: np.ndarray,
                   value: np.ndarray, block_ids: np.ndarray, token_offsets: np.ndarray,
                   stride_block: int, stride_head: int, stride_token: int,
                   num_blocks: int) -> None:
    """Guarded metal_write_kv_batch on host arrays (see oracle_write_kv_batch)."""
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    bids = np.ascontiguousarray(block_ids, dtype=np.int64)
    offs = np.ascontiguousarray(token_offsets, dtype=np.int64)
    T, KV, D = key.shape
    lib().oracle_write_kv_batch(_p(k_cache), _p(v_cache), _p(key), _p(value), _p(bids), _p(offs),
                                T, KV, D, stride_block, stride_head, stride_token, num_blocks)


def ref_write_kv_batch(k_cache: np.ndarray, v_cache: np.ndarray, key: np.ndarray,
                       value: np.ndarray, block_ids: np.ndarray, token_offsets: np.ndarray,
                       stride_block: int, stride_head: int, stride_token: int) -> None:
    """Call the reference's metal_write_kv_batch (kv_write.c:33-78) on host arrays."""
    l = ref_lib()
    if l is None:
        raise RuntimeError("oracle/_ref/libkv_write_ref.so not available")
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    bids = np.ascontiguousarray(block_ids, dtype=np.int64)
    offs = np.ascontiguousarray(token_offsets, dtype=np.int64)
    T, KV, D = key.shape
    l.metal_write_kv_batch(_p(k_cache), _p(v_cache), _p(key), _p(value), _p(bids), _p(offs), T,
                           KV, D, stride_block, stride_head, stride_token)


def ref_write_kv_single(k_cache: np.ndarray, v_cache: np.ndarray, key: np.ndarray,
                        value: np.ndarray, block_id: int, token_offset: int,
                        stride_block: int, stride_head: int, stride_token: int) -> None:
    l = ref_lib()
    if l is None:
        raise RuntimeError("oracle/_ref/libkv_write_ref.so not available")
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    KV, D = key.shape[-2:]
    l.metal_write_kv_single(_p(k_cache), _p(v_cache), _p(key), _p(value), int(block_id),
                            int(token_offset), KV, D, stride_block, stride_head, stride_token)
