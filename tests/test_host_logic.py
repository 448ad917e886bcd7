"""Host-side logic on the CPU: validation rules, strides, parameter packing,
metadata construction and the backend's static surface and error conventions.

Cases follow the reference's own unit tests (tests/unit/test_engine.py:320-423)
and the error behaviour of metal_attn.py / engine/kv_cache.py.
"""
import struct
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from vllm_apple_amd import backend, indexing
from vllm_apple_amd.engine.attention import (FusedAttentionParams, PagedAttentionOp,
                                             PagedAttentionParams)
from vllm_apple_amd.engine.kv_write import KVWriteParams
from vllm_apple_amd.kv_cache import HipKVCache, KVCacheDescriptor


def _cache(num_blocks=100, block_size=16):
    return HipKVCache(KVCacheDescriptor(num_blocks, block_size, 2, 64, 1), device="cpu")


# -- KV cache validation (engine/kv_cache.py:300-420, test_engine.py:343-423) --------
def test_valid_slot_mapping():
    _cache().validate_slot_mapping(np.array([0, 1, 15, 100, 1599], dtype=np.int32))


def test_invalid_slot_oob():
    with pytest.raises(ValueError, match="Slot mapping contains index 2000"):
        _cache().validate_slot_mapping(np.array([0, 1, 2000], dtype=np.int32))


def test_negative_one_slot_allowed_and_minus_two_rejected():
    c = _cache()
    c.validate_slot_mapping(np.array([0, -1, 10, -1, 20], dtype=np.int32))
    with pytest.raises(ValueError, match="invalid index -2"):
        c.validate_slot_mapping(np.array([0, -2, 10], dtype=np.int32))


def test_slot_mapping_torch_and_empty():
    c = _cache()
    c.validate_slot_mapping(torch.tensor([0, 10, 100], dtype=torch.int32))
    c.validate_slot_mapping(np.array([], dtype=np.int32))


def test_block_table_validation():
    c = _cache(num_blocks=8)
    c.validate_block_table(np.array([[0, 7, -1]], dtype=np.int32))
    with pytest.raises(ValueError, match="Block table contains index 8 >= num_blocks 8"):
        c.validate_block_table(np.array([[0, 8]], dtype=np.int32))
    with pytest.raises(ValueError, match="invalid index -3"):
        c.validate_block_table(torch.tensor([[0, -3]], dtype=torch.int32))


def test_descriptor_rules():
    with pytest.raises(ValueError, match="head_size must be 32/64/96/128"):
        KVCacheDescriptor(4, 16, 2, 80, 1)
    with pytest.raises(ValueError, match="num_blocks must be >= 1"):
        KVCacheDescriptor(0, 16, 2, 64, 1)
    d = KVCacheDescriptor(10, 16, 8, 128, 2)
    assert d.block_size_bytes == 8 * 16 * 128 * 2 * 2
    assert d.total_cache_bytes == d.block_size_bytes * 10 * 2
    # bf16 blocks are as large as fp16 ones, and the sizes equal what
    # HipKVCache allocates (the reference's formula counted 4 bytes for
    # anything not fp16).
    b = KVCacheDescriptor(10, 16, 8, 128, 2, dtype=torch.bfloat16)
    assert b.block_size_bytes == d.block_size_bytes
    c = HipKVCache(b, device="cpu", zero=False)
    k, v = c.get_buffers(0)
    assert b.total_cache_bytes == c._storage.numel() * c._storage.element_size()
    assert b.block_size_bytes == (k[0].numel() + v[0].numel()) * k.element_size()


def test_strides_match_reference():
    """test_engine.py:320-341."""
    c = HipKVCache(KVCacheDescriptor(4, 16, 8, 128, 1), device="cpu")
    assert c.strides["block"] == 16384 and c.strides["head"] == 2048 and c.strides["token"] == 128
    k, v = c.get_buffers(0)
    assert k.shape == (4, 8, 16, 128)
    assert k.stride()[:3] == (16384, 2048, 128)
    assert c.get_slot_offset(37) == (2, 5)
    assert c.get_element_offset(2, 3, 5) == 2 * 16384 + 3 * 2048 + 5 * 128
    op = PagedAttentionOp(None, 8, 32, 128, 16)
    assert (op.new_kv_stride_token, op.new_kv_stride_head) == (1024, 128)


# -- parameter structs keep the reference packing ------------------------------------
def test_param_struct_packing():
    op = PagedAttentionOp(None, num_kv_heads=8, num_query_heads=32, head_size=128,
                          block_size=16)
    fp = op.fused_params(num_seqs=4, max_seq_len=100, max_blocks_per_seq=7)
    raw = fp.to_bytes()
    assert len(raw) == 4 + 20 * 4
    vals = struct.unpack("f" + "I" * 20, raw)
    assert vals[1:9] == (4, 100, 7, 128, 16, 8, 32, 4)
    assert abs(vals[0] - 1 / 128 ** 0.5) < 1e-7
    pp = PagedAttentionParams(*([1.0] + [2] * 18))
    assert len(pp.to_bytes()) == 4 + 18 * 4
    kp = KVWriteParams(1, 2, 3, 4, 5, 6, 7, 8, 9)
    assert struct.unpack("I" * 9, kp.to_bytes()) == (1, 2, 3, 4, 5, 6, 7, 8, 9)
    assert isinstance(fp, FusedAttentionParams)


# -- index rules (runner.py:526-683, apple_model_runner.py:1188-1278) ---------------
def test_token_to_seq_rules():
    tok = indexing.derive_token_to_seq(torch.tensor([0, 3, 3, 5]), 3, 5)
    assert tok.tolist() == [0, 0, 0, 2, 2]
    with pytest.raises(ValueError, match="expected 4"):
        indexing.derive_token_to_seq(torch.tensor([0, 3, 5]), 3, 5)
    with pytest.raises(ValueError, match="must be 0"):
        indexing.derive_token_to_seq(torch.tensor([1, 3, 5]), 2, 5)
    with pytest.raises(ValueError, match="must equal num_tokens"):
        indexing.derive_token_to_seq(torch.tensor([0, 3, 4]), 2, 5)
    with pytest.raises(ValueError, match="non-decreasing"):
        indexing.derive_token_to_seq(torch.tensor([0, 4, 3, 5]), 3, 5)
    with pytest.raises(ValueError, match="requires query_start_locs"):
        indexing.derive_token_to_seq(None, 1, 1)


def test_positions_and_capacity():
    pos = indexing.positions_from_lengths(torch.tensor([0, 1, 4]), torch.tensor([513, 10]))
    assert pos.tolist() == [512, 7, 8, 9]
    bt = torch.zeros((2, 4), dtype=torch.int32)
    assert indexing.check_block_capacity(torch.tensor([64, 10]), bt, 16) == 64
    with pytest.raises(ValueError, match="exceeds block_table capacity"):
        indexing.check_block_capacity(torch.tensor([65]), bt[:1], 16)


def test_slot_mapping_and_block_table_from_lists():
    slots = indexing.slot_mapping_from_blocks([[7, 2], [5]], [[0, 17, 40], [15, 16]], 16)
    assert slots.tolist() == [112, 33, 40, 95, 16]
    bt = indexing.block_table_from_lists([[7, 2], [], [5]])
    assert bt.tolist() == [[7, 2], [-1, -1], [5, -1]]


# -- backend static surface (metal_attn.py:124-199) ----------------------------------
def test_backend_surface():
    B = backend.HipAttentionBackend
    assert B.accept_output_buffer is True
    assert B.get_supported_dtypes() == [torch.float16, torch.bfloat16]
    assert B.get_supported_head_sizes() == [32, 64, 96, 128]
    assert B.get_kv_cache_shape(10, 16, 8, 128) == (2, 10, 16, 8, 128)
    assert B.use_cascade_attention() is False
    assert B.get_kv_cache_device() == "cuda"
    assert B.get_impl_cls() is backend.HipAttentionImpl
    assert B.get_builder_cls() is backend.HipAttentionMetadataBuilder
    assert B.supports_attn_type(backend.AttentionType.DECODER)
    assert not B.supports_attn_type(backend.AttentionType.ENCODER_DECODER)


def _impl(**kw):
    args = dict(num_heads=32, head_size=128, scale=0.1, num_kv_heads=8, alibi_slopes=None,
                sliding_window=None, kv_cache_dtype="auto")
    args.update(kw)
    return backend.HipAttentionImpl(**args)


def test_sliding_window_rules(monkeypatch):
    """A window is accepted only where attending over the whole context gives
    the same result: no context longer than the window.  With max_model_len
    known, a shorter window is refused at construction; without it, each
    step's longest context is checked in forward."""
    monkeypatch.setattr(backend, "_max_model_len", lambda: 4096)
    with pytest.raises(NotImplementedError, match="sliding_window"):
        _impl(sliding_window=2048)
    impl = _impl(sliding_window=4096)
    assert impl.sliding_window == (-1, -1) and impl._window is None
    monkeypatch.setattr(backend, "_max_model_len", lambda: None)
    impl = _impl(sliding_window=4096)
    assert impl._window == 4096
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    out = torch.ones_like(q)
    md = backend.HipAttentionMetadata(
        num_actual_tokens=2, max_query_len=1, query_start_loc=torch.tensor([0, 1, 2]),
        max_seq_len=4097, seq_lens=torch.tensor([4097, 10]), block_table=torch.zeros(2, 1),
        slot_mapping=torch.zeros(2), num_decode_tokens=2)
    with pytest.raises(NotImplementedError, match="exceeds sliding_window=4096"):
        impl.forward(None, q, q[:, :8], q[:, :8], None, md, output=out)
    with pytest.raises(NotImplementedError):
        _impl(sliding_window=0)


def test_impl_error_conventions():
    with pytest.raises(NotImplementedError, match="FP8"):
        _impl(kv_cache_dtype="fp8")
    with pytest.raises(ValueError):
        _impl(head_size=80)
    impl = _impl()
    assert impl.sliding_window == (-1, -1)
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    out = torch.ones_like(q)
    with pytest.raises(AssertionError):
        impl.forward(None, q, q[:, :8], q[:, :8], None, None, output=None)
    with pytest.raises(NotImplementedError):
        impl.forward(None, q, q[:, :8], q[:, :8], None, None, output=out, output_scale=q)
    # attn_metadata None (warm-up): output returned untouched
    assert impl.forward(None, q, q[:, :8], q[:, :8], None, None, output=out) is out
    assert torch.all(out == 1)


def test_split_decodes_and_prefills():
    f = backend.split_decodes_and_prefills
    assert f([0, 1, 2, 3]) == (3, 0, 3, 0)
    assert f([0, 1, 2, 10, 12]) == (2, 2, 2, 10)
    assert f([0, 5, 9]) == (0, 2, 0, 9)
    assert f([0]) == (0, 0, 0, 0)


def test_split_decodes_and_prefills_require_uniform():
    """Hand-worked cases of vLLM's rule with require_uniform=True, the form the
    reference's builder calls (metal_attn.py:302-308).  Decodes are the leading
    requests whose query length equals the first one's."""
    f = backend.split_decodes_and_prefills
    # Every query at most the threshold of 1: all decodes, whatever the lengths.
    assert f([0, 1, 1, 2], 1, require_uniform=True) == (3, 0, 2, 0)
    # A zero-length request after decodes: a prefill under the uniform rule
    # (its length differs from the first), a decode under the plain one.
    assert f([0, 1, 2, 2, 7], 1, require_uniform=True) == (2, 2, 2, 5)
    assert f([0, 1, 2, 2, 7], 1) == (3, 1, 2, 5)
    # Threshold 4 (speculative decode): uniform keeps only equal lengths.
    assert f([0, 3, 6, 8, 20], 4, require_uniform=True) == (2, 2, 6, 14)
    assert f([0, 3, 6, 8, 20], 4) == (3, 1, 8, 12)
    # With a threshold above 1, all-short batches still split on unequal
    # lengths under the uniform rule.
    assert f([0, 3, 6, 8], 4, require_uniform=True) == (2, 1, 6, 2)
    assert f([0, 3, 6, 8], 4) == (3, 0, 8, 0)
    # First request longer than the threshold: no decodes.
    assert f([0, 9, 10], 4, require_uniform=True) == (0, 2, 0, 10)
    # Mixed 1-token decodes then prefills: both rules agree at threshold 1.
    for qsl in ([0, 1, 2, 10, 12], [0, 1, 2, 3], [0, 5, 9]):
        assert f(qsl, 1, require_uniform=True) == f(qsl, 1)


def test_metadata_builder():
    cm = SimpleNamespace(num_actual_tokens=12, max_query_len=8,
                         query_start_loc=torch.tensor([0, 1, 2, 10, 12], dtype=torch.int32),
                         query_start_loc_cpu=torch.tensor([0, 1, 2, 10, 12]),
                         max_seq_len=900, seq_lens=torch.tensor([5, 900, 8, 2]),
                         seq_lens_cpu=torch.tensor([5, 900, 8, 2]),
                         block_table_tensor=torch.zeros(4, 57, dtype=torch.int32),
                         slot_mapping=torch.zeros(12, dtype=torch.int64), causal=True)
    md = backend.HipAttentionMetadataBuilder().build(0, cm)
    assert md.num_decode_tokens == 2 and md.num_actual_tokens == 12
    assert md.query_start_loc_cpu == [0, 1, 2, 10, 12]
    assert md.seq_lens_cpu == [5, 900, 8, 2]


def test_ops_reject_cpu_tensors():
    """No CPU fallback: the HIP path refuses host tensors loudly."""
    from vllm_apple_amd import kernels

    x = torch.zeros(4, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="no CPU fallback"):
        kernels.rms_norm(x, torch.ones(128, dtype=torch.float16), 1e-6)


def test_partition_choice_small_batches():
    """Split-K choices the cost model makes where the launch leaves CUs idle,
    each the fastest (or within 6 %) of the partitions measured on MI355X
    (kernels.py, _LONE_WG_SPEEDUP), and the headline / ragged choices
    unchanged."""
    from vllm_apple_amd import kernels as K

    K._partition_cache.clear()
    assert K.choose_partition_size([8192], 8, 256) == 256
    assert K.choose_partition_size([4096] * 2, 8, 256) == 256
    assert K.choose_partition_size([2048] * 8, 8, 256) == 512
    assert K.choose_partition_size([1024] * 4, 8, 256) == 128
    assert K.choose_partition_size([4096] * 16, 8, 256) == 1024
    assert K.choose_partition_size([32768], 8, 256) == 1024
    assert K.choose_partition_size([162, 125, 444, 341], 2, 256) >= 444  # C1: unsplit
    assert K.choose_partition_size([8192] * 32, 8, 256) == 8192          # headline: unsplit
    assert K.choose_partition_size(list(range(1024, 8192, 224)), 8, 256) == K.PARTITION_BALANCED


def test_prefill_split_choice():
    """Key splits only for unequal contexts: C3 (four equal 2560-token
    contexts) stays whole; C5's prefill chunks (256 tokens over contexts up to
    16k, one of them far longer than the per-slot share) are split into pieces
    of a multiple of 1024 keys, shorter than the longest context."""
    from vllm_apple_amd import kernels as K

    K._prefill_split_cache.clear()
    assert K.choose_prefill_split([2560] * 4, [512] * 4, 8, 32, 256) == 0
    c5 = [16000, 600, 900, 2000, 3000, 1200, 800, 700]
    sp = K.choose_prefill_split(c5, [256] * 8, 8, 32, 256)
    assert sp > 0 and sp % 1024 == 0 and sp < 16000
    # decodes (query length 0 here) and empty sequences carry no prefill work
    assert K.choose_prefill_split([16000, 500], [0, 0], 8, 32, 256) == 0
    # short contexts never split
    assert K.choose_prefill_split([2000, 100], [64, 64], 8, 32, 256) == 0


def test_prefill_split_workspace_is_bounded():
    """One 256-token chunk at a 128k context beside 31 short 248-token
    prefills: the share-based piece (10240 keys, 13 pieces over 7944 tokens)
    would need 1.72 GB of partials.  The pieces grow until the workspace the
    kernel asks for (counted over the longest prefill context) fits the cap."""
    from vllm_apple_amd import _lib, kernels as K

    K._prefill_split_cache.clear()
    ctx = [131072] + [248] * 31
    ql = [256] + [248] * 31
    cap = K.PREFILL_SPLIT_MAX_WORKSPACE
    sp = K.choose_prefill_split(ctx, ql, 8, 32, 256)
    assert sp > 0 and sp % 1024 == 0
    tokens = sum(ql)
    pieces = -(-131072 // sp)
    need = tokens * 32 * pieces * 130 * 4
    assert pieces >= 2 and need <= cap
    # The library's own sizing agrees when max_seq_len is the longest prefill
    # context.
    p = _lib.VaaAttnParams()
    p.head_size, p.block_size, p.num_kv_heads, p.num_query_heads = 128, 16, 8, 32
    p.queries_per_kv, p.num_seqs, p.max_blocks_per_seq, p.num_blocks = 4, 32, 8192, 1 << 16
    p.max_seq_len = 131072
    assert K.prefill_workspace_size(p, tokens, sp) == need
    # Without the cap the piece count would be the share-based one.
    K._prefill_split_cache.clear()
    free = K.choose_prefill_split(ctx, ql, 8, 32, 256, max_workspace_bytes=1 << 40)
    assert free < sp and tokens * 32 * -(-131072 // free) * 130 * 4 > cap
    # A cap too small for two pieces drops the split.
    K._prefill_split_cache.clear()
    assert K.choose_prefill_split(ctx, ql, 8, 32, 256, max_workspace_bytes=1 << 20) == 0
