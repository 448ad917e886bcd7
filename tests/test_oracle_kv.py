"""Pin the C oracle for KV writes and index rules (CPU only).

Checks: against the reference's own kv_write.c (compiled into oracle/_ref),
against the reference's known-answer test (tests/metal/test_kv_cache_layout.py:68-131),
against torch scatter (base_attn.py:308-342) for the vLLM layout, and against
integer invariants on exhaustive small tables.
"""
import numpy as np
import pytest
import torch

import oracle.kv as okv
from oracle import ref_torch


def _cache(nb, kv, bs, d, layout, seed):
    rs = np.random.RandomState(seed)
    shape = (nb, kv, bs, d) if layout == "kernel" else (nb, bs, kv, d)
    return rs.randn(*shape).astype(np.float16), rs.randn(*shape).astype(np.float16)


def test_known_answer_block3_offset5():
    """test_kv_cache_layout.py:68-131: write 1.5/2.5 at block 3, offset 5."""
    nb, kv, bs, d = 16, 4, 16, 128
    kc = np.zeros((nb, kv, bs, d), np.float16)
    vc = np.zeros_like(kc)
    key = np.full((1, kv, d), 1.5, np.float16)
    val = np.full((1, kv, d), 2.5, np.float16)
    okv.kv_write_slots(kc, vc, key, val, np.array([3 * bs + 5]))
    for h in range(kv):
        assert np.all(kc[3, h, 5] == 1.5) and np.all(vc[3, h, 5] == 2.5)
    assert np.count_nonzero(kc) == kv * d and np.count_nonzero(vc) == kv * d


def test_slots_match_reference_c():
    if okv.ref_lib() is None:
        pytest.skip("reference kv_write.c not built (no /root/reference and no oracle/_ref)")
    nb, kv, bs, d, T = 50, 8, 16, 128, 300
    kc, vc = _cache(nb, kv, bs, d, "kernel", 1)
    rs = np.random.RandomState(2)
    key = rs.randn(T, kv, d).astype(np.float16)
    val = rs.randn(T, kv, d).astype(np.float16)
    slots = rs.permutation(nb * bs)[:T].astype(np.int64)
    a_k, a_v = kc.copy(), vc.copy()
    okv.kv_write_slots(a_k, a_v, key, val, slots)
    b_k, b_v = kc.copy(), vc.copy()
    okv.ref_write_kv_batch(b_k, b_v, key, val, slots // bs, slots % bs, kv * bs * d, bs * d, d)
    assert np.array_equal(a_k.view(np.uint16), b_k.view(np.uint16))
    assert np.array_equal(a_v.view(np.uint16), b_v.view(np.uint16))
    # single-token entry of the reference
    c_k, c_v = kc.copy(), vc.copy()
    for t in range(5):
        okv.ref_write_kv_single(c_k, c_v, key[t], val[t], slots[t] // bs, slots[t] % bs,
                                kv * bs * d, bs * d, d)
    e_k, e_v = kc.copy(), vc.copy()
    okv.kv_write_slots(e_k, e_v, key[:5], val[:5], slots[:5])
    assert np.array_equal(c_k.view(np.uint16), e_k.view(np.uint16))


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_write_kv_batch_guard(layout):
    """oracle_write_kv_batch: in-range tokens are the reference's kv_write.c
    byte for byte (on either layout's strides); a token with an offset at or
    past the block size, a negative offset or a block outside the pool
    changes nothing, not even the neighbouring block its row would reach."""
    nb, kv, bs, d, T = 12, 4, 16, 64, 40
    kc, vc = _cache(nb, kv, bs, d, layout, 11)
    sb, sh, st = okv.cache_strides(kc, layout)
    rs = np.random.RandomState(12)
    key = rs.randn(T, kv, d).astype(np.float16)
    val = rs.randn(T, kv, d).astype(np.float16)
    slots = rs.permutation(nb * bs)[:T].astype(np.int64)
    bids, offs = slots // bs, slots % bs
    a_k, a_v = kc.copy(), vc.copy()
    okv.write_kv_batch(a_k, a_v, key, val, bids, offs, sb, sh, st, nb)
    e_k, e_v = kc.copy(), vc.copy()
    okv.kv_write_slots(e_k, e_v, key, val, slots, layout)
    assert np.array_equal(a_k.view(np.uint16), e_k.view(np.uint16))
    assert np.array_equal(a_v.view(np.uint16), e_v.view(np.uint16))
    if okv.ref_lib() is not None:
        r_k, r_v = kc.copy(), vc.copy()
        okv.ref_write_kv_batch(r_k, r_v, key, val, bids, offs, sb, sh, st)
        assert np.array_equal(a_k.view(np.uint16), r_k.view(np.uint16))
    # Bad indices: a middle block with offset bs and bs + 3 (the reference
    # would write into block 6), offset -1, block -1 and block nb.
    bad_b = np.array([5, 5, 5, -1, nb], dtype=np.int64)
    bad_o = np.array([bs, bs + 3, -1, 0, 0], dtype=np.int64)
    b_k, b_v = kc.copy(), vc.copy()
    okv.write_kv_batch(b_k, b_v, key[:5], val[:5], bad_b, bad_o, sb, sh, st, nb)
    assert np.array_equal(b_k.view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(b_v.view(np.uint16), vc.view(np.uint16))
    # The last valid offset still writes, and only its own block.
    c_k, c_v = kc.copy(), vc.copy()
    okv.write_kv_batch(c_k, c_v, key[:1], val[:1], np.array([5]), np.array([bs - 1]), sb, sh, st,
                       nb)
    changed = np.nonzero((c_k.view(np.uint16) != kc.view(np.uint16)).reshape(nb, -1).any(1))[0]
    assert changed.tolist() == [5]


def test_slots_vllm_layout_match_torch_scatter():
    nb, kv, bs, d, T = 20, 2, 16, 64, 100
    kc, vc = _cache(nb, kv, bs, d, "vllm", 3)
    rs = np.random.RandomState(4)
    key = rs.randn(T, kv, d).astype(np.float16)
    val = rs.randn(T, kv, d).astype(np.float16)
    slots = rs.permutation(nb * bs)[:T].astype(np.int64)
    slots[::9] = -1
    a_k, a_v = kc.copy(), vc.copy()
    okv.kv_write_slots(a_k, a_v, key, val, slots, "vllm")
    tk, tv = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    ref_torch.update_kv_cache_scatter(torch.from_numpy(key), torch.from_numpy(val), tk, tv,
                                      torch.from_numpy(slots))
    assert np.array_equal(a_k.view(np.uint16), tk.numpy().view(np.uint16))
    assert np.array_equal(a_v.view(np.uint16), tv.numpy().view(np.uint16))


def test_slot_write_is_a_permutation_invariant():
    """Every written slot holds its token; every other slot is untouched."""
    nb, kv, bs, d = 8, 2, 16, 32
    kc, vc = _cache(nb, kv, bs, d, "kernel", 5)
    rs = np.random.RandomState(6)
    slots = rs.permutation(nb * bs)[:70].astype(np.int64)
    key = rs.randn(70, kv, d).astype(np.float16)
    a_k, a_v = kc.copy(), vc.copy()
    okv.kv_write_slots(a_k, a_v, key, key, slots)
    touched = np.zeros((nb, bs), bool)
    for t, s in enumerate(slots):
        assert np.array_equal(a_k[s // bs, :, s % bs], key[t])
        touched[s // bs, s % bs] = True
    for b in range(nb):
        for o in range(bs):
            if not touched[b, o]:
                assert np.array_equal(a_k[b, :, o].view(np.uint16), kc[b, :, o].view(np.uint16))


def test_decode_write_equals_slot_write():
    """kv_write_decode == kv_write_slots with slot = bt[s, (L-1)//bs]*bs + (L-1)%bs."""
    nb, kv, bs, d, S, maxb = 64, 4, 16, 64, 9, 6
    kc, vc = _cache(nb, kv, bs, d, "kernel", 7)
    rs = np.random.RandomState(8)
    bt = rs.permutation(nb)[:S * maxb].reshape(S, maxb).astype(np.int32)
    lens = rs.randint(1, maxb * bs + 1, S).astype(np.int32)
    key = rs.randn(S, kv, d).astype(np.float16)
    val = rs.randn(S, kv, d).astype(np.float16)
    a_k, a_v = kc.copy(), vc.copy()
    okv.kv_write_decode(a_k, a_v, key, val, bt, lens)
    slots = np.array([bt[s, (L - 1) // bs] * bs + (L - 1) % bs for s, L in enumerate(lens)])
    b_k, b_v = kc.copy(), vc.copy()
    okv.kv_write_slots(b_k, b_v, key, val, slots)
    assert np.array_equal(a_k.view(np.uint16), b_k.view(np.uint16))
    assert np.array_equal(a_v.view(np.uint16), b_v.view(np.uint16))


def test_decode_write_guards():
    nb, kv, bs, d = 8, 1, 16, 32
    kc, vc = _cache(nb, kv, bs, d, "kernel", 9)
    bt = np.array([[0, 1], [2, -1], [3, 4]], np.int32)
    lens = np.array([0, 20, 40], np.int32)  # L<=0; invalid block; past the table
    key = np.ones((3, kv, d), np.float16)
    a_k, a_v = kc.copy(), vc.copy()
    okv.kv_write_decode(a_k, a_v, key, key, bt, lens)
    assert np.array_equal(a_k.view(np.uint16), kc.view(np.uint16))


def test_token_index_exhaustive_small():
    """token_to_seq / positions == repeat_interleave rule for every small qsl."""
    rs = np.random.RandomState(10)
    for _ in range(200):
        S = rs.randint(1, 6)
        qlens = rs.randint(0, 5, S)
        qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
        seq_lens = (qlens + rs.randint(0, 30, S)).astype(np.int32)
        T = int(qsl[-1]) + rs.randint(0, 3)
        tok, pos = okv.token_index(qsl, seq_lens, T)
        rt = torch.repeat_interleave(torch.arange(S, dtype=torch.int32),
                                     torch.from_numpy(qlens.astype(np.int64))).numpy()
        assert np.array_equal(tok[:qsl[-1]], rt)
        assert np.all(tok[qsl[-1]:] == -1) and np.all(pos[qsl[-1]:] == -1)
        for s in range(S):
            assert np.array_equal(pos[qsl[s]:qsl[s + 1]],
                                  np.arange(seq_lens[s] - qlens[s], seq_lens[s]))


def test_slot_mapping_rule_and_fallback():
    bs = 16
    bt = np.array([[7, 2, -1, -1], [5, -1, -1, -1]], np.int32)
    tok = np.array([0, 0, 0, 1, 1, -1, 3], np.int32)
    pos = np.array([0, 17, 40, 15, 16, 3, 3], np.int32)
    slots = okv.slot_mapping(bt, bs, tok, pos)
    # block list too short -> slot = pos (apple_model_runner.py:1220-1221)
    assert slots.tolist() == [7 * 16, 2 * 16 + 1, 40, 5 * 16 + 15, 16, -1, -1]
