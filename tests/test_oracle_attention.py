"""Pin the attention oracle (CPU only).

decode/prefill (fp64 numpy) are checked against: torch SDPA on the gathered
rows (the library routine of the reference's PyTorch path), the token-serial
fp32 loop that mirrors the Metal kernel, the reference's known-answer test
(seq_len 1 -> V, tests/metal/test_metal_kernels.py:380-438), closed forms, and
the reference torch path restatement (oracle.ref_torch).
A plausible mistake -- a wrong GQA head map, a missing scale, an off-by-one
context, a transposed layout -- fails at least one of these (see the planted
mistakes at the end).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.attention as oat
from oracle import ref_torch

from helpers import assert_close


def _paged(S, H, KV, D, lens, bs=16, layout="kernel", seed=0):
    rs = np.random.RandomState(seed)
    nblk = [(L + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 3
    maxb = max(max(nblk), 1)
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = rs.randn(*shape).astype(np.float16)
    vc = rs.randn(*shape).astype(np.float16)
    perm = rs.permutation(nb).astype(np.int32)
    bt = np.full((S, maxb), -1, np.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    q = rs.randn(S, H, D).astype(np.float16)
    return kc, vc, bt, np.array(lens, np.int32), q


def _sdpa_decode(q, kc, vc, bt, lens, scale, layout):
    S, H, D = q.shape
    KV = kc.shape[1] if layout == "kernel" else kc.shape[2]
    out = np.zeros((S, H, D))
    for s in range(S):
        if lens[s] <= 0:
            continue
        K, _ = oat.gather(kc, bt[s], lens[s], layout)
        V, _ = oat.gather(vc, bt[s], lens[s], layout)
        kt = torch.from_numpy(K).transpose(0, 1).repeat_interleave(H // KV, 0)
        vt = torch.from_numpy(V).transpose(0, 1).repeat_interleave(H // KV, 0)
        qt = torch.from_numpy(q[s].astype(np.float64))[:, None, :]
        out[s] = F.scaled_dot_product_attention(qt, kt, vt, scale=scale)[:, 0, :].numpy()
    return out


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
@pytest.mark.parametrize("H,KV,D", [(14, 2, 64), (32, 8, 128), (8, 8, 32)])
def test_decode_vs_sdpa(layout, H, KV, D):
    lens = [1, 17, 100, 0, 333]
    kc, vc, bt, L, q = _paged(5, H, KV, D, lens, layout=layout, seed=1)
    scale = 1 / math.sqrt(D)
    got = oat.decode(q, kc, vc, bt, L, scale, layout)
    ref = _sdpa_decode(q, kc, vc, bt, L, scale, layout)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_decode_vs_metal_structured_loop():
    kc, vc, bt, L, q = _paged(3, 4, 2, 32, [40, 3, 16], seed=2)
    got = oat.decode(q, kc, vc, bt, L, 0.2)
    loop = oat.decode_loop_fp32(q, kc, vc, bt, L, 0.2)
    np.testing.assert_allclose(got, loop, rtol=1e-5, atol=1e-5)


def test_decode_vs_reference_torch_path():
    """The reference's own PyTorch decode (mps_attn.py:284-357) on the same data."""
    kc, vc, bt, L, q = _paged(4, 14, 2, 64, [16, 90, 512, 200], layout="vllm", seed=3)
    ref = ref_torch.decode_sdpa(torch.from_numpy(q).float(), torch.from_numpy(kc).float(),
                                torch.from_numpy(vc).float(), torch.from_numpy(bt),
                                L.tolist(), 1 / 8, 2).numpy()
    got = oat.decode(q, kc, vc, bt, L, 1 / 8, "vllm")
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_decode_known_answer_seq_len_one():
    kc, vc, bt, L, q = _paged(1, 32, 4, 64, [1], seed=4)
    got = oat.decode(q, kc, vc, bt, L, 0.125)
    v = vc[bt[0, 0], :, 0, :].astype(np.float64)
    assert np.array_equal(got[0], np.repeat(v, 8, axis=0))


def test_decode_closed_forms():
    kc, vc, bt, L, q = _paged(1, 4, 1, 32, [48], seed=5)
    # all keys equal -> mean of V
    kc[:] = kc[bt[0, 0], :, 0:1, :]
    got = oat.decode(q, kc, vc, bt, L, 0.3)
    V, _ = oat.gather(vc, bt[0], 48, "kernel")
    np.testing.assert_allclose(got[0], np.repeat(V.mean(0), 4, axis=0), rtol=1e-12, atol=1e-12)
    # one dominant key -> its value row
    kc2, vc2, bt2, L2, q2 = _paged(1, 2, 1, 32, [48], seed=6)
    q2[:] = 1
    blk, off = bt2[0, 1], 7
    kc2[blk, 0, off, :] = 60.0
    got2 = oat.decode(q2, kc2, vc2, bt2, L2, 1.0)
    np.testing.assert_allclose(got2[0, 0], vc2[blk, 0, off].astype(np.float64), atol=1e-9)


@pytest.mark.parametrize("part", [16, 100, 512, 4096])
def test_merge_of_partials_is_decode(part):
    """Splitting each context into partitions and merging their states gives
    the unsplit decode: exact in real arithmetic for any partition size, so
    a dropped weight, a wrong sign in the exponent or a missing normalisation
    fails.  Wide groups (G = 20) and empty sequences included."""
    lens = [0, 1, 15, 700, 3001]
    kc, vc, bt, L, q = _paged(5, 40, 2, 64, lens, seed=31)
    scale = 1 / 8
    po, lse, n = oat.decode_partials(q, kc, vc, bt, L, scale, part)
    got, LSE = oat.merge_states(po, lse, n)
    ref = oat.decode(q, kc, vc, bt, L, scale)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert np.all(np.isneginf(LSE[0])) and not np.any(got[0])
    # LSE of the whole context from the scores directly.
    K, _ = oat.gather(kc, bt[4], lens[4], "kernel")
    sc = np.einsum("hd,lhd->hl", q[4].astype(np.float64), K[:, np.arange(40) // 20]) * scale
    direct = np.log(np.exp(sc - sc.max(1, keepdims=True)).sum(1)) + sc.max(1)
    assert np.allclose(LSE[4], direct, rtol=1e-12)


def test_merge_states_closed_forms():
    rs = np.random.RandomState(3)
    o = rs.randn(2, 3, 4, 8)
    lse = rs.randn(2, 3, 4)
    # One partition: unchanged.
    got, LSE = oat.merge_states(o[:, :, :1], lse[:, :, :1])
    assert np.array_equal(got, o[:, :, 0]) and np.allclose(LSE, lse[:, :, 0])
    # lse 0 and ln 3: weights 1/4 and 3/4, LSE = ln 4.
    two = np.stack([np.zeros((1, 1)), np.full((1, 1), math.log(3.0))], axis=-1)
    got, LSE = oat.merge_states(o[:1, :1, :2], two)
    assert np.allclose(got[0, 0], 0.25 * o[0, 0, 0] + 0.75 * o[0, 0, 1], rtol=1e-14)
    assert np.isclose(LSE[0, 0], math.log(4.0))
    # Empty partitions (-inf) and partitions past num_parts are ignored.
    l2 = lse.copy()
    l2[:, :, 2] = -np.inf
    a, _ = oat.merge_states(o, l2, np.array([4, 4]))
    b, _ = oat.merge_states(np.delete(o, 2, axis=2), np.delete(lse, 2, axis=2))
    assert np.allclose(a, b, rtol=1e-14)
    c, _ = oat.merge_states(o, lse, np.array([3, 3]))
    d, _ = oat.merge_states(o[:, :, :3], lse[:, :, :3])
    assert np.array_equal(c, d)


def test_prefill_without_prefix_is_causal_sdpa():
    kc, vc, bt, _, _ = _paged(1, 8, 2, 64, [40], seed=7)
    rs = np.random.RandomState(8)
    q = rs.randn(40, 8, 64).astype(np.float16)
    tok = np.zeros(40, np.int32)
    pos = np.arange(40, dtype=np.int32)
    got, w = oat.prefill(q, kc, vc, bt, tok, pos, 0.125)
    K, _ = oat.gather(kc, bt[0], 40, "kernel")
    V, _ = oat.gather(vc, bt[0], 40, "kernel")
    qt = torch.from_numpy(q.astype(np.float64)).transpose(0, 1)
    kt = torch.from_numpy(K).transpose(0, 1).repeat_interleave(4, 0)
    vt = torch.from_numpy(V).transpose(0, 1).repeat_interleave(4, 0)
    ref = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=0.125).transpose(0, 1)
    assert w.all()
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-12)


def test_prefill_last_row_equals_decode():
    """The chunk's last token attends to the whole context: a decode of length L."""
    kc, vc, bt, L, _ = _paged(2, 16, 4, 64, [70, 33], seed=9)
    rs = np.random.RandomState(10)
    q = rs.randn(2, 16, 64).astype(np.float16)
    got, _ = oat.prefill(q, kc, vc, bt, np.array([0, 1], np.int32),
                         np.array([69, 32], np.int32), 0.1)
    dec = oat.decode(q, kc, vc, bt, L, 0.1)
    np.testing.assert_allclose(got, dec, rtol=1e-12, atol=1e-12)


def test_prefill_vs_reference_torch_prefix_path():
    kc, vc, bt, L, _ = _paged(2, 8, 2, 32, [50, 37], layout="vllm", seed=11)
    rs = np.random.RandomState(12)
    new = [20, 37]
    q = rs.randn(sum(new), 8, 32).astype(np.float16)
    tok = np.array([0] * 20 + [1] * 37, np.int32)
    pos = np.array(list(range(30, 50)) + list(range(37)), np.int32)
    got, w = oat.prefill(q, kc, vc, bt, tok, pos, 0.2, "vllm")
    ref = ref_torch.prefill_sdpa_prefix(torch.from_numpy(q).double(), torch.from_numpy(kc).double(),
                                        torch.from_numpy(vc).double(), torch.from_numpy(bt),
                                        [0, 20, 57], [50, 37], 0.2, 2).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-10)


def test_prefill_unwritten_rows_rules():
    kc, vc, bt, _, _ = _paged(2, 4, 1, 32, [32, 32], seed=13)
    q = np.ones((5, 4, 32), np.float16)
    tok = np.array([0, -1, 5, 0, 1], np.int32)
    pos = np.array([3, 3, 3, -1, 40], np.int32)  # last: context past the table
    _, w = oat.prefill(q, kc, vc, bt, tok, pos, 0.1)
    assert w.tolist() == [True, False, False, False, False]
    bt2 = bt.copy()
    bt2[0, 0] = -1
    _, w2 = oat.prefill(q, kc, vc, bt2, tok, pos, 0.1)
    assert not w2[0]


# -- planted mistakes: each must be caught by one of the pins above ----------


def _planted_decode_wrong_gqa(q, kc, vc, bt, L, scale):
    """GQA map h % KV instead of h // (H/KV)."""
    S, H, D = q.shape
    KV = kc.shape[1]
    out = np.zeros((S, H, D))
    for s in range(S):
        K, _ = oat.gather(kc, bt[s], L[s], "kernel")
        V, _ = oat.gather(vc, bt[s], L[s], "kernel")
        for h in range(H):
            sc = K[:, h % KV] @ q[s, h].astype(np.float64) * scale
            p = np.exp(sc - sc.max())
            out[s, h] = p @ V[:, h % KV] / p.sum()
    return out


def test_planted_mistake_is_caught():
    kc, vc, bt, L, q = _paged(2, 8, 2, 32, [30, 20], seed=14)
    ref = _sdpa_decode(q, kc, vc, bt, L, 0.2, "kernel")
    bad = _planted_decode_wrong_gqa(q, kc, vc, bt, L, 0.2)
    assert not np.allclose(bad, ref, atol=1e-3)
    with pytest.raises(AssertionError):
        assert_close(bad, ref)
