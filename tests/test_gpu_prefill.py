"""Chunked-prefill paged attention (MFMA) vs the oracle."""
import numpy as np
import pytest
import torch

from helpers import assert_close, host

import oracle.attention as oat
import oracle.kv as okv

pytestmark = pytest.mark.gpu


def _prefill_case(ctx, new, H, KV, D, bs=16, seed=0, layout="kernel", extra_blocks=4):
    """Sequences of total length ctx[s] whose last new[s] tokens are queries."""
    g = torch.Generator().manual_seed(seed)
    nblk = [(L + bs - 1) // bs for L in ctx]
    nb = sum(nblk) + extra_blocks
    maxb = max(nblk)
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = torch.randn(shape, generator=g).half()
    vc = torch.randn(shape, generator=g).half()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((len(ctx), maxb), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    tok, pos = [], []
    for s, (L, n) in enumerate(zip(ctx, new)):
        tok += [s] * n
        pos += list(range(L - n, L))
    T = len(tok)
    q = torch.randn(T, H, D, generator=g).half()
    return kc, vc, bt, torch.tensor(tok, dtype=torch.int32), torch.tensor(pos, dtype=torch.int32), q


def _run(kc, vc, bt, tok, pos, q, layout="kernel", rows=None):
    from vllm_apple_amd import kernels

    D = q.shape[2]
    scale = 1.0 / np.sqrt(D)
    sentinel = torch.full(q.shape, 7.0, dtype=torch.float16, device="cuda")
    out = kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok.cuda(), pos.cuda(),
                                scale=scale, layout=layout, output=sentinel)
    torch.cuda.synchronize()
    ref, written = oat.prefill(host(q), host(kc), host(vc), host(bt), host(tok), host(pos), scale,
                               layout, rows=rows)
    return host(out), ref, written


def test_prefill_single_seq_with_prefix(gpu):
    kc, vc, bt, tok, pos, q = _prefill_case([300], [100], 32, 8, 128, seed=1)
    out, ref, w = _run(kc, vc, bt, tok, pos, q)
    assert w.all()
    assert_close(out, ref, what="prefill prefix")


@pytest.mark.parametrize("D", [32, 64, 96, 128])
@pytest.mark.parametrize("H,KV", [(14, 2), (32, 8), (8, 8), (16, 1), (6, 2), (8, 4)])
def test_prefill_shapes(gpu, D, H, KV):
    print(f"[case] prefill D={D} H={H} KV={KV}", flush=True)
    kc, vc, bt, tok, pos, q = _prefill_case([77, 150, 40], [40, 64, 40], H, KV, D, seed=2)
    out, ref, w = _run(kc, vc, bt, tok, pos, q)
    assert_close(out, ref, what=f"prefill D={D} H={H} KV={KV}")


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_prefill_c3_shape_all_rows(gpu, layout):
    """C3 shape: 4 x (2048 cached + 512 new); every one of the 2048 rows
    against the fp64 oracle."""
    print(f"[case] C3 all rows {layout}", flush=True)
    kc, vc, bt, tok, pos, q = _prefill_case([2560] * 4, [512] * 4, 32, 8, 128, seed=3,
                                            layout=layout)
    out, ref, w = _run(kc, vc, bt, tok, pos, q, layout=layout)
    assert w.all()
    assert_close(out, ref, what=f"C3 rows {layout}")


@pytest.mark.parametrize("bs", [32, 64])
def test_prefill_larger_block_size(gpu, bs):
    kc, vc, bt, tok, pos, q = _prefill_case([300, 77], [120, 77], 32, 8, 128, bs=bs, seed=11)
    out, ref, w = _run(kc, vc, bt, tok, pos, q)
    assert w.all()
    assert_close(out, ref, what=f"prefill bs={bs}")


def test_prefill_no_prefix_is_causal_chunk(gpu):
    """Without a cached prefix the result is within-chunk causal attention
    (where the reference's SDPA prefill, base_attn.py:223-306, is valid)."""
    import torch.nn.functional as F

    kc, vc, bt, tok, pos, q = _prefill_case([64], [64], 8, 2, 64, seed=5)
    out, ref, w = _run(kc, vc, bt, tok, pos, q)
    k_rows, _ = oat.gather(host(kc), host(bt)[0], 64, "kernel")
    v_rows, _ = oat.gather(host(vc), host(bt)[0], 64, "kernel")
    qt = torch.from_numpy(host(q).astype(np.float32)).transpose(0, 1)
    kt = torch.from_numpy(k_rows.astype(np.float32)).transpose(0, 1).repeat_interleave(4, 0)
    vt = torch.from_numpy(v_rows.astype(np.float32)).transpose(0, 1).repeat_interleave(4, 0)
    sd = F.scaled_dot_product_attention(qt[None], kt[None], vt[None], is_causal=True,
                                        scale=1 / 8)[0].transpose(0, 1)
    assert_close(out, sd.numpy(), what="prefill vs causal SDPA")


def test_prefill_mixed_tile_and_shuffled_tokens(gpu):
    """Tokens of several sequences share a 32-token tile, in shuffled order."""
    kc, vc, bt, tok, pos, q = _prefill_case([20, 5, 50, 9, 33], [7, 5, 11, 3, 30], 16, 4, 64, seed=6)
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(tok.numel(), generator=g)
    out, ref, w = _run(kc, vc, bt, tok[perm].contiguous(), pos[perm].contiguous(), q[perm].contiguous())
    assert w.all()
    assert_close(out, ref, what="prefill mixed tiles")


def test_prefill_unwritten_rows(gpu):
    """Invalid sequence / negative position / invalid block -> row left untouched."""
    kc, vc, bt, tok, pos, q = _prefill_case([48, 48], [16, 16], 8, 2, 64, seed=8)
    tok[0] = -1
    tok[1] = 9
    pos[2] = -4
    bt[1, 0] = -1  # every row of sequence 1 aborts
    out, ref, w = _run(kc, vc, bt, tok, pos, q)
    assert not w[0] and not w[1] and not w[2] and not w[16:].any()
    assert np.all(out[~w] == np.float16(7.0))
    assert_close(out[w], ref[w], what="prefill valid rows")


@pytest.mark.parametrize("bs", [16, 32])
def test_prefill_invalid_block_mid_context(gpu, bs):
    """An invalid entry inside the context aborts exactly the rows whose
    context reaches it (paged_attention_v2.metal:428); earlier rows of the
    same sequence are written, masked against the zero-filled block."""
    kc, vc, bt, tok, pos, q = _prefill_case([1300, 150], [80, 60], 8, 2, 128, bs=bs, seed=11)
    bad0 = 1250 // bs          # sequence 0: rows at positions >= bad0 * bs abort
    bt[0, bad0] = -1
    bad1 = 120 // bs           # sequence 1: an entry past num_blocks
    bt[1, bad1] = kc.shape[0] + 3
    out, ref, w = _run(kc, vc, bt, tok, pos, q)
    p = pos.numpy()
    t = tok.numpy()
    expect = np.where(t == 0, p < bad0 * bs, p < bad1 * bs)
    assert np.array_equal(w, expect)
    assert w.any() and (~w).any()
    assert np.all(out[~w] == np.float16(7.0))
    assert_close(out[w], ref[w], what="prefill rows before an invalid block")


def test_prefill_after_slot_write_c3_flow(gpu):
    """C3 flow: write the chunk's K/V through slot_mapping, then attend."""
    from vllm_apple_amd import kernels

    kc, vc, bt, tok, pos, q = _prefill_case([200, 130], [64, 64], 32, 8, 128, seed=9)
    g = torch.Generator().manual_seed(10)
    nk = torch.randn(128, 8, 128, generator=g).half()
    nv = torch.randn(128, 8, 128, generator=g).half()
    slots = okv.slot_mapping(host(bt), 16, host(tok), host(pos))
    kd, vd = kc.cuda(), vc.cuda()
    kernels.kv_write_slots(nk.cuda(), nv.cuda(), kd, vd, torch.from_numpy(slots).cuda())
    out = kernels.paged_prefill(q.cuda(), kd, vd, bt.cuda(), tok.cuda(), pos.cuda(),
                                scale=1 / np.sqrt(128))
    torch.cuda.synchronize()
    kr, vr = host(kc).copy(), host(vc).copy()
    okv.kv_write_slots(kr, vr, host(nk), host(nv), slots)
    assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16))
    ref, w = oat.prefill(host(q), kr, vr, host(bt), host(tok), host(pos), 1 / np.sqrt(128))
    assert_close(host(out), ref, what="C3 flow")


def test_prefill_and_decode_block_stride_past_32_bits(gpu):
    """Caches whose block stride is 2^31 elements (4 GiB): the prefill's
    fetch takes its 64-bit address path (the 32-bit fast path needs the byte
    strides to fit 32 bits), and decode reads the same views; both against
    the oracle on compact host copies of the two blocks."""
    from vllm_apple_amd import kernels

    print("[case] prefill/decode, block stride 2^31 elements", flush=True)
    KV, bs, D, H = 2, 16, 64, 8
    sb = 1 << 31
    g = torch.Generator().manual_seed(21)
    kh = torch.randn(2, KV, bs, D, generator=g).half()
    vh = torch.randn(2, KV, bs, D, generator=g).half()
    bufs = []
    views = []
    for h_ in (kh, vh):
        buf = torch.empty(sb + KV * bs * D, dtype=torch.float16, device="cuda")
        v = buf.as_strided((2, KV, bs, D), (sb, bs * D, D, 1))
        v.copy_(h_.cuda())
        bufs.append(buf)
        views.append(v)
    kc, vc = views
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    tok = torch.zeros(20, dtype=torch.int32)
    pos = torch.arange(12, 32, dtype=torch.int32)
    q = torch.randn(20, H, D, generator=g).half()
    scale = 1.0 / np.sqrt(D)
    out = kernels.paged_prefill(q.cuda(), kc, vc, bt.cuda(), tok.cuda(), pos.cuda(), scale=scale)
    qd = torch.randn(1, H, D, generator=g).half()
    outd = kernels.paged_decode(qd.cuda(), kc, vc, bt.cuda(), torch.tensor([29], dtype=torch.int32,
                                device="cuda"), scale=scale, max_seq_len=29)
    torch.cuda.synchronize()
    ref, w = oat.prefill(host(q), host(kh), host(vh), host(bt), host(tok), host(pos), scale)
    assert w.all()
    assert_close(host(out), ref, what="prefill, 4 GiB block stride")
    refd = oat.decode(host(qd), host(kh), host(vh), host(bt), np.array([29], np.int32), scale)
    assert_close(host(outd), refd, what="decode, 4 GiB block stride")
    del bufs, views, kc, vc
    torch.cuda.empty_cache()
