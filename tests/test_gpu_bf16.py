"""bfloat16 caches and activations through the same kernels (vaa_attn_params.dtype
= VAA_DTYPE_BF16) against the fp64 oracle.

The reference runs fp16 only and converts bf16 models at its boundary
(metal_attn.py:609-620); here bf16 runs natively, so a bf16 vLLM kv_cache needs
no fp16 copy.  KV writes stay bit-exact (they are 16-bit copies: the oracle
copies the bf16 bit patterns).  Attention is checked with the north-star
bound |d| <= 2e-3 + 1e-2 |ref| plus the rounding of the bf16 output (half a
bf16 ulp of ref).  The probabilities enter the PV product as a bf16 pair
hi + lo: as one bf16 value they had measured up to 0.93 of that bound on
short contexts.
"""
import math

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16

import oracle.attention as oat
import oracle.kv as okv

pytestmark = pytest.mark.gpu


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> its 16-bit patterns as a float16-typed numpy array (for
    the oracle's byte-exact copies)."""
    return t.detach().cpu().view(torch.float16).numpy()


def vals(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def _paged(S, H, KV, D, lens, bs=16, seed=0, layout="kernel"):
    g = torch.Generator().manual_seed(seed)
    nblk = [(L + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 4
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = torch.randn(shape, generator=g).bfloat16()
    vc = torch.randn(shape, generator=g).bfloat16()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((S, max(max(nblk), 1)), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    return kc, vc, bt, g


def test_kv_write_slots_bf16_bit_exact(gpu):
    from vllm_apple_amd import kernels

    kc, vc, bt, g = _paged(3, 8, 4, 128, [40, 17, 100], seed=1, layout="vllm")
    T = 20
    k = torch.randn(T, 4, 128, generator=g).bfloat16()
    v = torch.randn(T, 4, 128, generator=g).bfloat16()
    slots = torch.randperm(kc.shape[0] * 16, generator=g)[:T].to(torch.int64)
    slots[3] = -1
    kd, vd = kc.cuda(), vc.cuda()
    kernels.kv_write_slots(k.cuda(), v.cuda(), kd, vd, slots.cuda(), layout="vllm")
    torch.cuda.synchronize()
    kr, vr = bits(kc).copy(), bits(vc).copy()
    okv.kv_write_slots(kr, vr, bits(k), bits(v), slots.numpy(), "vllm")
    assert np.array_equal(bits(kd).view(np.uint16), kr.view(np.uint16))
    assert np.array_equal(bits(vd).view(np.uint16), vr.view(np.uint16))


@pytest.mark.parametrize("part", [0, 256, 2048, -1, -2])
@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_decode_bf16_fused_write(gpu, part, layout):
    """C2 shape (32q/8kv, D128) in bf16: fused KV write bit-exact, output vs fp64."""
    from vllm_apple_amd import kernels

    lens = [1, 33, 1024, 3000, 8192, 517]
    print(f"[case] bf16 decode part={part} layout={layout}", flush=True)
    kc, vc, bt, g = _paged(6, 32, 8, 128, lens, seed=2, layout=layout)
    q = torch.randn(6, 32, 128, generator=g).bfloat16()
    nk = torch.randn(6, 8, 128, generator=g).bfloat16()
    nv = torch.randn(6, 8, 128, generator=g).bfloat16()
    L = torch.tensor(lens, dtype=torch.int32)
    kd, vd = kc.cuda(), vc.cuda()
    out = kernels.paged_decode(q.cuda(), kd, vd, bt.cuda(), L.cuda(), scale=1 / math.sqrt(128),
                               max_seq_len=max(lens), layout=layout, new_keys=nk.cuda(),
                               new_values=nv.cuda(), partition_size=part)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    kr, vr = bits(kc).copy(), bits(vc).copy()
    okv.kv_write_decode(kr, vr, bits(nk), bits(nv), bt.numpy(), L.numpy(), layout)
    assert np.array_equal(bits(kd).view(np.uint16), kr.view(np.uint16)), "fused K write"
    assert np.array_equal(bits(vd).view(np.uint16), vr.view(np.uint16)), "fused V write"
    kv_vals = torch.from_numpy(kr.copy()).view(torch.bfloat16).float().numpy()
    vv_vals = torch.from_numpy(vr.copy()).view(torch.bfloat16).float().numpy()
    ref = oat.decode(vals(q), kv_vals, vv_vals, bt.numpy(), L.numpy(), 1 / math.sqrt(128), layout)
    assert_close_bf16(vals(out), ref, what="bf16 decode")


def test_decode_bf16_seq_len_one_is_value_exact(gpu):
    """L=1: the output is the new V, exactly, in bf16 too (tests/metal/test_metal_kernels.py:380-438)."""
    from vllm_apple_amd import kernels

    kc, vc, bt, g = _paged(1, 32, 4, 64, [1], seed=3)
    q = torch.randn(1, 32, 64, generator=g).bfloat16()
    nk = torch.randn(1, 4, 64, generator=g).bfloat16()
    nv = torch.randn(1, 4, 64, generator=g).bfloat16()
    out = kernels.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(),
                               torch.tensor([1], dtype=torch.int32).cuda(), scale=0.125,
                               max_seq_len=1, new_keys=nk.cuda(), new_values=nv.cuda())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), nv.repeat_interleave(8, dim=1))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("H,KV", [(32, 8), (14, 2), (8, 8)])
def test_prefill_bf16(gpu, D, H, KV):
    """Chunks after a cached prefix (C3-like) in bf16 against the fp64 oracle."""
    from vllm_apple_amd import kernels

    ctx, new = [700, 300], [200, 300]
    print(f"[case] bf16 prefill D={D} H={H} KV={KV}", flush=True)
    kc, vc, bt, g = _paged(2, H, KV, D, ctx, seed=4)
    tok, pos = [], []
    for s, (Ls, n) in enumerate(zip(ctx, new)):
        tok += [s] * n
        pos += list(range(Ls - n, Ls))
    T = len(tok)
    q = torch.randn(T, H, D, generator=g).bfloat16()
    tok_t = torch.tensor(tok, dtype=torch.int32)
    pos_t = torch.tensor(pos, dtype=torch.int32)
    out = kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok_t.cuda(),
                                pos_t.cuda(), scale=1 / math.sqrt(D))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    ref, written = oat.prefill(vals(q), vals(kc), vals(vc), bt.numpy(), tok_t.numpy(),
                               pos_t.numpy(), 1 / math.sqrt(D))
    assert written.all()
    assert_close_bf16(vals(out), ref, what=f"bf16 prefill D={D}")


def test_bf16_short_contexts(gpu):
    """Few keys with values of opposite sign: the case where one bf16
    probability per key (8 bits) reached the attention bound (up to 1.03 of
    it on 5 keys).  Decode (every split mode) and prefill with no prefix."""
    from vllm_apple_amd import kernels

    lens = [2, 3, 5, 9, 17, 40, 90, 200]
    kc, vc, bt, g = _paged(len(lens), 32, 8, 128, lens, seed=6)
    q = torch.randn(len(lens), 32, 128, generator=g).bfloat16()
    L = torch.tensor(lens, dtype=torch.int32)
    ref = oat.decode(vals(q), vals(kc), vals(vc), bt.numpy(), L.numpy(), 1 / math.sqrt(128))
    for part in (0, 128, -1, -2):
        out = kernels.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), L.cuda(),
                                   scale=1 / math.sqrt(128), max_seq_len=max(lens),
                                   partition_size=part)
        torch.cuda.synchronize()
        assert_close_bf16(vals(out), ref, what=f"bf16 short decode part={part}")
    ctx = [5, 9, 40]
    kc, vc, bt, g = _paged(3, 32, 8, 128, ctx, seed=7)
    tok = sum(([s] * n for s, n in enumerate(ctx)), [])
    pos = sum((list(range(n)) for n in ctx), [])
    q = torch.randn(len(tok), 32, 128, generator=g).bfloat16()
    tok_t = torch.tensor(tok, dtype=torch.int32)
    pos_t = torch.tensor(pos, dtype=torch.int32)
    out = kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok_t.cuda(),
                                pos_t.cuda(), scale=1 / math.sqrt(128))
    torch.cuda.synchronize()
    ref, written = oat.prefill(vals(q), vals(kc), vals(vc), bt.numpy(), tok_t.numpy(),
                               pos_t.numpy(), 1 / math.sqrt(128))
    assert written.all()
    assert_close_bf16(vals(out), ref, what="bf16 short prefill")


def test_mixed_dtypes_are_rejected(gpu):
    from vllm_apple_amd import kernels

    kc, vc, bt, g = _paged(1, 8, 8, 64, [10], seed=5)
    q = torch.randn(1, 8, 64, generator=g).half()
    with pytest.raises(ValueError, match="float16 or all bfloat16"):
        kernels.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(),
                             torch.tensor([10], dtype=torch.int32).cuda(), scale=0.125,
                             max_seq_len=10)
