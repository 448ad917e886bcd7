"""KV-cache writes on the GPU vs the C oracle and the reference's own kv_write.c.

Bit-exact: every byte of both caches must equal the oracle's.
"""
import numpy as np
import pytest
import torch

from helpers import host

import oracle.kv as okv

pytestmark = pytest.mark.gpu


def _caches(nb, kv, bs, d, layout, seed):
    g = torch.Generator().manual_seed(seed)
    shape = (nb, kv, bs, d) if layout == "kernel" else (nb, bs, kv, d)
    k = torch.randn(shape, generator=g).half()
    v = torch.randn(shape, generator=g).half()
    return k, v


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("kv,d", [(8, 128), (2, 64), (4, 96), (1, 32)])
def test_kv_write_slots_bit_exact(gpu, layout, slot_dtype, kv, d):
    from vllm_apple_amd import kernels

    nb, bs, T = 64, 16, 300
    print(f"[case] slots layout={layout} dtype={slot_dtype} kv={kv} d={d}", flush=True)
    kc, vc = _caches(nb, kv, bs, d, layout, 1)
    g = torch.Generator().manual_seed(2)
    key = torch.randn(T, kv, d, generator=g).half()
    val = torch.randn(T, kv, d, generator=g).half()
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int64)
    slots[::7] = -1                       # padding
    slots[5] = nb * bs + 3                # past capacity: skipped by the guard
    kc_ref, vc_ref = host(kc).copy(), host(vc).copy()
    okv.kv_write_slots(kc_ref, vc_ref, host(key), host(val), host(slots), layout)

    kd, vd = kc.cuda(), vc.cuda()
    kernels.kv_write_slots(key.cuda(), val.cuda(), kd, vd, slots.to(slot_dtype).cuda(), layout=layout)
    torch.cuda.synchronize()
    assert np.array_equal(host(kd).view(np.uint16), kc_ref.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vc_ref.view(np.uint16))


def test_kv_write_slots_strided_source(gpu):
    """new K/V as views into a fused [T, (H+2KV)*D] projection (vLLM qkv split)."""
    from vllm_apple_amd import kernels

    nb, kv, bs, d, H, T = 32, 8, 16, 128, 32, 100
    kc, vc = _caches(nb, kv, bs, d, "vllm", 3)
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(T, (H + 2 * kv) * d, generator=g).half()
    key = qkv[:, H * d:(H + kv) * d].view(T, kv, d)
    val = qkv[:, (H + kv) * d:].view(T, kv, d)
    slots = torch.randperm(nb * bs, generator=g)[:T]
    kc_ref, vc_ref = host(kc).copy(), host(vc).copy()
    okv.kv_write_slots(kc_ref, vc_ref, host(key), host(val), host(slots), "vllm")
    qd = qkv.cuda()
    kd, vd = kc.cuda(), vc.cuda()
    kernels.kv_write_slots(qd[:, H * d:(H + kv) * d].view(T, kv, d),
                           qd[:, (H + kv) * d:].view(T, kv, d), kd, vd, slots.cuda(),
                           layout="vllm")
    torch.cuda.synchronize()
    assert np.array_equal(host(kd).view(np.uint16), kc_ref.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vc_ref.view(np.uint16))


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_kv_write_decode_bit_exact(gpu, layout):
    from vllm_apple_amd import kernels

    nb, kv, bs, d, S, maxb = 128, 4, 16, 128, 12, 8
    kc, vc = _caches(nb, kv, bs, d, layout, 5)
    g = torch.Generator().manual_seed(6)
    bt = torch.randperm(nb, generator=g)[:S * maxb].view(S, maxb).to(torch.int32)
    lens = torch.randint(1, maxb * bs + 1, (S,), generator=g).to(torch.int32)
    lens[0] = 0                   # no write
    lens[1] = maxb * bs + 5       # block index past the table: no write
    bt[2, (int(lens[2]) - 1) // bs] = -1  # invalid block: no write
    key = torch.randn(S, kv, d, generator=g).half()
    val = torch.randn(S, kv, d, generator=g).half()
    kc_ref, vc_ref = host(kc).copy(), host(vc).copy()
    okv.kv_write_decode(kc_ref, vc_ref, host(key), host(val), host(bt), host(lens), layout)
    kd, vd = kc.cuda(), vc.cuda()
    kernels.kv_write_decode(key.cuda(), val.cuda(), kd, vd, bt.cuda(), lens.cuda(), layout=layout)
    torch.cuda.synchronize()
    assert np.array_equal(host(kd).view(np.uint16), kc_ref.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vc_ref.view(np.uint16))


def test_write_kv_batch_matches_reference_c(gpu):
    """Device metal_write_kv_batch/single vs the reference's kv_write.c on the host."""
    from vllm_apple_amd import kernels

    if okv.ref_lib() is None:
        pytest.skip("oracle/_ref not built")
    nb, kv, bs, d, T = 40, 8, 16, 128, 77
    kc, vc = _caches(nb, kv, bs, d, "kernel", 7)
    g = torch.Generator().manual_seed(8)
    key = torch.randn(T, kv, d, generator=g).half()
    val = torch.randn(T, kv, d, generator=g).half()
    slots = torch.randperm(nb * bs, generator=g)[:T]
    bids, offs = slots // bs, slots % bs
    sb, sh, st = kv * bs * d, bs * d, d
    kc_ref, vc_ref = host(kc).copy(), host(vc).copy()
    okv.ref_write_kv_batch(kc_ref, vc_ref, host(key), host(val), host(bids), host(offs), sb, sh, st)
    okv.ref_write_kv_single(kc_ref, vc_ref, host(key[3]), host(val[3]), 39, 15, sb, sh, st)
    kd, vd = kc.cuda(), vc.cuda()
    kernels.write_kv_batch(kd, vd, key.cuda(), val.cuda(), bids.cuda(), offs.cuda(), sb, sh, st, nb)
    kernels.write_kv_single(kd, vd, key[3].contiguous().cuda(), val[3].contiguous().cuda(), 39, 15,
                            sb, sh, st, nb)
    torch.cuda.synchronize()
    assert np.array_equal(host(kd).view(np.uint16), kc_ref.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vc_ref.view(np.uint16))


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_write_kv_batch_offset_guard(gpu, layout):
    """Offsets at or past the block size aimed at a middle block (in-bounds
    memory: without the guard they would land in the next block) are skipped,
    as are negative offsets and blocks outside the pool; the valid tokens of
    the same call are written bit-exactly; the single-token entry point
    rejects such indices on the host."""
    from vllm_apple_amd import kernels

    nb, kv, bs, d = 16, 8, 16, 128
    print(f"[case] write_kv_batch offset guard layout={layout}", flush=True)
    kc, vc = _caches(nb, kv, bs, d, layout, 21)
    sb, sh, st = okv.cache_strides(host(kc), layout)
    g = torch.Generator().manual_seed(22)
    T = 9
    key = torch.randn(T, kv, d, generator=g).half()
    val = torch.randn(T, kv, d, generator=g).half()
    bids = torch.tensor([7, 7, 7, 7, -1, nb, 3, 7, nb - 1], dtype=torch.int64)
    offs = torch.tensor([bs, bs + 1, 2 * bs - 1, -1, 0, 0, 4, bs - 1, bs], dtype=torch.int64)
    kc_ref, vc_ref = host(kc).copy(), host(vc).copy()
    okv.write_kv_batch(kc_ref, vc_ref, host(key), host(val), host(bids), host(offs), sb, sh, st, nb)
    kd, vd = kc.cuda(), vc.cuda()
    kernels.write_kv_batch(kd, vd, key.cuda(), val.cuda(), bids.cuda(), offs.cuda(), sb, sh, st, nb)
    torch.cuda.synchronize()
    got_k, got_v = host(kd).view(np.uint16), host(vd).view(np.uint16)
    assert np.array_equal(got_k, kc_ref.view(np.uint16))
    assert np.array_equal(got_v, vc_ref.view(np.uint16))
    # Block 8 (the neighbour of block 7) is byte-identical to the input.
    assert np.array_equal(got_k[8], host(kc).view(np.uint16)[8])
    assert np.array_equal(got_v[8], host(vc).view(np.uint16)[8])
    # Only blocks 3 and 7 changed (offsets 4 and bs - 1).
    changed = np.nonzero((got_k != host(kc).view(np.uint16)).reshape(nb, -1).any(1))[0]
    assert changed.tolist() == [3, 7]
    for b, o in ((7, bs), (7, -1), (-1, 0), (nb, 0)):
        with pytest.raises(ValueError, match="vaa_write_kv_single"):
            kernels.write_kv_single(kd, vd, key[0].contiguous().cuda(), val[0].contiguous().cuda(),
                                    b, o, sb, sh, st, nb)
    torch.cuda.synchronize()
    assert np.array_equal(host(kd).view(np.uint16), got_k)


def test_kv_write_empty_and_all_padding(gpu):
    from vllm_apple_amd import kernels

    kc, vc = _caches(8, 2, 16, 64, "kernel", 9)
    kd, vd = kc.cuda(), vc.cuda()
    key = torch.zeros(0, 2, 64, dtype=torch.float16, device="cuda")
    kernels.kv_write_slots(key, key, kd, vd, torch.zeros(0, dtype=torch.int64, device="cuda"))
    key = torch.ones(5, 2, 64, dtype=torch.float16, device="cuda")
    kernels.kv_write_slots(key, key, kd, vd, torch.full((5,), -1, dtype=torch.int64, device="cuda"))
    torch.cuda.synchronize()
    assert np.array_equal(host(kd).view(np.uint16), host(kc).view(np.uint16))
