"""Head sizes other than 32/64/96/128 (any multiple of 8 up to 128), as the
reference's generic kernels take any head size up to 128
(paged_attention_fused.metal:208-233, paged_attention_v2.metal:73-87,
engine/ops/attention.py:268-290).  The kernels compute at the next multiple
of 32 with the tail masked; these tests check every output row against the
fp64 oracle, the fused and slot KV writes bit for bit over the whole cache,
and that nothing past the last row of an output or cache is touched (canary
tails behind each tensor)."""
import numpy as np
import pytest
import torch

from helpers import assert_close, canaried, decode_case, host, prefill_case, tail_ok

import oracle.attention as oat
import oracle.kv as okv

pytestmark = pytest.mark.gpu

@pytest.mark.parametrize("D", [8, 40, 72, 80, 112])
@pytest.mark.parametrize("H,KV", [(32, 8), (14, 2)])
@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_decode_padded_head_sizes(gpu, D, H, KV, layout):
    """Fused KV write + decode at head sizes that are not a multiple of 32,
    unsplit, fixed partitions, balanced and shared balanced splits."""
    from vllm_apple_amd import kernels

    lens = [1, 15, 17, 300, 1000, 2096]
    kc, vc, bt, L, q, nk, nv = decode_case(6, H, KV, D, lens, layout, seed=D + H)
    scale = 1.0 / np.sqrt(D)
    kr, vr = host(kc).copy(), host(vc).copy()
    okv.kv_write_decode(kr, vr, host(nk), host(nv), host(bt), host(L), layout)
    ref = oat.decode(host(q), kr, vr, host(bt), host(L), scale, layout)
    for part in (0, 128, kernels.PARTITION_BALANCED, kernels.PARTITION_BALANCED_SHARED):
        print(f"[case] decode D={D} H={H} KV={KV} {layout} part={part}", flush=True)
        kb, kd = canaried(kc)
        vb, vd = canaried(vc)
        ob, out = canaried(torch.zeros(q.shape, dtype=torch.float16))
        kernels.paged_decode(q.cuda(), kd, vd, bt.cuda(), L.cuda(), scale=scale,
                             max_seq_len=max(lens), layout=layout, output=out,
                             new_keys=nk.cuda(), new_values=nv.cuda(), partition_size=part)
        torch.cuda.synchronize()
        assert_close(host(out), ref, what=f"decode D={D} {layout} part={part}")
        assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16)), "fused K write"
        assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16)), "fused V write"
        assert tail_ok(kb) and tail_ok(vb) and tail_ok(ob), "write past the last row"


def test_decode_padded_unfused_and_seq_len_one(gpu):
    """Unfused decode reads the cache only; L = 1 returns the new V exactly
    (test_metal_kernels.py:380-438) at D = 80."""
    from vllm_apple_amd import kernels

    kc, vc, bt, L, q, nk, nv = decode_case(3, 16, 4, 80, [1, 700, 1], "kernel", seed=5)
    out = kernels.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), L.cuda(),
                               scale=1 / np.sqrt(80), max_seq_len=700, new_keys=nk.cuda(),
                               new_values=nv.cuda())
    torch.cuda.synchronize()
    o = host(out)
    for s in (0, 2):
        for h in range(16):
            assert np.array_equal(o[s, h].view(np.uint16), host(nv)[s, h // 4].view(np.uint16))
    kd = kc.cuda()
    out = kernels.paged_decode(q.cuda(), kd, vc.cuda(), bt.cuda(), L.cuda(),
                               scale=1 / np.sqrt(80), max_seq_len=700)
    torch.cuda.synchronize()
    ref = oat.decode(host(q), host(kc), host(vc), host(bt), host(L), 1 / np.sqrt(80), "kernel")
    assert_close(host(out), ref, what="unfused D=80")
    assert np.array_equal(host(kd).view(np.uint16), host(kc).view(np.uint16))


@pytest.mark.parametrize("D", [8, 40, 80, 112])
@pytest.mark.parametrize("H,KV", [(32, 8), (14, 2), (8, 8)])
@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_prefill_padded_head_sizes(gpu, D, H, KV, layout):
    """Chunked prefill (prefix + causal chunk) at padded head sizes, unsplit
    and with the key split; every row against the fp64 oracle."""
    from vllm_apple_amd import kernels

    ctx, new = [77, 1500, 40, 700], [40, 96, 40, 33]
    kc, vc, bt, tok, pos, q = prefill_case(ctx, new, H, KV, D, layout, seed=3 * D + H)
    scale = 1.0 / np.sqrt(D)
    ref, written = oat.prefill(host(q), host(kc), host(vc), host(bt), host(tok), host(pos),
                               scale, layout)
    assert written.all()
    for split in (0, 256):
        print(f"[case] prefill D={D} H={H} KV={KV} {layout} split={split}", flush=True)
        ob, out = canaried(torch.zeros(q.shape, dtype=torch.float16))
        kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok.cuda(), pos.cuda(),
                              scale=scale, layout=layout, output=out, split_keys=split,
                              max_seq_len=max(ctx))
        torch.cuda.synchronize()
        assert_close(host(out), ref, what=f"prefill D={D} {layout} split={split}")
        assert tail_ok(ob), "write past the last output row"


@pytest.mark.parametrize("D", [40, 80, 112])
def test_kv_write_slots_padded_head_sizes(gpu, D):
    """The slot-mapping KV write at these head sizes, bit-exact with padding
    slots skipped, nothing written past the cache."""
    from vllm_apple_amd import kernels

    g = torch.Generator().manual_seed(D)
    nb, KV, bs, T = 40, 4, 16, 300
    kc = torch.randn(nb, KV, bs, D, generator=g).half()
    vc = torch.randn(nb, KV, bs, D, generator=g).half()
    k = torch.randn(T, KV, D, generator=g).half()
    v = torch.randn(T, KV, D, generator=g).half()
    perm = torch.randperm(nb * bs, generator=g).to(torch.int64)
    last = int((perm == nb * bs - 1).nonzero()[0])
    perm[0], perm[last] = nb * bs - 1, perm[0].item()  # the pool's last row, once
    slots = perm[:T].clone()
    slots[1::7] = -1
    kb, kd = canaried(kc)
    vb, vd = canaried(vc)
    kernels.kv_write_slots(k.cuda(), v.cuda(), kd, vd, slots.cuda())
    torch.cuda.synchronize()
    kr, vr = host(kc).copy(), host(vc).copy()
    okv.kv_write_slots(kr, vr, host(k), host(v), host(slots))
    assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16))
    assert tail_ok(kb) and tail_ok(vb)
