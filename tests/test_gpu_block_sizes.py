"""Block sizes that are not a multiple of 16, as the reference's engine ops
take any block_size (engine/ops/attention.py:175-228; its kernels walk the
tokens of a block one at a time, paged_attention_v2.metal:67-160).  A
16-token tile then spans several blocks and each of its rows finds its own
block.  Every output row is checked against the fp64 oracle, the fused KV
write bit for bit over the whole cache, nothing is written past the last row
of an output or cache, and missing blocks follow the reference's rules
(decode skips their tokens; prefill leaves the rows that reach one
unwritten)."""
import numpy as np
import pytest
import torch

from helpers import assert_close, canaried, decode_case, host, prefill_case, tail_ok

import oracle.attention as oat
import oracle.kv as okv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bs", [1, 8, 12, 24, 40])
@pytest.mark.parametrize("D,H,KV", [(128, 32, 8), (64, 14, 2)])
@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_decode_block_sizes(gpu, bs, D, H, KV, layout):
    """Fused KV write + decode, unsplit, fixed partitions, balanced and
    shared balanced splits."""
    from vllm_apple_amd import kernels

    lens = [1, 15, 17, 300, 1000, 2096]
    kc, vc, bt, L, q, nk, nv = decode_case(6, H, KV, D, lens, layout, seed=bs + D, bs=bs)
    scale = 1.0 / np.sqrt(D)
    kr, vr = host(kc).copy(), host(vc).copy()
    okv.kv_write_decode(kr, vr, host(nk), host(nv), host(bt), host(L), layout)
    ref = oat.decode(host(q), kr, vr, host(bt), host(L), scale, layout)
    for part in (0, 128, kernels.PARTITION_BALANCED, kernels.PARTITION_BALANCED_SHARED):
        print(f"[case] decode bs={bs} D={D} H={H} KV={KV} {layout} part={part}", flush=True)
        kb, kd = canaried(kc)
        vb, vd = canaried(vc)
        ob, out = canaried(torch.zeros(q.shape, dtype=torch.float16))
        kernels.paged_decode(q.cuda(), kd, vd, bt.cuda(), L.cuda(), scale=scale,
                             max_seq_len=max(lens), layout=layout, output=out,
                             new_keys=nk.cuda(), new_values=nv.cuda(), partition_size=part)
        torch.cuda.synchronize()
        assert_close(host(out), ref, what=f"decode bs={bs} D={D} {layout} part={part}")
        assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16)), "fused K write"
        assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16)), "fused V write"
        assert tail_ok(kb) and tail_ok(vb) and tail_ok(ob), "write past the last row"


@pytest.mark.parametrize("bs", [8, 12])
def test_decode_block_sizes_missing_blocks(gpu, bs):
    """Missing blocks (table entries -1 or past the pool) inside a context
    mask exactly their tokens, also where a 16-token tile spans a missing and
    a present block."""
    from vllm_apple_amd import kernels

    lens = [200, 517, 64, 1000]
    kc, vc, bt, L, q, nk, nv = decode_case(4, 16, 4, 128, lens, "kernel", seed=bs, bs=bs)
    bt[0, 3] = -1
    bt[1, 5] = kc.shape[0] + 7
    bt[1, 6] = -1
    bt[3, 0] = -1
    scale = 1.0 / np.sqrt(128)
    ref = oat.decode(host(q), host(kc), host(vc), host(bt), host(L), scale, "kernel")
    for part in (0, 128, kernels.PARTITION_BALANCED):
        print(f"[case] decode missing blocks bs={bs} part={part}", flush=True)
        out = kernels.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), L.cuda(),
                                   scale=scale, max_seq_len=max(lens), partition_size=part)
        torch.cuda.synchronize()
        assert_close(host(out), ref, what=f"decode missing blocks bs={bs} part={part}")


@pytest.mark.parametrize("bs", [1, 8, 12, 24, 40])
@pytest.mark.parametrize("D,H,KV", [(128, 32, 8), (64, 14, 2), (80, 8, 8)])
@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_prefill_block_sizes(gpu, bs, D, H, KV, layout):
    """Chunked prefill (prefix + causal chunk), unsplit and with the key
    split."""
    from vllm_apple_amd import kernels

    ctx, new = [77, 1500, 40, 700], [40, 96, 40, 33]
    kc, vc, bt, tok, pos, q = prefill_case(ctx, new, H, KV, D, layout, seed=7 * bs + D, bs=bs)
    scale = 1.0 / np.sqrt(D)
    ref, written = oat.prefill(host(q), host(kc), host(vc), host(bt), host(tok), host(pos),
                               scale, layout)
    assert written.all()
    for split in (0, 256):
        print(f"[case] prefill bs={bs} D={D} H={H} KV={KV} {layout} split={split}", flush=True)
        ob, out = canaried(torch.zeros(q.shape, dtype=torch.float16))
        kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok.cuda(), pos.cuda(),
                              scale=scale, layout=layout, output=out, split_keys=split,
                              max_seq_len=max(ctx))
        torch.cuda.synchronize()
        assert_close(host(out), ref, what=f"prefill bs={bs} D={D} {layout} split={split}")
        assert tail_ok(ob), "write past the last output row"


@pytest.mark.parametrize("bs", [8, 12])
def test_prefill_block_sizes_missing_block(gpu, bs):
    """A missing block inside a context: rows whose context reaches it are
    left unwritten (paged_attention_v2.metal:428), the rows before it are
    computed normally."""
    from vllm_apple_amd import kernels

    ctx, new = [300, 160], [120, 64]
    kc, vc, bt, tok, pos, q = prefill_case(ctx, new, 32, 8, 128, "kernel", seed=bs, bs=bs)
    bt[0, 250 // bs] = -1
    scale = 1.0 / np.sqrt(128)
    ref, written = oat.prefill(host(q), host(kc), host(vc), host(bt), host(tok), host(pos),
                               scale, "kernel")
    assert not written.all() and written.any()
    for split in (0, 64):
        print(f"[case] prefill missing block bs={bs} split={split}", flush=True)
        fill = torch.full(q.shape, 3.0, dtype=torch.float16)
        out = fill.cuda()
        kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok.cuda(), pos.cuda(),
                              scale=scale, output=out, split_keys=split, max_seq_len=max(ctx))
        torch.cuda.synchronize()
        o = host(out)
        assert_close(o[written], ref[written], what=f"prefill missing block bs={bs}")
        assert (o[~written] == 3.0).all(), "rows reaching the missing block were written"


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.float16).numpy()


def _bf16_from_bits(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(a.copy()).view(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("bs", [8, 24])
def test_bf16_block_sizes(gpu, bs):
    """bf16 caches at block sizes that are not a multiple of 16: fused-write
    decode in every split mode and prefill with the key split, against the
    fp64 oracle on the bf16 values (the bound plus the bf16 output rounding)."""
    from helpers import assert_close_bf16
    from vllm_apple_amd import kernels

    lens = [1, 17, 300, 1000, 2096]
    kc, vc, bt, L, q, nk, nv = decode_case(5, 32, 8, 128, lens, "kernel", seed=bs, bs=bs)
    kc, vc, q, nk, nv = (t.bfloat16() for t in (kc, vc, q, nk, nv))
    scale = 1.0 / np.sqrt(128)
    kr, vr = _bf16_bits(kc).copy(), _bf16_bits(vc).copy()
    okv.kv_write_decode(kr, vr, _bf16_bits(nk), _bf16_bits(nv), host(bt), host(L), "kernel")
    ref = oat.decode(q.float().numpy(), _bf16_from_bits(kr), _bf16_from_bits(vr), host(bt),
                     host(L), scale, "kernel")
    for part in (0, 128, kernels.PARTITION_BALANCED):
        print(f"[case] bf16 decode bs={bs} part={part}", flush=True)
        kd, vd = kc.cuda(), vc.cuda()
        out = kernels.paged_decode(q.cuda(), kd, vd, bt.cuda(), L.cuda(), scale=scale,
                                   max_seq_len=max(lens), new_keys=nk.cuda(),
                                   new_values=nv.cuda(), partition_size=part)
        torch.cuda.synchronize()
        assert_close_bf16(out.float().cpu().numpy(), ref, what=f"bf16 decode bs={bs} part={part}")
        assert np.array_equal(_bf16_bits(kd).view(np.uint16), kr.view(np.uint16)), "fused K"
        assert np.array_equal(_bf16_bits(vd).view(np.uint16), vr.view(np.uint16)), "fused V"

    ctx, new = [77, 1500, 700], [40, 96, 33]
    kc, vc, bt, tok, pos, q = prefill_case(ctx, new, 32, 8, 128, "kernel", seed=bs + 1, bs=bs)
    kc, vc, q = kc.bfloat16(), vc.bfloat16(), q.bfloat16()
    ref, written = oat.prefill(q.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                               host(bt), host(tok), host(pos), scale, "kernel")
    assert written.all()
    for split in (0, 256):
        print(f"[case] bf16 prefill bs={bs} split={split}", flush=True)
        out = kernels.paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), tok.cuda(),
                                    pos.cuda(), scale=scale, split_keys=split,
                                    max_seq_len=max(ctx))
        torch.cuda.synchronize()
        assert_close_bf16(out.float().cpu().numpy(), ref, what=f"bf16 prefill bs={bs}")
