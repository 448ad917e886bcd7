"""vaa_kv_stream_read (the read-only stream beside the decode roofline) on the
GPU: its checksum must equal the XOR of the same rows computed on the host,
bit for bit, in both cache layouts, with partial tiles, empty sequences and
invalid block-table entries."""
import numpy as np
import pytest
import torch

from helpers import host

pytestmark = pytest.mark.gpu


def _xor_rows(k, v, bt, lens, layout, piece=0):
    """Host checksum: XOR of every 32-bit word of the K and V rows of each
    (sequence, piece, kv head), pieces of `piece` tokens (0: the whole
    context), rows in invalid table entries skipped."""
    nb = k.shape[0]
    bs = k.shape[2] if layout == "kernel" else k.shape[1]
    kv = k.shape[1] if layout == "kernel" else k.shape[2]
    top = max(max(lens), 1)
    parts = -(-top // piece) if piece else 1
    out = np.zeros((len(lens), parts, kv), dtype=np.uint32)
    for s, L in enumerate(lens):
        for pos in range(max(L, 0)):
            bi = pos // bs
            if bi >= bt.shape[1]:
                break
            phys = int(bt[s, bi])
            if phys < 0 or phys >= nb:
                continue
            o, q = pos % bs, (pos // piece if piece else 0)
            for h in range(kv):
                for c in (k, v):
                    row = c[phys, h, o] if layout == "kernel" else c[phys, o, h]
                    out[s, q, h] ^= np.bitwise_xor.reduce(np.ascontiguousarray(row).view(np.uint32))
    return out


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
@pytest.mark.parametrize("kv,d,bs", [(8, 128, 16), (2, 64, 32), (4, 96, 16), (1, 32, 48)])
@pytest.mark.parametrize("piece", [0, 32, 48])
def test_kv_stream_checksum(gpu, layout, kv, d, bs, piece):
    from vllm_apple_amd import kernels

    print(f"[case] kv_stream layout={layout} kv={kv} d={d} bs={bs} piece={piece}", flush=True)
    g = torch.Generator().manual_seed(11)
    nb, max_blocks = 128, 12
    shape = (nb, kv, bs, d) if layout == "kernel" else (nb, bs, kv, d)
    kc = torch.randn(shape, generator=g).half()
    vc = torch.randn(shape, generator=g).half()
    lens = [0, 1, 15, 16, 17, bs * max_blocks, 5 * bs + 3, -4, 2 * bs]
    bt = torch.randperm(nb, generator=g)[:len(lens) * max_blocks].view(len(lens), max_blocks)
    bt = bt.to(torch.int32).clone()
    bt[6, 2] = -1          # a missing block inside a context
    bt[8, 1] = nb + 5      # past the cache: skipped
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    ref = _xor_rows(host(kc), host(vc), host(bt), lens, layout, piece)
    sink = kernels.kv_stream_read(kc.cuda(), vc.cuda(), bt.cuda(), seq_lens.cuda(), layout=layout,
                                  partition_size=piece, max_seq_len=max(lens))
    torch.cuda.synchronize()
    got = host(sink).view(np.uint32)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]


def test_kv_stream_headline_shape(gpu):
    """The headline decode's tables (B=32, every context 8192, 8 kv heads,
    D128): the checksum of each (sequence, kv head) against a torch reduction
    of the gathered rows on the device."""
    from vllm_apple_amd import kernels, workloads

    print("[case] kv_stream headline", flush=True)
    b = workloads.c2_decode(device=torch.device("cuda:0"), fixed_len=8192)
    sink = kernels.kv_stream_read(b.k_cache, b.v_cache, b.block_table, b.seq_lens)
    L = 8192
    nblk = L // 16
    rows = b.block_table[:, :nblk].long()                     # [B, nblk]
    got = sink[:, 0].cpu()
    for c in (b.k_cache, b.v_cache):
        x = c[rows]                                           # [B, nblk, KV, 16, D]
        x = x.permute(0, 2, 1, 3, 4).reshape(x.shape[0], x.shape[2], -1)
        w = x.contiguous().view(torch.int32)
        while w.shape[-1] > 1:
            half = w.shape[-1] // 2
            w = torch.bitwise_xor(w[..., :half], w[..., half:2 * half])
        if c is b.k_cache:
            ref = w[..., 0]
        else:
            ref = torch.bitwise_xor(ref, w[..., 0])
    assert torch.equal(got, ref.cpu())


def test_kv_stream_rejects_bad_arguments(gpu):
    """Unsupported head sizes and piece sizes fail before any launch, with the
    library's status mapped to the Python exception."""
    from vllm_apple_amd import kernels

    print("[case] kv_stream errors", flush=True)
    dev = torch.device("cuda:0")
    bt = torch.zeros((2, 4), dtype=torch.int32, device=dev)
    lens = torch.tensor([16, 40], dtype=torch.int32, device=dev)
    k80 = torch.zeros((8, 2, 16, 80), dtype=torch.float16, device=dev)
    with pytest.raises(NotImplementedError, match="head_size=80"):
        kernels.kv_stream_read(k80, k80.clone(), bt, lens)
    k = torch.zeros((8, 2, 16, 64), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="partition_size=24"):
        kernels.kv_stream_read(k, k.clone(), bt, lens, partition_size=24, max_seq_len=40)
    with pytest.raises(ValueError, match="max_seq_len"):
        kernels.kv_stream_read(k, k.clone(), bt, lens, partition_size=32)
    with pytest.raises(ValueError, match="sink"):
        kernels.kv_stream_read(k, k.clone(), bt, lens,
                               sink=torch.zeros(3, dtype=torch.int32, device=dev))
