"""The allocation-free decode entry point (vaa_paged_attention_decode_noalloc)
through the C ABI, against vaa_paged_attention_decode with a caller
workspace: bit-identical outputs and fused cache writes on two calls in a
row, the second smaller, in every split mode that fits the fixed array; a
split that does not fit is refused before anything runs."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(S, H, KV, D, lens, seed, bs=16):
    g = torch.Generator().manual_seed(seed)
    nblk = [(L + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 8
    kc = torch.randn(nb, KV, bs, D, generator=g).half()
    vc = torch.randn(nb, KV, bs, D, generator=g).half()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((S, max(nblk)), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    q = torch.randn(S, H, D, generator=g).half()
    nk = torch.randn(S, KV, D, generator=g).half()
    nv = torch.randn(S, KV, D, generator=g).half()
    return [t.cuda() for t in (kc, vc, bt, torch.tensor(lens, dtype=torch.int32), q, nk, nv)]


def _params(kc, vc, q, out, nk, lens, bt, part):
    from vllm_apple_amd import kernels

    return kernels.make_params(key_cache=kc, value_cache=vc, layout="kernel",
                               num_query_heads=q.shape[1], scale=1 / np.sqrt(q.shape[2]),
                               num_seqs=lens.numel(), max_seq_len=int(lens.max()),
                               max_blocks_per_seq=bt.shape[1], query=q, output=out, new_kv=nk,
                               partition_size=part)


def _both(case, part):
    """(out, K, V) from the workspace entry point and from the no-alloc one,
    each on its own copy of the caches."""
    from vllm_apple_amd import _lib

    kc, vc, bt, lens, q, nk, nv = case
    stream = _lib.stream_handle()
    res = []
    for noalloc in (False, True):
        k, v = kc.clone(), vc.clone()
        out = torch.full_like(q, 7.0)
        p = _params(k, v, q, out, nk, lens, bt, part)
        args = [ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(),
                lens.data_ptr(), out.data_ptr(), nk.data_ptr(), nv.data_ptr()]
        if noalloc:
            _lib.call("vaa_paged_attention_decode_noalloc", *args, stream)
        else:
            part_out = ctypes.c_int32(0)
            n = _lib.load().vaa_paged_attention_decode_workspace_size(ctypes.byref(p),
                                                                       ctypes.byref(part_out))
            ws = torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")
            _lib.call("vaa_paged_attention_decode", *args, ws.data_ptr(), n, stream)
        res.append((out, k, v))
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize("part", [0, 128, 512, -1, -2])
def test_noalloc_matches_workspace_entry_point(gpu, part):
    first = _case(9, 32, 8, 128, [5000, 1, 0, 300, 8192, 2049, 77, 4000, 16], seed=1)
    second = _case(3, 32, 8, 128, [700, 33, 1500], seed=2)
    print(f"[case] noalloc part={part}", flush=True)
    for case in (first, second):
        (o1, k1, v1), (o2, k2, v2) = _both(case, part)
        assert torch.equal(o1, o2), f"outputs differ (part={part})"
        assert torch.equal(k1, k2) and torch.equal(v1, v2), "fused writes differ"
        assert not torch.any(o2 == 7.0), "rows left unwritten"


def test_noalloc_refuses_oversized_split(gpu):
    from vllm_apple_amd import _lib

    cap = _lib.load().vaa_paged_attention_decode_noalloc_max_workspace()
    assert cap == 32 << 20
    # 64 sequences of 32768 tokens in 128-token partitions: 64 * 32 * 256
    # partial rows of 130 floats = 272 MB > the fixed array.
    kc = torch.zeros(8, 8, 16, 128, dtype=torch.float16, device="cuda")
    q = torch.zeros(64, 32, 128, dtype=torch.float16, device="cuda")
    lens = torch.full((64,), 32768, dtype=torch.int32, device="cuda")
    bt = torch.zeros(64, 2048, dtype=torch.int32, device="cuda")
    out = torch.zeros_like(q)
    p = _params(kc, kc, q, out, None, lens, bt, 128)
    with pytest.raises(ValueError, match="fixed"):
        _lib.call("vaa_paged_attention_decode_noalloc", ctypes.byref(p), q.data_ptr(),
                  kc.data_ptr(), kc.data_ptr(), bt.data_ptr(), lens.data_ptr(), out.data_ptr(),
                  None, None, _lib.stream_handle())
    torch.cuda.synchronize()
    assert not torch.any(out)
