"""Split-K chunked prefill (vaa_paged_attention_prefill_split) vs the oracle.

The key range of each context is cut into pieces of split_keys positions,
the pieces run as separate workgroups and a log-sum-exp merge combines them
(the partition/merge structure of paged_attention_v2.metal:49-261 applied to
the prefill semantics of :375-478).  Every case prints its name before
touching the GPU.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, host
from test_gpu_prefill import _prefill_case

import oracle.attention as oat

pytestmark = pytest.mark.gpu


def _run_split(kc, vc, bt, tok, pos, q, split, layout="kernel", max_seq_len=0,
               dtype=torch.float16):
    from vllm_apple_amd import kernels

    D = q.shape[2]
    scale = 1.0 / np.sqrt(D)
    kd, vd, qd = kc.to(dtype).cuda(), vc.to(dtype).cuda(), q.to(dtype).cuda()
    sentinel = torch.full(q.shape, 7.0, dtype=dtype, device="cuda")
    out = kernels.paged_prefill(qd, kd, vd, bt.cuda(), tok.cuda(), pos.cuda(), scale=scale,
                                layout=layout, output=sentinel, split_keys=split,
                                max_seq_len=max_seq_len)
    whole = kernels.paged_prefill(qd, kd, vd, bt.cuda(), tok.cuda(), pos.cuda(), scale=scale,
                                  layout=layout,
                                  output=torch.full(q.shape, 7.0, dtype=dtype, device="cuda"))
    torch.cuda.synchronize()

    def h(t):  # numpy has no bfloat16: bf16 goes to fp32 (exact)
        return host(t.float()) if t.dtype == torch.bfloat16 else host(t)

    ref, written = oat.prefill(h(qd), h(kd), h(vd), host(bt), host(tok), host(pos), scale,
                               layout)
    return h(out), h(whole), ref, written


@pytest.mark.parametrize("split", [64, 1024, 4096])
@pytest.mark.parametrize("D,H,KV", [(128, 32, 8), (64, 14, 2), (96, 8, 8)])
def test_split_unequal_contexts(gpu, split, D, H, KV):
    print(f"[case] split={split} D={D} H={H} KV={KV}", flush=True)
    kc, vc, bt, tok, pos, q = _prefill_case([5000, 150, 2100, 64], [96, 40, 64, 30], H, KV, D,
                                            seed=split + D)
    out, whole, ref, w = _run_split(kc, vc, bt, tok, pos, q, split)
    assert w.all()
    assert_close(out, ref, what=f"split {split}")
    # the same rows as the unsplit kernel, up to the merge's rounding
    assert_close(out, whole.astype(np.float64), atol=1e-3, rtol=5e-3, what="split vs whole")


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_split_c5_like_batch(gpu, layout):
    """C5's prefill shape: 8 chunks of 256 tokens over contexts up to 16k,
    split as the chooser picks, every row against the oracle."""
    from vllm_apple_amd import kernels

    print(f"[case] C5-like split layout={layout}", flush=True)
    ctx = [16000, 600, 900, 2000, 3000, 1200, 800, 700]
    kc, vc, bt, tok, pos, q = _prefill_case(ctx, [256] * 8, 32, 8, 128, seed=21, layout=layout)
    split = kernels.choose_prefill_split(ctx, [256] * 8, 8, 32, 256)
    assert split > 0
    out, whole, ref, w = _run_split(kc, vc, bt, tok, pos, q, split, layout=layout,
                                    max_seq_len=max(ctx))
    assert w.all()
    assert_close(out, ref, what="C5-like split")


def test_split_mixed_tiles_shuffled_and_bf16(gpu):
    """Tokens of several sequences in one tile, shuffled, bf16 storage."""
    print("[case] split mixed tiles bf16", flush=True)
    kc, vc, bt, tok, pos, q = _prefill_case([700, 5, 1500, 9, 300], [7, 5, 11, 3, 30], 16, 4, 64,
                                            seed=6)
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(tok.numel(), generator=g)
    out, whole, ref, w = _run_split(kc, vc, bt, tok[perm].contiguous(), pos[perm].contiguous(),
                                    q[perm].contiguous(), 256, dtype=torch.bfloat16)
    assert w.all()
    assert_close(out.astype(np.float32), ref, what="split mixed tiles bf16")


def test_split_unwritten_rows(gpu):
    """Invalid sequence / negative position / an invalid block inside a long
    context: the same rows as the unsplit kernel stay untouched, in every
    split (the abort mark travels with split 0's partial)."""
    print("[case] split unwritten rows", flush=True)
    kc, vc, bt, tok, pos, q = _prefill_case([2600, 300], [80, 60], 8, 2, 128, seed=11)
    tok[0] = -1
    pos[1] = -4
    bt[0, 2500 // 16] = -1  # rows of sequence 0 at positions >= 2496 abort
    out, whole, ref, w = _run_split(kc, vc, bt, tok, pos, q, 512)
    p, t = pos.numpy(), tok.numpy()
    expect = (t >= 0) & (p >= 0) & np.where(t == 0, p < (2500 // 16) * 16, True)
    assert np.array_equal(w, expect) and (~w).any() and w.any()
    assert np.all(out[~w] == np.float16(7.0))
    assert np.array_equal(out[~w], whole[~w])
    assert_close(out[w], ref[w], what="split valid rows")


def test_split_contexts_past_max_seq_len(gpu):
    """A max_seq_len below the longest context: the last split takes the
    excess and the rows stay exact."""
    print("[case] split past max_seq_len", flush=True)
    kc, vc, bt, tok, pos, q = _prefill_case([3000, 200], [64, 64], 8, 2, 64, seed=13)
    out, whole, ref, w = _run_split(kc, vc, bt, tok, pos, q, 1024, max_seq_len=1500)
    assert w.all()
    assert_close(out, ref, what="split past max_seq_len")
