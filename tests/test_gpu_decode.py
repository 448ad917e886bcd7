"""Paged decode attention (fused KV write, GQA, split-K + LSE merge) vs the oracle."""
import numpy as np
import pytest
import torch

from helpers import assert_close, bf16_half_ulp, host

import oracle.attention as oat
import oracle.kv as okv

pytestmark = pytest.mark.gpu


def _case(S, H, KV, D, lens, nb=None, bs=16, layout="kernel", seed=0, maxb=None):
    g = torch.Generator().manual_seed(seed)
    nblk = [(L + bs - 1) // bs for L in lens]
    maxb = maxb or max(max(nblk), 1)
    nb = nb or max(sum(nblk) + 4, 8)
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = torch.randn(shape, generator=g).half()
    vc = torch.randn(shape, generator=g).half()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((S, maxb), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    q = torch.randn(S, H, D, generator=g).half()
    nk = torch.randn(S, KV, D, generator=g).half()
    nv = torch.randn(S, KV, D, generator=g).half()
    return kc, vc, bt, torch.tensor(lens, dtype=torch.int32), q, nk, nv


def _run(kc, vc, bt, lens, q, nk, nv, *, layout="kernel", fused=True, part=0, scale=None):
    from vllm_apple_amd import kernels

    D = q.shape[2]
    scale = scale or 1.0 / np.sqrt(D)
    kd, vd = kc.cuda(), vc.cuda()
    out = kernels.paged_decode(q.cuda(), kd, vd, bt.cuda(), lens.cuda(), scale=scale,
                               max_seq_len=int(lens.max()) if lens.numel() else 0,
                               layout=layout, new_keys=nk.cuda() if fused else None,
                               new_values=nv.cuda() if fused else None, partition_size=part)
    torch.cuda.synchronize()
    # Oracle: write the new token first (when fused), then attend.
    kc_ref, vc_ref = host(kc).copy(), host(vc).copy()
    if fused:
        okv.kv_write_decode(kc_ref, vc_ref, host(nk), host(nv), host(bt), host(lens), layout)
    ref = oat.decode(host(q), kc_ref, vc_ref, host(bt), host(lens), scale, layout)
    return out, ref, kd, vd, kc_ref, vc_ref


@pytest.mark.parametrize("part", [0, 128, 256, 512, -1])
def test_decode_c1_shape(gpu, part):
    """C1 shape (14q/2kv, D64, GQA 7), fused write, several partition sizes."""
    lens = [37, 512, 16, 201]
    print(f"[case] C1 part={part}", flush=True)
    kc, vc, bt, L, q, nk, nv = _case(4, 14, 2, 64, lens, nb=256, seed=1, maxb=32)
    out, ref, kd, vd, kr, vr = _run(kc, vc, bt, L, q, nk, nv, part=part, scale=1 / 8)
    assert_close(host(out), ref, what="decode C1")
    assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16)), "fused K write"
    assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16)), "fused V write"


@pytest.mark.parametrize("layout", ["kernel", "vllm"])
def test_decode_c2_shape_uniform(gpu, layout):
    """C2 shape (32q/8kv, D128) with U{1024..8192} contexts, 6 sequences."""
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(1024, 8193, (6,), generator=g).tolist()
    print(f"[case] C2 layout={layout} lens={lens}", flush=True)
    kc, vc, bt, L, q, nk, nv = _case(6, 32, 8, 128, lens, seed=2, layout=layout)
    out, ref, kd, vd, kr, vr = _run(kc, vc, bt, L, q, nk, nv, layout=layout)
    assert_close(host(out), ref, what=f"decode C2 {layout}")
    assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16))


@pytest.mark.parametrize("D", [32, 64, 96, 128])
@pytest.mark.parametrize("H,KV", [(8, 8), (16, 4), (16, 2), (32, 2), (16, 1)])
def test_decode_head_shapes(gpu, D, H, KV):
    lens = [1, 15, 16, 17, 300, 1000]
    print(f"[case] shapes D={D} H={H} KV={KV}", flush=True)
    kc, vc, bt, L, q, nk, nv = _case(6, H, KV, D, lens, seed=3)
    for part in (128, -1):
        out, ref, *_ = _run(kc, vc, bt, L, q, nk, nv, part=part)
        assert_close(host(out), ref, what=f"decode D={D} H={H} KV={KV} part={part}")


@pytest.mark.parametrize("bs", [32, 64])
def test_decode_larger_block_size(gpu, bs):
    """block_size a multiple of 16 (tiles of 16 tokens inside larger blocks)."""
    lens = [1, 31, 33, 2000, 5000, 700]
    kc, vc, bt, L, q, nk, nv = _case(6, 32, 8, 128, lens, bs=bs, seed=13)
    for part in (0, 128, 1024, -1):
        out, ref, kd, vd, kr, vr = _run(kc, vc, bt, L, q, nk, nv, part=part)
        assert_close(host(out), ref, what=f"decode bs={bs} part={part}")
        assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16))


def test_decode_long_contexts_many_windows(gpu):
    """Runs longer than one 64-block window per wave (C4-like lengths)."""
    lens = [32768, 20000, 4096, 9999]
    kc, vc, bt, L, q, nk, nv = _case(4, 32, 8, 128, lens, seed=14)
    for part in (0, 8192, 32768, -1):
        out, ref, *_ = _run(kc, vc, bt, L, q, nk, nv, part=part)
        assert_close(host(out), ref, what=f"decode long part={part}")


def test_decode_unfused_reads_cache(gpu):
    lens = [100, 2000, 33]
    kc, vc, bt, L, q, nk, nv = _case(3, 32, 8, 128, lens, seed=4)
    out, ref, kd, vd, kr, vr = _run(kc, vc, bt, L, q, nk, nv, fused=False)
    assert_close(host(out), ref, what="decode unfused")
    assert np.array_equal(host(kd).view(np.uint16), host(kc).view(np.uint16))


def test_decode_seq_len_one_is_value_exact(gpu):
    """Known answer (tests/metal/test_metal_kernels.py:380-438): L=1 -> new V per GQA group."""
    kc, vc, bt, L, q, nk, nv = _case(1, 32, 4, 64, [1], nb=8, seed=5)
    out, *_ = _run(kc, vc, bt, L, q, nk, nv)
    expected = nv.repeat_interleave(8, dim=1)
    assert torch.equal(out.cpu(), expected)


def test_decode_zero_and_edge_lengths(gpu):
    lens = [0, 1, 16, 0, 4097]
    kc, vc, bt, L, q, nk, nv = _case(5, 16, 4, 128, lens, seed=6)
    for part in (256, -1):
        out, ref, *_ = _run(kc, vc, bt, L, q, nk, nv, part=part)
        assert_close(host(out), ref, what=f"decode edge lengths part={part}")
        assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[3]) == 0


def test_decode_split_matches_unsplit(gpu):
    lens = [5000, 3000, 7777]
    kc, vc, bt, L, q, nk, nv = _case(3, 32, 8, 128, lens, seed=7)
    a, ref, *_ = _run(kc, vc, bt, L, q, nk, nv, part=128)
    b, *_ = _run(kc, vc, bt, L, q, nk, nv, part=8192)
    c, *_ = _run(kc, vc, bt, L, q, nk, nv, part=-1)
    assert_close(host(a), ref, what="split 128")
    assert_close(host(b), ref, what="split 8192")
    assert_close(host(c), ref, what="balanced split")
    assert_close(host(a), host(b).astype(np.float64), what="split vs unsplit")
    assert_close(host(c), host(b).astype(np.float64), what="balanced vs unsplit")


def test_decode_outlier_keys_c4_style(gpu):
    """1% of key rows x8 (C4): softmax max-tracking across partitions."""
    lens = [9000, 4096, 12000]
    kc, vc, bt, L, q, nk, nv = _case(3, 32, 8, 128, lens, seed=8)
    g = torch.Generator().manual_seed(9)
    flat = kc.view(-1, 128)
    idx = torch.randint(0, flat.shape[0], (flat.shape[0] // 100,), generator=g)
    flat[idx] = (flat[idx].float() * 8).half()
    for part in (512, -1):
        out, ref, *_ = _run(kc, vc, bt, L, q, nk, nv, part=part)
        assert_close(host(out), ref, what=f"decode outliers part={part}")


def test_decode_invalid_block_is_masked(gpu):
    lens = [64, 64]
    kc, vc, bt, L, q, nk, nv = _case(2, 8, 2, 64, lens, seed=10)
    bt[0, 1] = -1
    bt[1, 2] = 10_000  # past capacity
    out, ref, *_ = _run(kc, vc, bt, L, q, nk, nv, fused=False)
    assert_close(host(out), ref, what="decode invalid blocks")


def test_decode_matches_pure_loop_oracle(gpu):
    """Small case against the token-serial fp32 loop that mirrors the Metal kernel."""
    lens = [45, 7]
    kc, vc, bt, L, q, nk, nv = _case(2, 4, 2, 32, lens, seed=12)
    out, *_ = _run(kc, vc, bt, L, q, nk, nv, fused=False)
    loop = oat.decode_loop_fp32(host(q), host(kc), host(vc), host(bt), host(L), 1 / np.sqrt(32))
    assert_close(host(out), loop, what="vs Metal-structured loop")


@pytest.mark.parametrize("mode", [-1, -2])
@pytest.mark.parametrize("seed", [21, 22])
def test_decode_balanced_ragged_batch(gpu, seed, mode):
    """Balanced split over many ragged sequences (empty ones included): every
    piece boundary (inside a sequence, between sequences, across workgroups)
    against the oracle, with the fused write bit-exact.  mode -1 is one
    8-wave workgroup per CU, -2 (shared) 4-wave workgroups, four per CU's
    worth of the split."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, 3000, (77,), generator=g)
    lens[::9] = 0
    lens[5] = 1
    lens = lens.tolist()
    print(f"[case] balanced ragged seed={seed} mode={mode}", flush=True)
    kc, vc, bt, L, q, nk, nv = _case(77, 16, 4, 128, lens, seed=seed)
    out, ref, kd, vd, kr, vr = _run(kc, vc, bt, L, q, nk, nv, part=mode)
    assert_close(host(out), ref, what="balanced ragged")
    assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16))
    assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16))
    zero = [i for i, n in enumerate(lens) if n == 0]
    assert torch.count_nonzero(out[zero]) == 0


def test_decode_balanced_workspace_reuse(gpu):
    """Two balanced calls in a row through one workspace, the second with fewer
    and shorter sequences: nothing from the first call leaks into the second."""
    from vllm_apple_amd import kernels

    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    for S, hi, seed in ((40, 9000, 31), (7, 700, 32)):
        g = torch.Generator().manual_seed(seed)
        lens = torch.randint(1, hi, (S,), generator=g).tolist()
        kc, vc, bt, L, q, nk, nv = _case(S, 32, 8, 128, lens, seed=seed)
        out = kernels.paged_decode(q.cuda(), kc.cuda(), vc.cuda(), bt.cuda(), L.cuda(),
                                   scale=1 / np.sqrt(128), max_seq_len=max(lens),
                                   partition_size=-2 if S == 7 else -1, workspace=ws)
        ref = oat.decode(host(q), host(kc), host(vc), host(bt), host(L), 1 / np.sqrt(128))
        assert_close(host(out), ref, what=f"balanced reuse S={S}")


def test_decode_graph_replay_after_workspace_growth(gpu):
    """A decode captured in a HIP graph keeps working after a later eager call
    grows the shared split-K workspace: the outgrown buffer stays allocated,
    so the replay neither reads freed memory nor writes into a tensor that
    was allocated after the growth."""
    from vllm_apple_amd import kernels

    torch.cuda.synchronize()
    small = [900, 1500, 300]
    kc, vc, bt, L, q, nk, nv = _case(3, 32, 8, 128, small, seed=41)
    kd, vd, btd, Ld, qd = kc.cuda(), vc.cuda(), bt.cuda(), L.cuda(), q.cuda()
    out = torch.empty_like(qd)
    kw = dict(scale=1 / np.sqrt(128), max_seq_len=max(small), partition_size=128)

    def step():
        kernels.paged_decode(qd, kd, vd, btd, Ld, output=out, **kw)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm-up: sizes the workspace for this call
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    # A longer eager decode needs a bigger workspace: the shared one grows.
    # Each 65536-token sequence needs 32 heads x 512 partitions x 130 floats.
    before = kernels.decode_workspace(0, qd.device)
    per_seq = 32 * 512 * 130 * 4
    n_big = before.numel() // per_seq + 1
    big = [65536 - 7 * i for i in range(n_big)]
    kc2, vc2, bt2, L2, q2, *_ = _case(n_big, 32, 2, 128, big, seed=42)
    kernels.paged_decode(q2.cuda(), kc2.cuda(), vc2.cuda(), bt2.cuda(), L2.cuda(),
                         scale=1 / np.sqrt(128), max_seq_len=max(big), partition_size=128)
    torch.cuda.synchronize()
    assert kernels.decode_workspace(0, qd.device).data_ptr() != before.data_ptr(), "no growth"
    del kc2, vc2, bt2, L2, q2, before
    # Tensors allocated after the growth, which may reuse freed blocks.
    sentinels = [torch.full((1 << 20,), 7.0, device="cuda") for _ in range(8)]
    ref = oat.decode(host(q), host(kc), host(vc), host(bt), host(L), 1 / np.sqrt(128))
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert_close(host(out), ref, what="graph replay after workspace growth")
        for t in sentinels:
            assert bool(torch.all(t == 7.0)), "a replay wrote into a later allocation"


@pytest.mark.parametrize("H,KV,D", [(48, 1, 128), (32, 1, 64), (40, 2, 128), (17, 1, 96),
                                    (64, 2, 32)])
def test_decode_wide_groups(gpu, H, KV, D):
    """GQA groups of more than 16 query heads (MQA with many heads): the group
    runs in chunks of at most 16 heads, each its own workgroup, against the
    oracle for the unsplit, fixed-partition and both balanced splits, with the
    fused write bit-exact (only the first chunk writes the new token)."""
    lens = [1, 16, 17, 700, 3000, 0, 4100]
    print(f"[case] wide groups H={H} KV={KV} D={D}", flush=True)
    kc, vc, bt, L, q, nk, nv = _case(len(lens), H, KV, D, lens, seed=50 + H)
    for part in (0, 128, 1024, -1, -2):
        out, ref, kd, vd, kr, vr = _run(kc, vc, bt, L, q, nk, nv, part=part)
        assert_close(host(out), ref, what=f"decode H={H} KV={KV} D={D} part={part}")
        assert np.array_equal(host(kd).view(np.uint16), kr.view(np.uint16)), "fused K write"
        assert np.array_equal(host(vd).view(np.uint16), vr.view(np.uint16)), "fused V write"
        assert torch.count_nonzero(out[5]) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_merge_attn_states(gpu, dtype):
    """vaa_merge_attn_states on partials of a split decode (computed exactly
    on the host) against the unsplit decode and the oracle merge, with
    ragged partition counts, empty sequences and chained LSE output."""
    from vllm_apple_amd import kernels

    lens = [0, 1, 300, 5000, 2047, 9000]
    kc, vc, bt, L, q, *_ = _case(len(lens), 32, 8, 128, lens, seed=61)
    scale = 1 / np.sqrt(128)
    po, lse, n = oat.decode_partials(host(q), host(kc), host(vc), host(bt), host(L), scale, 512)
    ref_out, ref_lse = oat.merge_states(po, lse, n)
    full = oat.decode(host(q), host(kc), host(vc), host(bt), host(L), scale)
    po_d = torch.from_numpy(po.astype(np.float32)).cuda()
    lse_d = torch.from_numpy(lse.astype(np.float32)).cuda()
    out_lse = torch.empty(lse.shape[:2], dtype=torch.float32, device="cuda")
    out = kernels.merge_attn_states(po_d, lse_d, num_parts=torch.from_numpy(n).cuda(),
                                    output_lse=out_lse, dtype=dtype)
    torch.cuda.synchronize()
    # fp16: the north-star bound; bf16: plus the bf16 output rounding.
    tol = {} if dtype == torch.float16 else dict(extra=bf16_half_ulp(full))
    assert_close(out.float().cpu().numpy(), full, what="merge vs unsplit decode", **tol)
    tol = {} if dtype == torch.float16 else dict(extra=bf16_half_ulp(ref_out))
    assert_close(out.float().cpu().numpy(), ref_out, what="merge vs oracle merge", **tol)
    got_lse = out_lse.cpu().numpy()
    assert np.all(np.isneginf(got_lse[0]))
    assert np.allclose(got_lse[1:], ref_lse[1:], rtol=1e-5, atol=1e-5)
    assert torch.count_nonzero(out[0]) == 0
    # Without num_parts the -inf partitions past each length are skipped too.
    out2 = kernels.merge_attn_states(po_d, lse_d, dtype=dtype)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
