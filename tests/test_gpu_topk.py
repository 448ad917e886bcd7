"""Top-k logits selection (vaa_topk_logits) against the oracle: indices and
value bits exact, including heavy ties, bf16, strided rows, odd vocab sizes."""
import numpy as np
import pytest
import torch

import oracle.topk as otk

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("V", [32000, 32768, 151936, 1001, 8, 32001])
@pytest.mark.parametrize("k", [1, 8, 50, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_topk_random_rows(gpu, V, k, dtype):
    from vllm_apple_amd import kernels

    print(f"[case] topk V={V} k={k} {dtype}", flush=True)
    g = torch.Generator().manual_seed(V + k)
    logits = (torch.randn(9, V, generator=g) * 4).to(dtype)
    if k > V:  # more than the vocabulary: refused before any launch
        with pytest.raises(ValueError, match="must be in 1"):
            kernels.topk_logits(logits.cuda(), k)
        return
    idx, vals = kernels.topk_logits(logits.cuda(), k)
    torch.cuda.synchronize()
    ref_idx, ref_vals = otk.topk(_bits(logits), k)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.array_equal(_bits(vals), ref_vals)


def test_topk_many_rows_one_chunk_each(gpu):
    """A batch that fills the GPU with one workgroup (or, with 2048 rows and
    more at k <= 64, one wave) per row: no workspace, no merge launch,
    including rows shorter than the register slices."""
    from vllm_apple_amd import kernels

    for T, V, k in ((1500, 3000, 50), (1100, 4096, 256), (2000, 77, 5), (5000, 3000, 50)):
        print(f"[case] topk one-chunk T={T} V={V} k={k}", flush=True)
        assert kernels.topk_workspace_size(T, V, k) == 0
        g = torch.Generator().manual_seed(T)
        logits = (torch.randn(T, V, generator=g) * 3).half()
        idx, vals = kernels.topk_logits(logits.cuda(), k)
        torch.cuda.synchronize()
        ref_idx, ref_vals = otk.topk(_bits(logits), k)
        assert np.array_equal(idx.cpu().numpy(), ref_idx)
        assert np.array_equal(_bits(vals), ref_vals)


def test_topk_heavy_ties_and_specials(gpu):
    """Few distinct values (ties decided by lower column), infinities, signed
    zeros, and a row that is constant."""
    from vllm_apple_amd import kernels

    rng = np.random.default_rng(3)
    x = rng.integers(-2, 3, size=(5, 20000)).astype(np.float16)
    x[1, 17] = np.inf
    x[1, 30:40] = -np.inf
    x[2, :] = np.float16(0.0)
    x[2, 5::2] = np.float16(-0.0)
    x[3, :] = np.float16(1.5)
    bits = x.view(np.uint16)
    t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.float16).cuda()
    for k in (1, 7, 64, 256):
        idx, vals = kernels.topk_logits(t, k)
        torch.cuda.synchronize()
        ref_idx, ref_vals = otk.topk(bits, k)
        assert np.array_equal(idx.cpu().numpy(), ref_idx), f"k={k}"
        assert np.array_equal(_bits(vals), ref_vals), f"k={k}"


def test_topk_strided_rows_and_outputs(gpu):
    from vllm_apple_amd import kernels

    g = torch.Generator().manual_seed(5)
    big = torch.randn(7, 4096 + 64, generator=g).half().cuda()
    logits = big[:, :4096]  # row stride 4160
    idx_buf = torch.full((7, 80), -7, dtype=torch.int32, device="cuda")
    val_buf = torch.zeros((7, 80), dtype=torch.float16, device="cuda")
    kernels.topk_logits(logits, 50, indices=idx_buf[:, :50], values=val_buf[:, :50])
    torch.cuda.synchronize()
    ref_idx, ref_vals = otk.topk(_bits(logits.contiguous()), 50)
    assert np.array_equal(idx_buf[:, :50].cpu().numpy(), ref_idx)
    assert np.array_equal(_bits(val_buf[:, :50].contiguous()), ref_vals)
    assert torch.all(idx_buf[:, 50:] == -7), "columns past k untouched"


def test_engine_topk_encode_and_reconstruct(gpu, monkeypatch):
    """EngineTopK.encode into (buffer, byte offset) outputs inside an ENCODE
    phase, then the runner's -inf reconstruction of the full rows."""
    from vllm_apple_amd.engine import EngineStepContext, EngineTopK, reconstruct_logits

    monkeypatch.setenv("VLLM_METAL_TOPK_K", "40")
    op = EngineTopK(None)
    assert op.k == 40
    T, V = 6, 5000
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(T, V, generator=g).half()
    lbuf = torch.zeros(64 + T * V, dtype=torch.float16, device="cuda")
    lbuf[64:] = logits.reshape(-1).cuda()
    ibuf = torch.zeros(16 + T * 40, dtype=torch.int32, device="cuda")
    vbuf = torch.zeros(16 + T * 40, dtype=torch.float16, device="cuda")
    ctx = EngineStepContext()
    with pytest.raises(RuntimeError):
        op.encode(ctx, (lbuf, 128), (ibuf, 64), (vbuf, 32), T, V)
    with ctx:
        op.encode(ctx, (lbuf, 128), (ibuf, 64), (vbuf, 32), T, V)
    torch.cuda.synchronize()
    idx = ibuf[16:].view(T, 40)
    vals = vbuf[16:].view(T, 40)
    ref_idx, ref_vals = otk.topk(_bits(logits), 40)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.array_equal(_bits(vals), ref_vals)
    full = reconstruct_logits(idx, vals, V).cpu()
    keep = torch.zeros(T, V, dtype=torch.bool)
    keep.scatter_(1, torch.from_numpy(ref_idx).long(), True)
    assert torch.equal(full[keep], logits[keep])
    assert torch.all(torch.isneginf(full[~keep]))


@pytest.mark.parametrize("T,k", [(256, 50), (64, 50), (32, 64), (40, 1)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_topk_bench_shape_one_wave_paths(gpu, T, k, dtype):
    """The bench's vocabulary (128256) at k <= 64, where each chunk and each
    row's merge runs on one wave: every row against the oracle, with some rows
    flat or tied so that the chunk and merge lists overflow and take the
    exact-key and ordered-compaction paths."""
    from vllm_apple_amd import kernels

    print(f"[case] topk bench shape T={T} k={k} {dtype}", flush=True)
    V = 128256
    g = torch.Generator().manual_seed(T * 1000 + k)
    logits = (torch.randn(T, V, generator=g) * 4).to(dtype)
    logits[1] = 0.5                                   # flat row: ties everywhere
    logits[2] = torch.randint(-2, 3, (V,), generator=g).to(dtype)  # five distinct values
    logits[3, ::97] = float("inf")                    # many equal maxima
    logits[4] = -float("inf")
    logits[4, 5000:5000 + 3] = 1.0
    assert kernels.topk_workspace_size(T, V, k) > 0   # chunked: the merge runs
    idx, vals = kernels.topk_logits(logits.cuda(), k)
    torch.cuda.synchronize()
    ref_idx, ref_vals = otk.topk(_bits(logits), k)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.array_equal(_bits(vals), ref_vals)


def test_topk_wave_path_ragged_tail_strided(gpu):
    """The one-wave-per-chunk path on strided rows whose length is not a
    multiple of 8 (the last chunk's tail is read element by element) and at
    k = 64, its largest k, with enough rows for the wave kernel."""
    from vllm_apple_amd import kernels

    T, V, k = 1400, 10001, 64
    print(f"[case] topk wave tail T={T} V={V} k={k}", flush=True)
    g = torch.Generator().manual_seed(17)
    big = (torch.randn(T, V + 7, generator=g) * 3).half()
    big[:, V - 1] = 30.0          # the tail's last column is every row's maximum
    big[::5, V - 3:V] = 30.0      # ties inside the tail
    logits = big.cuda()[:, :V]    # row stride V + 7 = 10008, a multiple of 8
    idx, vals = kernels.topk_logits(logits, k)
    torch.cuda.synchronize()
    ref_idx, ref_vals = otk.topk(_bits(big[:, :V].contiguous()), k)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.array_equal(_bits(vals), ref_vals)
