"""The gated-MLP up projection with the SwiGLU epilogue (vaa_gate_up_silu)
against the oracle (fp64 products, silu_mul of the unrounded values) within
the north-star tolerance, and against the reference's unfused order (two
GEMMs rounded to 16 bits, then silu_mul) within the rounding that the fusion
removes.  Covers 1, 2, 3, 5 and 7 k-steps (every end
position of the three-stage weight ring and the two-stage activation ring), token counts that leave a
partial token tile, fused and separate weights, strided rows and the C5 shape.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, host, assert_close_bf16

import oracle.layer_ops as olo

pytestmark = pytest.mark.gpu


def _inputs(T, H, I, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(dtype)
    w = (torch.randn(2 * I, H, generator=g) / H ** 0.5).to(dtype)
    return x, w


@pytest.mark.parametrize("T,H,I", [(1, 64, 128), (3, 128, 128), (37, 192, 256), (5, 320, 128),
                                   (70, 256, 128), (128, 320, 256), (100, 5120, 128),
                                   (129, 256, 128), (256, 320, 128), (300, 512, 384),
                                   (513, 448, 256), (1000, 1024, 512)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gate_up_silu_vs_oracle(gpu, T, H, I, dtype):
    from vllm_apple_amd import kernels

    print(f"[case] gate_up_silu T={T} H={H} I={I} {dtype}", flush=True)
    x, w = _inputs(T, H, I, dtype, T * 31 + H + I)
    xd, wd = x.cuda(), w.cuda()
    out = kernels.gate_up_silu(xd, wd)
    sep = kernels.gate_up_silu(xd, wd[:I].contiguous(), wd[I:].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), sep.view(torch.int16)), "fused vs separate"
    # The oracle takes the 16-bit inputs exactly (as fp64 for bf16).
    ref = olo.gate_up_silu(x.double().numpy(), w.double().numpy())
    if dtype == torch.float16:
        assert_close(host(out), ref, what=f"gate_up_silu {T}x{H}x{I}")
    else:  # bf16 outputs: the same bound plus the bf16 output rounding
        assert_close_bf16(out.cpu().double().numpy(), ref, what=f"gate_up_silu bf16 {T}x{H}x{I}")


def test_gate_up_silu_vs_unfused_reference_order(gpu):
    """The reference's order: gate and up GEMMs rounded to fp16, then
    silu_mul.  The fused output differs only by those two roundings."""
    from vllm_apple_amd import kernels

    print("[case] gate_up_silu vs unfused", flush=True)
    T, H, I = 129, 1024, 640
    x, w = _inputs(T, H, I, torch.float16, 3)
    xd, wd = x.cuda(), w.cuda()
    gu = (xd.float() @ wd.float().T).half()
    unfused = kernels.silu_mul(gu[:, :I], gu[:, I:])
    fused = kernels.gate_up_silu(xd, wd)
    torch.cuda.synchronize()
    assert_close(host(fused), host(unfused).astype(np.float64), atol=4e-3, rtol=4e-3,
                 what="fused vs unfused")


def test_gate_up_silu_strided_rows(gpu):
    """x a column window of a wider buffer, weights rows of a wider matrix,
    output rows padded: only the output window is written."""
    from vllm_apple_amd import kernels

    print("[case] gate_up_silu strided", flush=True)
    T, H, I = 70, 256, 256
    g = torch.Generator().manual_seed(11)
    xb = torch.randn(T, H + 64, generator=g).half()
    wb = (torch.randn(2 * I, H + 128, generator=g) / H ** 0.5).half()
    x, w = xb[:, 32:32 + H], wb[:, 64:64 + H]
    ob = torch.full((T, I + 8), 7.0, dtype=torch.float16).cuda()
    out = ob[:, :I]
    kernels.gate_up_silu(xb.cuda()[:, 32:32 + H], wb.cuda()[:, 64:64 + H], out=out)
    torch.cuda.synchronize()
    assert_close(host(out), olo.gate_up_silu(host(x), host(w)), what="strided")
    assert (host(ob[:, I:]) == 7.0).all(), "padding written"


def test_gate_up_silu_rejects_unsupported_shapes(gpu):
    from vllm_apple_amd import kernels

    print("[case] gate_up_silu errors", flush=True)
    x = torch.zeros(4, 96, dtype=torch.float16, device="cuda")
    with pytest.raises(Exception, match="multiple"):
        kernels.gate_up_silu(x, torch.zeros(256, 96, dtype=torch.float16, device="cuda"))
    x = torch.zeros(4, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(Exception, match="multiple"):
        kernels.gate_up_silu(x, torch.zeros(2 * 100, 128, dtype=torch.float16, device="cuda"))
    empty = kernels.gate_up_silu(torch.zeros(0, 128, dtype=torch.float16, device="cuda"),
                                 torch.zeros(256, 128, dtype=torch.float16, device="cuda"))
    assert empty.shape == (0, 128)


def test_gate_up_silu_c5_shape(gpu):
    """C5: 2104 tokens, hidden 5120, intermediate 32768.  Rows from the first
    and the last (partial) token tile and columns from the first, a middle and
    the last column tile against the oracle; every output finite."""
    from vllm_apple_amd import kernels

    print("[case] gate_up_silu C5 2104x5120x32768", flush=True)
    T, H, I = 2104, 5120, 32768
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(T, H, generator=g, device="cuda").half()
    w = (torch.randn(2 * I, H, generator=g, device="cuda") / H ** 0.5).half()
    out = kernels.gate_up_silu(x, w)
    torch.cuda.synchronize()
    o = host(out)
    assert np.isfinite(o.astype(np.float32)).all()
    rows = np.array([0, 1, 255, 256, 1031, 2047, 2048, 2100, 2103])
    cols = np.concatenate([np.arange(0, 128), np.arange(16384, 16512), np.arange(I - 128, I)])
    xs = host(x)[rows]
    wh = host(w)
    ref = olo.gate_up_silu(xs, wh[cols], wh[I + cols])
    assert_close(o[np.ix_(rows, cols)], ref, what="C5 rows x cols")


def test_gate_up_silu_graph_replays_match_eager(gpu):
    """Captured in a HIP graph and replayed three times, with eager work and
    synchronizations between the replays: every replay equals the eager
    result bit for bit."""
    from vllm_apple_amd import kernels

    print("[case] gate_up_silu graph replays", flush=True)
    T, H, I = 300, 512, 384
    x, w = _inputs(T, H, I, torch.float16, 21)
    xd, wd = x.cuda(), w.cuda()
    eager = kernels.gate_up_silu(xd, wd)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kernels.gate_up_silu(xd, wd, out=out)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kernels.gate_up_silu(xd, wd, out=out)
    for r in range(3):
        out.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {r}"


@pytest.mark.parametrize("library_route", [False, True])
@pytest.mark.parametrize("fused", [True, False])
def test_engine_mlp_encode(gpu, fused, library_route):
    """EngineMLP.encode (mlp.py:170-245): down_proj(silu(gate(x)) * up(x)) on
    (buffer, byte offset) views inside an ENCODE phase, against the oracle's
    activation rounded to fp16 and an fp64 down projection; through the fused
    kernel and, above fused_max_tokens, through the library GEMM + silu_mul
    route (which rounds the products to fp16 first, as the reference does)."""
    from vllm_apple_amd.engine import EngineMLP, EngineStepContext

    print(f"[case] EngineMLP fused={fused} library_route={library_route}", flush=True)
    T, H, I = 37, 256, 512
    x, w = _inputs(T, H, I, torch.float16, 8)
    g = torch.Generator().manual_seed(9)
    down = (torch.randn(H, I, generator=g) / I ** 0.5).half()
    mlp = EngineMLP(None, H, I)
    if library_route:
        mlp.fused_max_tokens = 16
    if fused:
        mlp.set_weights(gate_up_proj=w.cuda(), down_proj=down.cuda())
    else:
        mlp.set_weights(gate_proj=w[:I].contiguous().cuda(), up_proj=w[I:].contiguous().cuda(),
                        down_proj=down.cuda())
    buf = torch.zeros(2 * T * H + 64, dtype=torch.float16, device="cuda")
    buf[64:64 + T * H] = x.cuda().reshape(-1)
    with EngineStepContext() as ctx:
        mlp.encode(ctx, (buf, 128), (buf, 128 + 2 * T * H), T)
    torch.cuda.synchronize()
    out = host(buf[64 + T * H:64 + 2 * T * H].view(T, H))
    act = olo.gate_up_silu(host(x), host(w)).astype(np.float16).astype(np.float64)
    ref = act @ host(down).astype(np.float64).T
    assert_close(out, ref, what="EngineMLP")
