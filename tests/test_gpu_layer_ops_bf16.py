"""bf16 through the layer ops (RMSNorm, residual add + RMSNorm, NeoX RoPE,
SwiGLU): the dtype argument selects bf16 for every 16-bit tensor of a call.

The reference's layer ops are fp16 only (engine/ops/rmsnorm.py:78-173,
elementwise.py:114-239); bf16 models there convert at the boundary.  Checked
against the fp64 oracle on the bf16 input values with the north-star bound
|d| <= 2e-3 + 1e-2 |ref| plus the rounding of the bf16 output (half a bf16
ulp of ref; the arithmetic is fp32), and the fused op bit-identical to its
unfused steps in bf16, as in fp16.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close_bf16

import oracle.layer_ops as olo

pytestmark = pytest.mark.gpu



def vals(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().double().numpy()


@pytest.mark.parametrize("T,H", [(37, 5120), (9, 100), (5, 20480), (64, 896)])
@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm_bf16(gpu, T, H, residual):
    from vllm_apple_amd import kernels

    print(f"[case] bf16 rmsnorm T={T} H={H} res={residual}", flush=True)
    g = torch.Generator().manual_seed(T * 3 + H)
    x = torch.randn(T, H, generator=g).bfloat16()
    w = (torch.randn(H, generator=g) * 0.1 + 1).bfloat16()
    r = torch.randn(T, H, generator=g).bfloat16() if residual else None
    out = kernels.rms_norm(x.cuda(), w.cuda(), 1e-5, residual=r.cuda() if residual else None)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    ref = olo.rms_norm(vals(x), vals(w), 1e-5, vals(r) if residual else None)
    assert_close_bf16(vals(out), ref, what=f"bf16 rmsnorm {T}x{H}")


@pytest.mark.parametrize("T,H", [(37, 5120), (9, 100), (5, 20480)])
def test_add_rmsnorm_bf16_equals_three_steps(gpu, T, H):
    from vllm_apple_amd import kernels

    print(f"[case] bf16 add_rmsnorm T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(T + 2 * H)
    x = torch.randn(T, H, generator=g).bfloat16().cuda()
    r = torch.randn(T, H, generator=g).bfloat16().cuda()
    w = (torch.randn(H, generator=g) * 0.1 + 1).bfloat16().cuda()
    h = x + r  # one rounding to bf16
    out2 = kernels.rms_norm(h, w, 1e-6)
    x1, r1 = x.clone(), r.clone()
    kernels.add_rms_norm(x1, r1, w, 1e-6, out=x1)
    torch.cuda.synchronize()
    assert torch.equal(r1.view(torch.int16), h.view(torch.int16)), "residual"
    assert torch.equal(x1.view(torch.int16), out2.view(torch.int16)), "normed output"
    ref = olo.rms_norm(vals(h), vals(w), 1e-6)
    assert_close_bf16(vals(x1), ref, what="bf16 add_rmsnorm")


@pytest.mark.parametrize("T,H,KV,D,rot", [(33, 8, 2, 128, 64), (16, 14, 14, 64, 64),
                                          (9, 4, 1, 48, 48), (7, 4, 2, 12, 12)])
def test_rope_bf16(gpu, T, H, KV, D, rot):
    from vllm_apple_amd import kernels

    print(f"[case] bf16 rope T={T} H={H} KV={KV} D={D} rot={rot}", flush=True)
    g = torch.Generator().manual_seed(T + D + 1)
    maxp = 4096
    q = torch.randn(T, H, D, generator=g).bfloat16()
    k = torch.randn(T, KV, D, generator=g).bfloat16()
    pos = torch.randint(0, maxp, (T,), generator=g).to(torch.int32)
    pos[0] = 0
    pos[1] = maxp + 3  # outside the table: left unrotated
    cos, sin = olo.cos_sin(rot, maxp, 1e4)
    qd, kd = q.cuda(), k.cuda()
    kernels.rope_neox_(qd, kd, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(),
                       pos.cuda(), rotary_dim=rot)
    torch.cuda.synchronize()
    assert_close_bf16(vals(qd), olo.rope_neox(vals(q), pos.numpy(), cos, sin, rot),
                      what="bf16 rope q")
    assert_close_bf16(vals(kd), olo.rope_neox(vals(k), pos.numpy(), cos, sin, rot),
                      what="bf16 rope k")
    assert torch.equal(qd[0].cpu().view(torch.int16), q[0].view(torch.int16)), "position 0"
    assert torch.equal(qd[1].cpu().view(torch.int16), q[1].view(torch.int16)), "past the table"


@pytest.mark.parametrize("shape", [(2104, 4096), (3, 1000), (777,)])
def test_silu_mul_bf16(gpu, shape):
    from vllm_apple_amd import kernels

    g = torch.Generator().manual_seed(sum(shape) + 7)
    gate = (torch.randn(*shape, generator=g) * 3).bfloat16()
    up = torch.randn(*shape, generator=g).bfloat16()
    out = kernels.silu_mul(gate.cuda(), up.cuda())
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    assert_close_bf16(vals(out), olo.silu_mul(vals(gate), vals(up)), what=f"bf16 silu_mul {shape}")
    # Row-strided halves of a [T, 2I] projection output.
    both = torch.randn(6, 2 * 96, generator=g).bfloat16().cuda()
    o2 = kernels.silu_mul(both[:, :96], both[:, 96:])
    torch.cuda.synchronize()
    assert_close_bf16(vals(o2), olo.silu_mul(vals(both[:, :96]), vals(both[:, 96:])),
                      what="bf16 silu_mul strided")


def test_layer_ops_reject_mixed_dtypes(gpu):
    from vllm_apple_amd import kernels

    x = torch.randn(4, 64, device="cuda").bfloat16()
    w = torch.ones(64, device="cuda").half()
    with pytest.raises(ValueError):
        kernels.rms_norm(x, w, 1e-6)
    with pytest.raises(ValueError):
        kernels.silu_mul(x, x.half())


def test_engine_ops_take_bf16_buffers(gpu):
    """EngineRMSNorm and EngineElementwiseOps on bf16 (buffer, byte offset) views."""
    from vllm_apple_amd import kernels
    from vllm_apple_amd.engine import EngineElementwiseOps, EngineRMSNorm, EngineStepContext

    T, H = 12, 256
    g = torch.Generator().manual_seed(21)
    x = torch.randn(T, H, generator=g).bfloat16().cuda()
    w = (torch.randn(H, generator=g) * 0.1 + 1).bfloat16().cuda()
    buf = torch.zeros(32 + 3 * T * H, dtype=torch.bfloat16, device="cuda")
    buf[32:32 + T * H] = x.reshape(-1)
    norm = EngineRMSNorm(None, H, eps=1e-6, weight_buffer=w)
    ops = EngineElementwiseOps()
    with EngineStepContext() as ctx:
        norm.encode(ctx, (buf, 64), (buf, 64 + 2 * T * H), T)
        ops.encode_silu_mul(ctx, (buf, 64), (buf, 64 + 2 * T * H), (buf, 64 + 4 * T * H), T * H)
    torch.cuda.synchronize()
    y = buf[32 + T * H:32 + 2 * T * H].view(T, H)
    assert torch.equal(y.view(torch.int16), kernels.rms_norm(x, w, 1e-6).view(torch.int16))
    s = buf[32 + 2 * T * H:].view(T, H)
    assert torch.equal(s.view(torch.int16), kernels.silu_mul(x, y).view(torch.int16))
