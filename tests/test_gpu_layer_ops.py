"""RMSNorm, NeoX RoPE, SiLU*mul and the device index builders vs the oracle."""
import numpy as np
import pytest
import torch

from helpers import assert_close, host

import oracle.kv as okv
import oracle.layer_ops as olo

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H", [(4, 128), (2104, 5120), (7, 4096), (3, 8192), (5, 20480), (9, 100)])
@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm(gpu, T, H, residual):
    from vllm_apple_amd import kernels

    print(f"[case] rmsnorm T={T} H={H} res={residual}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + H)
    x = torch.randn(T, H, generator=g).half()
    w = (torch.randn(H, generator=g) * 0.1 + 1).half()
    r = torch.randn(T, H, generator=g).half() if residual else None
    out = kernels.rms_norm(x.cuda(), w.cuda(), 1e-5, residual=r.cuda() if residual else None)
    torch.cuda.synchronize()
    ref = olo.rms_norm(host(x), host(w), 1e-5, host(r) if residual else None)
    assert_close(host(out), ref, what=f"rmsnorm {T}x{H}")


@pytest.mark.parametrize("T,H", [(37, 5120), (4, 896), (2104, 4096), (5, 20480), (9, 100)])
def test_add_rmsnorm_equals_three_steps(gpu, T, H):
    """vaa_add_rmsnorm against the reference layer's residual add, copy and
    norm in place (runner.py:1107-1130), here torch's fp16 add, a copy and
    vaa_rmsnorm: residual and output equal bit for bit.  Covers the register
    path, the long-row two-pass path (H=20480) and the scalar path (H=100),
    and the output written over x."""
    from vllm_apple_amd import kernels

    print(f"[case] add_rmsnorm T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(T + H)
    x = torch.randn(T, H, generator=g).half().cuda()
    r = torch.randn(T, H, generator=g).half().cuda()
    w = (torch.randn(H, generator=g) * 0.1 + 1).half().cuda()
    h = x + r  # the reference's residual_add (half add)
    res2 = h.clone()  # encode_copy into the residual buffer
    out2 = kernels.rms_norm(h, w, 1e-6)  # EngineRMSNorm.encode
    x1, r1 = x.clone(), r.clone()
    kernels.add_rms_norm(x1, r1, w, 1e-6, out=x1)
    torch.cuda.synchronize()
    assert torch.equal(r1.view(torch.int16), res2.view(torch.int16)), "residual"
    assert torch.equal(x1.view(torch.int16), out2.view(torch.int16)), "normed output"


def test_add_rmsnorm_against_oracle_and_engine(gpu):
    from vllm_apple_amd import kernels
    from vllm_apple_amd.engine import EngineRMSNorm, EngineStepContext

    T, H = 50, 2048
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g).half()
    r = torch.randn(T, H, generator=g).half()
    w = (torch.randn(H, generator=g) * 0.1 + 1).half()
    h_ref = (host(x) + host(r)).astype(np.float16)  # one rounding, as a half add
    ref = olo.rms_norm(h_ref, host(w), 1e-5)
    rd = r.cuda()
    out = kernels.add_rms_norm(x.cuda(), rd, w.cuda(), 1e-5)
    torch.cuda.synchronize()
    assert np.array_equal(host(rd).view(np.uint16), h_ref.view(np.uint16)), "residual"
    assert_close(host(out), ref, what="add_rmsnorm")
    # Engine op on (buffer, byte offset) views inside an ENCODE phase.
    buf = torch.zeros(3 * T * H + 64, dtype=torch.float16, device="cuda")
    buf[64:64 + T * H] = x.cuda().reshape(-1)
    buf[64 + T * H:64 + 2 * T * H] = r.cuda().reshape(-1)
    norm = EngineRMSNorm(None, H, eps=1e-5, weight_buffer=w.cuda())
    with EngineStepContext() as ctx:
        norm.encode_residual_add_norm(ctx, (buf, 128), (buf, 128 + 2 * T * H), (buf, 128), T)
    torch.cuda.synchronize()
    assert torch.equal(buf[64:64 + T * H].view(T, H).cpu().view(torch.int16),
                       out.cpu().view(torch.int16))
    assert np.array_equal(host(buf[64 + T * H:64 + 2 * T * H].view(T, H)).view(np.uint16),
                          h_ref.view(np.uint16))


def test_rmsnorm_reference_known_case(gpu):
    """tests/metal/test_transformer_block.py:136-199 (seed 42, [4,128], eps 1e-6)."""
    from vllm_apple_amd import kernels

    rs = np.random.RandomState(42)
    x = rs.randn(4, 128).astype(np.float16)
    w = rs.randn(128).astype(np.float16)
    xf, wf = x.astype(np.float32), w.astype(np.float32)
    expected = (xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6) * wf).astype(np.float16)
    out = kernels.rms_norm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), 1e-6)
    np.testing.assert_allclose(host(out).astype(np.float32), expected.astype(np.float32),
                               rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("T,H,KV,D,rot", [(2104, 32, 8, 128, 128), (16, 14, 14, 64, 64),
                                          (33, 8, 2, 128, 64), (5, 4, 2, 96, 96), (9, 4, 1, 48, 48),
                                          (6, 3, 1, 20, 20), (4, 2, 2, 64, 16)])
def test_rope_neox(gpu, T, H, KV, D, rot):
    from vllm_apple_amd import kernels

    print(f"[case] rope T={T} H={H} KV={KV} D={D} rot={rot}", flush=True)
    g = torch.Generator().manual_seed(T + D)
    maxp = 16384
    q = torch.randn(T, H, D, generator=g).half()
    k = torch.randn(T, KV, D, generator=g).half()
    pos = torch.randint(0, maxp, (T,), generator=g).to(torch.int32)
    pos[0] = 0
    if T > 3:
        pos[1] = maxp + 5  # outside the table: left unrotated
    cos, sin = olo.cos_sin(rot, maxp, 1e6)
    qd, kd = q.cuda(), k.cuda()
    kernels.rope_neox_(qd, kd, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(),
                       pos.cuda(), rotary_dim=rot)
    torch.cuda.synchronize()
    assert_close(host(qd), olo.rope_neox(host(q), host(pos), cos, sin, rot), what="rope q")
    assert_close(host(kd), olo.rope_neox(host(k), host(pos), cos, sin, rot), what="rope k")
    assert torch.equal(qd[0].cpu(), q[0]), "position 0 is the identity"


def test_rope_table_matches_reference_construction(gpu):
    from vllm_apple_amd import kernels

    cos, sin = kernels.rope_cos_sin_cache(128, 4096, 1e6, device="cuda")
    c2, s2 = olo.cos_sin(128, 4096, 1e6)
    assert np.array_equal(host(cos), c2) and np.array_equal(host(sin), s2)


@pytest.mark.parametrize("shape", [(1024,), (2104, 32768), (3, 1001), (77,)])
def test_silu_mul(gpu, shape):
    from vllm_apple_amd import kernels

    g = torch.Generator().manual_seed(sum(shape))
    gate = torch.randn(*shape, generator=g).half()
    up = torch.randn(*shape, generator=g).half()
    out = kernels.silu_mul(gate.cuda(), up.cuda())
    torch.cuda.synchronize()
    assert_close(host(out), olo.silu_mul(host(gate), host(up)), what=f"silu_mul {shape}")


def test_silu_mul_strided_halves(gpu):
    """gate/up as the two halves of vLLM's [T, 2I] projection output."""
    from vllm_apple_amd import kernels

    g = torch.Generator().manual_seed(3)
    gu = torch.randn(37, 2 * 4096, generator=g).half()
    d = gu.cuda()
    out = kernels.silu_mul(d[:, :4096], d[:, 4096:])
    torch.cuda.synchronize()
    assert_close(host(out), olo.silu_mul(host(gu[:, :4096]), host(gu[:, 4096:])), what="silu 2d")


def test_silu_mul_extremes(gpu):
    from vllm_apple_amd import kernels

    gate = torch.tensor([-65504, -100, -20, -1, 0, 1, 20, 100, 65504, 0.5, -0.5, 3], dtype=torch.float16)
    up = torch.ones_like(gate)
    out = kernels.silu_mul(gate.cuda(), up.cuda()).cpu()
    ref = olo.silu_mul(gate.numpy(), up.numpy())
    finite = np.isfinite(ref) & (np.abs(ref) < 65504)
    assert_close(out.numpy()[finite], ref[finite], what="silu extremes")


def test_token_index_and_slots(gpu):
    from vllm_apple_amd import kernels

    qsl = np.array([0, 3, 3, 10, 11, 40], dtype=np.int32)   # includes an empty query
    seq_lens = np.array([50, 7, 7, 1, 29], dtype=np.int32)
    T = 42  # two tokens past the end -> -1
    tok, pos = kernels.build_token_index(torch.from_numpy(qsl).cuda(),
                                         torch.from_numpy(seq_lens).cuda(), T)
    rt, rp = okv.token_index(qsl, seq_lens, T)
    assert np.array_equal(host(tok), rt) and np.array_equal(host(pos), rp)
    bt = np.full((5, 4), -1, dtype=np.int32)
    bt[0, :4] = [9, 3, 7, 1]
    bt[2, :1] = [5]
    bt[4, :2] = [11, 12]
    slots = kernels.build_slot_mapping(torch.from_numpy(bt).cuda(), 16, tok, pos)
    torch.cuda.synchronize()
    assert np.array_equal(host(slots), okv.slot_mapping(bt, 16, rt, rp))
