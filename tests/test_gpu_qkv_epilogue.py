"""Fused QKV epilogue (bias + NeoX RoPE + KV write, one launch) on the GPU.

Two checks:
- bit-exact against the three steps the reference runs over its planar QKV
  buffer (engine/ops/qkv.py:391-416 bias add, elementwise.py:185-239 RoPE,
  kv_write.py:118-156 KV write), here as torch's in-place 16-bit add, this
  library's RoPE kernel and its KV write;
- against the oracle: the 16-bit bias add in numpy (exact), oracle RoPE in fp64
  and the oracle KV write; V and its cache rows bit-exact, Q and K (and the K
  cache rows) within |d| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close

import oracle.kv as okv
import oracle.layer_ops as olo

pytestmark = pytest.mark.gpu


def _case(T, H, KV, D, nb, bs=16, seed=0, dtype=torch.float16, layout="kernel", idx=torch.int64):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(T * (H + 2 * KV) * D, generator=g).to(dtype)
    bias = (torch.randn((H + 2 * KV) * D, generator=g) * 0.5).to(dtype)
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = torch.randn(shape, generator=g).to(dtype)
    vc = torch.randn(shape, generator=g).to(dtype)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(idx)
    slots[::7] = -1
    pos = torch.randint(0, 4000, (T,), generator=g).to(torch.int32)
    return qkv, bias, kc, vc, slots, pos


def _views(buf, T, H, KV, D):
    q = buf[:T * H * D].view(T, H, D)
    k = buf[T * H * D:T * (H + KV) * D].view(T, KV, D)
    v = buf[T * (H + KV) * D:].view(T, KV, D)
    return q, k, v


@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("rot", [128, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_epilogue_equals_three_step_path(gpu, with_bias, rot, dtype):
    from vllm_apple_amd import kernels

    T, H, KV, D, nb = 77, 32, 8, 128, 40
    print(f"[case] epilogue vs 3-step bias={with_bias} rot={rot} {dtype}", flush=True)
    qkv, bias, kc, vc, slots, pos = _case(T, H, KV, D, nb, seed=1, dtype=dtype)
    pos[3] = 5000  # past the table: biased, not rotated
    cos, sin = kernels.rope_cos_sin_cache(rot, 4096, 1e6, device="cuda")
    b = bias.cuda() if with_bias else None
    # Fused.
    buf1, kc1, vc1 = qkv.cuda(), kc.cuda(), vc.cuda()
    q1, k1, v1 = _views(buf1, T, H, KV, D)
    kernels.qkv_epilogue(q1, k1, v1, pos.cuda(), cos, sin, slots.cuda(), kc1, vc1, bias=b,
                         rotary_dim=rot)
    # Three steps.
    buf2, kc2, vc2 = qkv.cuda(), kc.cuda(), vc.cuda()
    q2, k2, v2 = _views(buf2, T, H, KV, D)
    if with_bias:
        q2 += b[:H * D].view(1, H, D)
        k2 += b[H * D:(H + KV) * D].view(1, KV, D)
        v2 += b[(H + KV) * D:].view(1, KV, D)
    kernels.rope_neox_(q2, k2, cos, sin, pos.cuda(), rotary_dim=rot)
    kernels.kv_write_slots(k2, v2, kc2, vc2, slots.cuda())
    torch.cuda.synchronize()
    assert torch.equal(buf1.view(torch.int16), buf2.view(torch.int16)), "q/k/v in place"
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16)), "K cache"
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16)), "V cache"


@pytest.mark.parametrize("layout,idx", [("kernel", torch.int64), ("vllm", torch.int32)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_epilogue_against_oracle(gpu, layout, idx, dtype):
    from vllm_apple_amd import kernels

    T, H, KV, D, nb = 50, 14, 2, 64, 16
    print(f"[case] epilogue oracle layout={layout} dtype={dtype}", flush=True)
    qkv, bias, kc, vc, slots, pos = _case(T, H, KV, D, nb, seed=2, dtype=dtype, layout=layout,
                                          idx=idx)
    cos, sin = kernels.rope_cos_sin_cache(D, 4096, 1e4, device="cuda")
    buf, kcd, vcd = qkv.cuda(), kc.cuda(), vc.cuda()
    q, k, v = _views(buf, T, H, KV, D)
    kernels.qkv_epilogue(q, k, v, pos.cuda(), cos, sin, slots.cuda(), kcd, vcd,
                         bias=bias.cuda(), layout=layout)
    torch.cuda.synchronize()

    def f(t):  # 16-bit values as float32
        return t.float().numpy()

    def bits(t):  # 16-bit patterns as a float16-typed array (byte copies in the oracle)
        return t.cpu().view(torch.float16).numpy()

    qh, kh, vh = _views(qkv, T, H, KV, D)
    # Bias add in the 16-bit type (torch on the host rounds once, as a half add does).
    qb = (qh + bias[:H * D].view(1, H, D))
    kb = (kh + bias[H * D:(H + KV) * D].view(1, KV, D))
    vb = (vh + bias[(H + KV) * D:].view(1, KV, D))
    cos_np, sin_np = olo.cos_sin(D, 4096, 1e4)
    q_ref = olo.rope_neox(f(qb), pos.numpy(), cos_np, sin_np)
    k_ref = olo.rope_neox(f(kb), pos.numpy(), cos_np, sin_np)
    qd, kd, vd = _views(buf.cpu(), T, H, KV, D)
    assert_close(f(qd), q_ref, what="q rotated")
    assert_close(f(kd), k_ref, what="k rotated")
    assert torch.equal(vd.view(torch.int16), vb.view(torch.int16)), "v biased in place"
    # Cache: V rows bit-exact; K rows equal the rotated keys the kernel wrote
    # back, and no other slot changes.
    kr, vr = bits(kc).copy(), bits(vc).copy()
    okv.kv_write_slots(kr, vr, bits(kd), bits(vb), slots.numpy().astype(np.int64), layout)
    assert np.array_equal(bits(kcd).view(np.uint16), kr.view(np.uint16)), "K cache"
    assert np.array_equal(bits(vcd).view(np.uint16), vr.view(np.uint16)), "V cache"
