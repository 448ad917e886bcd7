"""Pins oracle.layer_ops (RMSNorm, NeoX RoPE, SiLU*mul) on the CPU.

Each check comes from somewhere other than the oracle's own formula: a library
routine (torch F.rms_norm / F.silu), a different formulation of the same
mathematics (complex multiplication for RoPE, the reference test's rotate-half
form), or an invariant the mathematics fixes.  A planted mistake in the
oracle's style must fail at least one of them.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.layer_ops as olo


# -- RMSNorm (rmsnorm.py:93-123) -------------------------------------------------------
def test_rmsnorm_vs_torch_rms_norm():
    rs = np.random.RandomState(42)
    x = rs.randn(4, 128).astype(np.float16)  # test_transformer_block.py:136-199 case
    w = rs.randn(128).astype(np.float16)
    ref = F.rms_norm(torch.from_numpy(x).double(), (128,), torch.from_numpy(w).double(), 1e-6)
    np.testing.assert_allclose(olo.rms_norm(x, w, 1e-6), ref.numpy(), rtol=1e-12, atol=1e-12)


def test_rmsnorm_invariants():
    rs = np.random.RandomState(1)
    x = rs.randn(6, 5120).astype(np.float16)
    ones = np.ones(5120, dtype=np.float16)
    y = olo.rms_norm(x, ones, 0.0)
    # unit root-mean-square per row, and invariance to scaling the row
    np.testing.assert_allclose(np.sqrt((y ** 2).mean(-1)), 1.0, rtol=1e-12)
    y2 = olo.rms_norm((x.astype(np.float64) * 4.0), ones, 0.0)
    np.testing.assert_allclose(y2, y, rtol=1e-12)
    # eps matters for tiny rows: x = c (constant) -> c / sqrt(c^2 + eps)
    c = np.full((1, 8), 1e-3, dtype=np.float16)
    got = olo.rms_norm(c, np.ones(8, dtype=np.float16), 1e-5)
    cf = float(c[0, 0])
    np.testing.assert_allclose(got, cf / np.sqrt(cf * cf + 1e-5), rtol=1e-12)


def test_rmsnorm_residual_is_post_added():
    """rmsnorm.py:128-173: norm(x) * w + r (post-add, not vLLM's pre-add)."""
    rs = np.random.RandomState(2)
    x = rs.randn(3, 64).astype(np.float16)
    w = (rs.randn(64) * 0.1 + 1).astype(np.float16)
    r = rs.randn(3, 64).astype(np.float16)
    got = olo.rms_norm(x, w, 1e-5, r)
    ref = F.rms_norm(torch.from_numpy(x).double(), (64,), torch.from_numpy(w).double(), 1e-5)
    np.testing.assert_allclose(got, ref.numpy() + r.astype(np.float64), rtol=1e-12, atol=1e-12)


# -- NeoX RoPE (elementwise.py:185-239, table :680-697) ----------------------------------
def _complex_rope(x, pos, base, rot):
    """Pairs (i, i+rot/2) as z = a + ib multiplied by exp(i pos theta_i), fp64."""
    half = rot // 2
    theta = base ** (-np.arange(half, dtype=np.float64) / half)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * theta[None, :]
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:rot].astype(np.float64)
    z = z * np.exp(1j * ang)[:, None, :]
    y = x.astype(np.float64).copy()
    y[..., :half] = z.real
    y[..., half:rot] = z.imag
    return y


def test_cos_sin_table_matches_reference_test_construction():
    """test_rope_equiv.py:53-58: inv_freq = 1/base^(arange(0,rot,2)/rot), outer, cos/sin."""
    rot, maxp, base = 64, 4096, 10000.0
    cos, sin = olo.cos_sin(rot, maxp, base)
    inv = 1.0 / (base ** (torch.arange(0, rot, 2).float() / rot))
    # numpy's and torch's fp32 pow may round inv_freq one ulp apart; the angle
    # error then grows with the position, so compare the tables where it is small
    np.testing.assert_allclose(1.0 / (base ** (np.arange(32, dtype=np.float32) / 32)),
                               inv.numpy(), rtol=2.5e-7)
    fr = torch.outer(torch.arange(64).float(), inv)
    np.testing.assert_allclose(cos[:64], fr.cos().numpy(), atol=2e-6)
    np.testing.assert_allclose(sin[:64], fr.sin().numpy(), atol=2e-6)
    # whole table against fp64 cos/sin of the fp32 angles
    ang = np.outer(np.arange(maxp, dtype=np.float32),
                   1.0 / (base ** (np.arange(32, dtype=np.float32) / 32))).astype(np.float64)
    np.testing.assert_allclose(cos, np.cos(ang), atol=2e-7)
    np.testing.assert_allclose(sin, np.sin(ang), atol=2e-7)


@pytest.mark.parametrize("rot,D", [(64, 64), (128, 128), (32, 64)])
def test_rope_vs_complex_rotation(rot, D):
    rs = np.random.RandomState(rot + D)
    x = rs.randn(16, 14, D).astype(np.float16)
    pos = rs.randint(0, 2000, size=16)
    cos, sin = olo.cos_sin(rot, 2048, 1e4)
    got = olo.rope_neox(x, pos, cos, sin, rot)
    ref = _complex_rope(x, pos, 1e4, rot)
    # the oracle uses the fp32 table; fp32 angle rounding at pos < 2048 is < 1e-3 rad
    np.testing.assert_allclose(got, ref, atol=3e-3 * np.abs(x).max())
    # dims past rot stay bit-identical
    assert np.array_equal(got[..., rot:], x[..., rot:].astype(np.float64))


def test_rope_vs_reference_rotate_half_form():
    """test_rope_equiv.py:42-66 (14 heads, D64, 16 tokens, base 1e4), in fp32."""
    rs = np.random.RandomState(3)
    x = rs.randn(16, 14, 64).astype(np.float16)
    pos = np.arange(16)
    cos, sin = olo.cos_sin(64, 64, 1e4)
    xt = torch.from_numpy(x).float()
    c = torch.from_numpy(np.concatenate([cos, cos], -1))[pos].unsqueeze(1)
    s = torch.from_numpy(np.concatenate([sin, sin], -1))[pos].unsqueeze(1)
    rotated = torch.cat((-xt[..., 32:], xt[..., :32]), dim=-1)
    ref = (xt * c + rotated * s).numpy()
    np.testing.assert_allclose(olo.rope_neox(x, pos, cos, sin), ref, atol=1e-5)


def test_rope_invariants():
    rs = np.random.RandomState(4)
    x = rs.randn(8, 4, 128).astype(np.float16)
    cos, sin = olo.cos_sin(128, 16384, 1e6)
    # position 0 is the identity
    y0 = olo.rope_neox(x, np.zeros(8, dtype=np.int64), cos, sin)
    assert np.array_equal(y0, x.astype(np.float64))
    # per-pair norm is preserved
    pos = rs.randint(0, 16384, size=8)
    y = olo.rope_neox(x, pos, cos, sin)
    n_in = x[..., :64].astype(np.float64) ** 2 + x[..., 64:].astype(np.float64) ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-6)
    # R(a) R(b) = R(a + b) (table angles are fp32: compare at small positions)
    a, b = rs.randint(0, 100, size=8), rs.randint(0, 100, size=8)
    yab = olo.rope_neox(olo.rope_neox(x, a, cos, sin), b, cos, sin)
    np.testing.assert_allclose(yab, olo.rope_neox(x, a + b, cos, sin), atol=1e-4)
    # positions outside [0, max_position) are left untouched
    bad = np.array([-1, 16384, 5, 5, 5, 5, 5, 5])
    yb = olo.rope_neox(x, bad, cos, sin)
    assert np.array_equal(yb[:2], x[:2].astype(np.float64))


# -- SiLU * mul (elementwise.py:114-124) -------------------------------------------------
def test_silu_mul_vs_torch_and_limits():
    rs = np.random.RandomState(5)
    g = rs.randn(1024).astype(np.float16)  # test_transformer_block.py:205-255 size
    u = rs.randn(1024).astype(np.float16)
    ref = F.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()
    np.testing.assert_allclose(olo.silu_mul(g, u), ref.numpy(), rtol=1e-12, atol=1e-15)
    big = np.array([0.0, 30.0, -30.0], dtype=np.float16)
    one = np.ones(3, dtype=np.float16)
    got = olo.silu_mul(big, one)
    assert got[0] == 0.0
    np.testing.assert_allclose(got[1], 30.0, rtol=1e-12)
    assert abs(got[2]) < 1e-11


def test_planted_layer_op_mistakes_are_caught():
    """Plausible slips in the oracle's style fail the checks above."""
    rs = np.random.RandomState(6)
    x = rs.randn(4, 128).astype(np.float16)
    w = rs.randn(128).astype(np.float16)
    ref = F.rms_norm(torch.from_numpy(x).double(), (128,), torch.from_numpy(w).double(), 1e-6)
    xf = x.astype(np.float64)
    wrong_sum = xf / np.sqrt((xf ** 2).sum(-1, keepdims=True) + 1e-6) * w  # sum, not mean
    assert not np.allclose(wrong_sum, ref.numpy(), rtol=1e-3)
    # RoPE with interleaved pairs (GPT-J style) instead of NeoX halves
    x3 = rs.randn(4, 2, 64).astype(np.float16)
    pos = np.array([1, 7, 100, 900])
    cos, sin = olo.cos_sin(64, 1024, 1e4)
    y = x3.astype(np.float64).copy()
    a, b = y[..., 0::2].copy(), y[..., 1::2].copy()
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    y[..., 0::2], y[..., 1::2] = a * c - b * s, a * s + b * c
    assert not np.allclose(y, _complex_rope(x3, pos, 1e4, 64), atol=1e-2)
    # sign flip in the rotation
    r0 = x3[..., :32].astype(np.float64) * c + x3[..., 32:].astype(np.float64) * s
    assert not np.allclose(r0, _complex_rope(x3, pos, 1e4, 64)[..., :32], atol=1e-2)


# -- gated MLP up projection + SwiGLU (mlp.py:247-330) ----------------------------------
def test_gate_up_silu_vs_matmul_and_special_cases():
    rs = np.random.RandomState(7)
    T, H, I = 5, 96, 40
    x = rs.randn(T, H).astype(np.float16)
    wg = (rs.randn(I, H) / np.sqrt(H)).astype(np.float16)
    wu = (rs.randn(I, H) / np.sqrt(H)).astype(np.float16)
    # numpy's matmul composed with the pinned silu_mul
    g = np.matmul(x.astype(np.float64), wg.astype(np.float64).T)
    u = np.matmul(x.astype(np.float64), wu.astype(np.float64).T)
    got = olo.gate_up_silu(x, wg, wu)
    np.testing.assert_allclose(got, olo.silu_mul(g, u), rtol=1e-12, atol=1e-14)
    # one-hot activations select weight column h of both matrices
    eye = np.zeros((3, H), dtype=np.float16)
    hs = [0, 17, H - 1]
    for t, h in enumerate(hs):
        eye[t, h] = 1.0
    sel = olo.gate_up_silu(eye, wg, wu)
    for t, h in enumerate(hs):
        np.testing.assert_allclose(sel[t], olo.silu_mul(wg[:, h], wu[:, h]), rtol=1e-12)
    # a zero gate (silu(0) = 0) or a zero up projection gives zero
    assert not olo.gate_up_silu(x, np.zeros_like(wg), wu).any()
    assert not olo.gate_up_silu(x, wg, np.zeros_like(wu)).any()
    # fused [2I, H] weight: gate rows first
    fused = np.concatenate([wg, wu])
    np.testing.assert_array_equal(olo.gate_up_silu(x, fused), got)
    # planted: halves swapped (silu on the up projection) or a transposed product
    assert not np.allclose(olo.gate_up_silu(x, wu, wg), got, rtol=1e-3)
    sq = rs.randn(H, H).astype(np.float16)
    xs = rs.randn(2, H).astype(np.float16)
    assert not np.allclose(olo.gate_up_silu(xs, sq, sq.T.copy()),
                           olo.gate_up_silu(xs, sq, sq), rtol=1e-3)


# -- the torch CPU path bench.py times as the CPU baseline (oracle/ref_torch.py) --------
def test_ref_torch_layer_ops_vs_fp64_oracle():
    """ref_torch.rms_norm / rope_neox / silu_mul compute in fp16 as the
    reference's CPU path does; against the pinned fp64 oracle they stay
    within fp16 rounding (the kernels' own tolerance, 2e-3 + 1e-2 |ref|)."""
    import oracle.ref_torch as rt

    rs = np.random.RandomState(8)
    x = rs.randn(64, 5120).astype(np.float16)
    w = (rs.randn(5120) * 0.1 + 1).astype(np.float16)
    got = rt.rms_norm(torch.from_numpy(x), torch.from_numpy(w), 1e-6).double().numpy()
    ref = olo.rms_norm(x, w, 1e-6)
    assert np.all(np.abs(got - ref) <= 2e-3 + 1e-2 * np.abs(ref))

    for D, base in ((128, 1e6), (64, 1e4)):
        q = rs.randn(96, 8, D).astype(np.float16)
        pos = rs.randint(0, 16384, size=96)
        cos, sin = olo.cos_sin(D, 16384, base)
        got = rt.rope_neox(torch.from_numpy(q), torch.from_numpy(pos), torch.from_numpy(cos),
                           torch.from_numpy(sin)).double().numpy()
        ref = olo.rope_neox(q, pos, cos, sin)
        assert np.all(np.abs(got - ref) <= 2e-3 + 1e-2 * np.abs(ref)), D
        # a plausible slip (halves swapped in the rotation) is far outside
        t = torch.from_numpy(q).double()
        c = torch.from_numpy(np.concatenate([cos, cos], -1))[torch.from_numpy(pos)].unsqueeze(1)
        s = torch.from_numpy(np.concatenate([sin, sin], -1))[torch.from_numpy(pos)].unsqueeze(1)
        slip = (t * c + torch.cat((t[..., D // 2:], -t[..., :D // 2]), -1) * s).numpy()
        assert not np.all(np.abs(slip - ref) <= 2e-3 + 1e-2 * np.abs(ref))

    g = (rs.randn(32, 1024) * 4).astype(np.float16)
    u = rs.randn(32, 1024).astype(np.float16)
    got = rt.silu_mul(torch.from_numpy(g), torch.from_numpy(u)).double().numpy()
    ref = olo.silu_mul(g, u)
    assert np.all(np.abs(got - ref) <= 2e-3 + 1e-2 * np.abs(ref))


def test_ref_torch_layout_permute():
    """kernel_to_vllm_layout: cache[b, h, t, d] lands at [b, t, h, d]."""
    import oracle.ref_torch as rt

    c = torch.arange(3 * 2 * 4 * 5, dtype=torch.float32).view(3, 2, 4, 5)
    v = rt.kernel_to_vllm_layout(c)
    assert v.shape == (3, 4, 2, 5) and v.is_contiguous()
    for b, h, t, d in [(0, 0, 0, 0), (2, 1, 3, 4), (1, 0, 2, 3), (2, 1, 0, 1)]:
        assert v[b, t, h, d] == c[b, h, t, d]
