"""ORACLE (test infrastructure): layer ops next to attention, numpy.

rms_norm   vllm_apple/engine/ops/rmsnorm.py:93-123 (and :161-172 with a
           residual added after the norm): float(x) * rsqrt(mean(x^2)+eps) *
           float(w) [+ float(r)], evaluated in fp64 from the fp16 inputs.
rope_neox  vllm_apple/engine/ops/elementwise.py:185-239 with the cos/sin table
           of :680-697 (fp32 numpy): pairs (i, i+rot/2) rotated by
           (cos, sin)[positions[t], i], in fp64 from the fp32 table.
cos_sin    the table itself, same numpy float32 construction.
silu_mul   elementwise.py:114-124: g / (1 + exp(-g)) * u in fp64.
gate_up_silu  the gated MLP's first half, vllm_apple/engine/ops/mlp.py:247-330:
           gate = x W_gate^T and up = x W_up^T (transpose_B GEMMs, weights
           [I, H]; a fused gate_up_proj [2I, H] holds the gate rows first,
           :267-296), then silu_mul(gate, up); all in fp64 from the 16-bit
           inputs, the intermediates not rounded.

Pinning (tests/test_oracle_layer_ops.py): rms_norm against the reference
test's own formula (tests/metal/test_transformer_block.py:136-199, seed 42,
[4,128], eps 1e-6) and torch.nn.functional.rms_norm; rope_neox against the
reference's torch formula (tests/unit/test_rope_equiv.py:42-66), pos 0 ->
identity, per-pair norm preservation, and composition R(a)R(b) = R(a+b);
silu_mul against torch.nn.functional.silu and its closed-form limits;
gate_up_silu against numpy's matmul composed with the pinned silu_mul, one-hot
activations (which select weight column h, so a transposed operand fails),
zero gate or up weights, and the gate/up order of a fused weight.
"""
from __future__ import annotations

import numpy as np


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float,
             residual: np.ndarray | None = None) -> np.ndarray:
    xf = x.astype(np.float64)
    ms = np.mean(xf * xf, axis=-1, keepdims=True)
    y = xf * (1.0 / np.sqrt(ms + eps)) * w.astype(np.float64)
    if residual is not None:
        y = y + residual.astype(np.float64)
    return y


def cos_sin(rotary_dim: int, max_position: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    half = rotary_dim // 2
    inv_freq = 1.0 / (base ** (np.arange(0, half, dtype=np.float32) / half))
    pos = np.arange(max_position, dtype=np.float32)
    freqs = np.outer(pos, inv_freq)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def rope_neox(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray,
              rotary_dim: int | None = None) -> np.ndarray:
    """x [T, heads, D] fp16 -> rotated float64 copy (positions outside the table untouched)."""
    T, Hh, D = x.shape
    rot = rotary_dim or D
    half = rot // 2
    y = x.astype(np.float64).copy()
    pos = np.asarray(positions, dtype=np.int64)
    ok = (pos >= 0) & (pos < cos.shape[0])
    c = cos[np.where(ok, pos, 0)].astype(np.float64)[:, None, :]
    s = sin[np.where(ok, pos, 0)].astype(np.float64)[:, None, :]
    x0 = y[:, :, :half].copy()
    x1 = y[:, :, half:rot].copy()
    r0 = x0 * c - x1 * s
    r1 = x0 * s + x1 * c
    y[ok, :, :half] = r0[ok]
    y[ok, :, half:rot] = r1[ok]
    return y


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    gf = g.astype(np.float64)
    return gf / (1.0 + np.exp(-gf)) * u.astype(np.float64)


def gate_up_silu(x: np.ndarray, w_gate: np.ndarray, w_up: np.ndarray | None = None) -> np.ndarray:
    """silu(x W_gate^T) * (x W_up^T) in fp64; with w_up None, w_gate is the
    fused [2I, H] gate_up weight, gate rows first."""
    if w_up is None:
        half = w_gate.shape[0] // 2
        w_gate, w_up = w_gate[:half], w_gate[half:]
    xf = x.astype(np.float64)
    g = np.einsum("th,ih->ti", xf, w_gate.astype(np.float64))
    u = np.einsum("th,ih->ti", xf, w_up.astype(np.float64))
    return silu_mul(g, u)
