"""Shared test helpers: tolerance rule and host/device copies."""
from __future__ import annotations

import numpy as np

# north_star tolerance for attention / RMSNorm / SwiGLU (and applied to RoPE):
# |gpu - ref| <= ATOL + RTOL * |ref| against the fp32/fp64-accumulated oracle.
ATOL = 2e-3
RTOL = 1e-2


def assert_close(actual, expected, atol: float = ATOL, rtol: float = RTOL, what: str = "",
                 extra=None):
    """|actual - expected| <= atol + rtol |expected| (+ extra, elementwise)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    diff = np.abs(a - e)
    bound = atol + rtol * np.abs(e)
    if extra is not None:
        bound = bound + extra
    bad = diff > bound
    max_abs = float(diff.max()) if diff.size else 0.0
    rel = diff / np.maximum(np.abs(e), 1e-6)
    max_rel = float(rel.max()) if rel.size else 0.0
    if bad.any():
        i = np.unravel_index(np.argmax(diff - bound), diff.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} outside |d|<={atol}+{rtol}|ref|; "
            f"worst at {i}: got {a[i]}, ref {e[i]}; max_abs={max_abs:.3g} max_rel={max_rel:.3g}")
    return max_abs, max_rel


def host(t):
    """torch tensor -> numpy (fp16 stays fp16)."""
    return t.detach().cpu().numpy()


def bf16_half_ulp(x):
    """Half a unit in the last place of bfloat16 at |x| (8 significant bits,
    so 2^(e-8) in the binade [2^e, 2^(e+1))): the rounding of a bf16 output."""
    ax = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(ax, np.finfo(np.float32).tiny)))
    return np.where(ax > 0, np.exp2(e - 8), 0.0)


def assert_close_bf16(actual, expected, what: str = ""):
    """The north-star bound |d| <= 2e-3 + 1e-2 |ref| against the fp64 oracle
    on the bf16 input values, plus the rounding of the bf16 output itself
    (half a bf16 ulp of ref)."""
    return assert_close(actual, expected, what=what, extra=bf16_half_ulp(expected))
