"""Shared test helpers: tolerance rule and host/device copies."""
from __future__ import annotations

import numpy as np
import torch

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


# ---------------------------------------------------------- paged batches --
CANARY = 0x7BCD  # an fp16 bit pattern no kernel writes here
TAIL = 256


def canaried(t: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(device buffer, view): t's contents on the GPU followed by TAIL canary
    elements, so a write past t's last element shows in the buffer's tail."""
    buf = torch.full((t.numel() + TAIL,), CANARY, dtype=torch.int16).view(t.dtype)
    buf[:t.numel()] = t.reshape(-1)
    buf = buf.cuda()
    return buf, buf[:t.numel()].view(t.shape)


def tail_ok(buf: torch.Tensor) -> bool:
    return bool((buf[-TAIL:].view(torch.int16).cpu() == CANARY).all())


def decode_case(S, H, KV, D, lens, layout, seed, bs=16):
    """A paged decode batch: caches of N(0,1) rows in shuffled blocks (three
    spare), block tables padded with -1, q and the new token's K/V."""
    g = torch.Generator().manual_seed(seed)
    nblk = [(L + bs - 1) // bs for L in lens]
    maxb = max(nblk)
    nb = sum(nblk) + 3
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = torch.randn(shape, generator=g).half()
    vc = torch.randn(shape, generator=g).half()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((S, maxb), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    # The last sequence's last block is the pool's last one, so its new token
    # (offset bs - 1 when L % bs == 0) lands on the pool's last rows.
    s_last, b_last = S - 1, nblk[-1] - 1
    where = (bt == nb - 1).nonzero()
    if len(where):
        r, c = where[0].tolist()
        bt[r, c], bt[s_last, b_last] = bt[s_last, b_last].item(), nb - 1
    else:
        bt[s_last, b_last] = nb - 1
    q = torch.randn(S, H, D, generator=g).half()
    nk = torch.randn(S, KV, D, generator=g).half()
    nv = torch.randn(S, KV, D, generator=g).half()
    return kc, vc, bt, torch.tensor(lens, dtype=torch.int32), q, nk, nv


def prefill_case(ctx, new, H, KV, D, layout, seed, bs=16):
    """A chunked-prefill batch: sequence s has ctx[s] cached positions of
    which the last new[s] are its query tokens (causal within the chunk)."""
    g = torch.Generator().manual_seed(seed)
    nblk = [(L + bs - 1) // bs for L in ctx]
    nb = sum(nblk) + 2
    maxb = max(nblk)
    shape = (nb, KV, bs, D) if layout == "kernel" else (nb, bs, KV, D)
    kc = torch.randn(shape, generator=g).half()
    vc = torch.randn(shape, generator=g).half()
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((len(ctx), maxb), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    tok, pos = [], []
    for s, (L, n) in enumerate(zip(ctx, new)):
        tok += [s] * n
        pos += list(range(L - n, L))
    q = torch.randn(len(tok), H, D, generator=g).half()
    return (kc, vc, bt, torch.tensor(tok, dtype=torch.int32),
            torch.tensor(pos, dtype=torch.int32), q)
