"""Pins the top-k oracle (oracle/topk.py) on the CPU."""
import numpy as np
import torch

import oracle.topk as otk


def test_key_map_orders_every_fp16_value():
    """All 65536 fp16 bit patterns: key order == float order, except that -0
    sorts below +0 and NaNs sit outside the infinities."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float64)
    keys = otk.sort_keys(bits)
    ok = ~np.isnan(vals) & (vals != 0)
    order = np.argsort(keys[ok], kind="stable")
    assert np.all(np.diff(vals[ok][order]) > 0)
    pz, nz = np.uint16(0x0000), np.uint16(0x8000)
    assert otk.sort_keys(np.array([nz]))[0] + 1 == otk.sort_keys(np.array([pz]))[0]
    pinf, ninf = np.uint16(0x7C00), np.uint16(0xFC00)
    nan_keys = keys[np.isnan(vals)]
    kp, kn = otk.sort_keys(np.array([pinf, ninf]))
    assert np.all((nan_keys > kp) | (nan_keys < kn))


def test_matches_torch_topk_without_ties():
    """Rows of distinct finite fp16 values (sampled bit patterns, no -0): the
    oracle equals torch.topk in values and indices."""
    rng = np.random.default_rng(0)
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = allbits.view(np.float16)
    pool = allbits[np.isfinite(f) & (allbits != 0x8000)]
    bits = np.stack([rng.choice(pool, size=5000, replace=False) for _ in range(6)])
    h = torch.from_numpy(bits.view(np.float16).copy())
    for k in (1, 8, 50, 256):
        idx, vals = otk.topk(bits, k)
        tv, ti = torch.topk(h.float(), k, dim=1, sorted=True)
        assert np.array_equal(idx, ti.numpy())
        assert np.array_equal(vals.view(np.float16).astype(np.float32), tv.numpy())


def test_ties_go_to_lower_columns():
    rng = np.random.default_rng(1)
    vals = rng.integers(-3, 4, size=(4, 997)).astype(np.float16)  # 7 distinct values
    bits = vals.view(np.uint16)
    idx, vb = otk.topk(bits, 100)
    for t in range(4):
        v = vals[t][idx[t]].astype(np.float64)
        # value-descending, and within equal values columns ascending
        assert np.all(np.diff(v) <= 0)
        for a, b in zip(range(99), range(1, 100)):
            if v[a] == v[b]:
                assert idx[t][a] < idx[t][b]
        # every selected value >= every unselected one, brute force
        rest = np.setdiff1d(np.arange(997), idx[t])
        assert v.min() >= vals[t][rest].astype(np.float64).max()
        # the last selected value's columns are the lowest ones among its equals
        last = v[-1]
        eq_cols = np.nonzero(vals[t] == last)[0]
        taken = idx[t][v == last]
        assert np.array_equal(np.sort(taken), eq_cols[:taken.size])
