"""Writes the golden fixtures in this folder from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Each fixture is a small .npz holding seeded inputs and the oracle's expected
outputs for one operation, at shapes taken from the reference's own tests
where they state one (RMSNorm [4,128] seed 42, eps 1e-6:
tests/metal/test_transformer_block.py:136-199; RoPE 14 heads, D64, 16 tokens,
base 1e4: tests/unit/test_rope_equiv.py:14-66; SiLU 1024 elements:
test_transformer_block.py:205-255; decode 14q/2kv D64 bs16 as BASELINE
config C1).  tests/test_golden.py checks that the oracle still reproduces
them; tests/test_gpu_golden.py checks the HIP library against them.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

import oracle.attention as oat  # noqa: E402
import oracle.kv as okv  # noqa: E402
import oracle.layer_ops as olo  # noqa: E402


def _paged(rs, nb, KV, bs, D):
    return (rs.randn(nb, KV, bs, D).astype(np.float16), rs.randn(nb, KV, bs, D).astype(np.float16))


def _table(rs, nblk, nb):
    perm = rs.permutation(nb).astype(np.int32)
    bt = np.full((len(nblk), max(nblk)), -1, dtype=np.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    return bt


def kv_write():
    rs = np.random.RandomState(2001)
    nb, KV, bs, D, T = 6, 2, 16, 32, 10
    kc, vc = _paged(rs, nb, KV, bs, D)
    key = rs.randn(T, KV, D).astype(np.float16)
    value = rs.randn(T, KV, D).astype(np.float16)
    slots = rs.choice(nb * bs, size=T, replace=False).astype(np.int64)
    slots[[2, 7]] = -1  # padding tokens are skipped
    ko, vo = kc.copy(), vc.copy()
    okv.kv_write_slots(ko, vo, key, value, slots)
    # decode-position form: seq_lens include the new token; 0 -> no write
    bt = _table(rs, [2, 3, 1], nb)
    seq_lens = np.array([17, 48, 0], dtype=np.int32)
    nk = rs.randn(3, KV, D).astype(np.float16)
    nv = rs.randn(3, KV, D).astype(np.float16)
    kd, vd = kc.copy(), vc.copy()
    okv.kv_write_decode(kd, vd, nk, nv, bt, seq_lens)
    return dict(kc=kc, vc=vc, key=key, value=value, slots=slots, kc_slots=ko, vc_slots=vo,
                block_table=bt, seq_lens=seq_lens, new_k=nk, new_v=nv, kc_decode=kd,
                vc_decode=vd)


def decode():
    rs = np.random.RandomState(2002)
    H, KV, D, bs = 14, 2, 64, 16
    lens = np.array([1, 16, 17, 90], dtype=np.int32)
    nblk = [(int(L) + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 2
    kc, vc = _paged(rs, nb, KV, bs, D)
    bt = _table(rs, nblk, nb)
    q = rs.randn(len(lens), H, D).astype(np.float16)
    out = oat.decode(q, kc, vc, bt, lens, 1 / 8.0)
    return dict(query=q, kc=kc, vc=vc, block_table=bt, seq_lens=lens, scale=np.float64(1 / 8.0),
                out=out)


def prefill():
    rs = np.random.RandomState(2003)
    H, KV, D, bs = 8, 2, 64, 16
    ctx, new = [40, 23], [8, 23]
    nblk = [(L + bs - 1) // bs for L in ctx]
    nb = sum(nblk) + 1
    kc, vc = _paged(rs, nb, KV, bs, D)
    bt = _table(rs, nblk, nb)
    tok, pos = [], []
    for s, (L, n) in enumerate(zip(ctx, new)):
        tok += [s] * n
        pos += list(range(L - n, L))
    tok = np.array(tok, dtype=np.int32)
    pos = np.array(pos, dtype=np.int32)
    q = rs.randn(len(tok), H, D).astype(np.float16)
    out, written = oat.prefill(q, kc, vc, bt, tok, pos, 1 / 8.0)
    assert written.all()
    return dict(query=q, kc=kc, vc=vc, block_table=bt, token_to_seq=tok, positions=pos,
                scale=np.float64(1 / 8.0), out=out)


def layer_ops():
    rs = np.random.RandomState(42)
    x = rs.randn(4, 128).astype(np.float16)
    w = rs.randn(128).astype(np.float16)
    r = np.random.RandomState(2004).randn(4, 128).astype(np.float16)
    rs2 = np.random.RandomState(2005)
    q = rs2.randn(16, 14, 64).astype(np.float16)
    k = rs2.randn(16, 2, 64).astype(np.float16)
    pos = np.arange(16, dtype=np.int32)
    cos, sin = olo.cos_sin(64, 64, 1e4)
    g = rs2.randn(1024).astype(np.float16)
    u = rs2.randn(1024).astype(np.float16)
    return dict(rms_x=x, rms_w=w, rms_res=r, rms_eps=np.float64(1e-6),
                rms_out=olo.rms_norm(x, w, 1e-6), rms_out_res=olo.rms_norm(x, w, 1e-6, r),
                rope_q=q, rope_k=k, rope_pos=pos, rope_base=np.float64(1e4), rope_max_pos=np.int64(64),
                rope_q_out=olo.rope_neox(q, pos, cos, sin), rope_k_out=olo.rope_neox(k, pos, cos, sin),
                silu_g=g, silu_u=u, silu_out=olo.silu_mul(g, u))


def indexing():
    qsl = np.array([0, 1, 2, 10, 12], dtype=np.int32)
    seq_lens = np.array([5, 900, 8, 2], dtype=np.int32)
    tok, pos = okv.token_index(qsl, seq_lens, 12)
    bt = np.array([[3, -1], [0, 1], [7, -1], [9, 2]], dtype=np.int32)
    bt_big = np.zeros((4, 57), dtype=np.int32) - 1
    bt_big[:, :2] = bt
    slots = okv.slot_mapping(bt_big, 16, tok, pos)
    return dict(qsl=qsl, seq_lens=seq_lens, token_to_seq=tok, positions=pos,
                block_table=bt_big, slots=slots)


BUILDERS = {"kv_write": kv_write, "decode": decode, "prefill": prefill,
            "layer_ops": layer_ops, "indexing": indexing}


def _f32(d):
    """Expected float outputs are stored as float32 (well inside the tolerance)."""
    return {k: (v.astype(np.float32) if v.dtype == np.float64 and v.ndim else np.asarray(v))
            for k, v in d.items()}


def main():
    okv.build()
    for name, fn in BUILDERS.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **_f32(fn()))
        print(f"wrote {path.relative_to(REPO)} ({path.stat().st_size} B)")


if __name__ == "__main__":
    main()
