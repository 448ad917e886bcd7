"""The BASELINE configurations at their full sizes, built by the same workload
constructors bench.py times, checked against the fp64 oracle on every output
row and through size-independent properties:

- the fused decode write changes exactly the new tokens' cache rows, bit for
  bit as the oracle's write (kv_write.py:66-114 semantics);
- the split-K modes (balanced, fixed 512-token partitions) agree with each
  other and with the fp64 oracle;
- every output row is finite.

Each case prints its name before touching the GPU.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, host

import oracle.attention as oat
import oracle.kv as okv

pytestmark = pytest.mark.gpu


def _decode(b, out, partition):
    from vllm_apple_amd import kernels

    kernels.paged_decode(b.query, b.k_cache, b.v_cache, b.block_table, b.seq_lens,
                         scale=b.scale, max_seq_len=b.max_seq_len, output=out,
                         new_keys=b.new_k, new_values=b.new_v, partition_size=partition,
                         seq_lens_host=b.extra["seq_lens_host"])
    torch.cuda.synchronize()


def test_headline_c2_full_size(gpu):
    """Headline: B=32, every context 8192, 32q/8kv, D128, fused write, automatic
    split choice (unsplit at this shape)."""
    from vllm_apple_amd import workloads

    print("[case] headline C2 B=32 ctx=8192", flush=True)
    b = workloads.c2_decode(device=torch.device("cuda:0"), fixed_len=8192)
    kc0, vc0 = host(b.k_cache), host(b.v_cache)
    out = torch.empty_like(b.query)
    _decode(b, out, 0)
    o = host(out)
    assert np.all(np.isfinite(o.astype(np.float32)))
    # The fused write: exactly the oracle's write of all 32 new tokens.
    kr, vr = kc0.copy(), vc0.copy()
    okv.kv_write_decode(kr, vr, host(b.new_k), host(b.new_v), host(b.block_table),
                        host(b.seq_lens), "kernel")
    kd, vd = host(b.k_cache), host(b.v_cache)
    assert np.array_equal(kd.view(np.uint16), kr.view(np.uint16)), "fused K write"
    assert np.array_equal(vd.view(np.uint16), vr.view(np.uint16)), "fused V write"
    changed = np.count_nonzero(kd.view(np.uint16) != kc0.view(np.uint16))
    assert changed <= 32 * b.num_kv_heads * b.head_size
    # Every sequence's attention rows against the fp64 oracle.
    ref = oat.decode(host(b.query), kr, vr, host(b.block_table), host(b.seq_lens), b.scale,
                     "kernel")
    assert_close(o, ref, what="headline rows")


def test_c2_uniform_full_size_balanced(gpu):
    """C2 exactly as configured: B=32, contexts U[1024, 8192], the 18,750-block
    pool, fused write, through the automatically chosen split (the balanced
    one at these lengths); every sequence against the oracle and the fused
    write bit-exact."""
    from vllm_apple_amd import kernels, workloads

    print("[case] C2 B=32 ctx U[1024,8192]", flush=True)
    b = workloads.c2_decode(device=torch.device("cuda:0"))
    lens = b.extra["seq_lens_host"]
    assert b.k_cache.shape[0] == 18750
    auto = kernels.choose_partition_size(lens, b.num_kv_heads, kernels.device_cus(b.query.device))
    assert auto == kernels.PARTITION_BALANCED
    kc0, vc0 = host(b.k_cache), host(b.v_cache)
    out = torch.empty_like(b.query)
    _decode(b, out, 0)  # automatic: seq_lens_host picks the split
    kr, vr = kc0.copy(), vc0.copy()
    okv.kv_write_decode(kr, vr, host(b.new_k), host(b.new_v), host(b.block_table),
                        host(b.seq_lens), "kernel")
    assert np.array_equal(host(b.k_cache).view(np.uint16), kr.view(np.uint16)), "fused K write"
    assert np.array_equal(host(b.v_cache).view(np.uint16), vr.view(np.uint16)), "fused V write"
    ref = oat.decode(host(b.query), kr, vr, host(b.block_table), host(b.seq_lens), b.scale,
                     "kernel")
    assert_close(host(out), ref, what="C2 uniform rows")


def test_c4_full_size_split_modes(gpu):
    """C4: B=64, contexts log-uniform in [4096, 32768], 1 % of key rows scaled
    x8.  The balanced split (automatic choice) and the config's 512-token
    partitions agree, and both match the oracle on every sequence."""
    from vllm_apple_amd import kernels, workloads

    print("[case] C4 B=64 ctx logU[4k,32k]", flush=True)
    b = workloads.c4_long_decode(device=torch.device("cuda:0"))
    kc0, vc0 = host(b.k_cache), host(b.v_cache)
    lens = b.extra["seq_lens_host"]
    auto = kernels.choose_partition_size(lens, b.num_kv_heads, kernels.device_cus(b.query.device))
    assert auto == kernels.PARTITION_BALANCED
    out_bal = torch.empty_like(b.query)
    out_512 = torch.empty_like(b.query)
    _decode(b, out_bal, auto)
    _decode(b, out_512, 512)  # rewrites the same new tokens: idempotent
    ob, o5 = host(out_bal), host(out_512)
    assert_close(ob, o5.astype(np.float64), atol=1e-3, rtol=5e-3, what="balanced vs 512")
    kr, vr = kc0.copy(), vc0.copy()
    okv.kv_write_decode(kr, vr, host(b.new_k), host(b.new_v), host(b.block_table),
                        host(b.seq_lens), "kernel")
    assert np.array_equal(host(b.k_cache).view(np.uint16), kr.view(np.uint16)), "fused K write"
    ref = oat.decode(host(b.query), kr, vr, host(b.block_table), host(b.seq_lens), b.scale,
                     "kernel")
    assert_close(ob, ref, what="C4 balanced rows")
    assert_close(o5, ref, what="C4 512-partition rows")


@pytest.fixture(scope="module")
def c5_step(gpu):
    """C5 attention step as bench.py runs it: the step's K/V written through
    slot_mapping (2104 tokens), 56 decodes, 8 x 256-token prefill chunks over
    contexts U[256, 16384].  Returns the host copies the checks need."""
    from vllm_apple_amd import kernels, workloads

    print("[case] C5 attention step", flush=True)
    b = workloads.c5_mixed(device=torch.device("cuda:0"))
    nd = b.num_decode_tokens
    lens = b.extra["seq_lens_host"]
    kc0, vc0 = host(b.k_cache), host(b.v_cache)
    out = torch.empty_like(b.query)
    kernels.kv_write_slots(b.new_k, b.new_v, b.k_cache, b.v_cache, b.slot_mapping)
    kernels.paged_decode(b.query[:nd], b.k_cache, b.v_cache, b.block_table[:nd],
                         b.seq_lens[:nd], scale=b.scale, max_seq_len=max(lens[:nd]),
                         output=out[:nd], seq_lens_host=lens[:nd])
    kernels.paged_prefill(b.query[nd:], b.k_cache, b.v_cache, b.block_table,
                          b.token_to_seq[nd:], b.positions[nd:], scale=b.scale,
                          output=out[nd:])
    torch.cuda.synchronize()
    kr, vr = kc0.copy(), vc0.copy()
    okv.kv_write_slots(kr, vr, host(b.new_k), host(b.new_v), host(b.slot_mapping))
    return dict(out=host(out), kd=host(b.k_cache), vd=host(b.v_cache), kr=kr, vr=vr,
                q=host(b.query), bt=host(b.block_table), lens=host(b.seq_lens),
                tok=host(b.token_to_seq), pos=host(b.positions), nd=nd, scale=b.scale,
                num_seqs=b.num_seqs)


def test_c5_step_kv_write_and_decodes(c5_step):
    """The slot write is bit-exact over the whole cache; all 56 decode rows
    match the oracle."""
    c = c5_step
    assert np.array_equal(c["kd"].view(np.uint16), c["kr"].view(np.uint16)), "K write"
    assert np.array_equal(c["vd"].view(np.uint16), c["vr"].view(np.uint16)), "V write"
    nd = c["nd"]
    ref_d = oat.decode(c["q"][:nd], c["kr"], c["vr"], c["bt"][:nd], c["lens"][:nd], c["scale"],
                       "kernel")
    assert_close(c["out"][:nd], ref_d, what="C5 decode rows")


@pytest.mark.parametrize("chunk", range(8))
def test_c5_step_prefill_chunk(c5_step, chunk):
    """Every row of one 256-token prefill chunk against the oracle."""
    c = c5_step
    s = c["nd"] + chunk
    rows = np.nonzero(c["tok"] == s)[0]
    assert rows.size == 256
    ref_p, written = oat.prefill(c["q"], c["kr"], c["vr"], c["bt"], c["tok"], c["pos"],
                                 c["scale"], "kernel", rows=rows)
    assert written[rows].all()
    assert_close(c["out"][rows], ref_p[rows], what=f"C5 prefill chunk {chunk}")
