"""bench.py's CPU-baseline leg on the CPU: the host copy of a sequence subset
(blocks renumbered, slots remapped) runs the reference torch path to the same
rows as the fp64 oracle over the original batch, and the host description
names the thread count it used."""
import numpy as np
import torch

import bench
import oracle.attention as oat
import oracle.kv as okv
from helpers import assert_close
from vllm_apple_amd import workloads


def _ref_after_write(b):
    kc, vc = b.k_cache.numpy().copy(), b.v_cache.numpy().copy()
    okv.kv_write_slots(kc, vc, b.new_k.numpy(), b.new_v.numpy(), b.slot_mapping.numpy())
    return kc, vc


def test_host_step_decode_subset_matches_oracle():
    b = workloads.c1_decode()
    h = bench.HostStep(b, n=3)
    assert h.n == 3 and h.num_tokens == 3
    assert h.k.shape[0] == sum((L + 15) // 16 for L in b.extra["seq_lens_host"][:3])
    h.write()
    out = h.decode().numpy()
    kc, vc = _ref_after_write(b)
    ref = oat.decode(b.query.numpy()[:3], kc, vc, b.block_table.numpy()[:3],
                     b.seq_lens.numpy()[:3], b.scale, "kernel")
    assert_close(out, ref, what="host-step decode")


def test_host_step_mixed_prefill_matches_oracle():
    b = workloads.c3_prefill(cached=64, chunk=32, num_seqs=3)
    h = bench.HostStep(b)
    h.write()
    out = h.prefill(1, 3).numpy()
    kc, vc = _ref_after_write(b)
    rows = np.nonzero(b.token_to_seq.numpy() >= 1)[0]
    ref, _ = oat.prefill(b.query.numpy(), kc, vc, b.block_table.numpy(),
                         b.token_to_seq.numpy(), b.positions.numpy(), b.scale, "kernel",
                         rows=rows)
    assert_close(out, ref[rows], what="host-step prefill")


def test_cpu_env_and_record():
    env = bench.cpu_env()
    assert env["threads"] >= 1 and env["threads"] <= env["os_cpu_count"]
    assert env["torch"] == torch.__version__
    bench._CPU_ENV = env
    try:
        rec = bench.cpu_record(1.0, "GB/s", "x")
    finally:
        bench._CPU_ENV = None
    assert rec["cores"] == env["threads"] and rec["kind"] == "port"
    assert rec["host"]["cpu_model"] == env["cpu_model"]


def test_bench_refuses_more_than_one_gpu():
    """bench.py runs on one GPU: --gpus above 1 exits with status 2 and a JSON
    line that says so, before touching any device."""
    import json
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(repo / "bench.py"), "--gpus", "2", "--steps", "1",
                        "--warmup", "0"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]
