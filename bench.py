"""Headline benchmark: paged decode step on one MI355X.

Workload (BASELINE.json metric "paged-attn decode GB/s (% HBM peak) + tokens/sec
at B=32, 8k ctx, 32q/8kv hd128"): Mistral-Small-22B-shaped decode step, B=32
sequences all at 8192 tokens of context, 32 query heads / 8 kv heads,
head_dim 128, fp16, block_size 16, physical blocks shuffled across a pool sized
for 300k tokens.  One step = the fused KV write of each sequence's new token
plus paged GQA attention over the whole context (one partition per
sequence at this shape, so no merge launch): a single kernel launch, inputs
resident in HBM.

value       algorithmic bytes of the step / wall time per step (GB/s)
roofline    the decode kernel's algorithmic bytes / its average launch duration
            from HIP events on the launch stream bracketing the timed region,
            against 8 TB/s
cpu_baseline the reference's CPU torch path (per-sequence gather +
            repeat_interleave + SDPA, oracle/ref_torch.py) on the same inputs
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "vllm-apple_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
METRIC = "paged-attn decode GB/s (% HBM peak) + tokens/sec at B=32, 8k ctx, 32q/8kv hd128"


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--partition", type=int, default=0, help="split-K tokens (0 = auto)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefix", type=int, default=2048,
                    help="C3: cached tokens before each 512-token chunk (2048 = the config)")
    ap.add_argument("--split-keys", type=int, default=0,
                    help="C3: also time the prefill split into key pieces of this many keys "
                         "(a multiple of 64; 0 = unsplit only)")
    ap.add_argument("--tokens", type=int, default=2104,
                    help="C5mlp: tokens of the gate/up projection (2104 = the C5 step)")
    ap.add_argument("--workload", default="headline",
                    choices=["headline", "C1", "C2u", "C3", "C4", "C5", "C5mlp", "C2bf16", "topk",
                             "C3-launches", "all"],
                    help="headline = the contract line; the others print one JSON line per "
                         "BASELINE config (measurement record, not the driver's metric)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="calibration mode: time a plain device-to-device copy of this "
                         "many bytes instead of the decode step (for HBM counter scaling)")
    return ap.parse_args()


def copy_calibration(nbytes: int, steps: int, warmup: int) -> dict:
    """A plain copy kernel of known size: its FETCH_SIZE/WRITE_SIZE per launch
    calibrate the PMC-derived HBM traffic of the decode kernel."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"mode": "copy-calibration", "bytes_read_per_launch": nbytes,
            "bytes_written_per_launch": nbytes, "ms_per_copy": round(ms, 5),
            "copy_gb_s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def traffic_from_profile() -> float | None:
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if present."""
    f = REPO / "profiles" / "paged_decode_c2_8k_traffic.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            try:
                return float(line.split("=", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_env() -> dict:
    """The host the CPU baseline runs on.  Read before the GPU is touched
    (`nproc` runs as a child process)."""
    import subprocess

    total = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = total
    quota = None
    try:  # cgroup v2 CPU quota: "<quota> <period>" or "max <period>"
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(per))
    except (OSError, ValueError):
        pass
    try:
        nproc = int(subprocess.run(["nproc"], capture_output=True, text=True,
                                   timeout=10).stdout.strip())
    except (OSError, ValueError, subprocess.SubprocessError):
        nproc = None
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    import torch

    return {"os_cpu_count": total, "affinity_cpus": affinity, "cgroup_cpus": quota,
            "nproc": nproc, "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "cpu_model": model, "torch": torch.__version__,
            # torch.set_num_threads(os.cpu_count()), capped at the CPUs this
            # process may run on: threads beyond those only time-slice.
            "threads": max(1, min(total, affinity, quota or total))}


_CPU_ENV: dict | None = None


def _cpu_timed(fn, budget_s: float, min_runs: int = 5) -> tuple[float, int]:
    """One warm-up call, then at least min_runs timed calls (more while the
    budget lasts); returns (median seconds, runs)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s
                                    and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


class HostStep:
    """Host copies of a batch's sequences [0, n) in the vLLM layout the
    reference's torch path reads ([nb, bs, KV, D], fp16 storage): only the
    blocks those sequences use, renumbered, with their block table, slots and
    tokens.  Building it is not timed."""

    def __init__(self, b, n: int | None = None):
        import torch

        from oracle import ref_torch

        S = b.num_seqs
        n = S if n is None else min(n, S)
        lens = b.extra["seq_lens_host"][:n]
        bs = b.block_size
        nblk = [(L + bs - 1) // bs for L in lens]
        bt = b.block_table[:n].cpu()
        used = torch.cat([bt[s, :k] for s, k in enumerate(nblk)]).long()
        remap = torch.full((b.k_cache.shape[0],), -1, dtype=torch.int64)
        remap[used] = torch.arange(used.numel())
        self.k = ref_torch.kernel_to_vllm_layout(b.k_cache[used.to(b.k_cache.device)].cpu())
        self.v = ref_torch.kernel_to_vllm_layout(b.v_cache[used.to(b.v_cache.device)].cpu())
        self.bt = torch.full((n, max(nblk) if nblk else 1), -1, dtype=torch.int32)
        for s, k in enumerate(nblk):
            self.bt[s, :k] = remap[bt[s, :k].long()].to(torch.int32)
        qsl = b.query_start_loc.cpu()
        t1 = int(qsl[n])
        self.q = b.query[:t1].cpu()
        self.new_k, self.new_v = b.new_k[:t1].cpu(), b.new_v[:t1].cpu()
        slots = b.slot_mapping[:t1].cpu()
        self.slots = remap[slots // bs] * bs + slots % bs
        self.qsl = qsl[:n + 1].tolist()
        self.lens = list(lens)
        self.n, self.num_tokens = n, t1
        self.kv, self.scale = b.num_kv_heads, b.scale

    def write(self):
        from oracle import ref_torch

        ref_torch.update_kv_cache_scatter(self.new_k, self.new_v, self.k, self.v, self.slots)

    def decode(self, s0: int = 0, s1: int | None = None):
        """Decode sequences [s0, s1) (one query token each)."""
        from oracle import ref_torch

        s1 = self.n if s1 is None else s1
        t0, t1 = self.qsl[s0], self.qsl[s1]
        return ref_torch.decode_sdpa(self.q[t0:t1], self.k, self.v, self.bt[s0:s1],
                                     self.lens[s0:s1], self.scale, self.kv)

    def prefill(self, s0: int = 0, s1: int | None = None):
        """Chunked prefill of sequences [s0, s1) over their cached prefix."""
        from oracle import ref_torch

        s1 = self.n if s1 is None else s1
        t0 = self.qsl[s0]
        return ref_torch.prefill_sdpa_prefix(self.q[t0:self.qsl[s1]], self.k, self.v,
                                             self.bt[s0:s1],
                                             [x - t0 for x in self.qsl[s0:s1 + 1]],
                                             self.lens[s0:s1], self.scale, self.kv)


def cpu_record(value: float, unit: str, sample: str, **extra) -> dict:
    env = _CPU_ENV or {}
    rec = {"value": value, "unit": unit, "cores": env.get("threads"), "kind": "port",
           "sample": sample}
    rec.update(extra)
    rec["host"] = {k: env.get(k) for k in ("cpu_model", "nproc", "os_cpu_count",
                                           "affinity_cpus", "cgroup_cpus", "omp_num_threads",
                                           "torch")}
    return rec


def _cpu_threads() -> int:
    import torch

    threads = (_CPU_ENV or {}).get("threads") or 1
    torch.set_num_threads(threads)
    return threads


def cpu_decode_step(b, budget_s: float, n: int | None = None, what: str = "decode step") -> dict:
    """The reference's CPU step for a decode batch: the KV scatter of the new
    tokens (base_attn.py:308-342) then per-sequence gather + repeat_interleave
    + SDPA (mps_attn.py:284-357), on sequences [0, n) of the batch."""
    _cpu_threads()
    h = HostStep(b, n)

    def step():
        h.write()
        h.decode()

    med, runs = _cpu_timed(step, budget_s)
    lens = h.lens
    B, H, KV, D = h.n, b.num_q_heads, b.num_kv_heads, b.head_size
    alg = (sum(lens) * KV * D * 4 + 2 * B * H * D * 2 + 2 * 2 * B * KV * D * 2
           + sum((L + b.block_size - 1) // b.block_size for L in lens) * 4 + B * 4)
    sample = (f"{'all ' if h.n == b.num_seqs else ''}{h.n} of {b.num_seqs} sequences "
              f"(ctx mean {sum(lens) / len(lens):.0f}, max {max(lens)}) of the same {what}, "
              f"median of {runs} runs after 1 warm-up")
    return cpu_record(round(alg / med / 1e9, 3), "GB/s", sample, ms_per_step=round(med * 1e3, 3),
                      latency_us=round(med * 1e6, 1), tokens_per_s=round(h.n / med, 1),
                      algorithmic_bytes=alg)


MFMA_F16_PEAK_TFLOPS = 2500.0



def _timed(fn, steps: int, warmup: int) -> float:
    """Average GPU time (ms) of one call of fn.

    The calls are captured back to back in a HIP graph and the replay is timed
    with HIP events on the launch stream, so a short kernel is not starved by
    the host-side Python of its wrapper (a serving loop replays graphs the same
    way).  Falls back to timing `steps` eager calls between two events if the
    capture fails.
    """
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(steps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps
    except RuntimeError:
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _timed_eager(fn, steps: int) -> float:
    """Average time (ms) of `steps` eager calls of fn between two events on
    the launch stream (host-side launch cost included, as a caller sees it)."""
    import torch

    fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _timed_rot(fns, steps: int, warmup: int) -> float:
    """_timed over a rotation: call i runs fns[i % len(fns)], each on its own
    copy of the data, so the bytes touched per rotation exceed the 256 MB
    Infinity Cache and a bandwidth figure is not inflated by cache hits."""
    state = {"i": 0}

    def call():
        fns[state["i"] % len(fns)]()
        state["i"] += 1

    return _timed(call, steps, warmup)


def _copies(nbytes: int, floor: int = 1) -> int:
    """Copies of a working set of nbytes needed to touch more than 256 MB."""
    return max(floor, -(-300_000_000 // max(1, nbytes)))


def _copy_floor(moved_bytes: int, steps: int, warmup: int) -> float:
    """ms of a plain device copy (torch's copy_) that reads moved_bytes / 2 and
    writes moved_bytes / 2, timed over a rotation like the ops: the practical
    HBM floor for one pass of this size.  Below a few hundred MB a pass pays
    the launch, the first memory latency and the tail of its last wave, so even
    this copy stays well under the 8 TB/s peak (43 MB: about 54 %)."""
    import torch

    n = max(1, moved_bytes // 4)  # fp16 elements per copy
    dev = torch.device("cuda:0")
    sets = [(torch.empty(n, dtype=torch.float16, device=dev).normal_(),
             torch.empty(n, dtype=torch.float16, device=dev)) for _ in range(_copies(4 * n))]
    t = _timed_rot([lambda s=s_: s[1].copy_(s[0]) for s_ in sets], steps, warmup)
    del sets
    return t


def _vs_copy(t_op: float, moved_bytes: int, steps: int, warmup: int) -> dict:
    """The copy floor of an op's bytes and the op's time as a fraction of it."""
    t_c = _copy_floor(moved_bytes, steps, warmup)
    return {"copy_floor_ms": round(t_c, 5), "copy_floor_pct_hbm_peak":
            round(100 * moved_bytes / (t_c * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
            "op_vs_copy_floor": round(t_c / t_op, 3)}


def _decode_record(name: str, b, args, partition: int, note: str) -> dict:
    import torch

    from vllm_apple_amd import kernels

    out = torch.empty_like(b.query)
    lens = b.extra["seq_lens_host"]

    def step():
        kernels.paged_decode(b.query, b.k_cache, b.v_cache, b.block_table, b.seq_lens,
                             scale=b.scale, max_seq_len=b.max_seq_len, output=out,
                             new_keys=b.new_k, new_values=b.new_v, partition_size=partition,
                             seq_lens_host=lens)

    ms = _timed(step, args.steps, args.warmup)
    alg = b.decode_algorithmic_bytes()
    used = partition or kernels.choose_partition_size(lens, b.num_kv_heads,
                                                      kernels.device_cus(b.query.device))
    if used == kernels.PARTITION_BALANCED:
        used = "balanced"
    return {"workload": name, "note": note, "batch": b.num_seqs,
            "ctx_mean": round(sum(lens) / len(lens), 1), "ctx_max": max(lens),
            "partition": used, "ms_per_step": round(ms, 5),
            "algorithmic_bytes": alg, "gb_s": round(alg / (ms * 1e-3) / 1e9, 1),
            "pct_hbm_peak": round(100 * alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
            "tokens_per_s": round(b.num_seqs / (ms * 1e-3), 1)}


def _read_stream(b, args, partition: int) -> dict:
    """The K/V rows of a decode record read by vaa_kv_stream_read in the same
    pieces (partition tokens per workgroup, 0: one per sequence), timed like
    the record: the ceiling of that decomposition's stream."""
    import torch

    from vllm_apple_amd import kernels

    parts = -(-b.max_seq_len // partition) if partition else 1
    sink = torch.empty((b.num_seqs, parts, b.num_kv_heads), dtype=torch.int32,
                       device=b.k_cache.device)
    kv_bytes = int(b.seq_lens.sum().item()) * b.num_kv_heads * b.head_size * 2 * 2
    t = _timed(lambda: kernels.kv_stream_read(b.k_cache, b.v_cache, b.block_table, b.seq_lens,
                                              partition_size=partition,
                                              max_seq_len=b.max_seq_len, sink=sink),
               args.steps, args.warmup)
    gbs = kv_bytes / (t * 1e-3) / 1e9
    return {"kernel": "kv_stream_kernel<128>", "partition": partition or "none",
            "bytes": kv_bytes, "ms": round(t, 5), "gb_s": round(gbs, 1),
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}


def wl_c1(args) -> dict:
    import torch

    from vllm_apple_amd import workloads

    b = workloads.c1_decode(device=torch.device("cuda:0"))
    r = _decode_record("C1", b, args, 0, "Qwen2-0.5B decode, B=4, cache-resident: latency")
    r["latency_us"] = round(r["ms_per_step"] * 1e3, 2)
    if not args.no_cpu_baseline:
        r["cpu_baseline"] = cpu_decode_step(b, args.cpu_seconds)
    return r


def wl_c2u(args) -> dict:
    import torch

    from vllm_apple_amd import workloads

    b = workloads.c2_decode(device=torch.device("cuda:0"))
    r = _decode_record("C2u", b, args, 0, "ctx U{1024..8192}, split-K chosen from lengths")
    if not args.no_cpu_baseline:
        r["cpu_baseline"] = cpu_decode_step(b, args.cpu_seconds)
    return r


def wl_c4(args) -> dict:
    import torch

    from vllm_apple_amd import workloads

    b = workloads.c4_long_decode(device=torch.device("cuda:0"))
    r512 = _decode_record("C4", b, args, 512, "512-token partitions + LSE merge (config spec)")
    rauto = _decode_record("C4", b, args, 0, "partition chosen from lengths")
    r512["auto_partition"] = {k: rauto[k] for k in ("partition", "ms_per_step", "gb_s",
                                                   "pct_hbm_peak")}
    r512["read_stream"] = _read_stream(b, args, 512)
    r512["scaled_key_rows"] = b.extra["scaled_rows"]
    if not args.no_cpu_baseline:
        # A quarter of the batch keeps the sample to a few seconds per step.
        r512["cpu_baseline"] = cpu_decode_step(b, args.cpu_seconds, n=16)
    return r512


def _prefill_flops(b) -> float:
    """Causal-exact: 4 * D per (query token, head, attended key)."""
    ctx = (b.positions.double() + 1).sum().item()
    return 4.0 * b.head_size * b.num_q_heads * ctx


def wl_c3(args) -> dict:
    import torch

    from vllm_apple_amd import kernels, workloads

    b = workloads.c3_prefill(device=torch.device("cuda:0"), cached=args.prefix)
    out = torch.empty_like(b.query)
    # KV write: each rotation copy has its own new K/V and its own cache.
    T = b.query.shape[0]
    kv_bytes = 2 * 2 * T * b.num_kv_heads * b.head_size * 2 + T * 8
    kv_sets = [(b.new_k.clone(), b.new_v.clone(), b.k_cache.clone(), b.v_cache.clone())
               for _ in range(_copies(kv_bytes))]
    t_kv = _timed_rot([lambda s=s_: kernels.kv_write_slots(s[0], s[1], s[2], s[3], b.slot_mapping)
                       for s_ in kv_sets], args.steps, args.warmup)
    del kv_sets
    t_at = _timed(lambda: kernels.paged_prefill(b.query, b.k_cache, b.v_cache, b.block_table,
                                                b.token_to_seq, b.positions, scale=b.scale,
                                                output=out), args.steps, args.warmup)
    fl = _prefill_flops(b)
    bb = workloads.c3_prefill(device=torch.device("cuda:0"), dtype=torch.bfloat16,
                              cached=args.prefix)
    out_b = torch.empty_like(bb.query)
    t_bf = _timed(lambda: kernels.paged_prefill(bb.query, bb.k_cache, bb.v_cache, bb.block_table,
                                                bb.token_to_seq, bb.positions, scale=bb.scale,
                                                output=out_b), args.steps, args.warmup)
    rec = {"workload": "C3", "note": f"4 x ({args.prefix} cached + 512 new), causal chunk",
            "tokens": T, "kv_write_ms": round(t_kv, 5),
            "kv_write_gb_s": round(kv_bytes / (t_kv * 1e-3) / 1e9, 1),
            "kv_write_copy_floor": _vs_copy(t_kv, kv_bytes, args.steps, args.warmup),
            "prefill_ms": round(t_at, 5), "flops": fl,
            "tflop_s": round(fl / (t_at * 1e-3) / 1e12, 1),
            "mfma_util_pct": round(100 * fl / (t_at * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 2),
            "bf16_prefill_ms": round(t_bf, 5),
            "bf16_tflop_s": round(fl / (t_bf * 1e-3) / 1e12, 1)}
    if args.split_keys:
        t_sp = _timed(lambda: kernels.paged_prefill(b.query, b.k_cache, b.v_cache, b.block_table,
                                                    b.token_to_seq, b.positions, scale=b.scale,
                                                    output=out, split_keys=args.split_keys,
                                                    max_seq_len=args.prefix + 512),
                      args.steps, args.warmup)
        rec["split_keys"] = args.split_keys
        rec["prefill_split_ms"] = round(t_sp, 5)
    if not args.no_cpu_baseline:
        _cpu_threads()
        h = HostStep(b)
        t_w, n_w = _cpu_timed(h.write, args.cpu_seconds / 3)
        t_p, n_p = _cpu_timed(h.prefill, args.cpu_seconds * 2 / 3)
        rec["cpu_baseline"] = cpu_record(
            round(fl / t_p / 1e12, 4), "TFLOP/s",
            f"the whole C3 step: KV scatter of {T} tokens (median of {n_w} runs) and the "
            f"prefill of all 4 chunks over their prefixes (median of {n_p} runs), 1 warm-up each",
            kv_write_ms=round(t_w * 1e3, 3), kv_write_gb_s=round(kv_bytes / t_w / 1e9, 3),
            prefill_ms=round(t_p * 1e3, 3))
    return rec


def wl_c5(args) -> dict:
    import torch

    from vllm_apple_amd import kernels, workloads

    dev = torch.device("cuda:0")
    b = workloads.c5_mixed(device=dev)
    nd = b.num_decode_tokens
    T = b.query.shape[0]
    out = torch.empty_like(b.query)
    lens = b.extra["seq_lens_host"]

    def decode(shared=False):
        kernels.paged_decode(b.query[:nd], b.k_cache, b.v_cache, b.block_table[:nd],
                             b.seq_lens[:nd], scale=b.scale, max_seq_len=max(lens[:nd]),
                             output=out[:nd], seq_lens_host=lens[:nd], shared=shared)

    # The key split the backend chooses for these prefill chunks when they run
    # alone; next to the decode it runs them unsplit.
    qlens = [0] * nd + [256] * (b.num_seqs - nd)
    split = kernels.choose_prefill_split(lens, qlens, b.num_kv_heads, b.num_q_heads,
                                         kernels.device_cus(dev))

    def prefill(split_keys=0):
        kernels.paged_prefill(b.query[nd:], b.k_cache, b.v_cache, b.block_table,
                              b.token_to_seq[nd:], b.positions[nd:], scale=b.scale,
                              output=out[nd:], split_keys=split_keys, max_seq_len=max(lens))

    def attn_step():
        # As the backend runs a mixed step: the KV write, then prefill (current
        # stream) and decode (side stream, shared split) concurrently.
        kernels.kv_write_slots(b.new_k, b.new_v, b.k_cache, b.v_cache, b.slot_mapping)
        kernels.overlap(prefill, lambda: decode(shared=True), dev)

    def attn_step_serial():
        kernels.kv_write_slots(b.new_k, b.new_v, b.k_cache, b.v_cache, b.slot_mapping)
        decode()
        prefill(split)

    t_attn = _timed(attn_step, args.steps, args.warmup)
    t_attn_serial = _timed(attn_step_serial, args.steps, args.warmup)
    t_prefill = _timed(lambda: prefill(split), args.steps, args.warmup)
    t_prefill_whole = _timed(prefill, args.steps, args.warmup)
    t_decode = _timed(decode, args.steps, args.warmup)
    # Eager calls too: vLLM runs the attention of mixed batches outside graphs.
    t_attn_eager = _timed_eager(attn_step, args.steps)
    t_attn_serial_eager = _timed_eager(attn_step_serial, args.steps)
    # Layer ops: each timed over a rotation of input/output copies whose bytes
    # exceed the 256 MB Infinity Cache.
    x, w = b.extra["hidden"], b.extra["norm_weight"]
    y = torch.empty_like(x)
    eps = b.extra["eps"]
    norm_sets = [(x.clone(), torch.empty_like(x)) for _ in range(_copies(2 * x.numel() * 2))]
    t_norm = _timed_rot([lambda s=s_: kernels.rms_norm(s[0], w, eps, out=s[1])
                         for s_ in norm_sets], args.steps, args.warmup)
    del norm_sets
    cos, sin = kernels.rope_cos_sin_cache(b.head_size, 16384, b.extra["rope_base"], device=dev)
    q2, k2 = b.query.clone(), b.new_k.clone()
    rope_sets = [(q2.clone(), k2.clone())
                 for _ in range(_copies((q2.numel() + k2.numel()) * 2))]
    t_rope = _timed_rot([lambda s=s_: kernels.rope_neox_(s[0], s[1], cos, sin, b.positions)
                         for s_ in rope_sets], args.steps, args.warmup)
    del rope_sets
    # QKV epilogue over the step's planar QKV views: fused (one launch) against
    # the reference's three passes (bias add, RoPE, KV write).
    T_, H_, KV_, D_ = T, b.num_q_heads, b.num_kv_heads, b.head_size
    gq = torch.Generator(device=dev).manual_seed(7)
    qkv = torch.randn(T_ * (H_ + 2 * KV_) * D_, generator=gq, device=dev).half()
    bias = torch.randn((H_ + 2 * KV_) * D_, generator=gq, device=dev).half()
    def epi_views(buf):
        return (buf[:T_ * H_ * D_].view(T_, H_, D_),
                buf[T_ * H_ * D_:T_ * (H_ + KV_) * D_].view(T_, KV_, D_),
                buf[T_ * (H_ + KV_) * D_:].view(T_, KV_, D_))

    # Rotation: own QKV buffer and own (random, distinct) cache slots per copy.
    n_slots = b.k_cache.shape[0] * b.k_cache.shape[2]
    epi_sets = [(epi_views(qkv.clone()),
                 torch.randperm(n_slots, generator=gq, device=dev)[:T_].to(torch.int64))
                for _ in range(_copies(qkv.numel() * 2 * 2))]
    t_epi = _timed_rot([lambda s=s_: kernels.qkv_epilogue(*s[0], b.positions, cos, sin, s[1],
                                                          b.k_cache, b.v_cache, bias=bias)
                        for s_ in epi_sets], args.steps, args.warmup)

    def three_step(s):
        (qv, kv_, vv), slots = s
        qv.add_(bias[:H_ * D_].view(1, H_, D_))
        kv_.add_(bias[H_ * D_:(H_ + KV_) * D_].view(1, KV_, D_))
        vv.add_(bias[(H_ + KV_) * D_:].view(1, KV_, D_))
        kernels.rope_neox_(qv, kv_, cos, sin, b.positions)
        kernels.kv_write_slots(kv_, vv, b.k_cache, b.v_cache, slots)

    t_three = _timed_rot([lambda s=s_: three_step(s) for s_ in epi_sets], args.steps,
                         args.warmup)
    del epi_sets
    n_qkv = qkv.numel() * 2
    epi_bytes = 2 * n_qkv + bias.numel() * 2 + T_ * (D_ // 2) * 4 * 2 + T_ * 8 \
        + 2 * T_ * KV_ * D_ * 2
    # Residual add + RMSNorm: fused against the reference's residual add, copy
    # into the residual buffer and norm (three passes, 7 row-sized accesses).
    res_a = torch.randn(x.shape, generator=gq, device=dev).half()
    an_sets = [(x.clone(), res_a.clone(), torch.empty_like(x))
               for _ in range(_copies(3 * x.numel() * 2))]
    t_addnorm = _timed_rot([lambda s=s_: kernels.add_rms_norm(s[0], s[1], w, eps, out=s[2])
                            for s_ in an_sets], args.steps, args.warmup)

    def addnorm_three(s):
        torch.add(s[0], s[1], out=s[2])
        s[1].copy_(s[2])
        kernels.rms_norm(s[2], w, eps, out=s[2])

    t_addnorm3 = _timed_rot([lambda s=s_: addnorm_three(s) for s_ in an_sets], args.steps,
                            args.warmup)
    del an_sets
    addnorm_bytes = 4 * x.numel() * 2 + w.numel() * 2
    g, u = b.extra["gate"], b.extra["up"]
    act = torch.empty_like(g)
    t_silu = _timed(lambda: kernels.silu_mul(g, u, out=act), args.steps, args.warmup)
    H, KV, D = b.num_q_heads, b.num_kv_heads, b.head_size
    norm_bytes = 2 * x.numel() * 2 + w.numel() * 2
    rope_bytes = 2 * (q2.numel() + k2.numel()) * 2 + T * (D // 2) * 4 * 2 + T * 4
    silu_bytes = 3 * g.numel() * 2
    kv_read = sum(lens[:nd]) * KV * D * 4
    pre_ctx = (b.positions[nd:].double() + 1).sum().item()
    rec = {"workload": "C5", "note": "56 decodes + 8 x 256-token chunks; layer ops over 2104 tokens",
           "attention_step_ms": round(t_attn, 5),
           "attention_step_serial_ms": round(t_attn_serial, 5),
           "attention_step_eager_ms": round(t_attn_eager, 5),
           "attention_step_serial_eager_ms": round(t_attn_serial_eager, 5),
           "prefill_split_keys": split,
           "prefill_ms": round(t_prefill, 5), "prefill_unsplit_ms": round(t_prefill_whole, 5),
           "decode_ms": round(t_decode, 5),
           "attention_decode_kv_bytes": kv_read,
           "attention_prefill_flops": 4.0 * D * H * pre_ctx}
    rec["qkv_epilogue_three_pass_ms"] = round(t_three, 5)
    rec["add_rmsnorm_three_pass_ms"] = round(t_addnorm3, 5)
    for nm, t, by in (("rmsnorm", t_norm, norm_bytes), ("rope", t_rope, rope_bytes),
                      ("silu_mul", t_silu, silu_bytes), ("qkv_epilogue", t_epi, epi_bytes),
                      ("add_rmsnorm", t_addnorm, addnorm_bytes)):
        rec[nm] = {"ms": round(t, 5), "bytes": by, "gb_s": round(by / (t * 1e-3) / 1e9, 1),
                   "pct_hbm_peak": round(100 * by / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                   **_vs_copy(t, by, args.steps, args.warmup)}
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_c5(b, args.cpu_seconds,
                                     {"rmsnorm": norm_bytes, "rope": rope_bytes,
                                      "silu_mul": silu_bytes})
    return rec


def cpu_c5(b, budget_s: float, layer_bytes: dict) -> dict:
    """The reference's CPU path for the whole C5 step: the KV scatter of all
    2104 tokens, the 56 decodes, the 8 prefill chunks, then F.rms_norm over
    the hidden rows, NeoX RoPE (runner.py:1500-1524) over q and k, and
    F.silu(g) * u over the intermediate rows."""
    import torch

    import oracle.layer_ops as olo
    from oracle import ref_torch

    _cpu_threads()
    h = HostStep(b)
    nd = b.num_decode_tokens

    def attn():
        h.write()
        h.decode(0, nd)
        h.prefill(nd, h.n)

    t_att, n_att = _cpu_timed(attn, budget_s)
    x, w = b.extra["hidden"].cpu(), b.extra["norm_weight"].cpu()
    eps = b.extra["eps"]
    cos, sin = (torch.from_numpy(t) for t in olo.cos_sin(b.head_size, 16384,
                                                          b.extra["rope_base"]))
    pos = b.positions.cpu()
    g, u = b.extra["gate"].cpu(), b.extra["up"].cpu()
    parts = {}
    for nm, fn in (("rmsnorm", lambda: ref_torch.rms_norm(x, w, eps)),
                   ("rope", lambda: (ref_torch.rope_neox(h.q, pos, cos, sin),
                                     ref_torch.rope_neox(h.new_k, pos, cos, sin))),
                   ("silu_mul", lambda: ref_torch.silu_mul(g, u))):
        t, n = _cpu_timed(fn, budget_s / 6)
        parts[nm] = {"ms": round(t * 1e3, 3), "gb_s": round(layer_bytes[nm] / t / 1e9, 3),
                     "runs": n}
    return cpu_record(round(t_att * 1e3, 3), "ms per attention step",
                      f"the whole C5 step: KV scatter of {h.num_tokens} tokens + {nd} decodes + "
                      f"{h.n - nd} prefill chunks (median of {n_att} runs after 1 warm-up); "
                      f"layer ops over all {h.num_tokens} tokens",
                      layer_ops=parts)


def wl_c2bf16(args) -> dict:
    """The headline shape (B=32, all contexts 8192) with a bf16 cache and bf16
    activations: bf16 models run through the same kernels without an fp16 copy."""
    import torch

    from vllm_apple_amd import workloads

    b = workloads.c2_decode(device=torch.device("cuda:0"), fixed_len=8192,
                            dtype=torch.bfloat16)
    return _decode_record("C2-bf16", b, args, 0, "headline shape in bf16 (extension)")


def wl_c5mlp(args) -> dict:
    """C5's SwiGLU with its producer: the gated MLP's up projection
    (2104 tokens, or --tokens, hidden 5120, intermediate 32768; x N(0,1), the fused
    gate_up weight [65536, 5120] N(0, 1/5120)) with the SiLU*mul epilogue in
    one MFMA kernel, against the reference's order on this GPU: the
    projection as a library GEMM (torch.matmul, hipBLASLt) into a [T, 2I]
    buffer, then vaa_silu_mul over its halves."""
    import torch

    from vllm_apple_amd import kernels

    dev = torch.device("cuda:0")
    T, H, I = args.tokens, 5120, 32768
    g = torch.Generator(device=dev).manual_seed(55)
    x = torch.randn(T, H, generator=g, device=dev).half()
    w = (torch.randn(2 * I, H, generator=g, device=dev) / H ** 0.5).half()
    act = torch.empty(T, I, dtype=torch.float16, device=dev)
    gu = torch.empty(T, 2 * I, dtype=torch.float16, device=dev)
    t_fused = _timed(lambda: kernels.gate_up_silu(x, w, out=act), args.steps, args.warmup)
    t_gemm = _timed(lambda: torch.matmul(x, w.T, out=gu), args.steps, args.warmup)

    def unfused():
        torch.matmul(x, w.T, out=gu)
        kernels.silu_mul(gu[:, :I], gu[:, I:], out=act)

    t_unfused = _timed(unfused, args.steps, args.warmup)
    flops = 2.0 * T * H * 2 * I
    tf = flops / (t_fused * 1e-3) / 1e12
    return {"workload": "C5mlp", "note": f"gate_up projection + SwiGLU, {T} x 5120 -> 2 x 32768",
            "flops": flops,
            "gate_up_silu_ms": round(t_fused, 5), "gate_up_silu_tflops": round(tf, 1),
            "pct_mfma_peak_f16": round(100 * tf / MFMA_F16_PEAK_TFLOPS, 2),
            "library_gemm_ms": round(t_gemm, 5),
            "library_gemm_tflops": round(flops / (t_gemm * 1e-3) / 1e12, 1),
            "library_gemm_plus_silu_mul_ms": round(t_unfused, 5)}


def wl_topk(args) -> dict:
    """Top-k logits selection at the end of a step: k=50 (the reference's
    default) over a 128256-entry vocabulary (the 32q/8kv hd128 family's), for
    a decode batch of 32 rows and a 256-row batch.  torch.topk on the same
    rows is timed beside it as a library reference point."""
    import torch

    from vllm_apple_amd import kernels

    dev = torch.device("cuda:0")
    V, k = 128256, 50
    rec = {"workload": "topk", "note": f"vocab {V}, k={k}, fp16 logits resident in HBM"}
    for T in (32, 256):
        g = torch.Generator(device=dev).manual_seed(T)
        logits = (torch.randn(T, V, generator=g, device=dev) * 4).half()
        idx = torch.empty((T, k), dtype=torch.int32, device=dev)
        vals = torch.empty((T, k), dtype=torch.float16, device=dev)
        rows = [logits.clone() for _ in range(_copies(logits.numel() * 2))]
        t = _timed_rot([lambda lg=lg_: kernels.topk_logits(lg, k, indices=idx, values=vals)
                        for lg_ in rows], args.steps, args.warmup)
        del rows
        t_torch = _timed(lambda: torch.topk(logits, k, dim=1), args.steps, args.warmup)
        by = T * V * 2 + T * k * 6
        rec[f"T{T}"] = {"ms": round(t, 5), "bytes": by,
                        "gb_s": round(by / (t * 1e-3) / 1e9, 1),
                        "pct_hbm_peak": round(100 * by / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                        "torch_topk_ms": round(t_torch, 5)}
    return rec


def wl_c3_launches(args) -> dict:
    """Counter driver: `--steps` eager launches of the C3 prefill alone (no
    graph, no other kernels), for rocprofv3 --pmc passes over exactly the
    prefill dispatches."""
    import torch

    from vllm_apple_amd import kernels, workloads

    b = workloads.c3_prefill(device=torch.device("cuda:0"))
    out = torch.empty_like(b.query)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        kernels.paged_prefill(b.query, b.k_cache, b.v_cache, b.block_table, b.token_to_seq,
                              b.positions, scale=b.scale, output=out)
    torch.cuda.synchronize()
    return {"workload": "C3-launches", "launches": args.steps,
            "note": "eager C3 prefill launches for counter collection"}


WORKLOADS = {"C1": wl_c1, "C2u": wl_c2u, "C3": wl_c3, "C4": wl_c4, "C5": wl_c5,
             "C5mlp": wl_c5mlp, "C2bf16": wl_c2bf16, "topk": wl_topk,
             "C3-launches": wl_c3_launches}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is described, not built)"}))
        return 2
    global _CPU_ENV
    if not args.no_cpu_baseline and not args.copy_bytes:
        _CPU_ENV = cpu_env()
    import torch

    if args.copy_bytes:
        print(json.dumps(copy_calibration(args.copy_bytes, args.steps, args.warmup)))
        return 0

    from vllm_apple_amd import _lib, kernels, workloads

    _lib.load()
    if args.workload != "headline":
        names = (["C1", "C2u", "C3", "C4", "C5", "C5mlp", "C2bf16", "topk"] if args.workload == "all"
                 else [args.workload])
        for name in names:
            print(json.dumps(WORKLOADS[name](args)), flush=True)
        return 0
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b = workloads.c2_decode(device=dev, fixed_len=args.ctx, batch=args.batch)
    out = torch.empty_like(b.query)
    max_len = b.max_seq_len

    def step():
        kernels.paged_decode(b.query, b.k_cache, b.v_cache, b.block_table, b.seq_lens,
                             scale=b.scale, max_seq_len=max_len, output=out,
                             new_keys=b.new_k, new_values=b.new_v,
                             partition_size=args.partition)

    stream = torch.cuda.current_stream()
    # Spread of single launches (events around each launch; informational, not
    # part of the timed region).  It runs before the warm-up: from an idle GPU
    # this kernel needs about 150 launches to reach its steady speed (launches
    # 5-50 run 2-3 % slower than from 150 on), so with a short warm-up the
    # timed region would otherwise measure the clocks settling.
    n_iso = 50
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n_iso)]
    for e0, e1 in ev:
        e0.record(stream)
        step()
        e1.record(stream)
    torch.cuda.synchronize()
    kern_ms = sorted(e0.elapsed_time(e1) for e0, e1 in ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: K steps, synchronize on both sides (one rank: no barrier).
    # HIP events on the launch stream bracket the region; at this shape a step
    # is one launch of the decode kernel (one partition per sequence, no merge
    # launch), so the region's event time / K is that kernel's average launch
    # duration, gaps between launches included.
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_start.record(stream)
    for _ in range(args.steps):
        step()
    e_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_avg_ms = e_start.elapsed_time(e_end) / args.steps
    ms_per_step = wall * 1e3 / args.steps

    alg_bytes = b.decode_algorithmic_bytes()
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = alg_bytes / (kern_avg_ms * 1e-3) / 1e9
    traffic = traffic_from_profile()
    ws_bytes, part = kernels.decode_workspace_size(kernels.make_params(
        key_cache=b.k_cache, value_cache=b.v_cache, layout="kernel",
        num_query_heads=b.num_q_heads, scale=b.scale, num_seqs=b.num_seqs,
        max_seq_len=max_len, max_blocks_per_seq=b.block_table.shape[1],
        partition_size=args.partition))
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic N(0,1) q/k/v and cache, seeded (workloads.c2_decode seed 1002)",
        "config": {
            "workload": "C2-headline: Mistral-Small-22B-shaped fused KV write + paged decode, "
                        "all ctx=8192",
            "batch": args.batch, "ctx": args.ctx, "num_q_heads": b.num_q_heads,
            "num_kv_heads": b.num_kv_heads, "head_dim": b.head_size, "block_size": 16,
            "pool_blocks": int(b.k_cache.shape[0]), "split_k_partition": part,
            "algorithmic_bytes_per_step": alg_bytes,
            "launches_per_step": 1 if ws_bytes == 0 else 2,
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(args.batch / (ms_per_step * 1e-3), 1),
        "kernel_ms": {"avg_in_timed_region": round(kern_avg_ms, 5),
                      "single_launch_min": round(kern_ms[0], 5),
                      "single_launch_p50": round(kern_ms[len(kern_ms) // 2], 5),
                      "single_launch_p90": round(kern_ms[int(len(kern_ms) * 0.9)], 5)},
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_kernel<128>",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "device": torch.cuda.get_device_name(0),
    }
    # A measured streaming bandwidth beside the 8 TB/s peak: a plain device
    # copy (torch's copy_) moving the step's algorithmic bytes, half read and
    # half written, timed after the record's own region.  The decode's stream
    # is almost all reads, which HBM serves faster than a read/write mix.
    res["streaming_copy"] = _vs_copy(kern_avg_ms, alg_bytes, args.steps, args.warmup)
    # The measured ceiling of the decode's own stream: the same K and V rows
    # read through the same block tables by a kernel that does nothing else
    # with them (vaa_kv_stream_read), timed like the record's region.
    rs = _read_stream(b, args, 0)
    rs["decode_vs_read_stream"] = round(achieved / rs["gb_s"], 4)
    res["read_stream"] = rs
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_decode_step(b, args.cpu_seconds)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
