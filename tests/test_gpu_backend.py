"""The drop-in surfaces on the GPU: HipAttentionImpl.forward (vLLM mode) and the
engine ops (PagedAttentionOp, KVWriteOp, EngineRMSNorm, EngineRoPE,
EngineElementwiseOps) against the oracle."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close, host, assert_close_bf16

import oracle.attention as oat
import oracle.kv as okv
import oracle.layer_ops as olo

pytestmark = pytest.mark.gpu


def _mixed_batch(H=32, KV=8, D=128, bs=16, dec_lens=(37, 300, 1, 2049), pre=((500, 64), (90, 90)),
                 seed=0, dtype=torch.float16):
    """vLLM-mode batch: decodes first, then prefill chunks (total len, chunk len)."""
    g = torch.Generator().manual_seed(seed)
    lens = list(dec_lens) + [p[0] for p in pre]
    qlens = [1] * len(dec_lens) + [p[1] for p in pre]
    nblk = [(L + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 8
    kv_cache = torch.randn(2, nb, bs, KV, D, generator=g).to(dtype)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    maxb = max(nblk)
    bt = torch.full((len(lens), maxb), -1, dtype=torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    T = int(qsl[-1])
    tok, pos = okv.token_index(qsl, np.array(lens, np.int32), T)
    slots = okv.slot_mapping(bt.numpy(), bs, tok, pos)
    qkv = torch.randn(T, (H + 2 * KV) * D, generator=g).to(dtype)
    return dict(kv_cache=kv_cache, bt=bt, lens=torch.tensor(lens, dtype=torch.int32),
                qsl=torch.from_numpy(qsl), slots=torch.from_numpy(slots), qkv=qkv, tok=tok,
                pos=pos, num_decode=len(dec_lens), T=T, H=H, KV=KV, D=D)


def _metadata(b, dev):
    from vllm_apple_amd.backend import HipAttentionMetadata

    return HipAttentionMetadata(
        num_actual_tokens=b["T"], max_query_len=int((b["qsl"][1:] - b["qsl"][:-1]).max()),
        query_start_loc=b["qsl"].to(dev), max_seq_len=int(b["lens"].max()),
        seq_lens=b["lens"].to(dev), block_table=b["bt"].to(dev),
        slot_mapping=b["slots"].to(dev), num_decode_tokens=b["num_decode"])


def _oracle(b, scale):
    """KV write through slot_mapping, then decode rows + prefill rows (vLLM layout)."""
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    qkv = b["qkv"].to(torch.float16).numpy()
    q = qkv[:, :H * D].reshape(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].reshape(T, KV, D)
    v = qkv[:, (H + KV) * D:].reshape(T, KV, D)
    kc = b["kv_cache"][0].to(torch.float16).numpy().copy()
    vc = b["kv_cache"][1].to(torch.float16).numpy().copy()
    okv.kv_write_slots(kc, vc, k, v, b["slots"].numpy(), "vllm")
    nd = b["num_decode"]
    out = np.zeros((T, H, D))
    out[:nd] = oat.decode(q[:nd], kc, vc, b["bt"].numpy()[:nd], b["lens"].numpy()[:nd], scale,
                          "vllm")
    pre, w = oat.prefill(q, kc, vc, b["bt"].numpy(), b["tok"], b["pos"], scale, "vllm",
                         rows=np.arange(nd, T))
    out[nd:] = pre[nd:]
    return out, kc, vc


def test_forward_mixed_batch_vllm_cache(gpu):
    from vllm_apple_amd.backend import HipAttentionImpl

    b = _mixed_batch(seed=1)
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    kv_cache = b["kv_cache"].to(dev)
    out = torch.full((T, H, D), 9.0, dtype=torch.float16, device=dev)
    res = impl.forward(None, q, k, v, kv_cache, _metadata(b, dev), output=out)
    torch.cuda.synchronize()
    assert res is out
    ref, kc, vc = _oracle(b, scale)
    assert np.array_equal(host(kv_cache[0]).view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(host(kv_cache[1]).view(np.uint16), vc.view(np.uint16))
    assert_close(host(out), ref, what="forward mixed")


@pytest.mark.parametrize("bs", [8, 12, 32])
def test_forward_mixed_batch_block_sizes(gpu, bs):
    """forward on a vLLM cache whose block size is not 16 (the platform
    selects this backend for any block size, as the reference's does): KV
    write bit-exact, decode and prefill rows against the oracle."""
    from vllm_apple_amd.backend import HipAttentionImpl

    b = _mixed_batch(bs=bs, seed=11 + bs)
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    kv_cache = b["kv_cache"].to(dev)
    out = torch.zeros((T, H, D), dtype=torch.float16, device=dev)
    impl.forward(None, q, k, v, kv_cache, _metadata(b, dev), output=out)
    torch.cuda.synchronize()
    ref, kc, vc = _oracle(b, scale)
    assert np.array_equal(host(kv_cache[0]).view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(host(kv_cache[1]).view(np.uint16), vc.view(np.uint16))
    assert_close(host(out), ref, what=f"forward bs={bs}")


@pytest.mark.parametrize("H,KV", [(48, 1), (40, 2)])
def test_forward_mixed_batch_wide_groups(gpu, H, KV):
    """A layer whose GQA group has more than 16 query heads (MQA with 48
    heads) is accepted and runs on the HIP kernels: KV write bit-exact,
    decode and prefill rows against the oracle."""
    from vllm_apple_amd.backend import HipAttentionImpl

    b = _mixed_batch(H=H, KV=KV, seed=5, dec_lens=(37, 300, 1, 2049, 5000), pre=((500, 64),))
    D, T = b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    kv_cache = b["kv_cache"].to(dev)
    out = torch.zeros((T, H, D), dtype=torch.float16, device=dev)
    impl.forward(None, q, k, v, kv_cache, _metadata(b, dev), output=out)
    torch.cuda.synchronize()
    ref, kc, vc = _oracle(b, scale)
    assert np.array_equal(host(kv_cache[0]).view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(host(kv_cache[1]).view(np.uint16), vc.view(np.uint16))
    assert_close(host(out), ref, what=f"forward wide group H={H} KV={KV}")


def test_forward_bf16_native_cache(gpu):
    """bf16 model: the bf16 vLLM kv_cache is written in place (bit-exact 16-bit
    copies) and attention runs in bf16, with no fp16 copy of the cache and no
    conversions (the reference converts to fp16, metal_attn.py:609-620)."""
    from vllm_apple_amd.backend import HipAttentionImpl

    b = _mixed_batch(seed=2, dtype=torch.bfloat16, dec_lens=(40, 7, 1000), pre=((64, 20),))
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    kv_cache = b["kv_cache"].to(dev)
    out = torch.zeros((T, H, D), dtype=torch.bfloat16, device=dev)
    impl.forward(None, q, k, v, kv_cache, _metadata(b, dev), output=out)
    torch.cuda.synchronize()
    assert impl._shadow is None, "no fp16 copy of a bf16 cache"
    # Oracle: the KV write on the bf16 bit patterns, attention on their values.
    bits = lambda t: t.cpu().view(torch.float16).numpy()  # noqa: E731
    qkv_b = bits(b["qkv"])
    kc, vc = bits(b["kv_cache"][0]).copy(), bits(b["kv_cache"][1]).copy()
    okv.kv_write_slots(kc, vc, qkv_b[:, H * D:(H + KV) * D].reshape(T, KV, D),
                       qkv_b[:, (H + KV) * D:].reshape(T, KV, D), b["slots"].numpy(), "vllm")
    assert np.array_equal(bits(kv_cache[0]).view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(bits(kv_cache[1]).view(np.uint16), vc.view(np.uint16))
    val = lambda a: torch.from_numpy(a.copy()).view(torch.bfloat16).float().numpy()  # noqa: E731
    qv = b["qkv"].float().numpy()[:, :H * D].reshape(T, H, D)
    kcv, vcv = val(kc), val(vc)
    nd = b["num_decode"]
    ref = np.zeros((T, H, D))
    ref[:nd] = oat.decode(qv[:nd], kcv, vcv, b["bt"].numpy()[:nd], b["lens"].numpy()[:nd],
                          scale, "vllm")
    pre, _ = oat.prefill(qv, kcv, vcv, b["bt"].numpy(), b["tok"], b["pos"], scale, "vllm",
                         rows=np.arange(nd, T))
    ref[nd:] = pre[nd:]
    assert out.dtype == torch.bfloat16
    # The north-star bound plus the bf16 output rounding.
    assert_close_bf16(out.float().cpu().numpy(), ref, what="bf16 forward")


def test_forward_bf16_activations_fp16_cache(gpu):
    """bf16 activations over an fp16 cache: converted to the cache's type and
    the output converted back, as the reference does for its fp16 kernels."""
    from vllm_apple_amd.backend import HipAttentionImpl

    b = _mixed_batch(seed=6, dtype=torch.float16, dec_lens=(40, 7), pre=((64, 20),))
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv16 = b["qkv"].to(dev)
    qkv = qkv16.to(torch.bfloat16)
    b["qkv"] = qkv.to(torch.float16).cpu()   # the oracle sees the bf16-rounded inputs
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    kv_cache = b["kv_cache"].to(dev)
    out = torch.zeros((T, H, D), dtype=torch.bfloat16, device=dev)
    impl.forward(None, q, k, v, kv_cache, _metadata(b, dev), output=out)
    torch.cuda.synchronize()
    ref, kc, vc = _oracle(b, scale)
    assert np.array_equal(host(kv_cache[0]).view(np.uint16), kc.view(np.uint16))
    assert out.dtype == torch.bfloat16
    # bf16 output rounding (8-bit mantissa) on top of the fp16 path.
    assert_close(host(out.float()), ref, atol=2e-3, rtol=1e-2 + 2 ** -8, what="bf16 over fp16")


@pytest.mark.parametrize("causal", [False, True])
def test_forward_encoder_only(gpu, causal):
    """Encoder attention inside each sequence (base_attn.py:223-306): two calls
    in a row, the second with more tokens (the staging cache grows) and an
    empty sequence in the middle; every row against torch SDPA in fp32."""
    from vllm_apple_amd.backend import AttentionType, HipAttentionImpl, HipAttentionMetadata

    H, KV, D = 8, 2, 64
    impl = HipAttentionImpl(H, D, 0.125, KV, None, None, "auto",
                            attn_type=AttentionType.ENCODER_ONLY)
    dev = torch.device("cuda")
    for seed, lens in ((3, [5, 40, 17]), (4, [70, 0, 33, 129, 1])):
        print(f"[case] encoder causal={causal} lens={lens}", flush=True)
        g = torch.Generator().manual_seed(seed)
        T = sum(lens)
        q = torch.randn(T, H, D, generator=g).half()
        k = torch.randn(T, KV, D, generator=g).half()
        v = torch.randn(T, KV, D, generator=g).half()
        qsl = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
        md = HipAttentionMetadata(T, max(lens), qsl.to(dev), max(lens),
                                  torch.tensor(lens).to(dev), None, None)
        out = torch.zeros(T, H, D, dtype=torch.float16, device=dev)
        if causal:  # the staging path's causal form (forward passes is_causal=False,
            # as metal_attn.py:639-647 does)
            impl._attention_no_cache(q.to(dev), k.to(dev), v.to(dev), out, md, causal=True)
        else:
            impl.forward(None, q.to(dev), k.to(dev), v.to(dev), None, md, output=out)
        torch.cuda.synchronize()
        ref = torch.zeros(T, H, D)
        for s_ in range(len(lens)):
            a, e = int(qsl[s_]), int(qsl[s_ + 1])
            if e == a:
                continue
            qt = q[a:e].float().transpose(0, 1)
            kt = k[a:e].float().transpose(0, 1).repeat_interleave(4, 0)
            vt = v[a:e].float().transpose(0, 1).repeat_interleave(4, 0)
            ref[a:e] = F.scaled_dot_product_attention(qt, kt, vt, scale=0.125,
                                                      is_causal=causal).transpose(0, 1)
        assert_close(host(out), ref.numpy(), what=f"encoder-only causal={causal}")


def test_engine_ops_planar_qkv_decode_step(gpu):
    """Engine mode (runner.py:829-1176 order): RMSNorm -> (QKV given) -> RoPE on
    views of the planar [Q_all][K_all][V_all] buffer -> fused decode."""
    from vllm_apple_amd.engine import (EngineRMSNorm, EngineRoPE, EngineStepContext,
                                       PagedAttentionOp)

    H, KV, D, bs, S = 32, 8, 128, 16, 6
    g = torch.Generator().manual_seed(4)
    lens = [33, 1000, 16, 4097, 1, 250]
    nblk = [(L + bs - 1) // bs for L in lens]
    nb = sum(nblk) + 4
    kc = torch.randn(nb, KV, bs, D, generator=g).half()
    vc = torch.randn(nb, KV, bs, D, generator=g).half()
    maxb = 300
    bt = torch.full((S, maxb), -1, dtype=torch.int32)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off:off + n]
        off += n
    qkv = torch.randn(S * (H + 2 * KV) * D, generator=g).half()  # planar
    positions = torch.tensor([L - 1 for L in lens], dtype=torch.int32)
    dev = torch.device("cuda")
    qkv_d, kc_d, vc_d = qkv.to(dev), kc.to(dev), vc.to(dev)
    out_d = torch.zeros(S * H * D, dtype=torch.float16, device=dev)
    q_off, k_off, v_off = 0, S * H * D * 2, S * (H + KV) * D * 2
    rope = EngineRoPE(None, D, H, KV, max_position=8192, base=1e6)
    attn = PagedAttentionOp(None, KV, H, D, bs)
    with EngineStepContext() as ctx:
        rope.encode(ctx, (qkv_d, q_off), (qkv_d, k_off), positions.to(dev), S,
                    max_position_in_batch=int(positions.max()))
        attn.encode_decode_fused(ctx, qkv_d, qkv_d, qkv_d, kc_d, vc_d, bt.to(dev),
                                 torch.tensor(lens, dtype=torch.int32).to(dev), out_d, S,
                                 max(lens), maxb, query_offset=q_off, new_keys_offset=k_off,
                                 new_values_offset=v_off)
        ctx.end_encoding()
        ctx.wait_until_completed()
    # Oracle: rope (fp64 from the fp32 table), round to fp16 like the kernel's
    # in-place store, write K/V at seq_len-1, attend.
    cos, sin = olo.cos_sin(D, 8192, 1e6)
    qn = qkv[:S * H * D].view(S, H, D).numpy()
    kn = qkv[S * H * D:S * (H + KV) * D].view(S, KV, D).numpy()
    vn = qkv[S * (H + KV) * D:].view(S, KV, D).numpy()
    qr = olo.rope_neox(qn, positions.numpy(), cos, sin).astype(np.float16)
    kr = olo.rope_neox(kn, positions.numpy(), cos, sin).astype(np.float16)
    got_q = host(qkv_d[:S * H * D]).reshape(S, H, D)
    assert_close(got_q, qr.astype(np.float64), what="rope q (planar view)")
    kcr, vcr = kc.numpy().copy(), vc.numpy().copy()
    okv.kv_write_decode(kcr, vcr, host(qkv_d[q_off // 2 + S * H * D:]).reshape(-1)[:S * KV * D]
                        .reshape(S, KV, D), vn, bt.numpy(), np.array(lens, np.int32))
    ref = oat.decode(got_q, kcr, vcr, bt.numpy(), np.array(lens, np.int32), 1 / math.sqrt(D))
    assert_close(host(out_d).reshape(S, H, D), ref, what="engine fused decode")
    assert np.array_equal(host(kc_d).view(np.uint16), kcr.view(np.uint16))
    assert_close(host(qkv_d[S * H * D:S * (H + KV) * D]).reshape(S, KV, D),
                 kr.astype(np.float64), what="rope k (planar view)")


def test_engine_prefill_flow_and_layer_ops(gpu):
    """KVWriteOp.encode_prefill -> PagedAttentionOp.encode_prefill, then
    EngineRMSNorm (with residual) and encode_silu_mul."""
    from vllm_apple_amd.engine import (EngineElementwiseOps, EngineRMSNorm, KVWriteOp,
                                       PagedAttentionOp)

    H, KV, D, bs = 16, 4, 64, 16
    g = torch.Generator().manual_seed(5)
    ctx_lens, new = [100, 40], [30, 40]
    nblk = [(L + bs - 1) // bs for L in ctx_lens]
    nb = sum(nblk) + 2
    kc = torch.randn(nb, KV, bs, D, generator=g).half()
    vc = torch.randn(nb, KV, bs, D, generator=g).half()
    bt = torch.full((2, max(nblk)), -1, dtype=torch.int32)
    bt[0, :nblk[0]] = torch.arange(nblk[0], dtype=torch.int32)
    bt[1, :nblk[1]] = torch.arange(nblk[0], nblk[0] + nblk[1], dtype=torch.int32)
    qsl = np.array([0, 30, 70], np.int32)
    tok, pos = okv.token_index(qsl, np.array(ctx_lens, np.int32), 70)
    slots = okv.slot_mapping(bt.numpy(), bs, tok, pos)
    q = torch.randn(70, H, D, generator=g).half()
    nk = torch.randn(70, KV, D, generator=g).half()
    nv = torch.randn(70, KV, D, generator=g).half()
    dev = torch.device("cuda")
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    out = torch.zeros(70, H, D, dtype=torch.float16, device=dev)
    KVWriteOp(None, KV, D, bs).encode_prefill(None, nk.to(dev), nv.to(dev), kc_d, vc_d,
                                              torch.from_numpy(slots).to(torch.int32).to(dev), 70)
    PagedAttentionOp(None, KV, H, D, bs).encode_prefill(
        None, q.to(dev), kc_d, vc_d, bt.to(dev), torch.from_numpy(tok).to(dev),
        torch.from_numpy(pos).to(dev), out, 70, 2, 100, bt.shape[1])
    x = torch.randn(70, 512, generator=g).half()
    r = torch.randn(70, 512, generator=g).half()
    w = (torch.randn(512, generator=g) * 0.1 + 1).half()
    y = torch.empty(70, 512, dtype=torch.float16, device=dev)
    norm = EngineRMSNorm(None, 512, eps=1e-5, weight_buffer=w.to(dev))
    norm.encode(None, x.to(dev), y, 70, residual_buffer=r.to(dev))
    gate = torch.randn(70 * 256, generator=g).half()
    up = torch.randn(70 * 256, generator=g).half()
    act = torch.empty(70 * 256, dtype=torch.float16, device=dev)
    EngineElementwiseOps(None).encode_silu_mul(None, gate.to(dev), up.to(dev), act, 70 * 256)
    torch.cuda.synchronize()
    kr, vr = kc.numpy().copy(), vc.numpy().copy()
    okv.kv_write_slots(kr, vr, nk.numpy(), nv.numpy(), slots)
    assert np.array_equal(host(kc_d).view(np.uint16), kr.view(np.uint16))
    ref, _ = oat.prefill(q.numpy(), kr, vr, bt.numpy(), tok, pos, 1 / 8)
    assert_close(host(out), ref, what="engine prefill")
    assert_close(host(y), olo.rms_norm(x.numpy(), w.numpy(), 1e-5, r.numpy()), what="rmsnorm")
    assert_close(host(act), olo.silu_mul(gate.numpy(), up.numpy()), what="silu_mul")


def test_kv_cache_object_write_and_validate(gpu):
    from vllm_apple_amd.kv_cache import HipKVCache, KVCacheDescriptor

    c = HipKVCache(KVCacheDescriptor(16, 16, 4, 128, 2))
    key = np.full((4, 128), 1.5, np.float16)
    val = np.full((4, 128), 2.5, np.float16)
    c.write_kv(1, 3, 5, torch.from_numpy(key), torch.from_numpy(val))  # known answer
    torch.cuda.synchronize()
    k, v = c.get_buffers(1)
    assert torch.all(k[3, :, 5] == 1.5) and torch.all(v[3, :, 5] == 2.5)
    assert int(torch.count_nonzero(k)) == 4 * 128
    assert int(torch.count_nonzero(c.get_key_buffer(0))) == 0
    with pytest.raises(ValueError):
        c.write_kv(0, 0, 16, torch.from_numpy(key), torch.from_numpy(val))


def test_forward_mixed_overlap_matches_serial_and_graph_replays(gpu, monkeypatch):
    """A mixed step runs prefill (side stream) and decode (current stream)
    concurrently: bit-identical to running them in turn, and a HIP graph of
    the step replays to the eager result every time (with eager work and
    synchronizations between the replays)."""
    from vllm_apple_amd import backend as B
    from vllm_apple_amd.backend import HipAttentionImpl

    b = _mixed_batch(seed=9)
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    impl = HipAttentionImpl(H, D, 1 / math.sqrt(D), KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    md = _metadata(b, dev)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv(B.OVERLAP_ENV, mode)
        kv_cache = b["kv_cache"].to(dev)
        out = torch.zeros((T, H, D), dtype=torch.float16, device=dev)
        impl.forward(None, q, k, v, kv_cache, md, output=out)
        torch.cuda.synchronize()
        outs[mode] = (out.clone(), kv_cache.clone())
    assert torch.equal(outs["0"][0], outs["1"][0])
    assert torch.equal(outs["0"][1], outs["1"][1])
    # Graph capture of the overlapped step (the KV write is idempotent).
    monkeypatch.setenv(B.OVERLAP_ENV, "1")
    kv_cache = b["kv_cache"].to(dev)
    out = torch.zeros((T, H, D), dtype=torch.float16, device=dev)
    impl.forward(None, q, k, v, kv_cache, md, output=out)  # warm-up (workspaces)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        impl.forward(None, q, k, v, kv_cache, md, output=out)
    for r in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, outs["1"][0]), f"replay {r}"
        _ = (out.float() * 2).sum().item()  # eager work between replays


def test_forward_mixed_overlap_balanced_shared_split(gpu, monkeypatch):
    """A mixed step whose decodes take the balanced split (host lengths known,
    many ragged contexts): overlapped, decode runs the shared split beside the
    prefill; the result matches the oracle and the serial step within the
    attention tolerance (the two splits sum partials in a different order)."""
    from vllm_apple_amd import backend as B
    from vllm_apple_amd.backend import HipAttentionImpl

    g = torch.Generator().manual_seed(12)
    dec = torch.randint(300, 6000, (40,), generator=g).tolist()
    b = _mixed_batch(seed=12, dec_lens=tuple(dec), pre=((2000, 128), (700, 96)))
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    from vllm_apple_amd import kernels

    assert kernels.choose_partition_size(dec, KV, kernels.device_cus(dev)) == \
        kernels.PARTITION_BALANCED
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv(B.OVERLAP_ENV, mode)
        md = _metadata(b, dev)
        md._seq_lens_cpu = b["lens"].tolist()
        kv_cache = b["kv_cache"].to(dev)
        out = torch.zeros((T, H, D), dtype=torch.float16, device=dev)
        impl.forward(None, q, k, v, kv_cache, md, output=out)
        torch.cuda.synchronize()
        outs[mode] = host(out)
    ref, _, _ = _oracle(b, scale)
    assert_close(outs["1"], ref, what="overlapped mixed step (shared split)")
    assert_close(outs["0"], ref, what="serial mixed step")
    assert np.array_equal(outs["0"][len(dec):], outs["1"][len(dec):]), "prefill rows"


@pytest.mark.parametrize("dec_lens", [(), (37, 300)])
def test_forward_prefill_split_with_host_lengths(gpu, monkeypatch, dec_lens):
    """With the host lengths in the metadata, a prefill-only batch with one
    long context next to short ones runs the split-K prefill (the chooser's
    split); beside decodes (run concurrently) the prefill stays unsplit.
    Every row matches the oracle either way."""
    from vllm_apple_amd import kernels
    from vllm_apple_amd.backend import HipAttentionImpl

    print(f"[case] backend prefill split, decodes {dec_lens}", flush=True)
    b = _mixed_batch(seed=7, dec_lens=dec_lens, pre=((12000, 256), (300, 256), (700, 256)))
    H, KV, D, T = b["H"], b["KV"], b["D"], b["T"]
    scale = 1 / math.sqrt(D)
    impl = HipAttentionImpl(H, D, scale, KV, None, None, "auto")
    dev = torch.device("cuda")
    qkv = b["qkv"].to(dev)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
    v = qkv[:, (H + KV) * D:].view(T, KV, D)
    kv_cache = b["kv_cache"].to(dev)
    md = _metadata(b, dev)
    md._seq_lens_cpu = b["lens"].tolist()
    md._query_start_loc_cpu = b["qsl"].tolist()
    seen = []
    real = kernels.paged_prefill

    def spy(*args, **kw):
        seen.append(kw.get("split_keys", 0))
        return real(*args, **kw)

    monkeypatch.setattr(kernels, "paged_prefill", spy)
    out = torch.zeros((T, H, D), dtype=torch.float16, device=dev)
    impl.forward(None, q, k, v, kv_cache, md, output=out)
    torch.cuda.synchronize()
    assert seen and (seen[0] > 0) == (len(dec_lens) == 0)
    ref, kc, vc = _oracle(b, scale)
    assert_close(host(out), ref, what="forward with split prefill")
