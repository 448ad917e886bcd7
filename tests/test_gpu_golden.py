"""The HIP library against the committed golden fixtures (tests/golden/*.npz)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_close, host

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_golden_kv_write(gpu):
    from vllm_apple_amd import kernels

    g = load("kv_write")
    kc, vc = dev(g["kc"]), dev(g["vc"])
    kernels.kv_write_slots(dev(g["key"]), dev(g["value"]), kc, vc, dev(g["slots"]))
    torch.cuda.synchronize()
    assert np.array_equal(host(kc).view(np.uint16), g["kc_slots"].view(np.uint16))
    assert np.array_equal(host(vc).view(np.uint16), g["vc_slots"].view(np.uint16))
    kc, vc = dev(g["kc"]), dev(g["vc"])
    kernels.kv_write_decode(dev(g["new_k"]), dev(g["new_v"]), kc, vc, dev(g["block_table"]),
                            dev(g["seq_lens"]))
    torch.cuda.synchronize()
    assert np.array_equal(host(kc).view(np.uint16), g["kc_decode"].view(np.uint16))
    assert np.array_equal(host(vc).view(np.uint16), g["vc_decode"].view(np.uint16))


def test_golden_decode(gpu):
    from vllm_apple_amd import kernels

    d = load("decode")
    out = kernels.paged_decode(dev(d["query"]), dev(d["kc"]), dev(d["vc"]), dev(d["block_table"]),
                               dev(d["seq_lens"]), scale=float(d["scale"]),
                               max_seq_len=int(d["seq_lens"].max()))
    torch.cuda.synchronize()
    assert_close(host(out), d["out"], what="golden decode")


def test_golden_prefill(gpu):
    from vllm_apple_amd import kernels

    p = load("prefill")
    out = kernels.paged_prefill(dev(p["query"]), dev(p["kc"]), dev(p["vc"]), dev(p["block_table"]),
                                dev(p["token_to_seq"]), dev(p["positions"]),
                                scale=float(p["scale"]))
    torch.cuda.synchronize()
    assert_close(host(out), p["out"], what="golden prefill")


def test_golden_layer_ops(gpu):
    from vllm_apple_amd import kernels

    g = load("layer_ops")
    eps = float(g["rms_eps"])
    out = kernels.rms_norm(dev(g["rms_x"]), dev(g["rms_w"]), eps)
    out_r = kernels.rms_norm(dev(g["rms_x"]), dev(g["rms_w"]), eps, residual=dev(g["rms_res"]))
    cos, sin = kernels.rope_cos_sin_cache(64, int(g["rope_max_pos"]), float(g["rope_base"]))
    q, k = dev(g["rope_q"]), dev(g["rope_k"])
    kernels.rope_neox_(q, k, cos, sin, dev(g["rope_pos"]))
    s = kernels.silu_mul(dev(g["silu_g"]), dev(g["silu_u"]))
    torch.cuda.synchronize()
    assert_close(host(out), g["rms_out"], what="golden rmsnorm")
    assert_close(host(out_r), g["rms_out_res"], what="golden rmsnorm+residual")
    assert_close(host(q), g["rope_q_out"], what="golden rope q")
    assert_close(host(k), g["rope_k_out"], what="golden rope k")
    assert_close(host(s), g["silu_out"], what="golden silu_mul")


def test_golden_indexing(gpu):
    from vllm_apple_amd import kernels

    g = load("indexing")
    tok, pos = kernels.build_token_index(dev(g["qsl"]), dev(g["seq_lens"]), 12)
    slots = kernels.build_slot_mapping(dev(g["block_table"]), 16, tok, pos)
    torch.cuda.synchronize()
    assert host(tok).tolist() == g["token_to_seq"].tolist()
    assert host(pos).tolist() == g["positions"].tolist()
    assert host(slots).tolist() == g["slots"].tolist()
