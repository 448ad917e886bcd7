"""The committed golden fixtures (tests/golden/*.npz) on the CPU.

The oracle must still reproduce every fixture, and the index fixtures are also
checked against values worked out by hand from the reference's rules
(apple_model_runner.py:1188-1249, runner.py:526-546).
"""
from pathlib import Path

import numpy as np
import pytest

import oracle.attention as oat
import oracle.kv as okv
import oracle.layer_ops as olo

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


def test_kv_write_fixture():
    g = load("kv_write")
    ko, vo = g["kc"].copy(), g["vc"].copy()
    okv.kv_write_slots(ko, vo, g["key"], g["value"], g["slots"])
    assert np.array_equal(ko.view(np.uint16), g["kc_slots"].view(np.uint16))
    assert np.array_equal(vo.view(np.uint16), g["vc_slots"].view(np.uint16))
    kd, vd = g["kc"].copy(), g["vc"].copy()
    okv.kv_write_decode(kd, vd, g["new_k"], g["new_v"], g["block_table"], g["seq_lens"])
    assert np.array_equal(kd.view(np.uint16), g["kc_decode"].view(np.uint16))
    # hand check: sequence 0 (seq_len 17) writes position 16 = block bt[0,1], offset 0
    b = g["block_table"][0, 1]
    assert np.array_equal(g["kc_decode"][b, :, 0], g["new_k"][0])
    # padding slots (-1) leave every other slot untouched
    changed = np.any(g["kc_slots"] != g["kc"], axis=(1, 3))
    assert changed.sum() <= 8 * 2


def test_decode_and_prefill_fixtures():
    d = load("decode")
    out = oat.decode(d["query"], d["kc"], d["vc"], d["block_table"], d["seq_lens"],
                     float(d["scale"]))
    np.testing.assert_allclose(out, d["out"], rtol=1e-6, atol=1e-7)
    # seq_len 1: every head of a kv group returns that token's V exactly
    v0 = d["vc"][d["block_table"][0, 0], :, 0]
    np.testing.assert_allclose(d["out"][0], np.repeat(v0, 7, axis=0).astype(np.float32))
    p = load("prefill")
    out, w = oat.prefill(p["query"], p["kc"], p["vc"], p["block_table"], p["token_to_seq"],
                         p["positions"], float(p["scale"]))
    assert w.all()
    np.testing.assert_allclose(out, p["out"], rtol=1e-6, atol=1e-7)


def test_layer_op_fixtures():
    g = load("layer_ops")
    eps = float(g["rms_eps"])
    np.testing.assert_allclose(olo.rms_norm(g["rms_x"], g["rms_w"], eps), g["rms_out"], rtol=1e-6)
    np.testing.assert_allclose(olo.rms_norm(g["rms_x"], g["rms_w"], eps, g["rms_res"]),
                               g["rms_out_res"], rtol=1e-6, atol=1e-6)
    cos, sin = olo.cos_sin(64, int(g["rope_max_pos"]), float(g["rope_base"]))
    np.testing.assert_allclose(olo.rope_neox(g["rope_q"], g["rope_pos"], cos, sin),
                               g["rope_q_out"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(olo.rope_neox(g["rope_k"], g["rope_pos"], cos, sin),
                               g["rope_k_out"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(olo.silu_mul(g["silu_g"], g["silu_u"]), g["silu_out"],
                               rtol=1e-6, atol=1e-7)


def test_index_fixture_by_hand():
    g = load("indexing")
    # qsl [0,1,2,10,12], seq_lens [5,900,8,2]: the last (q1-q0) positions of each sequence
    assert g["token_to_seq"].tolist() == [0, 1, 2, 2, 2, 2, 2, 2, 2, 2, 3, 3]
    assert g["positions"].tolist() == [4, 899, 0, 1, 2, 3, 4, 5, 6, 7, 0, 1]
    # slot = bt[s, pos // 16] * 16 + pos % 16; seq 1 at position 899 needs block 56,
    # which is -1 in the table -> fallback slot = pos (apple_model_runner.py:1220-1221)
    assert g["slots"].tolist() == [52, 899, 112, 113, 114, 115, 116, 117, 118, 119, 144, 145]
    tok, pos = okv.token_index(g["qsl"], g["seq_lens"], 12)
    assert np.array_equal(tok, g["token_to_seq"]) and np.array_equal(pos, g["positions"])
    assert np.array_equal(okv.slot_mapping(g["block_table"], 16, tok, pos), g["slots"])


@pytest.mark.parametrize("name", ["kv_write", "decode", "prefill", "layer_ops", "indexing"])
def test_fixtures_are_small(name):
    assert (GOLDEN / f"{name}.npz").stat().st_size < 256 * 1024
