"""EngineMLP host logic (no GPU): the supported form and the reference's
errors for missing weights (mlp.py:170-200)."""
import pytest

from vllm_apple_amd.engine import EngineMLP


def test_engine_mlp_supported_forms():
    with pytest.raises(NotImplementedError):
        EngineMLP(None, 256, 512, gated=False)
    with pytest.raises(NotImplementedError):
        EngineMLP(None, 256, 512, activation="gelu")
    with pytest.raises(NotImplementedError):
        EngineMLP(None, 256, 512, bias=True)
    m = EngineMLP(None, 256, 512)
    with pytest.raises(NotImplementedError):
        m.set_weights(gate_up_proj=object(), down_proj=object(), gate_bias=object())
    assert m.get_params_dict() == {"hidden_size": 256, "intermediate_size": 512, "gated": True,
                                   "activation": "silu", "bias": False}
    assert m.get_output_size(3) == 3 * 256 * 2
    assert m.get_intermediate_size(3) == 3 * 512 * 2
    # Up to 1024 tokens the fused kernel; above, the library GEMM + silu_mul.
    assert EngineMLP.FUSED_MAX_TOKENS == 1024 and m.fused_max_tokens == 1024


def test_engine_mlp_missing_weights():
    m = EngineMLP(None, 256, 512)
    with pytest.raises(RuntimeError, match="Down projection"):
        m.encode(None, None, None, 1)
    m.set_weights(down_proj=object())
    with pytest.raises(RuntimeError, match="Gate and up"):
        m.encode(None, None, None, 1)
