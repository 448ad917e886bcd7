"""Backend selection rule (vllm_apple_amd.platform, mirror of platform.py:100-168)."""
import pytest
import torch

from vllm_apple_amd import platform as P


def sel(**kw):
    args = dict(head_size=128, dtype=torch.float16, kv_cache_dtype="auto", block_size=16,
                use_mla=False, has_sink=False, use_sparse=False)
    args.update(kw)
    return P.select_attn_backend(**args)


def test_supported_layers_get_the_hip_backend(monkeypatch):
    monkeypatch.delenv(P.ATTENTION_ENV, raising=False)
    for hs in (32, 64, 96, 128):
        for dt in (torch.float16, torch.bfloat16):
            for bs in (8, 12, 16, 32, 128):
                assert sel(head_size=hs, dtype=dt, block_size=bs) == P.BACKEND_CLS
    assert sel(kv_cache_dtype=None) == P.BACKEND_CLS
    assert P.HipAttentionPlatformMixin.get_attn_backend_cls(
        None, 64, torch.bfloat16, "auto", 16, False, False, False) == P.BACKEND_CLS


def test_unsupported_layers_fall_back(monkeypatch):
    monkeypatch.delenv(P.ATTENTION_ENV, raising=False)
    monkeypatch.delenv(P.FALLBACK_ENV, raising=False)
    for kw in (dict(head_size=256), dict(head_size=80), dict(dtype=torch.float32),
               dict(kv_cache_dtype="fp8_e4m3"), dict(has_sink=True)):
        assert sel(**kw) == P.DEFAULT_FALLBACK, kw
    monkeypatch.setenv(P.FALLBACK_ENV, "my.backend.Cls")
    assert sel(head_size=256) == "my.backend.Cls"
    monkeypatch.setenv(P.ATTENTION_ENV, "0")
    assert sel() == "my.backend.Cls"


def test_mla_and_sparse_raise():
    with pytest.raises(NotImplementedError):
        sel(use_mla=True)
    with pytest.raises(NotImplementedError):
        sel(use_sparse=True)


def test_register_without_vllm_or_gpu():
    """No vLLM here: the plugin declines, so vLLM would keep its own platform."""
    assert P.HipPlatform is None
    assert P.register() is None
