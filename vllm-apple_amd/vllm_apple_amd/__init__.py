"""MI355X-native paged-attention hot path of vllm-apple.

Layers:
  _lib       ctypes binding of libvllm_apple_amd.so (HIP kernels, C ABI)
  kernels    functional torch-tensor wrappers over the C ABI
  kv_cache   HBM-resident paged K/V cache with the reference's validation
  engine     encode-only ops mirroring vllm_apple/engine/ops/*
  backend    vLLM AttentionBackend/Impl mirror of metal_attn.py
  indexing   slot / block / token index rules of the reference runner
"""
from __future__ import annotations

__version__ = "0.1.0"


def build_library(verbose: bool = True):
    """Compile every HIP source for gfx950 into the in-tree shared library."""
    import importlib.util
    from pathlib import Path

    build_py = Path(__file__).resolve().parent.parent / "csrc" / "build.py"
    spec = importlib.util.spec_from_file_location("_vaa_build", build_py)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build(verbose=verbose)
