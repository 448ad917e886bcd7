"""ORACLE -- test infrastructure, never product code.

CPU restatements of the reference's algorithms on the paged-attention hot
path, used only as the checker by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  Nothing in vllm-apple_amd/ imports this.

Modules
  kv          ctypes loader of the C restatement (kv_oracle.c -> _build/liboracle.so)
              and of the reference's own kv_write.c compiled into _ref/
  attention   numpy fp64 paged decode / chunked-prefill attention, plus a
              pure-Python fp32 online-softmax loop that follows the Metal kernel
  layer_ops   RMSNorm, NeoX RoPE, SiLU*mul in fp32 numpy
  ref_torch   the reference's CPU torch path (scatter KV write, per-sequence
              gather + repeat_interleave + SDPA decode, F.rms_norm, ...): the
              CPU baseline timed by bench.py
  inputs      seeded generators of the BASELINE.json configurations

Pinning status of every function is listed in each module docstring.
"""
