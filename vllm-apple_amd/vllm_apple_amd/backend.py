"""vLLM attention backend on the HIP kernels: drop-in for METAL_ATTN.

Mirrors vllm_apple/v1/attention/backends/metal_attn.py:
  HipAttentionBackend           MetalAttentionBackend (:124-199)
  HipAttentionMetadata          MetalAttentionMetadata (:202-250)
  HipAttentionMetadataBuilder   MetalAttentionMetadataBuilder (:253-321)
  HipAttentionImpl              MetalAttentionImpl (:324-764), forward (:568-764)

Differences from the Metal backend, all on the device side:
  * vLLM's own kv_cache tensor [2, num_blocks, block_size, num_kv_heads, D] is
    read and written directly in HBM (the kernels take its strides), so there
    is no shadow cache and no host copy; the KV write is one launch.
  * Chunked-prefill tokens attend to the cached prefix plus the causal chunk
    (paged_attention_v2.metal:375-478 semantics) instead of the chunk alone.
  * Every call only enqueues on the current HIP stream; nothing synchronises.
vLLM is optional at import time: without it the classes use local stand-ins
for AttentionType and the abstract bases.
"""
from __future__ import annotations

import logging
import os
from dataclasses import dataclass
from typing import Any, ClassVar, Optional

import torch

from . import kernels

logger = logging.getLogger(__name__)

try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.attention.backends.abstract import (AttentionBackend, AttentionImpl,
                                                  AttentionType)
except Exception:  # noqa: BLE001
    AttentionBackend = object
    AttentionImpl = object

    class AttentionType:  # vllm/attention/backends/abstract.py values
        DECODER = "decoder"
        ENCODER = "encoder"
        ENCODER_ONLY = "encoder_only"
        ENCODER_DECODER = "encoder_decoder"


SUPPORTED_HEAD_SIZES = [32, 64, 96, 128]
BACKEND_NAME = "VAA_HIP_ATTN"


def _max_model_len() -> Optional[int]:
    """vLLM's max_model_len for the model being built, or None without vLLM
    (or outside a vLLM config context)."""
    try:  # pragma: no cover - vLLM is not installed in the build container
        from vllm.config import get_current_vllm_config
        return int(get_current_vllm_config().model_config.max_model_len)
    except Exception:  # noqa: BLE001
        return None


def is_quantized_kv_cache(kv_cache_dtype: str) -> bool:
    return kv_cache_dtype not in ("auto", "float16", "half", "fp16", "bfloat16", "bf16")


class HipAttentionBackend(AttentionBackend):
    accept_output_buffer: bool = True
    supported_dtypes: ClassVar[list] = [torch.float16, torch.bfloat16]

    @classmethod
    def get_supported_dtypes(cls) -> list:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_supported_head_sizes(cls) -> list:
        return list(SUPPORTED_HEAD_SIZES)

    @staticmethod
    def get_name() -> str:
        return BACKEND_NAME

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type in (AttentionType.DECODER, AttentionType.ENCODER,
                             AttentionType.ENCODER_ONLY)

    @staticmethod
    def get_impl_cls():
        return HipAttentionImpl

    @staticmethod
    def get_builder_cls():
        return HipAttentionMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple:
        """[2, num_blocks, block_size, num_kv_heads, head_size] (metal_attn.py:171-185)."""
        return 2, num_blocks, block_size, num_kv_heads, head_size

    @staticmethod
    def use_cascade_attention(*args, **kwargs) -> bool:
        return False

    @staticmethod
    def get_kv_cache_device() -> str:
        """The cache lives in HBM (the Metal backend returns "cpu": unified memory)."""
        return "cuda"


@dataclass
class HipAttentionMetadata:
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    scheduler_metadata: Optional[torch.Tensor] = None
    causal: bool = True
    num_decode_tokens: int = 0
    _query_start_loc_cpu: Optional[list] = None
    _seq_lens_cpu: Optional[list] = None

    @property
    def query_start_loc_cpu(self) -> list:
        if self._query_start_loc_cpu is None:
            self._query_start_loc_cpu = self.query_start_loc.tolist()
        return self._query_start_loc_cpu

    @property
    def seq_lens_cpu(self) -> list:
        if self._seq_lens_cpu is None:
            self._seq_lens_cpu = self.seq_lens.tolist()
        return self._seq_lens_cpu


def split_decodes_and_prefills(query_start_loc_cpu: list, decode_threshold: int = 1,
                               require_uniform: bool = False):
    """(num_decodes, num_prefills, num_decode_tokens, num_prefill_tokens) for a
    batch whose decode requests come first, as vLLM's reorder guarantees.

    Restates vLLM's split_decodes_and_prefills (vllm/v1/attention/backends/
    utils.py), which the reference calls with require_uniform=True
    (metal_attn.py:302-308):
      * every request is a decode when the longest query is at most
        decode_threshold (with require_uniform only when the threshold is 1);
      * no decodes when the first request's query is longer than the threshold;
      * otherwise the decodes are the leading requests up to the first
        "prefill": a query longer than the threshold, or, with
        require_uniform, a query whose length differs from the first one's.
    vLLM is not vendored with the reference, so this boundary is pinned by
    hand-worked cases only.
    """
    qsl = list(query_start_loc_cpu)
    num_reqs = len(qsl) - 1
    num_tokens = qsl[-1] if qsl else 0
    if num_reqs <= 0:
        return 0, 0, 0, 0
    lens = [qsl[i + 1] - qsl[i] for i in range(num_reqs)]
    if max(lens) <= decode_threshold and (not require_uniform or decode_threshold <= 1):
        return num_reqs, 0, num_tokens, 0
    if lens[0] > decode_threshold:
        return 0, num_reqs, 0, num_tokens
    if require_uniform:
        is_prefill = [n != lens[0] for n in lens]
    else:
        is_prefill = [n > decode_threshold for n in lens]
    if not any(is_prefill):
        return num_reqs, 0, num_tokens, 0
    first_prefill = is_prefill.index(True)
    num_decode_tokens = qsl[first_prefill]
    return (first_prefill, num_reqs - first_prefill, num_decode_tokens,
            num_tokens - num_decode_tokens)


try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.v1.attention.backends.utils import AttentionMetadataBuilder as _VllmBuilder
except Exception:  # noqa: BLE001
    _VllmBuilder = None


class HipAttentionMetadataBuilder(_VllmBuilder[HipAttentionMetadata]
                                  if _VllmBuilder is not None else object):
    """Builds HipAttentionMetadata from vLLM's CommonAttentionMetadata
    (MetalAttentionMetadataBuilder, metal_attn.py:253-321).  Derives from
    vLLM's AttentionMetadataBuilder when vLLM is importable."""

    reorder_batch_threshold: int = 1

    def __init__(self, kv_cache_spec: Any = None, layer_names: Optional[list] = None,
                 vllm_config: Any = None, device: Optional[torch.device] = None):
        if _VllmBuilder is not None:  # pragma: no cover - needs vLLM
            super().__init__(kv_cache_spec, layer_names or [], vllm_config, device)
            init_reorder = getattr(self, "_init_reorder_batch_threshold", None)
            if init_reorder is not None:
                init_reorder(1, False)
        # Decode requests (one query token) are reordered to the front of the
        # batch, as the reference's builder asks (metal_attn.py:265).
        self.reorder_batch_threshold = 1
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names or []
        self.vllm_config = vllm_config
        self.device = device
        self.block_size = getattr(kv_cache_spec, "block_size", 16)

    def build(self, common_prefix_len: int, common_attn_metadata: Any,
              fast_build: bool = False) -> HipAttentionMetadata:
        cm = common_attn_metadata
        qsl_cpu = getattr(cm, "query_start_loc_cpu", None)
        if qsl_cpu is None:
            qsl_cpu = cm.query_start_loc.cpu()
        qsl_list = qsl_cpu.tolist() if isinstance(qsl_cpu, torch.Tensor) else list(qsl_cpu)
        num_decode_tokens = 0
        if cm.causal:
            _, _, num_decode_tokens, _ = split_decodes_and_prefills(
                qsl_list, self.reorder_batch_threshold, require_uniform=True)
        seq_cpu = getattr(cm, "seq_lens_cpu", None)
        return HipAttentionMetadata(
            num_actual_tokens=cm.num_actual_tokens,
            max_query_len=cm.max_query_len,
            query_start_loc=cm.query_start_loc,
            max_seq_len=cm.max_seq_len,
            seq_lens=cm.seq_lens,
            block_table=cm.block_table_tensor,
            slot_mapping=cm.slot_mapping,
            scheduler_metadata=None,
            causal=cm.causal,
            num_decode_tokens=num_decode_tokens,
            _query_start_loc_cpu=qsl_list,
            _seq_lens_cpu=seq_cpu.tolist() if isinstance(seq_cpu, torch.Tensor) else seq_cpu,
        )


# Staging cache of the no-cache (encoder) path: grow-only, reused by calls
# ordered on one stream.
_no_cache_scratch = kernels._GrowOnlyScratch()

OVERLAP_ENV = "VLLM_VAA_OVERLAP"


def _overlap_enabled() -> bool:
    """Decode and prefill of a mixed step run concurrently unless
    VLLM_VAA_OVERLAP=0."""
    return os.environ.get(OVERLAP_ENV, "1") != "0"


class HipAttentionImpl(AttentionImpl):
    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: Optional[list], sliding_window: Optional[int],
                 kv_cache_dtype: str, logits_soft_cap: Optional[float] = None,
                 attn_type: str = AttentionType.DECODER,
                 kv_sharing_target_layer_name: Optional[str] = None,
                 sinks: Optional[torch.Tensor] = None) -> None:
        self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
        self._is_kv_shared = kv_sharing_target_layer_name is not None
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        if logits_soft_cap is not None:
            logger.warning("%s does not support logits softcap, outputs may be slightly off",
                           BACKEND_NAME)
        self.logits_soft_cap = logits_soft_cap or 0
        self.num_kv_heads = num_kv_heads
        if alibi_slopes is not None:
            logger.warning("%s does not support ALiBi slopes, ignoring", BACKEND_NAME)
        self.alibi_slopes = None
        # The kernels attend over the whole context.  A window of W keys
        # (vLLM's: query position p sees keys p-W+1 .. p) gives the same result
        # whenever no context is longer than W.  The reference keeps the window
        # and ignores it (metal_attn.py:377-382), which attends too far once a
        # context outgrows it; here a window shorter than the model's longest
        # context (vLLM's max_model_len) is refused, and when that length is
        # unknown every step's longest context is checked in forward.
        self._window: Optional[int] = None
        if sliding_window is not None:
            window = int(sliding_window)
            mml = _max_model_len()
            if window <= 0 or (mml is not None and window < mml):
                raise NotImplementedError(
                    f"sliding_window={sliding_window} is not supported by {BACKEND_NAME}: "
                    f"the kernels attend over the whole context (max_model_len={mml})")
            if mml is None:
                self._window = window
        self.sliding_window = (-1, -1)
        self.kv_cache_dtype = kv_cache_dtype
        self.num_queries_per_kv = num_heads // num_kv_heads
        if is_quantized_kv_cache(kv_cache_dtype):
            raise NotImplementedError(f"FP8 KV cache is unsupported in {BACKEND_NAME}")
        if head_size not in SUPPORTED_HEAD_SIZES:
            raise ValueError(f"head_size must be 32/64/96/128, got {head_size}")
        if num_heads % num_kv_heads != 0:
            raise ValueError(
                f"num_heads={num_heads} is not a multiple of num_kv_heads={num_kv_heads}")
        self.attn_type = attn_type
        self.sinks = sinks
        self._shadow: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ cache
    def _caches(self, kv_cache: torch.Tensor) -> tuple:
        """(key_cache, value_cache) in the vLLM layout [nb, bs, KV, D].

        An fp16 or bf16 kv_cache is used in place: the kernels take both
        element types, so bf16 models need neither the fp16 copy of the cache
        the Metal backend keeps (metal_attn.py:654-660) nor conversions.  Any
        other cache dtype gets a same-shaped fp16 cache kept per layer.
        """
        if kv_cache.dtype in kernels.ATTN_DTYPES:
            return kv_cache[0], kv_cache[1]
        if self._shadow is None or self._shadow.shape != kv_cache.shape:
            self._shadow = torch.zeros(kv_cache.shape, dtype=torch.float16,
                                       device=kv_cache.device)
        return self._shadow[0], self._shadow[1]

    # ---------------------------------------------------------------- forward
    def forward(self, layer: Any, query: torch.Tensor, key: Optional[torch.Tensor],
                value: Optional[torch.Tensor], kv_cache: torch.Tensor,
                attn_metadata: Optional[HipAttentionMetadata],
                output: Optional[torch.Tensor] = None,
                output_scale: Optional[torch.Tensor] = None,
                output_block_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError(
                "Fused output quantization is not yet supported for HipAttentionImpl")
        if attn_metadata is None:  # warm-up / profiling
            return output
        if self._window is not None and attn_metadata.max_seq_len > self._window:
            raise NotImplementedError(
                f"a context of {attn_metadata.max_seq_len} tokens exceeds "
                f"sliding_window={self._window}: {BACKEND_NAME} attends over the whole context")

        # The kernels run in the cache's element type (fp16 or bf16).  Only
        # activations of another type are converted, as the Metal backend
        # converts bf16 for its fp16 kernels (metal_attn.py:609-620).
        original_output = output
        if self.attn_type in (AttentionType.ENCODER_ONLY, AttentionType.ENCODER):
            work_dt = query.dtype if query.dtype in kernels.ATTN_DTYPES else torch.float16
        else:
            work_dt = kv_cache.dtype if kv_cache.dtype in kernels.ATTN_DTYPES else torch.float16
        conv = query.dtype != work_dt
        if conv:
            query = query.to(work_dt)
            key = key.to(work_dt) if key is not None else None
            value = value.to(work_dt) if value is not None else None
            output = torch.empty(output.shape, dtype=work_dt, device=output.device)

        n = attn_metadata.num_actual_tokens
        if self.attn_type in (AttentionType.ENCODER_ONLY, AttentionType.ENCODER):
            self._attention_no_cache(query[:n], key[:n], value[:n], output[:n], attn_metadata,
                                     causal=False)
        else:
            key_cache, value_cache = self._caches(kv_cache)
            if not self._is_kv_shared and key is not None and value is not None and n > 0:
                kernels.kv_write_slots(key[:n], value[:n], key_cache, value_cache,
                                       attn_metadata.slot_mapping[:n], layout="vllm")
            nd = attn_metadata.num_decode_tokens

            def decode(shared=False):
                # Host lengths, only if already cached (never a device sync here).
                lens_host = attn_metadata._seq_lens_cpu
                kernels.paged_decode(query[:nd], key_cache, value_cache,
                                     attn_metadata.block_table[:nd],
                                     attn_metadata.seq_lens[:nd], scale=self.scale,
                                     max_seq_len=attn_metadata.max_seq_len, layout="vllm",
                                     output=output[:nd],
                                     seq_lens_host=lens_host[:nd] if lens_host else None,
                                     shared=shared)

            overlapped = nd > 0 and n > nd and _overlap_enabled()

            def prefill():
                # Split long contexts when the host lengths are at hand (never
                # a device sync for them) and no decode runs beside the
                # prefill: next to a decode the unsplit prefill is better (its
                # long workgroups hold a few CUs and leave the rest to the
                # decode; C5 attention step 0.61 ms against 0.68-0.79 split).
                # The pieces are counted over the longest prefill context
                # (decode contexts do not matter), which bounds the workspace.
                split, longest = 0, 0
                lens_host = attn_metadata._seq_lens_cpu
                qsl_host = attn_metadata._query_start_loc_cpu
                if lens_host and qsl_host and not overlapped:
                    ql = [b - a if b - a > 1 else 0 for a, b in zip(qsl_host[:-1], qsl_host[1:])]
                    split = kernels.choose_prefill_split(
                        lens_host, ql, self.num_kv_heads, query.shape[1],
                        kernels.device_cus(query.device), head_size=self.head_size)
                    longest = max((l for l, q in zip(lens_host, ql) if q > 0), default=0)
                kernels.paged_prefill(query[nd:n], key_cache, value_cache,
                                      attn_metadata.block_table, tok[nd:n], pos[nd:n],
                                      scale=self.scale, layout="vllm", output=output[nd:n],
                                      split_keys=split, max_seq_len=longest if split else 0)

            if n > nd:
                tok, pos = kernels.build_token_index(attn_metadata.query_start_loc,
                                                     attn_metadata.seq_lens, n)
            if overlapped:
                # Mixed step: prefill (MFMA-bound, current stream, dispatched
                # first) and decode (HBM-bound, side stream, shared split) run
                # concurrently.
                kernels.overlap(prefill, lambda: decode(shared=True), query.device)
            else:
                if nd > 0:
                    decode()
                if n > nd:
                    prefill()
        if conv:
            original_output[:n].copy_(output[:n].to(original_output.dtype))
            return original_output
        return output

    def _attention_no_cache(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            output: torch.Tensor, attn_metadata: HipAttentionMetadata,
                            causal: bool) -> torch.Tensor:
        """Attention inside each sequence's own tokens (encoder / no KV cache),
        the semantics of _compute_attention_sdpa (base_attn.py:223-306).

        The tokens are staged into a scratch paged cache, one block-aligned
        range per sequence, and run through the prefill kernel; positions are
        the in-sequence index (causal) or the last index (bidirectional).
        """
        qsl = attn_metadata.query_start_loc_cpu
        num_seqs = len(qsl) - 1
        T = min(query.shape[0], qsl[-1] if num_seqs > 0 else 0)
        if T <= 0:
            return output
        bs = 16
        dev = query.device
        # Per-sequence tables on the host (num_seqs entries), per-token indices
        # on the device.
        start = torch.tensor(qsl[:-1], dtype=torch.int64)
        lens = torch.tensor(qsl[1:], dtype=torch.int64) - start
        nblk = (lens + bs - 1) // bs
        blk_off = torch.cumsum(nblk, 0) - nblk
        total, maxb = int(nblk.sum()), max(int(nblk.max()), 1)
        start_d, lens_d, nblk_d, off_d = (t.to(dev, non_blocking=True)
                                          for t in (start, lens, nblk, blk_off))
        seq = torch.repeat_interleave(torch.arange(num_seqs, device=dev), lens_d,
                                      output_size=qsl[-1])[:T]
        idx = torch.arange(T, device=dev) - start_d[seq]  # index inside the sequence
        slots = off_d[seq] * bs + idx
        pos = (idx if causal else lens_d[seq] - 1).to(torch.int32)
        j = torch.arange(maxb, device=dev)
        bt = torch.where(j[None, :] < nblk_d[:, None], off_d[:, None] + j[None, :],
                         torch.full_like(j[None, :], -1)).to(torch.int32)
        kv = key.shape[1]
        scratch = _no_cache_scratch.get(2 * total * bs * kv * self.head_size * query.element_size(),
                                        dev)
        kc = scratch[:total * bs * kv * self.head_size * query.element_size()].view(
            query.dtype).view(total, bs, kv, self.head_size)
        vc = scratch[kc.numel() * query.element_size():2 * kc.numel() * query.element_size()
                     ].view(query.dtype).view(total, bs, kv, self.head_size)
        kernels.kv_write_slots(key[:T], value[:T], kc, vc, slots, layout="vllm")
        kernels.paged_prefill(query[:T], kc, vc, bt, seq.to(torch.int32), pos, scale=self.scale,
                              layout="vllm", output=output[:T])
        return output
