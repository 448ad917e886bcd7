"""Encode-only ops mirroring vllm_apple/engine/ops/{attention,kv_write,rmsnorm,elementwise,topk,mlp}.py.

"Encode" here means: enqueue the HIP kernels on a stream and return without
waiting.  Every encode_* method keeps the reference's argument names and order;
its first argument, step_ctx, may be None (torch's current stream), a
torch.cuda.Stream, or any object with a `.stream` attribute.  Buffers are fp16
or int32 torch tensors on the GPU; byte offsets select a view into them like
the reference's (MTLBuffer, offset) pairs.
"""
from .attention import FusedAttentionParams, PagedAttentionOp, PagedAttentionParams
from .elementwise import EngineElementwiseOps, EngineRoPE
from .kv_write import KVWriteOp, KVWriteParams
from .mlp import EngineMLP, MLPConfig
from .rmsnorm import EngineRMSNorm, RMSNormConfig
from .step import EngineStepContext
from .topk import EngineTopK, reconstruct_logits

__all__ = [
    "EngineElementwiseOps",
    "EngineMLP",
    "EngineRMSNorm",
    "EngineRoPE",
    "EngineStepContext",
    "EngineTopK",
    "FusedAttentionParams",
    "KVWriteOp",
    "KVWriteParams",
    "MLPConfig",
    "PagedAttentionOp",
    "PagedAttentionParams",
    "RMSNormConfig",
    "reconstruct_logits",
]
