"""EngineMLP: mirror of vllm_apple/engine/ops/mlp.py's gated SiLU MLP on HIP.

encode (mlp.py:170-245 with _encode_gated_mlp, :247-384) computes
down_proj(silu(gate_proj(x)) * up_proj(x)).  The reference runs the gate and
up GEMMs into two [T, I] intermediates and a silu_mul pass over them; here
the first half is one MFMA kernel with the SwiGLU epilogue
(kernels.gate_up_silu), so only the activated [T, I] intermediate exists, and
the down projection is a plain library GEMM (torch.matmul on the step's
stream).  Weights keep the reference's layouts: gate_proj / up_proj [I, H]
or the fused gate_up_proj [2I, H] (gate rows first), down_proj [H, I].

Above FUSED_MAX_TOKENS tokens encode takes the reference's order instead: a
library GEMM into [T, 2I] and kernels.silu_mul over its halves.  On MI355X
(hidden 5120, intermediate 32768) the fused kernel leads up to 1024 tokens
(by 9 % at 16-64, 2-5 % at 256-1024) and hipBLASLt's GEMM leads at 2104 and
4096 tokens (3 and 8 %).

Only the gated SiLU form without biases is on this path; a standard MLP,
GELU or biases raise NotImplementedError.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional

import torch

from .. import kernels
from .step import resolve_stream, view


@dataclass
class MLPConfig:
    hidden_size: int
    intermediate_size: int
    gated: bool = True
    activation: str = "silu"
    bias: bool = False


class EngineMLP:
    # Token counts above this run the library GEMM + silu_mul route.
    FUSED_MAX_TOKENS = 1024

    def __init__(self, context: Any, hidden_size: int, intermediate_size: int,
                 gated: bool = True, activation: str = "silu", bias: bool = False):
        if not gated or activation != "silu" or bias:
            raise NotImplementedError("only the gated SiLU MLP without biases is supported")
        self._context = context
        self.config = MLPConfig(hidden_size=hidden_size, intermediate_size=intermediate_size,
                                gated=gated, activation=activation, bias=bias)
        self._gate_proj = None
        self._up_proj = None
        self._gate_up_proj = None
        self._down_proj = None
        self._fused_gate_up = False
        self._scratch: Optional[torch.Tensor] = None
        self._scratch_streams: set = set()
        self._gu: Optional[torch.Tensor] = None
        self._gu_streams: set = set()
        # Outgrown scratch buffers, kept alive (see _grow).
        self._retired: list = []
        self.fused_max_tokens = self.FUSED_MAX_TOKENS

    def set_weights(self, gate_proj: Optional[torch.Tensor] = None,
                    up_proj: Optional[torch.Tensor] = None,
                    down_proj: Optional[torch.Tensor] = None,
                    gate_up_proj: Optional[torch.Tensor] = None,
                    gate_bias: Optional[torch.Tensor] = None,
                    up_bias: Optional[torch.Tensor] = None,
                    down_bias: Optional[torch.Tensor] = None) -> None:
        """mlp.py:125-168: a fused gate_up_proj takes precedence over separate
        gate_proj / up_proj."""
        if gate_bias is not None or up_bias is not None or down_bias is not None:
            raise NotImplementedError("MLP biases are not supported")
        if gate_up_proj is not None:
            self._gate_up_proj, self._gate_proj, self._up_proj = gate_up_proj, None, None
            self._fused_gate_up = True
        else:
            self._gate_proj, self._up_proj, self._gate_up_proj = gate_proj, up_proj, None
            self._fused_gate_up = False
        self._down_proj = down_proj

    @staticmethod
    def _buf(x: Any):
        if isinstance(x, tuple):
            return x
        return x, 0

    def _grow(self, name: str, n: int, like: torch.Tensor,
              stream: torch.cuda.Stream) -> torch.Tensor:
        """A grow-only scratch of at least n elements kept in attribute
        `name`, allocated on the stream that writes and reads it.  An outgrown
        buffer is kept alive, never freed, as kernels._GrowOnlyScratch does: a
        HIP graph captured while it was current holds its address, and a
        replay must not write into memory the caching allocator has handed to
        another tensor.  Sizes grow at least 2x, so the kept buffers sum to
        less than the current one.  A scratch first made on another stream is
        marked as used on this one (record_stream)."""
        buf, streams = getattr(self, name), getattr(self, name + "_streams")
        if buf is None or buf.numel() < n or buf.dtype != like.dtype or buf.device != like.device:
            size = n
            if buf is not None:
                self._retired.append(buf)
                if buf.dtype == like.dtype and buf.device == like.device:
                    size = max(n, 2 * buf.numel())
            with torch.cuda.stream(stream):
                buf = torch.empty(size, dtype=like.dtype, device=like.device)
            setattr(self, name, buf)
            setattr(self, name + "_streams", {stream.cuda_stream})
        elif stream.cuda_stream not in streams:
            buf.record_stream(stream)
            streams.add(stream.cuda_stream)
        return buf

    def _intermediate(self, num_tokens: int, like: torch.Tensor,
                      stream: torch.cuda.Stream) -> torch.Tensor:
        """The activated [T, I] scratch."""
        n = num_tokens * self.config.intermediate_size
        return self._grow("_scratch", n, like, stream)[:n].view(num_tokens,
                                                                self.config.intermediate_size)

    def encode(self, step_ctx: Any, hidden_states: Any, output_buffer: Any, num_tokens: int,
               intermediate_buffer: Optional[Any] = None) -> None:
        if self._down_proj is None:
            raise RuntimeError("Down projection weights not set - call set_weights() first")
        if not self._fused_gate_up and (self._gate_proj is None or self._up_proj is None):
            raise RuntimeError("Gate and up projection weights not set for gated MLP. "
                               "Call set_weights(gate_proj=..., up_proj=...) or "
                               "set_weights(gate_up_proj=...)")
        stream = resolve_stream(step_ctx)
        H, I = self.config.hidden_size, self.config.intermediate_size
        hb, ho = self._buf(hidden_states)
        ob, oo = self._buf(output_buffer)
        x = view(hb, ho, (num_tokens, H), dtype=hb.dtype)
        out = view(ob, oo, (num_tokens, H), dtype=ob.dtype)
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        if intermediate_buffer is not None:
            ib, io = self._buf(intermediate_buffer)
            act = view(ib, io, (num_tokens, I), dtype=ib.dtype)
        else:
            act = self._intermediate(num_tokens, x, s)
        with torch.cuda.stream(s):
            if num_tokens <= self.fused_max_tokens:
                if self._fused_gate_up:
                    kernels.gate_up_silu(x, self._gate_up_proj, out=act, stream=s)
                else:
                    kernels.gate_up_silu(x, self._gate_proj, self._up_proj, out=act, stream=s)
            else:
                # The reference's order (mlp.py:247-330): both GEMMs into one
                # [T, 2I] scratch, then silu_mul over its halves.
                gu = self._grow("_gu", 2 * num_tokens * I, x, s)[:2 * num_tokens * I]
                gu = gu.view(num_tokens, 2 * I)
                if self._fused_gate_up:
                    torch.matmul(x, self._gate_up_proj.t(), out=gu)
                else:
                    torch.matmul(x, self._gate_proj.t(), out=gu[:, :I])
                    torch.matmul(x, self._up_proj.t(), out=gu[:, I:])
                kernels.silu_mul(gu[:, :I], gu[:, I:], out=act, stream=s)
            torch.matmul(act, self._down_proj.t(), out=out)

    def get_intermediate_size(self, num_tokens: int) -> int:
        """Bytes of intermediate buffer encode needs: the one activated
        [T, I] buffer (the reference needs three: gate, up and fused)."""
        return num_tokens * self.config.intermediate_size * 2

    def get_output_size(self, num_tokens: int) -> int:
        return num_tokens * self.config.hidden_size * 2

    def get_params_dict(self) -> Dict[str, Any]:
        return {"hidden_size": self.config.hidden_size,
                "intermediate_size": self.config.intermediate_size,
                "gated": self.config.gated, "activation": self.config.activation,
                "bias": self.config.bias}
