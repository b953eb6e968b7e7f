"""A Gated DeltaNet block (Qwen3.5's linear attention) on the GPU, as the
reference's Engine.linearAttend runs it (src/engine.ts:6646-6825): the
in_proj (q|k|v then z) and b|a projections, the causal convolution with
its state, the recurrence (a row at a time for short batches, in chunks
of 64 for prompt batches, as recurrenceChunks), the gated RMSNorm and
out_proj. The weights are ops.Q4Matrix (any layout); the projections run
as GEMVs up to 8 rows and as the MFMA GEMM above that."""
from __future__ import annotations

import torch

from . import lib as L
from . import ops

CHUNKED_ROWS = 64  # batches of at least this many rows run the chunked form


class LinearAttention:
    def __init__(self, in_proj: ops.Q4Matrix, ba: ops.Q4Matrix, out_proj: ops.Q4Matrix,
                 conv_taps: torch.Tensor, A: torch.Tensor, dt_bias: torch.Tensor,
                 norm_w: torch.Tensor, heads: int, key_dim: int, value_dim: int,
                 eps: float = 1e-6):
        H, dk, dv = heads, key_dim, value_dim
        self.H, self.dk, self.dv, self.eps = H, dk, dv, eps
        self.C = 2 * H * dk + H * dv  # conv channels: q | k | v
        if in_proj.N != self.C + H * dv or ba.N != 2 * H or out_proj.K != H * dv:
            raise ValueError("Gated DeltaNet: projection shapes do not match the heads")
        if conv_taps.shape[0] != self.C:
            raise ValueError(f"Gated DeltaNet: conv taps for {conv_taps.shape[0]} channels, "
                             f"expected {self.C}")
        self.in_proj, self.ba, self.out_proj = in_proj, ba, out_proj
        self.taps, self.A, self.dt, self.norm_w = conv_taps, A, dt_bias, norm_w
        dev = conv_taps.device
        W = conv_taps.shape[1]
        self.conv_state = [torch.zeros((max(W - 1, 1), self.C), device=dev) for _ in range(2)]
        self.state = torch.zeros((H, dk, dv), device=dev)

    @staticmethod
    def uses_gemm(m: ops.Q4Matrix, M: int) -> bool:
        return (M > 8 and m.N % 64 == 0 and m.K % 64 == 0 and
                m.layout in (L.LAYOUT_ROWGROUP, L.LAYOUT_Q8))

    def _project(self, m: ops.Q4Matrix, x16: torch.Tensor) -> torch.Tensor:
        M = x16.shape[0]
        if M <= 8:
            return ops.gemv(m, x16)
        if self.uses_gemm(m, M):
            return ops.gemm(m, x16)
        out = torch.empty((M, m.N), dtype=torch.float32, device=x16.device)
        for r in range(0, M, 8):
            ops.gemv(m, x16[r:r + 8], out=out[r:r + 8])
        return out

    def forward(self, x16: torch.Tensor) -> torch.Tensor:
        """Rows of the block's normed input (halves [M, D]) to its output
        (float32 [M, D]); the conv and recurrent states move on by M rows."""
        M = x16.shape[0]
        proj = self._project(self.in_proj, x16)
        ba = self._project(self.ba, x16)
        qkv = ops.delta_conv(proj, self.C, self.taps, self.conv_state[0], self.conv_state[1])
        self.conv_state.reverse()
        chunked = (M >= CHUNKED_ROWS and self.dk <= 128 and self.dv <= 128 and
                   self.dk % 4 == 0)
        rule = ops.delta_rule_chunked if chunked else ops.delta_rule
        o = rule(qkv, ba, self.A, self.dt, self.H, self.dk, self.dv, self.state)
        h16 = ops.delta_norm(o, self.H, self.dv, proj[:, self.C:], self.norm_w, self.eps)
        return self._project(self.out_proj, h16)
