"""A Gated DeltaNet block end to end (delta_layer.LinearAttention, the
reference's Engine.linearAttend) against the oracle's float64 composition
of the same steps: projections of the dequantized weights (rounded to
halves where the MFMA GEMM runs them, as the reference's f16 prompt plan
does), LIN_CONV, LIN_GATES + LIN_PREP + the delta rule, LIN_NORM (its
output rounded to halves, out_proj's input), out_proj. A prompt batch
(chunked) continued by decode rows equals the oracle over all the rows.
Outputs within rel-L2 1e-3 (the model-level bound: halves in the middle)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gguf_q4_0
from tests.model_oracle import dense_of

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _block(rng, D, H, dk, dv, W=4):
    from webgllm_amd import ops
    from webgllm_amd.delta_layer import LinearAttention
    C = 2 * H * dk + H * dv

    def q4(N, K):
        return ops.Q4Matrix.from_q4_0(torch.from_numpy(gguf_q4_0(rng, N, K)).cuda(), N, K)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    blk = LinearAttention(q4(C + H * dv, D), q4(2 * H, D), q4(D, H * dv),
                          t((rng.standard_normal((C, W)) * 0.5).astype(np.float32)),
                          t(-np.exp(rng.standard_normal(H) * 0.5).astype(np.float32)),
                          t((rng.standard_normal(H) * 0.5).astype(np.float32)),
                          t((1 + 0.1 * rng.standard_normal(dv)).astype(np.float32)), H, dk, dv)
    return blk


class _Oracle:
    """The block's steps in float64 on the oracle, carrying its states."""

    def __init__(self, blk):
        self.blk = blk
        self.w = [dense_of(m).astype(np.float64) for m in (blk.in_proj, blk.ba, blk.out_proj)]
        self.taps = blk.taps.cpu().numpy()
        self.A, self.dt = blk.A.cpu().numpy(), blk.dt.cpu().numpy()
        self.norm_w = blk.norm_w.cpu().numpy()
        self.conv = np.zeros((self.taps.shape[1] - 1, blk.C), np.float32)
        self.state = np.zeros((blk.H, blk.dk, blk.dv))

    def forward(self, x16):
        b = self.blk
        M = x16.shape[0]
        mats = (b.in_proj, b.ba, b.out_proj)
        w_in, w_ba, w_out = (w.astype(np.float16).astype(np.float64) if b.uses_gemm(m, M)
                             else w for w, m in zip(self.w, mats))
        x = x16.astype(np.float64)
        proj = x @ w_in.T
        ba = x @ w_ba.T
        qkv, self.conv = O.delta_conv(proj.astype(np.float32), b.C, self.taps, self.conv)
        o, self.state, _ = O.delta_rule(qkv.astype(np.float32), ba, self.A, self.dt, b.H, b.dk,
                                        b.dv, self.state)
        h = O.delta_norm(o.astype(np.float32), b.H, b.dv, proj[:, b.C:].astype(np.float32),
                         self.norm_w, b.eps)
        h16 = np.clip(h, -65504, 65504).astype(np.float16).astype(np.float64)
        return h16 @ w_out.T


@pytest.mark.parametrize("D,H,dk,dv,rows", [(512, 4, 64, 64, [1, 1, 5]),
                                            (1024, 16, 128, 128, [100, 3, 1]),
                                            (256, 2, 32, 48, [70, 9, 2])])
def test_block_matches_oracle(hip, D, H, dk, dv, rows):
    rng = np.random.default_rng(D + H + dk)
    blk = _block(rng, D, H, dk, dv)
    ref = _Oracle(blk)
    for M in rows:
        x = (rng.standard_normal((M, D)) * 0.5).astype(np.float16)
        y = blk.forward(torch.from_numpy(x).cuda())
        want = ref.forward(x)
        torch.cuda.synchronize()
        assert _rel(y.cpu().numpy(), want) < 1e-3, M
    assert _rel(blk.state.cpu().numpy(), ref.state) < 1e-3
    assert _rel(blk.conv_state[0].cpu().numpy()[:3], ref.conv) < 1e-5
