"""The GEMV epilogues (prescaled norm in, residual + next norm's input and
sums of squares out, SwiGLU, RoPE + KV cache writes) against the oracle,
for every layout and row count."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import rel_l2
from tests.model_oracle import dense_of

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _h(t):
    return O.halves_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))


def _matrix(fmt, N, K, seed, row_order=None):
    from webgllm_amd import engine as E
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.__new__(E.Weights)
    w.shape = shape
    w.device = "cuda"
    w.g = torch.Generator(device="cuda")
    w.g.manual_seed(seed)
    return w.matrix(N, K, row_order)


FMTS = ["q4_0", "nbits", "q4_k", "q4_k_rowgroup", "q4_k_records", "q8_0", "q6_k"]


def _tol(fmt, tight):
    # Q4_K records weigh a block's zero term as dmin m, not packQ4_K's d'
    # half(dmin m / d') that the oracle computes: the 1e-3 rel-L2 parity bar
    # then, rather than the float32 sums' tighter margin
    return 1e-3 if fmt == "q4_k_records" else tight


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [1, 2, 5])
@pytest.mark.parametrize("N,K", [(512, 1024), (256, 4096), (1024, 14336)])
def test_store_normed_residual_prescaled_out(hip, fmt, M, N, K):
    from webgllm_amd import lib as L, ops
    rng = np.random.default_rng(N + K + M)
    m = _matrix(fmt, N, K, seed=M)
    W = dense_of(m).astype(np.float64)
    # input: a residual row h (K) and its prescaled half with norm weights
    hin = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    x16 = O.f32_to_h2(hin * nw / np.float32(32))
    parts_in = (hin.astype(np.float32).reshape(M, K // 4, 4) ** 2).sum(-1).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    w_next = rng.uniform(0.5, 1.5, N).astype(np.float32)
    y = _t(res.copy())
    out16 = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    parts_out = torch.zeros((M, N // 4), dtype=torch.float32, device="cuda")
    pin, wn, wn2 = _t(parts_in), _t(nw), _t(w_next)
    ep = L.Epilogue(mode=L.EPI_STORE, norm_parts=pin.data_ptr(), n_parts=K // 4,
                    ld_parts_in=K // 4, norm_count=K, eps=1e-5, norm_mult=32.0,
                    residual=y.data_ptr(), ld_residual=N, out16=out16.data_ptr(), ld_out16=N,
                    out16_w=wn2.data_ptr(), norm_mult_out=32.0, parts_out=parts_out.data_ptr(),
                    ld_parts_out=N // 4)
    ops.gemv(m, _t(x16.view(np.int16)), out=y, epilogue=ep)
    r = 32.0 / np.sqrt((hin.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5)
    want = res + (O.halves_to_f32(x16).astype(np.float64) @ W.T) * r
    got = y.cpu().numpy()
    # float32 sums (products exact): well inside the 1e-3 bar
    assert rel_l2(got, want) <= _tol(fmt, 1e-4)
    assert rel_l2(_h(out16), got * w_next / 32) <= 1e-3
    want_parts = (got.astype(np.float64).reshape(M, N // 4, 4) ** 2).sum(-1)
    assert rel_l2(parts_out.cpu().numpy(), want_parts) <= 1e-4


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M", [1, 3])
def test_swiglu_epilogue(hip, fmt, M):
    from webgllm_amd import engine as E, lib as L, ops
    F, K = 768, 2048
    rng = np.random.default_rng(M)
    m = _matrix(fmt, 2 * F, K, seed=11, row_order=E.gate_up_row_order(F))
    W = dense_of(m).astype(np.float64)   # logical rows: gate then up
    x16 = O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
    out16 = torch.zeros((M, F), dtype=torch.int16, device="cuda")
    ops.gemv(m, _t(x16.view(np.int16)),
             epilogue=L.Epilogue(mode=L.EPI_SWIGLU, out16=out16.data_ptr(), ld_out16=F))
    gu = (O.halves_to_f32(x16).astype(np.float64) @ W.T).astype(np.float32)
    want = O.swiglu(gu)
    got = _h(out16)
    assert rel_l2(got, want) <= 1e-3
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -9 + 1e-3 * np.abs(want).max())


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "q4_k_records", "q8"])
# K = 4096 at 32/8 heads: more row groups than the grid's waves, where the
# rotation's table rows are fetched after the activations
@pytest.mark.parametrize("H,KV,hd,K", [(14, 2, 64, 1024), (32, 8, 128, 1024), (32, 8, 128, 4096)])
@pytest.mark.parametrize("M,pos0", [(1, 0), (1, 1500), (4, 1022)])
def test_rope_kv_epilogue(hip, fmt, H, KV, hd, K, M, pos0):
    from webgllm_amd import engine as E, lib as L, ops
    shape = E.ModelShape("t", K, 1, H, KV, hd, 4, 4, fmt)
    N = shape.qkv_rows
    rng = np.random.default_rng(H + M + pos0)
    m = _matrix(fmt, N, K, seed=5, row_order=E.qkv_row_order(shape))
    W = dense_of(m).astype(np.float64)
    x16 = O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
    ctx = 2048
    rope = O.rope_table(1e6, hd, hd, ctx)
    drope = _t(rope)
    pos = _t(np.array([pos0], np.int32))
    q = torch.zeros((M, H * hd), dtype=torch.float32, device="cuda")
    kc = torch.zeros((ctx, KV * hd), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    ep = L.Epilogue(mode=L.EPI_ROPE_KV, heads=H, kv_heads=KV, head_dim=hd, ctx=ctx,
                    rope_rows=rope.shape[0], rope=drope.data_ptr(), pos0=pos.data_ptr(),
                    q_out=q.data_ptr(), ld_q_out=H * hd, k_cache=kc.data_ptr(),
                    v_cache=vc.data_ptr())
    ops.gemv(m, _t(x16.view(np.int16)), epilogue=ep)
    qkv = (O.halves_to_f32(x16).astype(np.float64) @ W.T).astype(np.float32)
    qg = q.cpu().numpy()
    kg = kc.cpu().numpy().view(np.uint16)
    vg = vc.cpu().numpy().view(np.uint16)
    qd = H * hd
    for t in range(M):
        p = pos0 + t
        for h in range(H):
            want = O.head_prep(qkv[t, h * hd:(h + 1) * hd], None, rope, hd, hd, p, 0.0,
                               1 / math.sqrt(hd), False)
            got = qg[t, h * hd:(h + 1) * hd]
            assert rel_l2(got, want) <= _tol(fmt, 1e-4)
            assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max())
        for h in range(KV):
            want = O.f32_to_h2(O.head_prep(qkv[t, qd + h * hd:qd + (h + 1) * hd], None, rope, hd,
                                           hd, p, 0.0, 1.0, False))
            got = O.halves_to_f32(kg[p, h * hd:(h + 1) * hd])
            wf = O.halves_to_f32(want)
            # halves of float32 results that agree to ~1e-5 of the vector
            assert np.all(np.abs(got - wf) <= np.abs(wf) * 2 ** -10 + _tol(fmt, 1e-4) * np.abs(wf).max())
            vw = O.halves_to_f32(O.f32_to_h2(qkv[t, qd + KV * hd + h * hd:
                                                 qd + KV * hd + (h + 1) * hd]))
            vgot = O.halves_to_f32(vg[p, h * hd:(h + 1) * hd])
            assert np.all(np.abs(vgot - vw) <= np.abs(vw) * 2 ** -10 + _tol(fmt, 1e-4) * np.abs(vw).max())
    assert not np.any(kg[pos0 + M:])


@pytest.mark.parametrize("fmt", FMTS)
def test_embed_extras(hip, fmt):
    from webgllm_amd import lib as L, ops
    N, K = 256, 1024
    m = _matrix(fmt, N, K, seed=2)
    rng = np.random.default_rng(4)
    ids = np.array([3, 200, 77], np.int32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    dw = _t(w)
    out16 = torch.zeros((3, K), dtype=torch.int16, device="cuda")
    parts = torch.zeros((3, K // 4), dtype=torch.float32, device="cuda")
    h = ops.embed(m, _t(ids), epilogue=L.Epilogue(
        mode=L.EPI_STORE, out16=out16.data_ptr(), ld_out16=K, out16_w=dw.data_ptr(),
        norm_mult_out=32.0, parts_out=parts.data_ptr(), ld_parts_out=K // 4)).cpu().numpy()
    dense = dense_of(m)
    assert np.array_equal(h, dense[ids])
    assert np.array_equal(_h(out16), O.halves_to_f32(O.f32_to_h2(h * w / np.float32(32))))
    assert np.allclose(parts.cpu().numpy(), (h.astype(np.float64).reshape(3, -1, 4) ** 2).sum(-1),
                       rtol=1e-6)
