"""Prefill GEMM on MFMA against the oracle. Two references: the exact
dequantized weights in float64 (the rel-L2 <= 1e-3 parity bar), and
the weights rounded to halves the way the reference's dequantOut stores them
(src/gpu/kernels.ts:436-597), which the GEMM must match to float32
accumulation error."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import nbits, rel_l2
from tests.model_oracle import dense_of

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _matrix(fmt, N, K, seed):
    from webgllm_amd import engine as E
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.__new__(E.Weights)
    w.shape, w.device = shape, "cuda"
    w.g = torch.Generator(device="cuda")
    w.g.manual_seed(seed)
    return w.matrix(N, K)


def _check(m, M, seed, residual=False):
    from webgllm_amd import ops
    rng = np.random.default_rng(seed)
    K = m.K
    a = rng.standard_normal((M, K)).astype(np.float32)
    a16 = O.f32_to_h2(a)
    af = O.halves_to_f32(a16).astype(np.float64)
    W = dense_of(m)
    res = rng.standard_normal((M, m.N)).astype(np.float32) if residual else None
    out = _t(res.copy()) if residual else None
    got = ops.gemm(m, _t(a16.view(np.int16)), out=out,
                   residual=out if residual else None).cpu().numpy()
    base = res.astype(np.float64) if residual else 0.0
    want = base + af @ W.astype(np.float64).T
    # dequantOut's halves: (q - z) d rounded once to half
    W16 = O.halves_to_f32(O.f32_to_h2(W)).astype(np.float64)
    want16 = base + af @ W16.T
    return rel_l2(got, want), rel_l2(got, want16)


@pytest.mark.parametrize("N", [4096, 14336])
def test_c2_matmulnbits_prefill(hip, N):
    # 512 tokens x 4096 -> N, MatMulNBits with u8 zero points (the prefill workload)
    m = _matrix("nbits", N, 4096, seed=N)
    e, e16 = _check(m, 512, seed=1)
    print(f"N={N} rel-L2 vs exact {e:.2e}, vs half-rounded weights {e16:.2e}")
    assert e <= 1e-3
    assert e16 <= 1e-5


@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k_rowgroup", "q4_k_records", "q8_0",
                                 "q8"])
@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (37, 192, 128), (200, 512, 1024),
                                   (128, 1024, 2048)])
def test_gemm_shapes_and_formats(hip, fmt, M, N, K):
    if fmt.startswith("q4_k") and K % 256:
        pytest.skip("Q4_K rows are super-blocks of 256")
    m = _matrix(fmt, N, K, seed=M + N)
    e, e16 = _check(m, M, seed=M)
    assert e <= 1e-3
    # fractional zero points dequantize through float32 like the reference
    assert e16 <= 1e-5


def test_gemm_residual_in_place(hip):
    m = _matrix("q4_0", 256, 512, seed=3)
    e, e16 = _check(m, 64, seed=4, residual=True)
    assert e16 <= 1e-5


def test_gemm_rejects(hip):
    from webgllm_amd import ops, lib as L
    m = _matrix("q4_0", 96, 64, seed=1)   # N not a multiple of 64
    with pytest.raises(L.WgError, match="multiple of 64"):
        ops.gemm(m, torch.zeros((4, 64), dtype=torch.float16, device="cuda"))
    for fmt in ("q4_k", "q6_k"):
        m2 = _matrix(fmt, 64, 256, seed=1)
        with pytest.raises(L.WgError, match="row-group"):
            ops.gemm(m2, torch.zeros((4, 256), dtype=torch.float16, device="cuda"))


def test_gemm_8bit_c2_shape(hip):
    """An 8-bit gate|up-sized matrix at 512 rows (the prompt batches of a
    Q8_0 or requantized GGUF model): within float32 summation of the
    half-rounded weights."""
    m = _matrix("q8", 14336, 4096, seed=9)
    e, e16 = _check(m, 512, seed=2)
    assert e <= 1e-3
    assert e16 <= 1e-5


@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k_rowgroup", "q4_k_records", "q8_0"])
def test_gemm_every_tile(hip, fmt, tile):
    """Each tile shape (64 x 128, 128 x 128, 128 x 256), forced through the
    gemm_tile knob, on ragged rows (M = 200 leaves a partial 128-row tile)."""
    from webgllm_amd import lib as L
    m = _matrix(fmt, 512, 1024, seed=tile)
    L.tuning_set("gemm_tile", tile)
    try:
        e, e16 = _check(m, 200, seed=tile + 7)
    finally:
        L.tuning_set("gemm_tile", 0)
    assert e <= 1e-3
    assert e16 <= 1e-5


def test_gemm_column_map(hip):
    """col_of sends stored row n to output column col_of[n]: the mapped
    product equals the plain one with its columns permuted (bit for bit);
    an entry outside 0..N-1 leaves nothing written."""
    from webgllm_amd import ops
    N, K, M = 256, 512, 40
    m = _matrix("nbits", N, K, seed=4)
    rng = np.random.default_rng(3)
    a = _t(O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32)).view(np.int16))
    plain = ops.gemm(m, a).cpu().numpy()
    perm = rng.permutation(N).astype(np.int32)
    mapped = ops.gemm(m, a, col_of=_t(perm)).cpu().numpy()
    assert np.array_equal(mapped[:, perm], plain)
    perm[7] = N + 5  # out of range: column perm-less, stays as it was
    out = torch.full((M, N), 123.0, device="cuda")
    ops.gemm(m, a, out=out, col_of=_t(perm))
    got = out.cpu().numpy()
    ok = np.ones(N, bool)
    ok[7] = False
    assert np.array_equal(got[:, perm[ok]], plain[:, ok])
    missing = np.setdiff1d(np.arange(N), perm[ok])
    assert (got[:, missing] == 123.0).all()


@pytest.mark.parametrize("fmt,tile", [("q4_k_rowgroup", 0), ("q4_0", 1), ("nbits", 2),
                                      ("q8_0", 3), ("q8", 0)])
@pytest.mark.parametrize("M", [1, 77, 300])
def test_gemm_swiglu_equals_gemm_then_swiglu(hip, fmt, tile, M):
    """The fused gate|up GEMM + SwiGLU writes, bit for bit, what the GEMM
    (through the matrix's column map) then wg_swiglu write, with a row
    scale, on every tile shape and ragged row counts."""
    from webgllm_amd import engine as E, lib as L, ops
    F, K = 768, 1024
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.blank(shape, seed=M)
    m = w.matrix(2 * F, K, E.gate_up_row_order(F))
    rng = np.random.default_rng(M)
    a = _t(O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32)).view(np.int16))
    rs = _t(rng.uniform(0.5, 2.0, M).astype(np.float32))
    col = _t(np.asarray(m.row_order, np.int32))
    L.tuning_set("gemm_tile", tile)
    try:
        gu = ops.gemm(m, a, col_of=col, row_scale=rs)
        want = ops.swiglu(gu).cpu().numpy().view(np.uint16)
        got = ops.gemm_swiglu(m, a, row_scale=rs).cpu().numpy().view(np.uint16)
    finally:
        L.tuning_set("gemm_tile", 0)
    assert np.array_equal(got, want)


def test_gemm_swiglu_rejects(hip):
    from webgllm_amd import lib as L
    m = _matrix("q4_0", 128, 64, seed=1)
    lib = L.load()
    rc = lib.wg_q4_gemm_swiglu(C.byref(m.desc), 0x10000, 4, 64, 0x20000, 32, None, None)
    assert rc == -1 and "N / 2" in L.last_error()


@pytest.mark.parametrize("tile,ks", [(1, 2), (1, 4), (1, 8), (2, 2), (2, 4), (3, 2), (3, 4), (3, 8)])
@pytest.mark.parametrize("fmt", ["nbits", "q4_k_rowgroup", "q8"])
def test_gemm_split_k(hip, fmt, tile, ks):
    """K split 2, 4 or 8 ways (forced through gemm_splits) on each tile shape
    and ragged rows: within float32 summation of the half-rounded weights,
    the same bits on every repeat (the pairwise tree does not depend on
    which split ends last), and a residual added in place."""
    from webgllm_amd import lib as L, ops
    m = _matrix(fmt, 512, 2048, seed=ks + tile)
    L.tuning_set("gemm_tile", tile)
    L.tuning_set("gemm_splits", ks)
    try:
        e, e16 = _check(m, 200, seed=ks)
        er, er16 = _check(m, 77, seed=ks + 1, residual=True)
        rng = np.random.default_rng(ks)
        a = _t(O.f32_to_h2(rng.standard_normal((130, m.K)).astype(np.float32)).view(np.int16))
        first = ops.gemm(m, a)
        repeats = [ops.gemm(m, a) for _ in range(20)]
    finally:
        L.tuning_set("gemm_tile", 0)
        L.tuning_set("gemm_splits", 0)
    assert e <= 1e-3 and er <= 1e-3
    assert e16 <= 1e-5 and er16 <= 1e-5
    for r in repeats:
        assert torch.equal(r, first)


def test_gemm_split_k_first_launches(hip):
    """Every launch right after the split layout changes (tile shape, split
    count) equals the launch after it, bit for bit, and the unsplit result
    to float32 rounding: the first launch of a layout reads no partial of
    an earlier one."""
    from webgllm_amd import lib as L, ops
    m = _matrix("nbits", 4096, 4096, seed=6)
    rng = np.random.default_rng(6)
    a = _t(O.f32_to_h2(rng.standard_normal((512, 4096)).astype(np.float32)).view(np.int16))
    L.tuning_set("gemm_splits", 1)
    try:
        unsplit = ops.gemm(m, a)
        for tile, ks in [(2, 4), (1, 2), (2, 4), (2, 2), (1, 4), (2, 8), (1, 8), (3, 2), (3, 4),
                         (2, 4)]:
            L.tuning_set("gemm_tile", tile)
            L.tuning_set("gemm_splits", ks)
            c1 = ops.gemm(m, a)
            c2 = ops.gemm(m, a)
            assert torch.equal(c1, c2), (tile, ks)
            assert rel_l2(c1.cpu().numpy(), unsplit.cpu().numpy()) <= 1e-6, (tile, ks)
    finally:
        L.tuning_set("gemm_tile", 0)
        L.tuning_set("gemm_splits", 0)


def test_gemm_split_k_prefill_shape_in_graph(hip):
    """The 512 x 4096 -> 4096 prefill GEMM (split by default when eager)
    captured in a graph runs unsplit: every replay equals the unsplit result
    bit for bit, also with eager split launches on the capture stream
    between replays and after the stream's workspace has grown, and when
    replayed on another stream; the eager launches equal one another."""
    from webgllm_amd import lib as L, ops
    m = _matrix("nbits", 4096, 4096, seed=5)
    rng = np.random.default_rng(5)
    a = _t(O.f32_to_h2(rng.standard_normal((512, 4096)).astype(np.float32)).view(np.int16))
    L.tuning_set("gemm_splits", 1)
    try:
        unsplit = ops.gemm(m, a)
    finally:
        L.tuning_set("gemm_splits", 0)
    s = torch.cuda.Stream()
    out = torch.empty((512, 4096), device="cuda")
    with torch.cuda.stream(s):
        eager = ops.gemm(m, a)  # this stream's workspace
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ops.gemm(m, a, out=out)
        for i in range(4):
            out.fill_(float("nan"))
            g.replay()
            other = ops.gemm(m, a)
            torch.cuda.synchronize()
            assert torch.equal(out, unsplit), i
            assert torch.equal(other, eager), i
        # a 4-way split needs more room: the workspace grows (is freed and
        # allocated again)
        L.tuning_set("gemm_splits", 4)
        try:
            four = ops.gemm(m, a)
        finally:
            L.tuning_set("gemm_splits", 0)
        torch.cuda.synchronize()
        assert rel_l2(four.cpu().numpy(), unsplit.cpu().numpy()) <= 1e-6
    out.fill_(float("nan"))
    g.replay()  # on the current stream, not the capture stream
    torch.cuda.synchronize()
    assert torch.equal(out, unsplit)
    assert rel_l2(eager.cpu().numpy(), unsplit.cpu().numpy()) <= 1e-6


@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k_rowgroup", "q8"])
@pytest.mark.parametrize("K,ks", [(64, 1), (256, 2), (2048, 1), (2048, 4)])
@pytest.mark.parametrize("M", [1, 200, 640])
def test_gemm_pingpong_same_bits(hip, fmt, K, ks, M):
    """The 128 x 256 tile's two schedules, the wave groups half a step apart
    (gemm_pingpong 1) and in lock-step (0), add the same products in the
    same order: the same bits, plain and fused with SwiGLU, at one K step,
    fewer steps than the ring's stages, and split K (test_gemm_every_tile
    holds the default, lock-step, form to the oracle)."""
    from webgllm_amd import engine as E, lib as L, ops
    if fmt == "q4_k_rowgroup" and K % 256:
        pytest.skip("Q4_K rows are whole 256-weight super-blocks")
    N = 512
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.blank(shape, seed=M + K)
    m = w.matrix(N, K, E.gate_up_row_order(N // 2))
    rng = np.random.default_rng(M + K + ks)
    a = _t(O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32)).view(np.int16))
    got = {}
    L.tuning_set("gemm_tile", 3)
    L.tuning_set("gemm_splits", ks)
    try:
        for pp in (1, 0):
            L.tuning_set("gemm_pingpong", pp)
            got[pp] = (ops.gemm(m, a), ops.gemm_swiglu(m, a))
            torch.cuda.synchronize()
    finally:
        L.tuning_set("gemm_pingpong", 0)
        L.tuning_set("gemm_tile", 0)
        L.tuning_set("gemm_splits", 0)
    assert torch.equal(got[1][0].view(torch.int32), got[0][0].view(torch.int32))
    assert torch.equal(got[1][1].view(torch.int16), got[0][1].view(torch.int16))
