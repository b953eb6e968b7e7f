"""Q4_K matrices kept as Q4_K records (WG_ZERO_Q4K): packQ4_K's quants with
the file's d, dmin and 6-bit scales and mins, 0.5625 bytes a weight.

- The repack: the records and quants put back into Q4_K super-blocks and
  packed by the oracle's packQ4_K (src/repack.ts:100-168) give the oracle's
  packing of the file's bytes, and the quants are the half-zero-point
  repack's, bit for bit (constant sub-blocks, extreme d and dmin, src_rows).
- Dequant, the embedding and the prefill GEMM rebuild packQ4_K's halves:
  bit for bit what the half-zero-point matrix of the same rows gives.
- The GEMVs weigh a block as half(d sc) q - dmin m: against the float64
  oracle in test_gemv_gpu; here against the half-zero-point GEMV of the
  same rows, every kernel form (stream, few-token, row-group), within
  the zero term's half rounding."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import random_q4_k_bytes, rel_l2

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _pair(rng, N, K, zero_every=5, extreme=False, src_rows=None):
    from webgllm_amd import ops
    src = random_q4_k_bytes(rng, N, K, zero_scale_every=zero_every, extreme=extreme)
    dsrc = ops.to_device_bytes(src)
    sr = None if src_rows is None else torch.tensor(src_rows, dtype=torch.int32, device="cuda")
    f16 = ops.Q4Matrix.from_q4_k(dsrc, N, K, native=False, src_rows=sr)
    rec = ops.Q4Matrix.from_q4_k(dsrc, N, K, native=False, src_rows=sr, records=True)
    torch.cuda.synchronize()
    return src, f16, rec


@pytest.mark.parametrize("N,K,extreme,zero_every,order", [
    (8, 256, False, 1, False), (64, 1024, True, 3, False), (1024, 4096, False, 7, True),
    (4, 512, True, 1, True)])
def test_repack_records_against_packq4k(hip, N, K, extreme, zero_every, order):
    from webgllm_amd import lib as L
    rng = np.random.default_rng(N + K)
    src_rows = rng.permutation(N).tolist() if order else None
    src, f16, rec = _pair(rng, N, K, zero_every, extreme, src_rows)
    assert rec.zero == L.ZERO_Q4K and rec.zeros is None
    assert rec.quants.numel() + rec.scales.numel() * 2 == N * K // 256 * 144
    # the stored rows: source row src_rows[i] at row i
    rows = np.asarray(src_rows if order else range(N))
    stored = src.reshape(N, -1)[rows].reshape(-1)
    want = O.QuantMatrix(N, K, "halves")
    O.pack_q4_k(want, 0, stored, N)
    back = O.q4k_from_records(_np(rec.quants), _np(rec.scales).view(np.uint8), N, K)
    got = O.QuantMatrix(N, K, "halves")
    O.pack_q4_k(got, 0, back.reshape(-1), N)
    assert np.array_equal(got.quants, want.quants)
    assert np.array_equal(got.scales, want.scales)
    assert np.array_equal(got.zero_halves, want.zero_halves)
    # the quants are the half-zero-point repack's (15s in constant blocks)
    assert np.array_equal(_np(rec.quants), _np(f16.quants))
    assert np.array_equal(_np(f16.quants).view(np.uint32), want.quants)


@pytest.mark.parametrize("N,K,extreme", [(64, 1024, False), (256, 2048, True), (4, 4096, False)])
def test_dequant_and_embedding_equal_the_half_zero_form(hip, N, K, extreme):
    from webgllm_amd import ops
    rng = np.random.default_rng(3 * N + K)
    _, f16, rec = _pair(rng, N, K, zero_every=2, extreme=extreme)
    a, b = f16.dequant(0, N), rec.dequant(0, N)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    ids = torch.tensor([0, N - 1, N // 2, -1, N, 3 % N], dtype=torch.int32, device="cuda")
    ea = ops.embed(f16, ids)
    eb = ops.embed(rec, ids)
    torch.cuda.synchronize()
    assert torch.equal(ea.view(torch.int32), eb.view(torch.int32))
    assert torch.equal(ea[0].view(torch.int32), a[0].view(torch.int32)) and not ea[3].any()


@pytest.mark.parametrize("N,K,M", [(256, 1024, 64), (4096, 4096, 300), (1024, 14336, 40)])
def test_gemm_equals_the_half_zero_form(hip, N, K, M):
    from webgllm_amd import ops
    rng = np.random.default_rng(N + K + M)
    _, f16, rec = _pair(rng, N, K, zero_every=4)
    a = torch.from_numpy(O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
                         .view(np.int16)).cuda()
    ya = ops.gemm(f16, a)
    yb = ops.gemm(rec, a, kept=False)  # the library's rebuild each call
    yc = ops.gemm(rec, a)              # the kept halves (wg_q4k_record_halves)
    torch.cuda.synchronize()
    assert torch.equal(ya.view(torch.int32), yb.view(torch.int32))
    assert torch.equal(ya.view(torch.int32), yc.view(torch.int32))
    sa = ops.gemm_swiglu(f16, a)
    sb = ops.gemm_swiglu(rec, a, kept=False)
    sc = ops.gemm_swiglu(rec, a)
    torch.cuda.synchronize()
    assert torch.equal(sa.view(torch.int16), sb.view(torch.int16))
    assert torch.equal(sa.view(torch.int16), sc.view(torch.int16))
    # the kept halves are the half-zero-point repack's arrays, made again
    # after the rows are repacked
    rec.prompt_desc()
    assert torch.equal(rec._halves[0], f16.scales) and torch.equal(rec._halves[1], f16.zeros)
    rec.repack_q4_k(0, 4, ops.to_device_bytes(np.zeros(K // 256 * 144 * 4, np.uint8)))
    assert rec._halves is None
    rec.prompt_desc()
    torch.cuda.synchronize()
    # (all-zero super-blocks: constant blocks of scale -0)
    assert not (rec._halves[0][:K // 32 * 4] & 0x7FFF).any()


def test_gemm_refuses_capture(hip):
    from webgllm_amd import ops
    rng = np.random.default_rng(9)
    _, _, rec = _pair(rng, 256, 512)
    a = torch.zeros((64, 512), dtype=torch.int16, device="cuda")
    out = torch.zeros((64, 256), device="cuda")
    st = torch.cuda.Stream()
    raised = None
    with torch.cuda.stream(st):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            try:
                ops.gemm(rec, a, out=out, kept=False)
            except Exception as e:  # refused before any launch: nothing captured
                raised = e
            out.zero_()  # (a graph of one fill, not an empty one)
    torch.cuda.synchronize()
    assert raised is not None and "under capture" in str(raised)


@pytest.fixture(params=["mfma", "vector"])
def few_path(request):
    from webgllm_amd import lib as L
    old = L.tuning_get("gemv_mfma")
    L.tuning_set("gemv_mfma", 2 if request.param == "mfma" else 0)
    yield request.param
    L.tuning_set("gemv_mfma", old)


@pytest.mark.parametrize("N,K", [(2048, 2048), (6144, 4096), (4096, 14336), (100, 4096),
                                 (28672, 4096), (264, 18432)])
@pytest.mark.parametrize("M", [1, 2, 5, 8])
def test_gemv_close_to_the_half_zero_form(hip, few_path, N, K, M):
    """Every GEMV form the records take (the streaming kernel at 1-2 rows,
    the few-token one at 3-8, the row-group kernel past 256 blocks a row;
    the MFMA form declines them) against the half-zero-point matrix's
    GEMV: the same quants and d', a zero term within a half's rounding."""
    from webgllm_amd import ops
    rng = np.random.default_rng(N + K * 7 + M)
    _, f16, rec = _pair(rng, N, K, zero_every=6)
    x = torch.from_numpy(O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
                         .view(np.int16)).cuda()
    ya = ops.gemv(f16, x)
    yb = ops.gemv(rec, x)
    torch.cuda.synchronize()
    err = rel_l2(_np(yb), _np(ya))
    print(f"{few_path} N={N} K={K} M={M} rel-L2 {err:.2e}")
    assert err <= 2e-4


@pytest.mark.parametrize("N,K", [(2048, 4096), (6144, 2048), (4096, 14336)])
def test_few_rows_take_the_kept_halves(hip, N, K):
    """With its halves kept, a records matrix's 3-8-row GEMVs at K <= 4096
    run on the half-zero-point form (the MFMA kernel): its bits; deeper
    rows and 1-2 rows stay on the records."""
    from webgllm_amd import ops
    rng = np.random.default_rng(N + K)
    _, f16, rec = _pair(rng, N, K, zero_every=5)
    rec.prompt_desc()
    for M in (1, 5, 8):
        x = torch.from_numpy(O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
                             .view(np.int16)).cuda()
        ya, yb = ops.gemv(f16, x), ops.gemv(rec, x)
        torch.cuda.synchronize()
        if M >= 3 and K <= 4096:
            assert torch.equal(ya.view(torch.int32), yb.view(torch.int32)), M
        else:
            assert rel_l2(_np(yb), _np(ya)) <= 2e-4, M
