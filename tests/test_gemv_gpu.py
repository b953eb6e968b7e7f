"""Decode / few-token GEMV against the oracle (fp64 over the reference's
dequantized weights): rel-L2 <= 1e-3, the parity bar (in practice
~1e-6: products are exact and sums float32)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gguf_q4_0, nbits, random_q4_k_bytes, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _x16(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float32)
    h = O.f32_to_h2(x)
    return h, O.halves_to_f32(h)


def _q4_0(rng, N, K):
    from webgllm_amd import ops
    src = gguf_q4_0(rng, N, K)
    want = O.QuantMatrix(N, K, False)
    O.pack_q4_0(want, 0, src, N)
    return ops.Q4Matrix.from_q4_0(ops.to_device_bytes(src), N, K), want


def _nbits(rng, N, K):
    from webgllm_amd import ops
    q, s, z = nbits(rng, N, K)
    want = O.QuantMatrix(N, K, True)
    O.pack_nbits(want, 0, q, s, z, N)
    m = ops.Q4Matrix.from_nbits(ops.to_device_bytes(q), ops.to_device_bytes(s),
                                ops.to_device_bytes(z), N, K)
    return m, want


def _q4_k(rng, N, K, native=False, records=False):
    from webgllm_amd import ops
    src = random_q4_k_bytes(rng, N, K, zero_scale_every=5)
    want = O.QuantMatrix(N, K, "halves")
    O.pack_q4_k(want, 0, src, N)
    return ops.Q4Matrix.from_q4_k(ops.to_device_bytes(src), N, K, native=native,
                                  records=records), want


MAKERS = {"q4_0": _q4_0, "nbits": _nbits, "q4_k": _q4_k,
          "q4_k_native": lambda rng, N, K: _q4_k(rng, N, K, native=True),
          "q4_k_records": lambda rng, N, K: _q4_k(rng, N, K, native=False, records=True)}


@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k", "q4_k_native", "q4_k_records"])
@pytest.mark.parametrize("N,K", [(2048, 2048), (896, 896), (4864, 896), (896, 4864), (64, 32),
                                 (1024, 4096)])
@pytest.mark.parametrize("M", [1, 5])
def test_gemv_matches_oracle(hip, fmt, N, K, M):
    from webgllm_amd import ops
    if fmt.startswith("q4_k") and K % 256:
        pytest.skip("Q4_K rows are super-blocks of 256")
    rng = np.random.default_rng(N * 31 + K + M)
    m, want_m = MAKERS[fmt](rng, N, K)
    h, xf = _x16(rng, M, K)
    y = ops.gemv(m, torch.from_numpy(h.view(np.int16)).cuda())
    torch.cuda.synchronize()
    want = O.gemv_f64(want_m, xf)
    err = rel_l2(y.cpu().numpy(), want)
    print(f"{fmt} N={N} K={K} M={M} rel-L2 {err:.2e}")
    assert err <= TOL
    # every row's greedy pick agrees
    got = y.cpu().numpy()
    for t in range(M):
        assert O.argmax(got[t])[0] == O.argmax(want[t].astype(np.float32))[0]


@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 7, 8])
def test_gemv_every_row_count(hip, M):
    from webgllm_amd import ops
    rng = np.random.default_rng(100 + M)
    m, want_m = _nbits(rng, 256, 1024)
    h, xf = _x16(rng, M, 1024)
    y = ops.gemv(m, torch.from_numpy(h.view(np.int16)).cuda())
    assert rel_l2(y.cpu().numpy(), O.gemv_f64(want_m, xf)) <= TOL


def test_gemv_epilogue_residual_and_scale(hip):
    from webgllm_amd import ops
    rng = np.random.default_rng(7)
    N, K, M = 512, 1024, 3
    m, want_m = _q4_0(rng, N, K)
    h, xf = _x16(rng, M, K)
    res = rng.standard_normal((M, N)).astype(np.float32)
    rs = np.array([0.5, 2.0, -1.0], np.float32)
    y = torch.from_numpy(res.copy()).cuda()
    ops.gemv(m, torch.from_numpy(h.view(np.int16)).cuda(), out=y, residual=y,
             row_scale=torch.from_numpy(rs).cuda())
    want = res + rs[:, None] * O.gemv_f64(want_m, xf)
    assert rel_l2(y.cpu().numpy(), want) <= 1e-5


def test_gemv_closed_forms(hip):
    from webgllm_amd import ops
    rng = np.random.default_rng(9)
    N, K = 128, 512
    m, want_m = _q4_0(rng, N, K)
    dense = want_m.dense()
    # one-hot x -> column k of W (exact up to float32)
    x = np.zeros((1, K), np.float32)
    x[0, 77] = 1
    y = ops.gemv(m, torch.from_numpy(O.f32_to_h2(x).view(np.int16)).cuda())
    assert np.allclose(y.cpu().numpy()[0], dense[:, 77], rtol=0, atol=1e-7)
    # x = 1 -> row sums
    y = ops.gemv(m, torch.ones((1, K), dtype=torch.float16, device="cuda"))
    assert rel_l2(y.cpu().numpy()[0], dense.astype(np.float64).sum(1)) < 1e-6
    # all nibbles at the zero point -> 0, up to float32 rounding of the two
    # block sums (sum q a and z sum a are formed in different orders)
    z = ops.Q4Matrix(N, K)
    z.quants.fill_(0x88)
    z.scales.fill_(0x3C00)
    x = torch.randn((2, K), device="cuda").half()
    y = ops.gemv(z, x)
    bound = 8 * x.float().abs().sum(1, keepdim=True) * 2 ** -20
    assert torch.all(y.abs() <= bound)


@pytest.fixture(params=["mfma", "vector"])
def few_path(request):
    """The few-token GEMV on MFMA for every row count (knob 2), or on the
    vector kernels only (knob 0)."""
    from webgllm_amd import lib as L
    old = L.tuning_get("gemv_mfma")
    L.tuning_set("gemv_mfma", 2 if request.param == "mfma" else 0)
    yield request.param
    L.tuning_set("gemv_mfma", old)


@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k", "q4_k_records"])
@pytest.mark.parametrize("N,K", [(2048, 2048), (36, 96), (100, 4096), (4864, 896), (512, 32),
                                 (264, 1568), (2048, 8192)])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_gemv_paths_match_oracle(hip, few_path, fmt, N, K, M):
    """Both few-token paths within rel-L2 1e-5 of the float64 oracle:
    partial last tiles (N = 36, 100, 264: row groups that are not a
    multiple of 4), an odd block count (K = 96, 1568), a single block,
    K split over 8 waves (4096), and K = 8192, which the MFMA kernel leaves
    to the vector one."""
    from webgllm_amd import ops
    if fmt.startswith("q4_k") and K % 256:
        pytest.skip("Q4_K rows are super-blocks of 256")
    rng = np.random.default_rng(N * 7 + K * 3 + M)
    m, want_m = MAKERS[fmt](rng, N, K)
    h, xf = _x16(rng, M, K)
    y = ops.gemv(m, torch.from_numpy(h.view(np.int16)).cuda())
    torch.cuda.synchronize()
    err = rel_l2(y.cpu().numpy(), O.gemv_f64(want_m, xf))
    print(f"{few_path} {fmt} N={N} K={K} M={M} rel-L2 {err:.2e}")
    # (Q4_K records weigh a block's zero term as dmin m, not packQ4_K's d'
    # half(dmin m / d'): within a half's rounding of it)
    assert err <= (1e-3 if fmt == "q4_k_records" else 1e-4)
