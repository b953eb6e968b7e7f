"""8-bit and Q6_K matrices through the C-ABI: the GPU packers and quantizer
byte-exact against the oracle, the dequant bit-exact (the reference's own
Q6_K vectors included), and the GEMV against the reference's float32 block
forms and a float64 product."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import encode_q6_k, rel_l2

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _np(t):
    return t.detach().cpu().numpy()


def _q8_0_bytes(rng, rows, K):
    b = rng.integers(0, 256, rows * (K // 32) * 34, dtype=np.uint8).reshape(-1, 34)
    d = rng.uniform(1e-4, 3e-3, b.shape[0]).astype(np.float16).view(np.uint16)
    b[:, 0], b[:, 1] = d & 255, d >> 8
    return b.reshape(-1)


def _q6_k_bytes(rng, rows, K):
    b = rng.integers(0, 256, rows * (K // 256) * 210, dtype=np.uint8).reshape(-1, 210)
    d = rng.uniform(1e-5, 1e-4, b.shape[0]).astype(np.float16).view(np.uint16)
    b[:, 208], b[:, 209] = d & 255, d >> 8
    return b.reshape(-1)


def _oracle_of(m):
    from webgllm_amd import lib as L
    wm = O.WideMatrix(m.N, m.K, 8 if m.layout == L.LAYOUT_Q8 else 6)
    wm.quants[:] = _np(m.quants)
    wm.scales[:] = _np(m.scales).view(np.uint16)
    return wm


@pytest.mark.parametrize("N,K", [(8, 32), (64, 4096), (36, 1056)])
def test_repack_q8_0_matches_oracle(hip, N, K):
    from webgllm_amd import lib as L, ops
    rng = np.random.default_rng(N + K)
    src = _q8_0_bytes(rng, N + 8, K)
    perm = rng.permutation(N + 8)[:N // 2].astype(np.int32)
    m = ops.Q4Matrix(N, K, L.LAYOUT_Q8)
    m.repack_q8_0(0, N // 2, _t(src), _t(perm))
    m.repack_q8_0(N // 2, N // 2, _t(src))
    torch.cuda.synchronize()
    want = O.WideMatrix(N, K, 8)
    O.pack_q8_0(want, 0, src, N // 2, src_rows=perm)
    O.pack_q8_0(want, N // 2, src, N // 2)
    assert np.array_equal(_np(m.quants), want.quants)
    assert np.array_equal(_np(m.scales).view(np.uint16), want.scales)
    # matrixRow, bit-exact, against dequantizeQ8_0 of the source rows
    rows = O.dequantize_q8_0(src, N + 8, K)
    got = _np(m.dequant())
    assert np.array_equal(got[:N // 2], rows[perm])
    assert np.array_equal(got[N // 2:], rows[:N // 2])


def _edge_rows(K):
    v = np.random.default_rng(7).standard_normal((8, K)).astype(np.float32) * 0.05
    v[0, :8] = [127, 2.5, -2.5, 0.49, -0.5, 126.6, -127, 3.0]
    v[1, :32] = 0.0
    v[1, 32] = np.nan
    v[1, 64] = np.inf
    v[1, 65] = -np.inf
    tiny = np.float32(127 * 1.25 * 2.0 ** -24)
    v[2, :3] = [tiny, -tiny, tiny / 2]
    v[2, 32:64] = np.float32(2.0 ** -30)  # max / 127 rounds to a zero half
    v[3, :32] = 70000.0 * 127  # max / 127 overflows to an infinite half
    v[3, 1] = -1.0
    return v


@pytest.mark.parametrize("N,K", [(8, 128), (128, 2048)])
def test_quantize_q8_matches_oracle(hip, N, K):
    from webgllm_amd import lib as L, ops
    v = np.random.default_rng(K).standard_normal((N, K)).astype(np.float32) * 0.03
    v[:8] = _edge_rows(K)
    m = ops.Q4Matrix(N, K, L.LAYOUT_Q8)
    m.quantize_q8(4, N - 4, _t(v[4:]))
    m.quantize_q8(0, 4, _t(v[:4]))
    torch.cuda.synchronize()
    want = O.WideMatrix(N, K, 8)
    O.quantize_q8(want, 4, v[4:])
    O.quantize_q8(want, 0, v[:4])
    assert np.array_equal(_np(m.scales).view(np.uint16), want.scales)
    assert np.array_equal(_np(m.quants), want.quants)


@pytest.mark.parametrize("N,K", [(8, 256), (40, 4096), (12, 2816)])
def test_repack_q6_k_matches_oracle(hip, N, K):
    from webgllm_amd import lib as L, ops
    rng = np.random.default_rng(N * K)
    src = _q6_k_bytes(rng, N + 4, K)
    perm = rng.permutation(N + 4)[:N].astype(np.int32)
    m = ops.Q4Matrix(N, K, L.LAYOUT_Q6K)
    m.repack_q6_k(0, N, _t(src), _t(perm))
    torch.cuda.synchronize()
    want = O.WideMatrix(N, K, 6)
    O.pack_q6_k(want, 0, src, N, src_rows=perm)
    assert np.array_equal(_np(m.quants), want.quants)
    assert np.array_equal(_np(m.scales).view(np.uint16), want.scales)
    rows = O.dequantize_q6_k(src, N + 4, K)
    assert np.array_equal(_np(m.dequant()), rows[perm])


@pytest.mark.parametrize("kind", ["expanded", "split"])
def test_q6_k_reference_vectors_on_the_device(hip, kind):
    """The reference's Q6_K layout vectors (src/q6-expanded.test.ts:7-46,
    src/q6-split.test.ts:6-28): packed on the GPU, dequantized and embedded
    there, equal to dequantizeQ6_K bit for bit."""
    from tests.test_oracle import _q6k_reference_matrix
    from webgllm_amd import ops
    rows, K, raw = _q6k_reference_matrix(kind)
    m = ops.Q4Matrix.from_q6_k(_t(raw), rows, K)
    want = O.dequantize_q6_k(raw, rows, K)
    assert np.array_equal(_np(m.dequant()), want)
    ids = np.array([rows - 1, 0, 5, rows, -1], np.int32)  # the last two outside: zeros
    h = _np(ops.embed(m, _t(ids)))
    assert np.array_equal(h[:3], want[ids[:3]])
    assert not h[3:].any()


def test_q6_k_known_codes_through_gemv(hip):
    """Codes packed by ggml's loop, times a one-hot activation, read back
    every weight d * sc * (q - 32) through the GEMV."""
    from webgllm_amd import ops
    rng = np.random.default_rng(2)
    N, K = 4, 256
    q = rng.integers(0, 64, (N, 256))
    sc = rng.integers(-128, 128, (N, 16))
    d_bits = np.array([O.to_half(v) for v in (1.0, 0.5, 0.25, 2.0)])
    m = ops.Q4Matrix.from_q6_k(_t(encode_q6_k(q, sc, d_bits)), N, K)
    eye = np.eye(8, K, dtype=np.float32)
    for k0 in range(0, K, 8):
        x16 = O.f32_to_h2(np.roll(eye, k0, axis=1))
        y = _np(ops.gemv(m, _t(x16.view(np.int16))))
        d = np.array([O.from_half(int(h)) for h in d_bits])
        want = (d[:, None] * sc[:, (k0 + np.arange(8)) // 16] * (q[:, k0:k0 + 8] - 32)).T
        assert np.array_equal(y, want.astype(np.float32))


def _wide(fmt, N, K, seed):
    from tests.test_epilogue_gpu import _matrix
    return _matrix(fmt, N, K, seed)


WIDE = ["q8_0", "q8", "q6_k"]


@pytest.mark.parametrize("fmt", WIDE)
@pytest.mark.parametrize("M", [1, 2, 3, 8])
@pytest.mark.parametrize("N,K", [(512, 1024), (256, 4096), (128, 14336), (1024, 2816)])
def test_gemv_wide_against_block_form_and_f64(hip, fmt, M, N, K):
    from webgllm_amd import ops
    if fmt == "q6_k" and K % 256:
        pytest.skip("Q6_K rows are whole super-blocks")
    m = _wide(fmt, N, K, seed=M + N)
    rng = np.random.default_rng(M + K)
    x16 = O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
    got = _np(ops.gemv(m, _t(x16.view(np.int16))))
    wm = _oracle_of(m)
    block = wm.matmul(x16)
    f64 = O.halves_to_f32(x16).astype(np.float64) @ wm.dense().astype(np.float64).T
    assert rel_l2(got, block) <= 1e-5
    assert rel_l2(got, f64) <= 1e-5
    assert np.max(np.abs(got - f64)) <= 1e-4 * np.abs(f64).max()


@pytest.mark.parametrize("fmt,K", [
    ("q8", 8192),     # 4 parts of 64 blocks
    ("q8", 16896),    # more blocks than 4 parts of 128: one wave per row group
    ("q6_k", 6144),   # 2 parts
    ("q6_k", 8448),   # 33 super-blocks: parts rounded to even chunk counts
    ("q6_k", 18432),  # 4 parts, 2 chunks a lane
])
@pytest.mark.parametrize("M", [1, 2])
def test_gemv_wide_launch_shapes(hip, fmt, K, M):
    """Every launch shape of the 1- and 2-token GEMV (K split into 1, 2 or 4
    parts, 1 or 2 chunks a lane, and the one-wave-per-row-group form)."""
    from webgllm_amd import ops
    N = 64
    m = _wide(fmt, N, K, seed=K)
    x16 = O.f32_to_h2(np.random.default_rng(K).standard_normal((M, K)).astype(np.float32))
    got = _np(ops.gemv(m, _t(x16.view(np.int16))))
    f64 = O.halves_to_f32(x16).astype(np.float64) @ _oracle_of(m).dense().astype(np.float64).T
    assert rel_l2(got, f64) <= 1e-5


@pytest.mark.parametrize("fmt", WIDE)
def test_embed_wide(hip, fmt):
    from webgllm_amd import ops
    N, K = 256, 1024
    m = _wide(fmt, N, K, seed=4)
    ids = np.array([255, 0, 17, 300, -2], np.int32)
    h = _np(ops.embed(m, _t(ids)))
    dense = _oracle_of(m).dense()
    assert np.array_equal(h[:3], dense[ids[:3]])
    assert not h[3:].any()
