"""Load-time repacking and dequant on the GPU against the oracle: bit-exact
(the reference's packers, src/repack.ts, and matrixRow, :865-891)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gguf_q4_0, nbits, random_q4_0_bytes, random_q4_k_bytes

pytestmark = pytest.mark.gpu


def _np(t):
    return t.cpu().numpy()


def _same_floats(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("N,K,perm", [(8, 64, False), (64, 256, True), (2048, 2048, False)])
def test_repack_q4_0_bit_exact(hip, N, K, perm):
    from webgllm_amd import ops
    rng = np.random.default_rng(N + K)
    src = random_q4_0_bytes(rng, N, K) if N < 2048 else gguf_q4_0(rng, N, K)
    order = rng.permutation(N).astype(np.int32) if perm else None
    want = O.QuantMatrix(N, K, False)
    O.pack_q4_0(want, 0, src, N, order)
    m = ops.Q4Matrix(N, K)
    m.repack_q4_0(0, N, ops.to_device_bytes(src),
                  torch.from_numpy(order).cuda() if perm else None)
    assert np.array_equal(_np(m.quants).view(np.uint32), want.quants)
    assert np.array_equal(_np(m.scales).view(np.uint16), want.scales)
    rows = slice(0, min(N, 256))
    _same_floats(_np(m.dequant(0, rows.stop)), want.dense()[rows])


def test_repack_q4_0_row_offset(hip):
    from webgllm_amd import ops
    rng = np.random.default_rng(3)
    src = random_q4_0_bytes(rng, 4, 128)
    want = O.QuantMatrix(12, 128, False)
    O.pack_q4_0(want, 4, src, 4)
    m = ops.Q4Matrix(12, 128)
    m.repack_q4_0(4, 4, ops.to_device_bytes(src))
    assert np.array_equal(_np(m.quants).view(np.uint32), want.quants)
    _same_floats(_np(m.dequant()), want.dense())


@pytest.mark.parametrize("N,K,zp", [(16, 96, True), (64, 512, False), (4096, 4096, True)])
def test_repack_nbits_bit_exact(hip, N, K, zp):
    from webgllm_amd import ops
    rng = np.random.default_rng(K)
    quant, scales, zpk = nbits(rng, N, K, with_zp=zp)
    want = O.QuantMatrix(N, K, True)
    O.pack_nbits(want, 0, quant, scales, zpk, N)
    m = ops.Q4Matrix.from_nbits(ops.to_device_bytes(quant), ops.to_device_bytes(scales),
                                ops.to_device_bytes(zpk) if zp else None, N, K)
    assert np.array_equal(_np(m.quants).view(np.uint32), want.quants)
    assert np.array_equal(_np(m.scales).view(np.uint16), want.scales)
    if zp:
        assert np.array_equal(_np(m.zeros), want.zeros)
    rows = min(N, 128)
    got = _np(m.dequant(0, rows))
    _same_floats(got, want.dense()[:rows])
    # and against the raw-rows dequant of load-onnx.ts:471-501
    for n in (0, rows - 1):
        _same_floats(got[n], O.dequantize_nbits_row(K, quant, scales, zpk, n))


@pytest.mark.parametrize("N,K,extreme,zero_every", [(8, 512, False, 0), (8, 256, False, 1),
                                                    (64, 1024, True, 3), (1024, 4096, False, 7)])
def test_repack_q4_k_bit_exact(hip, N, K, extreme, zero_every):
    from webgllm_amd import ops
    rng = np.random.default_rng(N * 7 + K)
    src = random_q4_k_bytes(rng, N, K, zero_scale_every=zero_every, extreme=extreme)
    want = O.QuantMatrix(N, K, "halves")
    O.pack_q4_k(want, 0, src, N)
    dsrc = ops.to_device_bytes(src)
    m = ops.Q4Matrix.from_q4_k(dsrc, N, K, native=False)
    assert np.array_equal(_np(m.quants).view(np.uint32), want.quants)
    assert np.array_equal(_np(m.scales).view(np.uint16), want.scales)
    assert np.array_equal(_np(m.zeros).view(np.uint16), want.zero_halves)
    rows = min(N, 128)
    dense = want.dense()[:rows]
    _same_floats(_np(m.dequant(0, rows)), dense)
    # The native super-block layout rebuilds the same (d', z') in registers.
    nat = ops.Q4Matrix.from_q4_k(dsrc, N, K, native=True)
    _same_floats(_np(nat.dequant(0, rows)), dense)
