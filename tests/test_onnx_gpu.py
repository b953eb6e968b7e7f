"""MatMulNBits weights of ONNX files into the device layout (upload_nbits:
4-bit through wg_repack_nbits on the GPU, 8-bit dequantized and requantized
there), against the oracle's packMatMulNBits, dequantizeNBitsRow and
quantizeQ8, bit for bit. The reference's fixture graphs carry no weights
(their data files are not shipped): layer 0's tensors are written at the
graph's external offsets into a sparse data file here."""
import os
import shutil

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import onnx_writer as W
from tests.helpers import nbits

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")


def _np(t):
    return t.detach().cpu().numpy()


def _same(a, b):
    assert np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def _with_data(tmp_path, fixture, modules, rng):
    """The fixture graph beside a sparse data file holding random MatMulNBits
    weights (the helper's quantized normal rows) for `modules`."""
    from webgllm_amd.onnx import OnnxFile, OnnxModel
    d = tmp_path / fixture
    d.mkdir()
    shutil.copy(os.path.join(GOLDEN, fixture, "model_q4f16.onnx"), d / "model_q4f16.onnx")
    f = OnnxFile(d / "model_q4f16.onnx")
    m = OnnxModel(f)
    written = {}
    with open(d / "model_q4f16.onnx_data", "wb") as out:
        for mod in modules:
            w = m.nbits(mod)
            quant, scales, zp = nbits(rng, w.N, w.K, with_zp=w.zp is not None)
            for t, data in ((w.quant, quant), (w.scales, scales), (w.zp, zp)):
                if t is None:
                    continue
                raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
                assert t.external is not None and raw.size == t.external[2]
                out.seek(t.external[1])
                out.write(raw.tobytes())
            written[mod] = (w, quant, scales, zp)
    return f, m, written


@pytest.mark.parametrize("fixture", ["lfm2-350m", "lfm2-1.2b-tool"])
def test_fixture_layer0_uploads_bit_exact(hip, tmp_path, fixture):
    from webgllm_amd.onnx import upload_nbits
    rng = np.random.default_rng(3)
    mods = ["/model/layers.0/mlp/gate_proj/", "/model/layers.0/mlp/down_proj/"]
    f, m, written = _with_data(tmp_path, fixture, mods, rng)
    for mod in mods:
        w, quant, scales, zp = written[mod]
        dev = upload_nbits(f, m.nbits(mod))
        want = O.QuantMatrix(w.N, w.K, zp is not None)
        O.pack_nbits(want, 0, quant, scales, zp, w.N)
        assert np.array_equal(_np(dev.quants).view(np.uint32), want.quants)
        assert np.array_equal(_np(dev.scales).view(np.uint16), want.scales)
        rows = 64
        got = _np(dev.dequant(0, rows))
        _same(got, want.dense()[:rows])
        for n in (0, rows - 1):  # dequantizeNBitsRow, load-onnx.ts:471-501
            _same(got[n], O.dequantize_nbits_row(w.K, quant, scales, zp, n))
    f.close()


@pytest.mark.parametrize("zp", [True, False])
@pytest.mark.parametrize("scale_type", [W.FLOAT16, W.FLOAT])
def test_8bit_and_float_scales(hip, tmp_path, zp, scale_type):
    """An 8-bit MatMulNBits weight is stored as the reference stores it
    (src/load-onnx.ts:208-225): scale * (q - zero point) (128 without zero
    points) requantized by quantizeQ8; float32 scales become the nearest
    halves first (halfBytes). A 4-bit weight with float32 scales too."""
    from webgllm_amd.onnx import OnnxFile, OnnxModel, upload_nbits
    rng = np.random.default_rng(9 + zp + scale_type)
    N, K = 8, 96
    blocks = K // 32
    s32 = rng.uniform(0.001, 0.05, N * blocks).astype(np.float32)
    halves = np.array([O.to_half(float(v)) for v in s32], np.uint16)
    scales = s32.tobytes() if scale_type == W.FLOAT else halves.tobytes()
    q8 = rng.integers(0, 256, N * K, dtype=np.uint8)
    z8 = rng.integers(100, 156, N * blocks, dtype=np.uint8)
    n8, i8 = W.matmul_nbits("/model/layers.0/mlp/up_proj/", N, K, 8, q8.tobytes(), scales,
                            z8.tobytes() if zp else None, scale_type=scale_type)
    q4, _, z4 = nbits(rng, N, K, with_zp=zp)
    n4, i4 = W.matmul_nbits("/model/layers.0/mlp/gate_proj/", N, K, 4, q4.tobytes(), scales,
                            z4.tobytes() if zp else None, scale_type=scale_type)
    p = tmp_path / "m.onnx"
    p.write_bytes(W.model(W.graph("g", [n8, n4], i8 + i4)))
    f = OnnxFile(p)
    m = OnnxModel(f)
    got8 = upload_nbits(f, m.nbits("/model/layers.0/mlp/up_proj/"))
    zz = z8.reshape(N, blocks).astype(np.float64) if zp else np.full((N, blocks), 128.0)
    s = np.array([O.from_half(int(h)) for h in halves]).reshape(N, blocks)
    rows = (s[:, :, None] * (q8.reshape(N, blocks, 32) - zz[:, :, None])).reshape(N, K)
    want8 = O.WideMatrix(N, K, 8)
    O.quantize_q8(want8, 0, rows.astype(np.float32))
    _same(_np(got8.dequant()), want8.dense())
    got4 = upload_nbits(f, m.nbits("/model/layers.0/mlp/gate_proj/"))
    want4 = O.QuantMatrix(N, K, zp)
    O.pack_nbits(want4, 0, q4, halves, z4 if zp else None, N)
    _same(_np(got4.dequant()), want4.dense())
    f.close()
