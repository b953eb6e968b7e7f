"""The Node N-API addon (webgllm_amd/node: webgllm_hip.node and index.js's
HipGpu) run by Node itself, as the reference's TypeScript engine would
load it in place of its WebGL2 backend (src/gpu/gl.ts:47). The script
tests/node/addon_test.js makes its own assertions and prints what it read;
this side compares that with the Python readers and the oracle.

- CPU: the QuantMatrix sizes (src/weights.ts:153-178), GpuError codes and
  messages of rejected calls, TypeErrors for wrong handles, and the GGUF
  and ONNX readers (a written GGUF file; the reference's LFM2-350M fixture
  graph) against webgllm_amd.gguf / webgllm_amd.onnx.
- GPU: textures written, zeroed, read whole and by rectangle behind
  polled fences, cancelled reads, disposed handles, and a GGUF Q4_0 matrix
  repacked and multiplied through HipGpu.ops: dequant bit-exact, GEMV
  within rel-L2 1e-4 of the float64 oracle, greedy picks equal."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from tests import gguf_writer as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "tests", "node", "addon_test.js")
ADDON = os.path.join(ROOT, "webgllm_amd", "node", "webgllm_hip.node")
FIXTURE = os.path.join(ROOT, "tests", "golden", "onnx", "lfm2-350m", "model_q4f16.onnx")


def _node():
    node = shutil.which("node")
    if node is None:
        pytest.skip("no node on this machine")
    if not os.path.exists(ADDON):
        pytest.fail("webgllm_amd/node/webgllm_hip.node is not built (run __graft_entry__.build())")
    return node


def _run(args, timeout=120):
    p = subprocess.run([_node(), SCRIPT] + args, capture_output=True, text=True, timeout=timeout)
    assert p.returncode == 0, p.stderr[-4000:]
    return json.loads(p.stdout.strip().splitlines()[-1])


def test_addon_sizes_errors_and_readers(tmp_path):
    from webgllm_amd import gguf as G
    from webgllm_amd.onnx import OnnxFile
    rng = np.random.default_rng(0)
    meta = [("general.architecture", W.STRING, "lfm2"), ("t.u32", W.U32, 4000000000),
            ("t.i32", W.I32, -7), ("t.f32", W.F32, 0.5), ("t.bool", W.BOOL, True),
            ("t.ints", W.ARRAY, (W.I32, [0, 4, 0, 4]))]
    tensors = [("a.weight", (64, 2), 0, rng.standard_normal(128).astype(np.float32)),
               ("b.weight", (32, 3), 2, rng.integers(0, 256, 3 * 18, dtype=np.uint8))]
    path = tmp_path / "t.gguf"
    W.write_gguf(path, meta, tensors)
    out = _run(["cpu", str(path), FIXTURE])
    with G.GgufFile(path) as f:
        g = out["gguf"]
        assert g["version"] == f.version and g["dataOffset"] == f.data_offset
        want = [[t.name, list(t.dims), t.type, t.offset, t.nbytes]
                for t in sorted(f.tensors.values(), key=lambda t: t.index)]
        assert g["tensors"] == want
        m = g["meta"]
        assert m["general.architecture"] == "lfm2" and m["t.u32"] == 4000000000
        assert m["t.i32"] == -7 and m["t.f32"] == 0.5 and m["t.bool"] is True
        assert m["t.ints"] == {"type": W.I32, "length": 4}
    with OnnxFile(FIXTURE) as f:
        o = out["onnx"]
        assert o["name"] == f.name
        assert o["nodes"] == [[n.name, n.op_type, n.domain, n.inputs, n.outputs,
                               sorted(n.attributes)] for n in f.nodes]
        inits = [[t.name, list(t.dims), t.data_type] + (list(t.external) if t.external else
                                                        [None, None, None])
                 for t in f.initializers.values()]
        assert o["initializers"] == inits
        assert len(o["nodes"]) > 100 and len(o["initializers"]) > 50


@pytest.mark.gpu
def test_addon_textures_and_q4_0_gemv(hip, tmp_path):
    from oracle import oracle as O
    from tests.helpers import rel_l2
    rng = np.random.default_rng(9)
    N, K, M = 1024, 2048, 3
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    src = O.quantize_q4_0(w)
    x16 = O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
    (tmp_path / "q4_0.bin").write_bytes(np.ascontiguousarray(src).tobytes())
    (tmp_path / "x16.bin").write_bytes(np.ascontiguousarray(x16).tobytes())
    (tmp_path / "gemv.json").write_text(json.dumps({"N": N, "K": K, "M": M}))
    # Q4_K blocks for a Q4_K-records matrix (N4 x K, zero scales in some)
    from tests.helpers import random_q4_k_bytes
    N4 = 64
    src4 = random_q4_k_bytes(rng, N4, K, zero_scale_every=3)
    (tmp_path / "q4_k.bin").write_bytes(np.ascontiguousarray(src4).tobytes())
    out = _run(["gpu", str(tmp_path)])
    qm = O.QuantMatrix(N, K, False)
    O.pack_q4_0(qm, 0, src, N)
    y = np.frombuffer((tmp_path / "y.bin").read_bytes(), np.float32).reshape(M, N)
    want = O.gemv_f64(qm, O.halves_to_f32(x16))
    assert rel_l2(y, want) <= 1e-4
    assert out["picks"] == [O.argmax(y[m])[0] for m in range(M)]
    dq = np.frombuffer((tmp_path / "dequant.bin").read_bytes(), np.float32).reshape(4, K)
    assert np.array_equal(dq.view(np.uint32), qm.dense()[8:12].view(np.uint32))
    # the records matrix's kept halves are packQ4_K's, its dequant packQ4_K's rows
    q4 = O.QuantMatrix(N4, K, "halves")
    O.pack_q4_k(q4, 0, src4, N4)
    halves = np.frombuffer((tmp_path / "q4k_halves.bin").read_bytes(), np.uint16)
    assert np.array_equal(halves[:q4.scales.size], q4.scales)
    assert np.array_equal(halves[q4.scales.size:], q4.zero_halves)
    dq4 = np.frombuffer((tmp_path / "q4k_dequant.bin").read_bytes(), np.float32).reshape(4, K)
    assert np.array_equal(dq4.view(np.uint32), q4.dense()[4:8].view(np.uint32))
    assert 1 <= out["staging"]["slots"] <= 18
