"""An LFM2 ONNX export end to end: the reference's LFM2-350M fixture graph
(onnxruntime-genai's q4f16 export; its weights are not shipped) beside a
data file holding seeded weights at every offset the graph gives, loaded by
load_onnx into the engine. Every device matrix is the oracle's
packMatMulNBits of the file's rows in the order the loader must place them
(gate|up interleaved, in_proj's B, C, x, q|k|v), bit for bit; norms, conv
taps and the embedding are the file's values; and the engine's prompt
logits and greedy tokens are the oracle decoder's. The float16 embedding of
the LFM2-1.2B-Tool export quantizes to 8 bits in chunks the same as at
once, and as the oracle's quantizeQ8."""
import json
import os
import shutil

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import rel_l2
from tests.model_oracle import OracleModel

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")


def _np(t):
    return t.detach().cpu().numpy()


def _fixture(tmp_path, fixture):
    d = tmp_path / fixture
    d.mkdir()
    for name in ("model_q4f16.onnx", "config.json"):
        shutil.copy(os.path.join(GOLDEN, fixture, name), d / name)
    with open(d / "config.json") as fh:
        return d / "model_q4f16.onnx", json.load(fh)


def _put(out, t, arr):
    raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    assert t.external is not None and raw.size == t.external[2], t.name
    out.seek(t.external[1])
    out.write(raw.tobytes())


def _halves(rng, n, lo, hi):
    return rng.uniform(lo, hi, n).astype(np.float16)


def write_weights(path, cfg, seed):
    """Seeded weights for every tensor the loader reads, at the graph's
    offsets: 4-bit quants and zero points any byte, half scales near a
    trained layer's, norms near 1, conv taps N(0, 0.3); the LM head's own
    copy of the 4-bit embedding (the export's tied head) the same bytes."""
    from webgllm_amd.load_onnx import plan_onnx
    from webgllm_amd.onnx import OnnxFile, OnnxModel
    rng = np.random.default_rng(seed)
    with OnnxFile(path) as f:
        m = OnnxModel(f)
        plan = plan_onnx(m, cfg)
        with open(str(path) + "_data", "wb") as out:
            for lp in plan.layers:
                for t in lp.norms:
                    _put(out, t, (1 + 0.1 * rng.standard_normal(t.dims)).astype(np.float16))
                if lp.type == "conv":
                    k = lp.extra[0]
                    _put(out, k, (0.3 * rng.standard_normal(k.dims)).astype(np.float16))
                for w in lp.matrices.values():
                    _put(out, w.quant, rng.integers(0, 256, w.quant.external[2], np.uint8))
                    _put(out, w.scales, _halves(rng, w.scales.external[2] // 2, 0.002, 0.005))
                    if w.zp is not None:
                        _put(out, w.zp, rng.integers(0, 256, w.zp.external[2], np.uint8))
            t = plan.final_norm
            _put(out, t, (1 + 0.1 * rng.standard_normal(t.dims)).astype(np.float16))
            e = plan.embedding
            assert e.kind == "q4"
            quant = rng.integers(0, 256, e.quant.external[2], np.uint8)
            _put(out, e.quant, quant)
            _put(out, e.scales, _halves(rng, e.scales.external[2] // 2, 0.01, 0.03))
            _put(out, e.zp, rng.integers(0, 256, e.zp.external[2], np.uint8))
            head = m.nbits("/lm_head/")
            if head.quant.name != e.quant.name:
                _put(out, head.quant, quant)
    return plan


@pytest.fixture(scope="module")
def lfm2_350m(tmp_path_factory):
    path, cfg = _fixture(tmp_path_factory.mktemp("onnx"), "lfm2-350m")
    plan = write_weights(path, cfg, seed=11)
    return path, cfg, plan


def _rows(f, w, order=None):
    """A 4-bit weight's file rows: quants [N][K/2], half scales [N][K/32],
    zero points [N][ceil(K/64)]."""
    blocks = w.K // 32
    q = np.asarray(f.data(w.quant)).reshape(w.N, blocks * 16)
    s = np.asarray(f.data(w.scales)).view(np.uint16).reshape(w.N, blocks)
    z = np.asarray(f.data(w.zp)).reshape(w.N, -(-blocks // 2))
    return q, s, z


def _expect(f, parts, order=None):
    """The oracle's packMatMulNBits of the parts' rows ([(NBits, [(start,
    rows)])]) stacked, stored in `order` (stored row p = logical row
    order[p])."""
    qs, ss, zs = [], [], []
    for w, segs in parts:
        q, s, z = _rows(f, w)
        for a, n in segs:
            qs.append(q[a:a + n])
            ss.append(s[a:a + n])
            zs.append(z[a:a + n])
    q, s, z = np.concatenate(qs), np.concatenate(ss), np.concatenate(zs)
    if order is not None:
        q, s, z = q[order], s[order], z[order]
    N, K = q.shape[0], q.shape[1] * 2
    qm = O.QuantMatrix(N, K, True)
    O.pack_nbits(qm, 0, q.reshape(-1), s.reshape(-1), z.reshape(-1), N)
    return qm


def _same_matrix(dev, want, what):
    assert np.array_equal(_np(dev.quants).view(np.uint32), want.quants), what
    assert np.array_equal(_np(dev.scales).view(np.uint16), want.scales), what
    assert np.array_equal(_np(dev.zeros), want.zeros), what


def _halves_of(f, t):
    return np.asarray(f.data(t)).view(np.float16).astype(np.float32)


def test_loaded_onnx_matrices_are_the_files(hip, lfm2_350m):
    from webgllm_amd import engine as E
    from webgllm_amd.load_onnx import load_onnx
    from webgllm_amd.onnx import OnnxFile
    path, cfg, plan = lfm2_350m
    w = load_onnx(str(path))
    s = w.shape
    assert s == plan.shape
    D, F = s.hidden, s.intermediate
    with OnnxFile(path) as f:
        for i, (lp, lw) in enumerate(zip(plan.layers, w.layers)):
            mm = lp.matrices

            def whole(x):
                return (x, [(0, x.N)])
            if lp.type == "conv":
                _same_matrix(lw["in_proj"], _expect(f, [(mm["in_proj"], [(x.start, x.rows)
                                                                         for x in lp.bcx])]),
                             f"layer {i} in_proj")
                _same_matrix(lw["out_proj"], _expect(f, [whole(mm["out_proj"])]),
                             f"layer {i} out_proj")
                assert np.array_equal(_np(lw["taps"]),
                                      _halves_of(f, lp.extra[0]).reshape(D, s.conv_kernel))
            else:
                _same_matrix(lw["qkv"], _expect(f, [whole(mm["q"]), whole(mm["k"]),
                                                    whole(mm["v"])]), f"layer {i} qkv")
                _same_matrix(lw["o"], _expect(f, [whole(mm["o"])]), f"layer {i} o")
                assert np.array_equal(_np(lw["q_norm"]), _halves_of(f, lp.extra[0]))
                assert np.array_equal(_np(lw["k_norm"]), _halves_of(f, lp.extra[1]))
            _same_matrix(lw["gate_up"], _expect(f, [whole(mm["gate"]), whole(mm["up"])],
                                                E.gate_up_row_order(F)), f"layer {i} gate_up")
            _same_matrix(lw["down"], _expect(f, [whole(mm["down"])]), f"layer {i} down")
            assert np.array_equal(_np(lw["op_norm"]), _halves_of(f, lp.norms[0]))
            assert np.array_equal(_np(lw["ffn_norm"]), _halves_of(f, lp.norms[1]))
        assert np.array_equal(_np(w.final_norm), _halves_of(f, plan.final_norm))
        e = plan.embedding
        from webgllm_amd.onnx import NBits
        emb = NBits("embedding", None, e.N, D, 4, 32, e.quant, e.scales, e.zp)
        _same_matrix(w.embedding, _expect(f, [(emb, [(0, e.N)])]), "embedding")


def test_onnx_model_decodes_the_oracles_tokens(hip, lfm2_350m):
    from webgllm_amd.engine import Engine
    from webgllm_amd.load_onnx import load_onnx
    path, _, _ = lfm2_350m
    w = load_onnx(str(path))
    eng, orc = Engine(w, 256), OracleModel(w, 256)
    rng = np.random.default_rng(5)
    prompt = [int(x) for x in rng.integers(0, w.shape.vocab, 21)]
    print(f"onnx lfm2-350m: prompt of {len(prompt)}", flush=True)
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok())
    assert rel_l2(eng.logits[:len(prompt) % 8].cpu().numpy(), logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    first = int(picks[-1])
    assert eng.decode(first, 8) == orc.decode(first, 8)


def test_float16_embedding_quantizes_in_chunks_as_at_once(hip, tmp_path):
    """LFM2-1.2B-Tool's float16 embedding (65536 x 2048, read by a plain
    Gather; the head a MatMul over it transposed): each row ((r * 7 + k) mod
    33) - 16, exact in halves, as the reference's test writes it; the
    loader's chunks are bit for bit the whole matrix quantized at once, the
    first chunk the oracle's quantizeQ8, and the values within a step."""
    from webgllm_amd import ops
    from webgllm_amd.load_onnx import _Uploader, plan_onnx
    from webgllm_amd.onnx import OnnxFile, OnnxModel
    path, cfg = _fixture(tmp_path, "lfm2-1.2b-tool")
    with OnnxFile(path) as f:
        plan = plan_onnx(OnnxModel(f), cfg)
        e = plan.embedding
        N, D = e.weight.dims
        r = np.arange(N, dtype=np.int64)[:, None]
        k = np.arange(D, dtype=np.int64)[None, :]
        vals = (((r * 7 + k) % 33) - 16).astype(np.float16)
        with open(str(path) + "_data", "wb") as out:
            _put(out, e.weight, vals)
    with OnnxFile(path) as f:
        chunk = 4096
        got = _Uploader(f, "cuda").embedding(e, D, chunk_rows=chunk)
        whole = ops.Q4Matrix.from_floats_q8(torch.from_numpy(vals).cuda().float())
        torch.cuda.synchronize()
        assert torch.equal(got.quants, whole.quants)
        assert torch.equal(got.scales, whole.scales)
        wm = O.WideMatrix(chunk, D, 8)
        O.quantize_q8(wm, 0, vals[:chunk].astype(np.float32))
        assert np.array_equal(_np(got.quants)[:wm.quants.size].view(np.uint8),
                              wm.quants.view(np.uint8))
        assert np.array_equal(_np(got.scales)[:wm.scales.size].view(np.uint16), wm.scales)
        dense = _np(got.dequant(0, 64))
        assert np.abs(dense - vals[:64].astype(np.float32)).max() < 0.07
