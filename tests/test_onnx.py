"""The ONNX reader (wg_onnx_*, the library's host code) and the MatMulNBits
lookups (src/load-onnx.ts:717-830): the reference's two fixture graphs
(src/test-fixtures/lfm2-350m-onnx and lfm2-1.2b-tool-onnx, copied under
tests/golden/onnx; their weights live in data files the fixtures do not
ship) read the same as by an independent decoder written here, the facts
the reference's tests state about them, and models written from the wire
format covering every field kind and error. CPU only."""
import os
import struct

import pytest

from tests import onnx_writer as W

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")
FIXTURES = [os.path.join(GOLDEN, "lfm2-350m", "model_q4f16.onnx"),
            os.path.join(GOLDEN, "lfm2-1.2b-tool", "model_q4f16.onnx")]


# --- an independent wire-format decoder --------------------------------------

def _fields(buf: bytes):
    """(field, wire, value) of one message: ints, or bytes for wire 2."""
    pos, out = 0, []
    while pos < len(buf):
        k, pos = _varint(buf, pos)
        field, wire = k >> 3, k & 7
        if wire == 0:
            v, pos = _varint(buf, pos)
        elif wire == 2:
            n, pos = _varint(buf, pos)
            v, pos = buf[pos:pos + n], pos + n
        elif wire == 1:
            v, pos = buf[pos:pos + 8], pos + 8
        elif wire == 5:
            v, pos = buf[pos:pos + 4], pos + 4
        else:
            raise ValueError(wire)
        out.append((field, wire, v))
    return out


def _varint(buf, pos):
    v = shift = 0
    while True:
        b = buf[pos]
        pos += 1
        v |= (b & 0x7F) << shift
        shift += 7
        if b < 0x80:
            return v, pos


def _packed(wire, v):
    if wire != 2:
        return [v]
    out, pos = [], 0
    while pos < len(v):
        x, pos = _varint(v, pos)
        out.append(x)
    return out


def _decode(path):
    data = open(path, "rb").read()
    g = [v for f, w, v in _fields(data) if f == 7][0]
    nodes, inits = [], []
    for f, w, v in _fields(g):
        if f == 1:
            n = {"in": [], "out": [], "name": "", "op": ""}
            for nf, nw, nv in _fields(v):
                if nf == 1:
                    n["in"].append(nv.decode())
                elif nf == 2:
                    n["out"].append(nv.decode())
                elif nf == 3:
                    n["name"] = nv.decode()
                elif nf == 4:
                    n["op"] = nv.decode()
            nodes.append(n)
        elif f == 5:
            t = {"dims": [], "ext": {}, "type": 0, "name": ""}
            for tf, tw, tv in _fields(v):
                if tf == 1:
                    t["dims"] += _packed(tw, tv)
                elif tf == 2:
                    t["type"] = tv
                elif tf == 8:
                    t["name"] = tv.decode()
                elif tf == 13:
                    kv = {ef: ev.decode() for ef, _, ev in _fields(tv)}
                    t["ext"][kv[1]] = kv[2]
            inits.append(t)
    return nodes, inits


@pytest.mark.parametrize("path", FIXTURES)
def test_fixture_graph_matches_independent_decoder(path):
    from webgllm_amd.onnx import OnnxFile
    nodes, inits = _decode(path)
    with OnnxFile(path) as f:
        assert [(n.name, n.op_type, n.inputs, n.outputs) for n in f.nodes] == \
            [(n["name"], n["op"], n["in"], n["out"]) for n in nodes]
        assert list(f.initializers) == [t["name"] for t in inits]
        for t in inits:
            got = f.initializers[t["name"]]
            assert list(got.dims) == t["dims"] and got.data_type == t["type"]
            if t["ext"]:
                assert got.external == (t["ext"]["location"], int(t["ext"].get("offset", 0)),
                                        int(t["ext"].get("length", -1)))
            else:
                assert got.external is None


def test_tool_export_facts():
    """src/load-onnx-layouts.test.ts:11-24 on onnx-community's LFM2-1.2B-Tool
    export: 4-bit weights named `model.layers.0.mlp.gate_proj.MatMul.weight_Q4`
    with no zero points, the conv's split sizes from a Constant node, a
    float16 embedding, one data file `model_q4f16.onnx_data`."""
    from webgllm_amd.onnx import FLOAT16, INT64, OnnxFile, OnnxModel
    with OnnxFile(FIXTURES[1]) as f:
        m = OnnxModel(f)
        w = m.nbits("/model/layers.0/mlp/gate_proj/")
        assert w.quant.name == "model.layers.0.mlp.gate_proj.MatMul.weight_Q4" and w.zp is None
        assert (w.N, w.K, w.bits) == (8192, 2048, 4)
        emb = f.initializers["model.embed_tokens.weight"]
        assert emb.data_type == FLOAT16 and emb.dims == (65536, 2048)
        assert {t.external[0] for t in f.initializers.values() if t.external} == \
            {"model_q4f16.onnx_data"}
        split = [n for n in f.nodes if n.op_type == "Split" and "/conv/" in n.name][0]
        sizes = m.constant(split.inputs[1])
        assert sizes.data_type == INT64 and m.producers[split.inputs[1]].op_type == "Constant"
        assert [int(v) for v in _int64s(sizes)] == [2048, 2048, 2048]


def _int64s(t):
    """onnxInt64s (src/onnx.ts:325-340)."""
    if t.int64_data:
        return t.int64_data
    raw = bytes(t.raw)
    return list(struct.unpack(f"<{len(raw) // 8}q", raw))


def test_genai_export_lookups():
    """The onnxruntime-genai export (LFM2-350M): nodes named by module path,
    zero points beside every weight, shapes as config.json states (the FFN
    width after LFM2's block_auto_adjust_ff_dim: 2/3 of block_ff_dim, times
    the multiplier, up to a multiple of block_multiple_of; the reference
    reads it from the weights, src/load-onnx.ts:1386-1397)."""
    import json
    import math
    from webgllm_amd.onnx import OnnxFile, OnnxModel
    cfg = json.load(open(os.path.join(GOLDEN, "lfm2-350m", "config.json")))
    D = cfg["hidden_size"]
    F = int(cfg["block_ffn_dim_multiplier"] * int(2 * cfg["block_ff_dim"] / 3))
    F = cfg["block_multiple_of"] * math.ceil(F / cfg["block_multiple_of"])
    with OnnxFile(FIXTURES[0]) as f:
        m = OnnxModel(f)
        for i in range(cfg["num_hidden_layers"]):
            for mod, (N, K) in (("mlp/gate_proj", (F, D)), ("mlp/up_proj", (F, D)),
                                ("mlp/down_proj", (D, F))):
                w = m.nbits(f"/model/layers.{i}/{mod}/")
                assert (w.N, w.K, w.bits, w.block_size) == (N, K, 4, 32)
                assert w.zp is not None and w.zp.dims == (N, (K // 32 + 1) // 2)
        assert not m.has_nbits("/model/layers.99/mlp/gate_proj/")


def test_written_model_round_trip(tmp_path):
    from webgllm_amd.onnx import OnnxFile
    const = W.tensor("c", (3,), W.INT64, int64s=[5, -1, 1 << 40], packed=False)
    attrs = [W.attr("axis", 2, i=-1), W.attr("alpha", 1, f=0.25), W.attr("mode", 3, s="nearest"),
             W.attr("value", 4, t=const), W.attr("fs", 6, floats=[1.0, -2.5]),
             W.attr("is", 7, ints=[3, -4, 5], packed=False), W.attr("ps", 7, ints=[7, 8]),
             W.attr("ss", 8, strings=["a", "bc"])]
    g = W.graph("g", [W.node("n0", "Custom", ["x", "", "w"], ["y"], attrs, domain="d.x"),
                      W.node("n1", "Constant", [], ["k"], [W.attr("value", 4, t=const)])],
                [W.tensor("w", (2, 3), W.FLOAT, raw=struct.pack("<6f", *range(6)), packed=False),
                 W.tensor("e", (4, 8), W.UINT8, external=("w.bin", 4096, 32)),
                 W.tensor("fd", (2,), W.FLOAT, floats=[0.5, 1.5]),
                 W.tensor("empty", (0,), W.FLOAT)],
                ["x"], ["y"])
    path = tmp_path / "m.onnx"
    path.write_bytes(W.model(g))
    with OnnxFile(path) as f:
        assert f.name == "g" and list(f.initializers) == ["w", "e", "fd", "empty"]
        w = f.initializers["w"]
        assert w.dims == (2, 3) and w.data_type == W.FLOAT and w.external is None
        assert struct.unpack("<6f", bytes(f.data(w))) == tuple(float(v) for v in range(6))
        assert f.initializers["e"].external == ("w.bin", 4096, 32)
        assert f.initializers["fd"].float_data == [0.5, 1.5]
        assert f.initializers["empty"].dims == (0,) and f.data(f.initializers["empty"]).size == 0
        n0, n1 = f.nodes
        assert (n0.name, n0.op_type, n0.domain, n0.inputs, n0.outputs) == \
            ("n0", "Custom", "d.x", ["x", "", "w"], ["y"])
        a = n0.attributes
        assert a["axis"].i == -1 and a["alpha"].f == 0.25 and a["mode"].s == b"nearest"
        assert a["value"].t.int64_data == [5, -1, 1 << 40] and a["value"].t.name == "c"
        assert a["fs"].floats == [1.0, -2.5] and a["is"].ints == [3, -4, 5]
        assert a["ps"].ints == [7, 8] and a["ss"].type == 8
        assert n1.attributes["value"].t.int64_data == [5, -1, 1 << 40]
        assert "c" not in f.initializers  # attribute tensors are not initializers


def test_reader_errors(tmp_path):
    from webgllm_amd import lib as L
    from webgllm_amd.onnx import OnnxFile
    good = W.model(W.graph("g", [W.node("n", "Relu", ["x"], ["y"])],
                           [W.tensor("w", (2,), W.FLOAT, raw=b"\0" * 8)]))
    cases = {"truncated": (good[:-5], "truncated message"),
             "no graph": (W.f_varint(1, 8), "no graph in the model"),
             "group": (W.f_bytes(7, W.key(3, 3)), "unsupported wire type 3")}
    for name, (data, msg) in cases.items():
        p = tmp_path / f"{name}.onnx"
        p.write_bytes(data)
        with pytest.raises(L.WgError, match=msg):
            OnnxFile(p)
    with pytest.raises(L.WgError, match="No such file"):
        OnnxFile(tmp_path / "missing.onnx")


def test_external_data_stays_in_the_model_folder(tmp_path):
    """An external data location must name a file inside the model's folder:
    absolute paths, .. parts and a symbolic link leading out are refused
    before anything is mapped; a plain name (or a subfolder) is read."""
    from webgllm_amd.onnx import OnnxFile
    outside = tmp_path / "secret.bin"
    outside.write_bytes(bytes(range(64)))
    model_dir = tmp_path / "model"
    (model_dir / "sub").mkdir(parents=True)
    (model_dir / "w.bin").write_bytes(bytes(range(32)) * 2)
    (model_dir / "sub" / "v.bin").write_bytes(bytes(range(16)) * 4)
    (model_dir / "link.bin").symlink_to(outside)
    locations = {"abs": str(outside), "up": "../secret.bin", "deep": "sub/../../secret.bin",
                 "link": "link.bin", "ok": "w.bin", "sub": "sub/v.bin"}
    inits = [W.tensor(k, (8,), W.UINT8, external=(v, 8, 8)) for k, v in locations.items()]
    path = model_dir / "m.onnx"
    path.write_bytes(W.model(W.graph("g", [], inits)))
    with OnnxFile(path) as f:
        for name in ("abs", "up", "deep", "link"):
            with pytest.raises(ValueError, match="external data location"):
                f.data(f.initializers[name])
        assert bytes(f.data(f.initializers["ok"])) == bytes(range(8, 16))
        assert bytes(f.data(f.initializers["sub"])) == bytes(range(8, 16))


def _nbits_model(tmp_path, **kw):
    from webgllm_amd.onnx import OnnxFile, OnnxModel
    N, K = kw.pop("N", 8), kw.pop("K", 64)
    bits, bs = kw.pop("bits", 4), kw.pop("block_size", 32)
    blocks = -(-K // bs)
    qbytes = N * blocks * bs * bits // 8
    n, inits = W.matmul_nbits("/model/layers.0/mlp/gate_proj/", N, K, bits, b"\0" * qbytes,
                              b"\0" * (2 * N * blocks), block_size=bs, **kw)
    p = tmp_path / "nb.onnx"
    p.write_bytes(W.model(W.graph("g", [n], inits)))
    return OnnxModel(OnnxFile(p))


def test_nbits_checks(tmp_path):
    """wideNBits and nbits (src/load-onnx.ts:783-830): 4-bit in blocks of 32,
    8-bit in multiples of 32, no g_idx or bias, the quants' element count."""
    m = _nbits_model(tmp_path)
    assert m.nbits("/model/layers.0/mlp/gate_proj/").N == 8
    with pytest.raises(ValueError, match="not 4-bit in blocks of 32"):
        _nbits_model(tmp_path, bits=2).nbits("/model/layers.0/mlp/gate_proj/")
    with pytest.raises(ValueError, match="not 4-bit in blocks of 32"):
        _nbits_model(tmp_path, block_size=64).nbits("/model/layers.0/mlp/gate_proj/")
    w = _nbits_model(tmp_path, bits=8, block_size=64).wide_nbits("/model/layers.0/mlp/gate_proj/")
    assert (w.bits, w.block_size) == (8, 64)
    with pytest.raises(ValueError, match="not in blocks of 32"):
        _nbits_model(tmp_path, bits=8, block_size=64).nbits("/model/layers.0/mlp/gate_proj/")
    with pytest.raises(ValueError, match="g_idx or bias"):
        _nbits_model(tmp_path, extra_inputs=["", "bias"]).nbits("/model/layers.0/mlp/gate_proj/")
    with pytest.raises(ValueError, match="240 elements, expected 256"):
        _nbits_model(tmp_path, quant_dims=(8, 2, 15)).nbits("/model/layers.0/mlp/gate_proj/")
    with pytest.raises(ValueError, match="no MatMulNBits node"):
        m.nbits("/model/layers.1/mlp/gate_proj/")


def test_two_nodes_for_one_module(tmp_path):
    from webgllm_amd.onnx import OnnxFile, OnnxModel
    n, inits = W.matmul_nbits("/model/layers.0/mlp/up_proj/", 4, 32, 4, b"\0" * 64, b"\0" * 8)
    n2 = W.node("/model/layers.0/mlp/up_proj/Other", "MatMulNBits", ["a", "b"], ["c"])
    p = tmp_path / "two.onnx"
    p.write_bytes(W.model(W.graph("g", [n, n2], inits)))
    with pytest.raises(ValueError, match="2 MatMulNBits nodes"):
        OnnxModel(OnnxFile(p)).nbits_node("/model/layers.0/mlp/up_proj/")
