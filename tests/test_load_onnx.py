"""The ONNX loader's plan over the reference's two fixture graphs (LFM2-350M's
onnxruntime-genai export, LFM2-1.2B-Tool's transformers.js export), with
the facts the reference's tests state about them
(src/load-onnx-layouts.test.ts) and edited copies of the graphs for the
refusals: the shapes and layout found from the graph alone, every read
listed before any data is read. CPU only (the graph reader is host code)."""
import copy
import json
import os

import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")


def _paths(fixture):
    d = os.path.join(GOLDEN, fixture)
    with open(os.path.join(d, "config.json")) as fh:
        return os.path.join(d, "model_q4f16.onnx"), json.load(fh)


class _Edited:
    """A copy of a parsed graph whose nodes and initializers can be changed."""

    def __init__(self, f):
        self.nodes = [copy.copy(n) for n in f.nodes]
        for n in self.nodes:
            n.inputs, n.outputs, n.attributes = list(n.inputs), list(n.outputs), \
                dict(n.attributes)
        self.initializers = dict(f.initializers)
        self.name, self.path = f.name, f.path


@pytest.fixture
def graph():
    from webgllm_amd.onnx import OnnxFile
    opened = []

    def open_(fixture):
        path, cfg = _paths(fixture)
        f = OnnxFile(path)
        opened.append(f)
        return _Edited(f), cfg
    yield open_
    for f in opened:
        f.close()


def _plan(g, cfg):
    from webgllm_amd.load_onnx import plan_onnx
    from webgllm_amd.onnx import OnnxModel
    return plan_onnx(OnnxModel(g), cfg)


def _check(g, cfg):
    from webgllm_amd.load_onnx import check_model
    from webgllm_amd.onnx import OnnxModel
    return check_model(OnnxModel(g), cfg)


@pytest.mark.parametrize("fixture", ["lfm2-350m", "lfm2-1.2b-tool"])
def test_fixture_graphs_pass_the_check(fixture):
    from webgllm_amd.load_onnx import check_onnx
    path, cfg = _paths(fixture)
    assert check_onnx(path, cfg) == ["model_q4f16.onnx_data"]


def test_lfm2_350m_plan(graph):
    """onnxruntime-genai's export: a GatherBlockQuantized 4-bit embedding
    tied to the MatMulNBits head, zero points, the MLP width the weights
    have (4608, where config.json says 6656 with block_auto_adjust_ff_dim),
    GroupQueryAttention rotating every dim of a head."""
    g, cfg = graph("lfm2-350m")
    p = _plan(g, cfg)
    s = p.shape
    assert (s.hidden, s.layers, s.heads, s.kv_heads, s.head_dim) == (1024, 16, 16, 8, 64)
    assert (s.intermediate, s.vocab, s.conv_kernel) == (4608, 65536, 3)
    assert s.conv_layers == (0, 1, 3, 4, 6, 7, 9, 11, 13, 15)
    assert (s.rope_theta, s.eps, s.qk_norm) == (1e6, 1e-5, True)
    assert s.extra["bos"] == 1 and s.extra["eos"] == 7
    assert p.embedding.kind == "q4" and p.embedding.N == 65536
    assert p.embedding.zp is not None
    assert p.final_norm.name == "model.layers.16.final_norm_layernorm.weight"
    # the Split's outputs 0 and 2 are multiplied before the convolution, 1 after it
    assert [(x.start, x.rows) for x in p.layers[0].bcx] == [(0, 1024), (1024, 1024),
                                                            (2048, 1024)]
    assert p.layers[2].type == "full_attention" and p.layers[2].rope_sin is None
    # reads in the loader's order: norms, operator matrices, the kernel, the MLP
    assert [r[0] for r in p.reads[:3]] == ["model.layers.0.operator_layernorm.weight",
                                           "model.layers.0.ffn_layernorm.weight",
                                           "model_layers_0_conv_in_proj_MatMul_weight_quant"]
    # the embedding in chunks of 2048 rows: quants, scales, zero points each
    emb = [r for r in p.reads if r[0].startswith("model_embed_tokens")]
    assert len(emb) == 3 * 32
    assert emb[3][2] - emb[0][2] == 2048 * 512


def test_lfm2_tool_plan(graph):
    """transformers.js's export: weights named model.layers.0.mlp.gate_proj.
    MatMul.weight_Q4 without zero points, split sizes from a Constant node,
    a float16 embedding read by a plain Gather with the head a MatMul over
    it transposed: quantized to 8 bits at load."""
    g, cfg = graph("lfm2-1.2b-tool")
    p = _plan(g, cfg)
    s = p.shape
    assert (s.hidden, s.heads, s.kv_heads, s.intermediate, s.vocab) == (2048, 32, 8, 8192, 65536)
    assert p.embedding.kind == "float" and s.embed_fmt == "q8"
    assert p.layers[0].matrices["gate"].zp is None
    assert [(x.start, x.rows) for x in p.layers[0].bcx] == [(0, 2048), (2048, 2048),
                                                            (4096, 2048)]


def test_c_is_found_by_following_the_graph(graph):
    """With the Split's outputs used the other way round (output 0 after the
    convolution), in_proj's rows are placed B, C, x all the same."""
    g, cfg = graph("lfm2-350m")
    pre = "/model/layers.0/conv/"
    mul1 = next(n for n in g.nodes if n.name == pre + "Mul_1")
    mul2 = next(n for n in g.nodes if n.name == pre + "Mul_2")
    assert mul1.inputs[0] == pre + "Split/output_0" and mul2.inputs[0] == pre + "Split/output_1"
    mul1.inputs[0], mul2.inputs[0] = pre + "Split/output_1", pre + "Split/output_0"
    p = _plan(g, cfg)
    assert [(x.start, x.rows) for x in p.layers[0].bcx] == [(1024, 1024), (0, 1024),
                                                            (2048, 1024)]


def test_a_projection_is_found_by_the_weights_it_reads(graph):
    g, cfg = graph("lfm2-350m")
    node = next(n for n in g.nodes if n.name == "/model/layers.0/mlp/gate_proj/MatMul_Quant")
    node.name = "/other/gate/MatMul_Quant"
    assert _check(g, cfg) == ["model_q4f16.onnx_data"]
    p = _plan(g, cfg)
    assert p.layers[0].matrices["gate"].node.name == "/other/gate/MatMul_Quant"


def test_a_plain_matmul_head_with_its_own_weights_is_refused(graph):
    from webgllm_amd.onnx import FLOAT16, OnnxNode, OnnxTensor
    g, cfg = graph("lfm2-350m")
    i = next(j for j, n in enumerate(g.nodes) if n.name == "/lm_head/MatMul_Quant")
    head = g.nodes[i]
    D, V = cfg["hidden_size"], cfg["vocab_size"]
    g.initializers["lm_head.weight"] = OnnxTensor(
        "lm_head.weight", (D, V), FLOAT16, 0, external=("model_q4f16.onnx_data", 0, D * V * 2))
    g.nodes[i] = OnnxNode("/lm_head/MatMul", "MatMul", "", [head.inputs[0], "lm_head.weight"],
                          list(head.outputs), {})
    with pytest.raises(ValueError, match="LM head"):
        _check(g, cfg)


def test_a_float_embedding_short_of_its_rows_is_refused(graph):
    g, cfg = graph("lfm2-1.2b-tool")
    emb = g.initializers["model.embed_tokens.weight"]
    loc, off, n = emb.external
    g.initializers[emb.name] = _with(emb, external=(loc, off, n // 2))
    with pytest.raises(ValueError, match=r"model\.embed_tokens\.weight has \d+ bytes, expected"):
        _check(g, cfg)


def test_an_embedding_whose_rows_are_not_a_multiple_of_4_is_refused(graph):
    g, cfg = graph("lfm2-1.2b-tool")
    emb = g.initializers["model.embed_tokens.weight"]
    rows, D = emb.dims[0] - 1, emb.dims[1]
    loc, off, _ = emb.external
    g.initializers[emb.name] = _with(emb, dims=(rows, D), external=(loc, off, rows * D * 2))
    with pytest.raises(ValueError, match="65535 rows, not a multiple of 4"):
        _check(g, dict(cfg, vocab_size=rows))


@pytest.mark.parametrize("edit,match", [
    (lambda c: c.update(layer_types=["sliding_attention" if t == "full_attention" else t
                                     for t in c["layer_types"]]), "sliding_attention layers"),
    (lambda c: c.update(rope_parameters={"rope_theta": 1e6, "partial_rotary_factor": 0.5}),
     "partial RoPE"),
    (lambda c: c.update(rope_parameters={"rope_type": "yarn", "rope_theta": 1e6}), "yarn RoPE"),
    (lambda c: c.update(intermediate_size=1000, block_auto_adjust_ff_dim=False),
     "intermediate_size 1000"),
    (lambda c: c.update(vocab_size=1000), "vocab_size 1000"),
    (lambda c: c.pop("layer_types"), "neither layer_types"),
    (lambda c: c.update(num_hidden_layers=15), "16 layer types for 15 layers"),
])
def test_configs_off_the_engines_path_are_refused(graph, edit, match):
    g, cfg = graph("lfm2-350m")
    cfg = json.loads(json.dumps(cfg))
    edit(cfg)
    with pytest.raises(ValueError, match=match):
        _check(g, cfg)


def test_interleaved_or_partial_rotary_graphs_are_refused(graph):
    g, cfg = graph("lfm2-350m")
    gqa = next(n for n in g.nodes if n.name == "/model/layers.2/attn/GroupQueryAttention")
    a = gqa.attributes["rotary_interleaved"]
    gqa.attributes["rotary_interleaved"] = _with(a, i=1)
    with pytest.raises(ValueError, match="non-interleaved"):
        _check(g, cfg)
    gqa.attributes["rotary_interleaved"] = a
    cos = g.initializers["cos_cache"]
    g.initializers["cos_cache"] = _with(cos, dims=(cos.dims[0], 16))
    with pytest.raises(ValueError, match="rotates 32 of each head's 64 dims"):
        _check(g, cfg)


def test_an_attention_gate_is_refused(graph):
    from webgllm_amd.onnx import OnnxNode
    g, cfg = graph("lfm2-350m")
    q = next(n for n in g.nodes if n.name == "/model/layers.2/attn/q_proj/MatMul_Quant")
    g.nodes.append(OnnxNode("/model/layers.2/attn/gate_proj/MatMul_Quant", "MatMulNBits", "",
                            list(q.inputs), ["gate_out"], dict(q.attributes)))
    with pytest.raises(ValueError, match="output gate"):
        _check(g, cfg)


def _with(obj, **kw):
    out = copy.copy(obj)
    for k, v in kw.items():
        setattr(out, k, v)
    return out
