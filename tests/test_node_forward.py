"""A whole LFM2-shaped forward driven from Node through HipGpu alone
(tests/node/lfm2_forward.js), as the reference's Engine.forwardBatch drives
its WebGL2 backend (src/engine.ts:8875-9303): weights uploaded as GGUF Q4_0
blocks and repacked by the addon; a 40-token prompt through the prefill
GEMMs; 8 greedy decode steps through the few-token GEMVs and their
epilogues; one verify batch of the last token and 4 drafts (two the true
continuation, two random) whose accept and conv-state rollback run on the
device (src/handler.ts:1811-1887, src/engine.ts:8063-8086); two more steps
after the rollback. Every step's logits are within rel-L2 1e-3 of the
oracle decoder's (tests/model_oracle.py, float64 matmuls over the oracle's
dequantized weights) and every pick equals the oracle's."""
import copy
import dataclasses
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import rel_l2
from tests.model_oracle import OracleModel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "tests", "node", "lfm2_forward.js")
ADDON = os.path.join(ROOT, "webgllm_amd", "node", "webgllm_hip.node")


def _q4_0_blocks(rng, N, K, sigma):
    """GGUF Q4_0 blocks of an N(0, sigma) matrix by ggml's reference
    quantizer (the oracle's)."""
    return O.quantize_q4_0((rng.standard_normal((N, K)) * sigma).astype(np.float32))


def _dense_q4_0(src, N, K):
    qm = O.QuantMatrix(N, K, False)
    O.pack_q4_0(qm, 0, src, N)
    return qm.dense()


def _model(tmp, seed=5):
    from webgllm_amd import engine as E
    shape = dataclasses.replace(E.LFM2_12B, name="lfm2-small", hidden=512, layers=4, heads=8,
                                kv_heads=2, head_dim=64, intermediate=1024, vocab=4096,
                                conv_layers=(0, 1, 3))
    rng = np.random.default_rng(seed)
    D, F, hd = shape.hidden, shape.intermediate, shape.head_dim
    tensors, dense_layers = {}, []

    def put(name, arr):
        fn = name + ".bin"
        (tmp / fn).write_bytes(np.ascontiguousarray(arr).tobytes())
        tensors[name] = fn

    def matrix(name, N, K, sigma=0.05):
        src = _q4_0_blocks(rng, N, K, sigma)
        put(name, src)
        return _dense_q4_0(src, N, K)

    def norm(name, n):
        v = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        put(name, v)
        return v

    emb = matrix("embedding", shape.vocab, D, sigma=0.05)
    final = norm("final_norm", D)
    types = []
    for i in range(shape.layers):
        p = f"layers.{i}."
        lw = {"op_norm": norm(p + "op_norm", D), "ffn_norm": norm(p + "ffn_norm", D)}
        lw["gate_up"] = matrix(p + "gate_up", 2 * F, D)
        lw["down"] = matrix(p + "down", D, F)
        if shape.layer_type(i) == "conv":
            types.append("conv")
            lw["in_proj"] = matrix(p + "in_proj", 3 * D, D)
            lw["out_proj"] = matrix(p + "out_proj", D, D)
            taps = (rng.standard_normal((D, shape.conv_kernel)) * 0.5).astype(np.float32)
            put(p + "taps", taps)
            lw["taps"] = taps
        else:
            types.append("attn")
            lw["qkv"] = matrix(p + "qkv", shape.qkv_rows, D)
            lw["o"] = matrix(p + "o", D, shape.heads * hd)
            lw["q_norm"] = norm(p + "q_norm", hd)
            lw["k_norm"] = norm(p + "k_norm", hd)
        dense_layers.append(lw)
    return shape, tensors, types, emb, final, dense_layers


@pytest.mark.gpu
def test_node_lfm2_prompt_decode_verify_rollback(hip, tmp_path):
    node = shutil.which("node")
    if node is None:
        pytest.skip("no node on this machine")
    assert os.path.exists(ADDON), "webgllm_amd/node/webgllm_hip.node is not built"
    ctx = 256
    shape, tensors, types, emb, final, layers = _model(tmp_path)
    orc = OracleModel.from_dense(shape, emb, final, layers, ctx)
    rng = np.random.default_rng(11)
    prompt = [int(t) for t in rng.integers(0, shape.vocab, 40)]
    # the oracle: the prompt (its layers' weights rounded to halves, as the
    # prefill GEMMs read them), 8 greedy steps, then the truth ahead
    p_logits, p_picks = orc.forward(prompt, f16_weights=True, batch=len(prompt))
    steps, truth_logits, t = [], [], p_picks[-1]
    for _ in range(8):
        lo, p = orc.forward_rows([t])
        truth_logits.append(lo[0])
        t = p[0]
        steps.append(t)
    before = copy.deepcopy((orc.k, orc.v, orc.state, orc.position))
    seq = []
    u = t
    for _ in range(3):
        _, p = orc.forward_rows([u])
        u = p[0]
        seq.append(u)
    drafts = seq[:2] + [int(v) for v in rng.integers(0, shape.vocab, 2)]
    orc.k, orc.v, orc.state, orc.position = copy.deepcopy(before)
    v_logits, v_picks = orc.forward_rows([t] + drafts)
    kept = 1
    while kept < 5 and v_picks[kept - 1] == drafts[kept - 1]:
        kept += 1
    assert kept >= 3  # the two true drafts are kept
    # the oracle's state after keeping `kept` rows: the batch's first rows run alone
    orc.k, orc.v, orc.state, orc.position = copy.deepcopy(before)
    orc.forward_rows(([t] + drafts)[:kept])
    after, after_logits, u = [], [], v_picks[kept - 1]
    for _ in range(2):
        lo, p = orc.forward_rows([u])
        after_logits.append(lo[0])
        u = p[0]
        after.append(u)

    cfg = {"hidden": shape.hidden, "intermediate": shape.intermediate, "heads": shape.heads,
           "kvHeads": shape.kv_heads, "headDim": shape.head_dim, "vocab": shape.vocab,
           "convKernel": shape.conv_kernel, "eps": shape.eps, "ropeTheta": shape.rope_theta,
           "ctx": ctx, "maxPrompt": 64, "layerTypes": types, "tensors": tensors,
           "prompt": prompt, "decodeSteps": 8, "drafts": drafts, "afterSteps": 2}
    (tmp_path / "model.json").write_text(json.dumps(cfg))
    print(f"node {SCRIPT} {tmp_path}", flush=True)
    r = subprocess.run([node, SCRIPT, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-4000:]
    out = json.loads((tmp_path / "out.json").read_text())
    V = shape.vocab

    def logits(name, M):
        return np.frombuffer((tmp_path / f"logits_{name}.bin").read_bytes(),
                             np.float32).reshape(M, V)

    by = {s["name"]: s for s in out["steps"]}
    assert by["prompt"]["picks"] == list(p_picks)
    assert rel_l2(logits("prompt", 8), p_logits) <= 1e-3
    for s in range(8):
        assert by[f"decode{s}"]["picks"] == [steps[s]], s
        assert rel_l2(logits(f"decode{s}", 1)[0], truth_logits[s]) <= 1e-3, s
    assert by["verify"]["picks"] == list(v_picks)
    assert rel_l2(logits("verify", 5), v_logits) <= 1e-3
    assert out["verify"]["kept"] == kept
    assert out["verify"]["written"] == list(v_picks[:kept])
    assert out["verify"]["position"] == len(prompt) + 8 + kept
    for s in range(2):
        assert by[f"after{s}"]["picks"] == [after[s]], s
        assert rel_l2(logits(f"after{s}", 1)[0], after_logits[s]) <= 1e-3, s
