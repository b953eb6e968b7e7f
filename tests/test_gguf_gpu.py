"""GGUF files through the loader onto the device: rowsToFloats bit-exact per
ggml type, every loaded matrix equal (row for row, in logical order) to the
oracle's reading of the file's own tensors by the reference's storage rules
(src/load-gguf.ts:475-555), and the loaded model decoding the oracle
decoder's tokens. The files are written here from the format (tests/
gguf_writer.py), shaped as LFM2 GGUFs are (src/lfm2-gguf.test.ts:11-39)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import gguf_writer as W
from tests.helpers import rel_l2
from tests.model_oracle import OracleModel, dense_of

pytestmark = pytest.mark.gpu

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 3, 8, 12, 13, 14


def _blocks(rng, t, rows, K):
    """Random ggml blocks of type t, their scales as the engine's own random
    weights have them (weights of about 0.02): a random model's conditioning
    depends on them, and with larger or differently biased weights even a
    float32 run of the oracle drifts from its float64 run by 1e-3."""
    w, b = W.BLOCK[t]
    n = rows * K // w
    raw = rng.integers(0, 256, (n, b), dtype=np.uint8)

    def halves(lo, hi):
        return rng.uniform(lo, hi, n).astype(np.float16).view(np.uint16)
    if t == Q4_0:
        h = halves(0.002, 0.006)
        raw[:, 0], raw[:, 1] = h & 255, h >> 8
    elif t == Q8_0:
        h = halves(1e-4, 3e-4)
        raw[:, 0], raw[:, 1] = h & 255, h >> 8
    elif t == Q4_1:
        d, m = halves(0.002, 0.005), halves(-0.04, -0.02)
        raw[:, 0], raw[:, 1], raw[:, 2], raw[:, 3] = d & 255, d >> 8, m & 255, m >> 8
    elif t == Q4_K:
        d, m = halves(1e-4, 2e-4), halves(4e-4, 8e-4)
        raw[:, 0], raw[:, 1], raw[:, 2], raw[:, 3] = d & 255, d >> 8, m & 255, m >> 8
    elif t == Q5_K:
        d, m = halves(5e-5, 1e-4), halves(4e-4, 8e-4)
        raw[:, 0], raw[:, 1], raw[:, 2], raw[:, 3] = d & 255, d >> 8, m & 255, m >> 8
    elif t == Q6_K:
        h = halves(1e-5, 2e-5)
        raw[:, 208], raw[:, 209] = h & 255, h >> 8
    elif t == F16:
        return (rng.standard_normal(rows * K) * 0.02).astype(np.float16)
    elif t == F32:
        return (rng.standard_normal(rows * K) * 0.02).astype(np.float32)
    return raw.reshape(-1)


MIXES = {
    # every layer matrix in one type, as Q4_0 and Q8_0 files have them
    "q4_0": dict(default=Q4_0),
    "q8_0": dict(default=Q8_0),
    # a Q4_K_M-like mix: 4-bit Q4_K, Q6_K values and down projections (their
    # fused matrices then go to 8 bits through floats), a Q5_K and a Q4_1
    # tensor (unsloth's quants have a few), an F16 projection
    "q4_k_m": dict(default=Q4_K, attn_v=Q6_K, ffn_down=Q6_K,
                   **{"blk.2.ffn_down": Q5_K, "blk.0.shortconv.out_proj": Q4_1,
                      "blk.2.shortconv.out_proj": F16}),
}


def lfm2_file(path, layers=3, kv=(0, 2, 0), mix="q4_0", emb=Q6_K, arch="lfm2", sliding=0,
              output_head=False, seed=0, D=256, heads=4, hd=64, F=512, vocab=1024):
    """An LFM2 GGUF: conv layers where kv is 0, attention elsewhere; returns
    the path (and keeps the tensors on the returned path's `.tensors`)."""
    rng = np.random.default_rng(seed)
    types = MIXES[mix]
    tensors = []

    def ty(name):
        for key in (name, name.split(".", 2)[-1]):
            if key in types:
                return types[key]
        return types["default"]

    def mat(name, K, rows):
        t = ty(name)
        tensors.append((name + ".weight", (K, rows), t, _blocks(rng, t, rows, K)))

    def vec(name, n, shape=None, scale=0.1, base=1.0):
        v = (base + scale * rng.standard_normal(n)).astype(np.float32)
        tensors.append((name + ".weight", shape or (n,), F32, v))

    for i in range(layers):
        p = f"blk.{i}."
        vec(p + "attn_norm", D)
        vec(p + "ffn_norm", D)
        if kv[i] == 0:
            mat(p + "shortconv.in_proj", D, 3 * D)
            mat(p + "shortconv.out_proj", D, D)
            vec(p + "shortconv.conv", 3 * D, (3, D), scale=0.5, base=0.0)
        else:
            mat(p + "attn_q", D, heads * hd)
            mat(p + "attn_k", D, kv[i] * hd)
            mat(p + "attn_v", D, kv[i] * hd)
            mat(p + "attn_output", heads * hd, D)
            vec(p + "attn_q_norm", hd)
            vec(p + "attn_k_norm", hd)
        mat(p + "ffn_gate", D, F)
        mat(p + "ffn_up", D, F)
        mat(p + "ffn_down", F, D)
    vec("token_embd_norm", D)
    tensors.append(("token_embd.weight", (D, vocab), emb, _blocks(rng, emb, vocab, D)))
    if output_head:
        tensors.append(("output.weight", (D, vocab), emb, _blocks(rng, emb, vocab, D)))
    meta = [("general.architecture", W.STRING, arch), ("general.name", W.STRING, "tiny-lfm2"),
            (f"{arch}.block_count", W.U32, layers), (f"{arch}.embedding_length", W.U32, D),
            (f"{arch}.attention.head_count", W.U32, heads),
            (f"{arch}.attention.head_count_kv", W.ARRAY, (W.I32, list(kv))),
            (f"{arch}.feed_forward_length", W.U32, F),
            (f"{arch}.context_length", W.U32, 128000),
            (f"{arch}.rope.freq_base", W.F32, 1000000.0),
            (f"{arch}.attention.layer_norm_rms_epsilon", W.F32, 1e-5),
            (f"{arch}.shortconv.l_cache", W.U32, 3),
            (f"{arch}.attention.sliding_window", W.U32, sliding)]
    W.write_gguf(path, meta, tensors)
    lfm2_file.tensors = {n: (dims, t, data) for n, dims, t, data in tensors}
    return path


def _floats(t, data, rows, K):
    """The oracle's rowsToFloats (src/load-gguf.ts:557-580)."""
    if t == F32:
        return np.asarray(data, np.float32).reshape(rows, K)
    if t == F16:
        return np.asarray(data, np.float16).astype(np.float32).reshape(rows, K)
    fn = {Q8_0: O.dequantize_q8_0, Q4_1: O.dequantize_q4_1, Q4_K: O.dequantize_q4_k,
          Q5_K: O.dequantize_q5_k, Q6_K: O.dequantize_q6_k}[t]
    return fn(np.asarray(data, np.uint8), rows, K)


def _expected(tensors, names, K):
    """A fused matrix as the reference's loader stores it (matrixStorage +
    packRows), dequantized by the oracle, rows in logical order."""
    parts = [tensors[n] for n in names]
    types = {t for _, t, _ in parts}
    N = sum(d[1] for d, _, _ in parts)
    if types == {Q4_K} and K % 256 == 0:
        out = []
        for dims, _, data in parts:
            qm = O.QuantMatrix(dims[1], K, "halves")
            O.pack_q4_k(qm, 0, data, dims[1])
            out.append(qm.dense())
        return np.concatenate(out)
    if types == {Q4_0}:
        out = []
        for dims, _, data in parts:
            qm = O.QuantMatrix(dims[1], K)
            O.pack_q4_0(qm, 0, data, dims[1])
            out.append(qm.dense())
        return np.concatenate(out)
    if types == {Q8_0}:
        return np.concatenate([O.dequantize_q8_0(data, dims[1], K) for dims, _, data in parts])
    wm = O.WideMatrix(N, K, 8)
    O.quantize_q8(wm, 0, np.concatenate([_floats(t, data, dims[1], K)
                                         for dims, t, data in parts]))
    return wm.dense()


@pytest.mark.parametrize("t,K", [(F32, 96), (F16, 7), (Q8_0, 64), (Q4_1, 96), (Q4_K, 512),
                                 (Q5_K, 256), (Q6_K, 768)])
def test_rows_to_floats_bit_exact(hip, t, K):
    from webgllm_amd import lib as L
    rng = np.random.default_rng(t + K)
    rows = 6
    data = _blocks(rng, t, rows, K)
    if t == Q4_K:  # a zero-scale sub-block and extreme halves too
        from tests.helpers import random_q4_k_bytes
        data = random_q4_k_bytes(rng, rows, K, zero_scale_every=3, extreme=True)
    src = torch.from_numpy(np.ascontiguousarray(data).view(np.uint8).copy()).cuda()
    out = torch.empty((rows, K), dtype=torch.float32, device="cuda")
    L.check(L.load().wg_rows_to_floats(t, src.data_ptr(), rows, K, out.data_ptr(), None))
    torch.cuda.synchronize()
    want = _floats(t, data, rows, K)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rows_to_floats_rejects(hip):
    from webgllm_amd import lib as L
    lib = L.load()
    assert lib.wg_rows_to_floats(Q4_0, 0x1000, 1, 32, 0x2000, None) == -6
    assert lib.wg_rows_to_floats(Q4_K, 0x1000, 1, 96, 0x2000, None) == -1


@pytest.mark.parametrize("mix,emb", [("q4_0", Q6_K), ("q8_0", Q8_0), ("q4_k_m", Q6_K),
                                     ("q4_0", F16)])
def test_loaded_matrices_are_the_files(hip, tmp_path, mix, emb):
    from webgllm_amd import lib as L
    from webgllm_amd.load_gguf import load_gguf
    path = lfm2_file(tmp_path / "m.gguf", mix=mix, emb=emb)
    tensors = lfm2_file.tensors
    w = load_gguf(path)
    s = w.shape
    D, F = s.hidden, s.intermediate
    for i, lw in enumerate(w.layers):
        p = f"blk.{i}."
        fused = {"gate_up": ([p + "ffn_gate.weight", p + "ffn_up.weight"], D),
                 "down": ([p + "ffn_down.weight"], F)}
        if s.layer_type(i) == "conv":
            fused["in_proj"] = ([p + "shortconv.in_proj.weight"], D)
            fused["out_proj"] = ([p + "shortconv.out_proj.weight"], D)
            taps = tensors[p + "shortconv.conv.weight"][2].reshape(D, 3)
            assert np.array_equal(lw["taps"].cpu().numpy(), taps)
        else:
            fused["qkv"] = ([p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"], D)
            fused["o"] = ([p + "attn_output.weight"], s.heads * s.head_dim)
            assert np.array_equal(lw["q_norm"].cpu().numpy(), tensors[p + "attn_q_norm.weight"][2])
        for key, (names, K) in fused.items():
            want = _expected(tensors, names, K)
            got = dense_of(lw[key])
            assert got.shape == want.shape, key
            assert np.array_equal(got, want), f"layer {i} {key}"
        for norm, name in (("op_norm", "attn_norm"), ("ffn_norm", "ffn_norm")):
            assert np.array_equal(lw[norm].cpu().numpy(), tensors[p + name + ".weight"][2])
    assert np.array_equal(w.final_norm.cpu().numpy(), tensors["token_embd_norm.weight"][2])
    dims, t, data = tensors["token_embd.weight"]
    if t == Q6_K:
        want = O.dequantize_q6_k(data, dims[1], D)
        assert w.embedding.layout == L.LAYOUT_Q6K
    elif t == Q8_0:
        want = O.dequantize_q8_0(data, dims[1], D)
    else:
        wm = O.WideMatrix(dims[1], D, 8)
        O.quantize_q8(wm, 0, _floats(t, data, dims[1], D))
        want = wm.dense()
    assert np.array_equal(dense_of(w.embedding), want)
    if mix == "q4_k_m":  # the storage the rules pick
        assert w.layers[1]["qkv"].layout == L.LAYOUT_Q8          # Q4_K q, k + Q6_K v
        assert w.layers[1]["o"].zero == L.ZERO_Q4K               # Q4_K alone: 4 bits
        assert w.layers[0]["down"].layout == L.LAYOUT_Q8         # Q6_K


@pytest.mark.parametrize("mix,emb", [("q4_0", Q6_K), ("q4_k_m", Q6_K), ("q8_0", Q8_0)])
def test_loaded_model_decodes_the_oracles_tokens(hip, tmp_path, mix, emb):
    from webgllm_amd.engine import Engine
    from webgllm_amd.load_gguf import load_gguf
    w = load_gguf(lfm2_file(tmp_path / "m.gguf", mix=mix, emb=emb, seed=3))
    eng, orc = Engine(w, 256), OracleModel(w, 256)
    rng = np.random.default_rng(7)
    prompt = [int(x) for x in rng.integers(0, w.shape.vocab, 21)]
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok())
    assert rel_l2(eng.logits[:len(prompt) % 8].cpu().numpy(), logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    first = int(picks[-1])
    assert eng.decode(first, 10) == orc.decode(first, 10)
