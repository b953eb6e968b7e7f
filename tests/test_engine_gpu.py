"""End-to-end decode and speculative verify through the HIP kernels against
the CPU decoder over the oracle: identical greedy tokens, logits within
rel-L2 1e-3 (the parity bar)."""
import numpy as np
import pytest
import torch

from tests.helpers import rel_l2
from tests.model_oracle import OracleModel

pytestmark = pytest.mark.gpu


def _shape(fmt, conv_layers=(), qk_norm=False, layers=3, hidden=256, heads=4, kv=2, hd=64,
           inter=512, vocab=1024, embed_fmt=None):
    from webgllm_amd.engine import ModelShape
    return ModelShape(f"tiny-{fmt}", hidden, layers, heads, kv, hd, inter, vocab, fmt,
                      qk_norm=qk_norm, conv_layers=conv_layers, embed_fmt=embed_fmt)


FAMILIES = {
    "llama-q4_k": dict(fmt="q4_k"),
    "qwen-nbits": dict(fmt="nbits", heads=7, kv=1),
    "lfm2-q4_0": dict(fmt="q4_0", conv_layers=(0, 2), qk_norm=True),
    "q4_k-rowgroup": dict(fmt="q4_k_rowgroup"),
    "q4_k-records": dict(fmt="q4_k_records"),
    # as real GGUF files: a Q6_K embedding and output head; Q8_0 tensors; and
    # tensors the loader requantizes to 8 bits (Q4_K_M's Q6_K/Q5_K ones)
    "gguf-q4_k-q6_k-head": dict(fmt="q4_k_rowgroup", embed_fmt="q6_k"),
    "gguf-q8_0": dict(fmt="q8_0", conv_layers=(1,), qk_norm=True),
    "gguf-requant-q8": dict(fmt="q8", embed_fmt="q6_k", heads=7, kv=1),
}


def _pair(family, seed=0, ctx=256, **kw):
    from webgllm_amd.engine import Engine, Weights
    args = dict(FAMILIES[family])
    args.update(kw)
    w = Weights(_shape(**args), seed=seed)
    return Engine(w, ctx), OracleModel(w, ctx)


def _prompt(rng, n, vocab):
    return [int(t) for t in rng.integers(0, vocab, n)]


@pytest.mark.parametrize("family", list(FAMILIES))
def test_prompt_logits_and_greedy_decode(hip, family):
    eng, orc = _pair(family)
    rng = np.random.default_rng(1)
    prompt = _prompt(rng, 21, eng.shape.vocab)
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok())
    got = eng.logits[:len(prompt) % 8 or 8].cpu().numpy()
    assert rel_l2(got, logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    # greedy decode by graph replay
    first = int(picks[-1])
    toks = eng.decode(first, 12)
    toks_o = orc.decode(first, 12)
    assert toks == toks_o


@pytest.mark.parametrize("family", ["lfm2-q4_0", "llama-q4_k"])
def test_verify_accept_matches_sequential(hip, family):
    """A token and 4 drafts in one batch, keeping the agreeing prefix + 1
    (src/handler.ts:1811-1887, Engine.accept src/engine.ts:8063-8086): the
    tokens written equal sequential greedy decoding."""
    eng, orc = _pair(family, seed=3)
    rng = np.random.default_rng(5)
    prompt = _prompt(rng, 10, eng.shape.vocab)
    token = int(eng.forward(prompt).cpu().numpy()[-1])
    seq = orc.forward(prompt)[1][-1]
    assert token == seq
    want = orc.decode(token, 12)
    written = []
    while len(written) < 10:
        # drafts: the true continuation for the first k, then random ids
        k = len(written) % 3
        truth = want[len(written):len(written) + 4]
        drafts = truth[:k] + [int(x) for x in rng.integers(0, eng.shape.vocab, 4 - k)]
        rows = eng.forward([token] + drafts, draft=True).cpu().numpy()
        kept = 1
        for i in range(4):
            if rows[i] != drafts[i]:
                break
            kept += 1
        eng.accept(kept)
        new = [int(x) for x in rows[:kept]]
        written += new
        token = new[-1]
    assert written[:10] == want[:10]


def test_graph_replay_equals_eager(hip):
    eng, _ = _pair("lfm2-q4_0", seed=7)
    rng = np.random.default_rng(9)
    prompt = _prompt(rng, 9, eng.shape.vocab)
    first = int(eng.forward(prompt).cpu().numpy()[-1])
    p = eng.position
    toks_graph = eng.decode(first, 8)
    # eager replay of the same steps from the same state
    eng2, _ = _pair("lfm2-q4_0", seed=7)
    eng2.forward(prompt)
    t, eager = first, []
    for _ in range(8):
        t = int(eng2.forward([t]).cpu().numpy()[0])
        eager.append(t)
    assert eng.position == p + 8
    assert toks_graph == eager


def test_engine_errors(hip):
    eng, _ = _pair("llama-q4_k", ctx=32)
    with pytest.raises(ValueError, match="cache holds"):
        eng.forward(list(range(33)))
    with pytest.raises(ValueError, match="8 tokens at most"):
        eng.forward(list(range(9)), draft=True)
    with pytest.raises(ValueError, match="No draft batch"):
        eng.accept(1)
    eng.forward([1, 2, 3], draft=True)
    with pytest.raises(ValueError, match="keep 4 of a 3"):
        eng.accept(4)


@pytest.mark.parametrize("name,layers", [("qwen2", 2), ("llama3", 2), ("lfm2", 3)])
def test_full_width_shapes(hip, name, layers):
    """The workloads' real widths, heads and vocabularies (fewer layers, so
    the CPU decoder stays quick): identical greedy tokens."""
    from webgllm_amd import engine as E
    import dataclasses
    base = {"qwen2": E.QWEN2_05B, "llama3": E.LLAMA3_8B, "lfm2": E.LFM2_12B}[name]
    conv = tuple(i for i in base.conv_layers if i < layers)
    if name == "lfm2":
        conv = (0, 2)
    shape = dataclasses.replace(base, layers=layers, conv_layers=conv)
    w = E.Weights(shape, seed=11)
    ctx = 128
    eng, orc = E.Engine(w, ctx), OracleModel(w, ctx)
    rng = np.random.default_rng(2)
    prompt = _prompt(rng, 12, shape.vocab)
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok())
    got = eng.logits[:4].cpu().numpy()
    assert rel_l2(got, logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    first = int(picks[-1])
    assert eng.decode(first, 4) == orc.decode(first, 4)


@pytest.mark.parametrize("family", ["q4_k-rowgroup", "lfm2-q4_0", "qwen-nbits"])
def test_long_prompt_through_gemm_batches(hip, family, monkeypatch):
    """A 600-token prompt: rows 0..591 in GEMM batches of 512 and 80 (MFMA
    GEMMs, flash prefill attention, batched short conv), the last 8 through
    the few-token path. Logits of the last batch and the greedy tokens after
    it match the CPU decoder."""
    from webgllm_amd import engine as E
    monkeypatch.setattr(E, "PREFILL_ROWS", 512)
    eng, orc = _pair(family, seed=23, ctx=640)
    assert eng._prefill_ok()
    rng = np.random.default_rng(17)
    prompt = _prompt(rng, 600, eng.shape.vocab)
    assert E.PREFILL_ROWS < 592
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok())
    assert rel_l2(eng.logits[:8].cpu().numpy(), logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    first = int(picks[-1])
    assert eng.decode(first, 6) == orc.decode(first, 6)


def test_capture_leaves_the_cache_alone(hip):
    """Capturing the decode step after a prompt runs it once eagerly: every
    cache row before the current position stays as the prompt wrote it, and
    graph replay then decodes as the CPU decoder does."""
    eng, orc = _pair("qwen-nbits", seed=0)
    rng = np.random.default_rng(1)
    prompt = _prompt(rng, 21, eng.shape.vocab)
    first = int(eng.forward(prompt).cpu()[-1])
    orc.forward(prompt)
    before = {i: (k[:21].clone(), v[:21].clone()) for i, (k, v) in
              enumerate(zip(eng.k_cache.values(), eng.v_cache.values()))}
    eng.capture_step(first)
    for i, (k, v) in enumerate(zip(eng.k_cache.values(), eng.v_cache.values())):
        assert torch.equal(k[:21], before[i][0]) and torch.equal(v[:21], before[i][1])
    assert eng.decode(first, 12) == orc.decode(first, 12)


@pytest.mark.parametrize("family,freq", [("llama-q4_k", 0.0), ("lfm2-q4_0", 0.0),
                                         ("gguf-q4_k-q6_k-head", 0.0), ("llama-q4_k", 0.4),
                                         ("lfm2-q4_0", 0.25)])
def test_sampled_generate_with_penalties(hip, family, freq):
    """Sampled decoding through the GPU's candidate pick and the host
    sampler (or, with a frequency penalty, the whole row read back and
    penalized on the host): at temperature 0 with repetition, presence and
    frequency penalties it writes the oracle decoder's penalized greedy
    tokens (the host sampler over the oracle's full logits); at temperature
    0.8 two seeded runs write the same tokens."""
    import random as pyrandom
    from webgllm_amd.sampler import Sampler
    eng, orc = _pair(family, seed=2)
    rng = np.random.default_rng(11)
    prompt = _prompt(rng, 13, eng.shape.vocab)
    # a small vocabulary repeats tokens, so the frequency counts matter
    got = eng.generate(prompt, 12, Sampler(0, 40, repetition_penalty=1.3,
                                           presence_penalty=0.2, frequency_penalty=freq))
    s = Sampler(0, 40, repetition_penalty=1.3, presence_penalty=0.2, frequency_penalty=freq)
    s.see(prompt)
    want, tokens = [], prompt
    for _ in range(12):
        logits, _ = orc.forward(tokens)
        t = s.sample(np.ascontiguousarray(logits[-1], np.float32))
        want.append(t)
        s.see([t], True)
        tokens = [t]
    assert got == want
    runs = []
    for _ in range(2):
        e2, _ = _pair(family, seed=2)
        r = pyrandom.Random(5)
        runs.append(e2.generate(prompt, 10, Sampler(0.8, 50, top_p=0.95,
                                                    repetition_penalty=1.1), r.random))
    assert runs[0] == runs[1] and all(0 <= t < eng.shape.vocab for t in runs[0])


@pytest.mark.parametrize("family", ["llama-q4_k", "lfm2-q4_0"])
def test_sampled_generate_guess_changes_no_token(hip, family):
    """The guessed forward (the row's greedy pick run ahead while the host
    draws, src/engine.ts:8095-8150) changes no token: seeded runs with and
    without it write the same tokens, at temperatures where guesses both
    hit and miss (LFM2's conv states put back after a miss), and leave the
    engine at the same position with the same state: the next forward's
    logits are equal bit for bit."""
    import random as pyrandom
    from webgllm_amd.sampler import Sampler
    rng = np.random.default_rng(21)
    hits = misses = 0
    for temp, steps in ((0.9, 16), (0.05, 16)):
        runs, ends = [], []
        for guess in (False, True):
            e, _ = _pair(family, seed=3)
            prompt = _prompt(np.random.default_rng(31), 9, e.shape.vocab)
            toks = e.generate(prompt, steps, Sampler(temp, 40, repetition_penalty=1.1),
                              pyrandom.Random(7).random, guess=guess)
            runs.append(toks)
            if guess:
                hits += e.guess_hits
                misses += e.guess_misses
                assert e.guess_hits + e.guess_misses == steps - 1
            e.forward([toks[-1]])
            ends.append((e.position, e.logits[:1].clone()))
        assert runs[0] == runs[1]
        assert ends[0][0] == ends[1][0] == 9 + steps
        assert torch.equal(ends[0][1], ends[1][1])
    assert hits > 0 and misses > 0, (hits, misses)


def test_sampled_generate_without_top_k_reads_the_row(hip):
    """top_k 0 at temperature 0.7: the GPU's chunks could not hold the
    whole distribution, so the row is read back and sampled on the host;
    two seeded runs write the same tokens. And the two paths' distributions
    for one row are the same set of (token, probability), bit for bit: the
    GPU's candidates of a top-40 pick and the host's whole penalized row.
    (Their draws may differ: a draw walks the distribution in its heap
    order, which depends on the order the candidates come in.)"""
    import random as pyrandom
    from webgllm_amd.sampler import GpuPick, Sampler
    eng, _ = _pair("llama-q4_k", seed=4)
    rng = np.random.default_rng(12)
    prompt = _prompt(rng, 11, eng.shape.vocab)
    runs = []
    for _ in range(2):
        e2, _ = _pair("llama-q4_k", seed=4)
        runs.append(e2.generate(prompt, 8, Sampler(0.7, 0, repetition_penalty=1.1),
                                pyrandom.Random(9).random))
    assert runs[0] == runs[1] and all(0 <= t < eng.shape.vocab for t in runs[0])
    eng.forward(prompt)
    row = eng.logits[(len(prompt) - 1) % 8]
    s_gpu = Sampler(0.7, 40, repetition_penalty=1.1, presence_penalty=0.3)
    s_host = Sampler(0.7, 40, repetition_penalty=1.1, presence_penalty=0.3)
    pick = GpuPick(eng.shape.vocab, 64)
    pick.see(s_gpu.see(prompt))
    s_host.see(prompt)
    d_gpu = pick(row, s_gpu)
    d_host = s_host.distribution(row.cpu().numpy().copy(), penalize=True)
    a, b = np.argsort(d_gpu.ids), np.argsort(d_host.ids)
    assert d_gpu.ids.size == d_host.ids.size == 40
    assert np.array_equal(d_gpu.ids[a], d_host.ids[b])
    assert np.array_equal(d_gpu.p[a], d_host.p[b])


def _host_verify_recording(eng, token, truth, rng, steps):
    """The host verify loop (forward(draft=True) + accept) for `steps`
    steps, drafts partly the true continuation: (tokens written, kept
    counts, the drafts fed)."""
    written, kept_log, fed = [], [], []
    for s in range(steps):
        k = s % 3
        nxt = truth[len(written):len(written) + 4]
        drafts = nxt[:k] + [int(x) for x in rng.integers(0, eng.shape.vocab, 4 - len(nxt[:k]))]
        fed.append(drafts)
        rows = eng.forward([token] + drafts, draft=True).cpu().numpy()
        kept = 1
        for i in range(4):
            if rows[i] != drafts[i]:
                break
            kept += 1
        eng.accept(kept)
        kept_log.append(kept)
        written += [int(x) for x in rows[:kept]]
        token = written[-1]
    return written, kept_log, fed


@pytest.mark.parametrize("family,table", [("lfm2-q4_0", 1024), ("lfm2-q4_0", 3),
                                          ("llama-q4_k", 1024)])
def test_graph_verify_equals_host_verify(hip, family, table, monkeypatch):
    """Verify steps replayed as one captured graph each (drafts from a
    device table, picks, accept and conv rollback on the device) write the
    host loop's tokens and keep its counts, step for step; with a table of
    3 rows the run is split and read back between parts."""
    from webgllm_amd import engine as E
    eng, orc = _pair(family, seed=3)
    rng = np.random.default_rng(5)
    prompt = _prompt(rng, 10, eng.shape.vocab)
    token = int(eng.forward(prompt).cpu()[-1])
    orc.forward(prompt)
    truth = orc.decode(token, 64)  # 12 steps keep at most 3 each here
    written, kept, fed = _host_verify_recording(eng, token, truth, rng, 12)
    assert written == truth[:len(written)]
    eng2, _ = _pair(family, seed=3)
    monkeypatch.setattr(E.Engine, "VERIFY_TABLE", table)
    eng2.forward(prompt)
    p0 = eng2.position
    tokens, kept2 = eng2.verify_drafts(token, fed)
    assert kept2 == kept
    assert tokens == written
    assert eng2.position == p0 + sum(kept)
    # and it goes on from there as sequential decoding does
    assert eng2.decode(tokens[-1], 4) == truth[len(written):len(written) + 4]



def test_cache_grows_on_demand(hip):
    """The attention caches start at KV_START positions and grow as the
    prompt and the decode need them (whole KV_STEP steps, at least doubling):
    the rows already written are kept, the decode graph captured over the
    smaller caches is captured again, and the tokens are the oracle
    decoder's across the growth; reset shrinks the caches back."""
    from webgllm_amd import engine as E
    eng, orc = _pair("lfm2-q4_0", seed=2, ctx=3000)
    assert eng.kv_positions == E.KV_START == 1024
    rng = np.random.default_rng(9)
    prompt = _prompt(rng, 1016, eng.shape.vocab)
    picks = eng.forward(prompt).cpu().numpy()
    assert eng.kv_positions == 1024
    _, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok(), batch=128)
    assert list(picks) == list(picks_o)
    first = int(picks[-1])
    toks = eng.decode(first, 4)
    assert eng.kv_positions == 1024
    layer = next(iter(eng.k_cache))
    kept_k = eng.k_cache[layer][:1020].clone()
    kept_v = eng.v_cache[layer][:1020].clone()
    graph = eng.graph
    toks += eng.decode(toks[-1], 12)  # positions 1020 .. 1031: 2048 positions
    assert eng.kv_positions == 2048 and eng.graph is not graph
    assert torch.equal(eng.k_cache[layer][:1020], kept_k)
    assert torch.equal(eng.v_cache[layer][:1020], kept_v)
    assert toks == orc.decode(first, 16)
    with pytest.raises(ValueError, match="holds 3000 tokens"):
        eng.reserve(3001)
    eng.reset()
    orc.reset()
    assert eng.kv_positions == 1024
    short = _prompt(rng, 12, eng.shape.vocab)
    first = int(eng.forward(short).cpu()[-1])
    orc.forward(short)
    assert eng.decode(first, 6) == orc.decode(first, 6)


@pytest.mark.parametrize("family", ["lfm2-q4_0", "llama-q4_k"])
def test_verify_grows_the_cache(hip, family):
    """Verify steps whose run passes the caches' size: the run reserves its
    room first (the verify graph captured again over the new caches) and
    writes the host loop's tokens, which are the oracle decoder's."""
    eng, orc = _pair(family, seed=4, ctx=2048)
    rng = np.random.default_rng(6)
    prompt = _prompt(rng, 1018, eng.shape.vocab)
    token = int(eng.forward(prompt).cpu()[-1])
    orc.forward(prompt, f16_weights=eng._prefill_ok(), batch=128)
    truth = orc.decode(token, 64)
    written, kept, fed = _host_verify_recording(eng, token, truth, rng, 12)
    assert written == truth[:len(written)]
    eng2, _ = _pair(family, seed=4, ctx=2048)
    eng2.forward(prompt)
    eng2.capture_verify(5)  # over the 1024-position caches
    assert eng2.kv_positions == 1024
    tokens, kept2 = eng2.verify_drafts(token, fed)
    assert eng2.kv_positions == 2048
    assert kept2 == kept and tokens == written
