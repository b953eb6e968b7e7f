"""The three model workloads at their stated sizes.

- Qwen2-0.5B shape (24 layers, MatMulNBits): a 512-token prompt, then
  greedy decode past position 520 in a 1024-token cache, against the
  float64 decoder over the oracle (identical tokens, logits rel-L2 <= 1e-3).
- Llama-3-8B shape (32 layers, Q4_K) in a 4096-token cache, near its end:
  one token layer by layer against the oracle (each layer's output given
  the same input and the same cache), the head's logits and pick; a
  replayed token graph equals the eager per-op path bit for bit; a verify
  batch equals sequential decoding; every logit finite.
- LFM2-1.2B shape (16 layers: 10 short-conv, 6 attention): verify batches
  of 5 (a token and 4 drafts, some agreeing, most random) with KV and conv
  state rollback write the oracle decoder's sequential greedy tokens, and
  every kept row's logits are the oracle's at that position.

Verify semantics follow src/handler.ts:1811-1887 and Engine.accept
(src/engine.ts:8063-8086): keep the longest agreeing prefix + 1.
"""
import dataclasses

import numpy as np
import pytest
import torch

from tests.helpers import rel_l2
from tests.model_oracle import OracleModel

pytestmark = pytest.mark.gpu


def _prompt(rng, n, vocab):
    return [int(t) for t in rng.integers(0, vocab, n)]


def _finite(t: torch.Tensor) -> bool:
    return bool(torch.isfinite(t).all())


def _verify_loop(eng, token, truth, rng, want_logits=None, total=None):
    """Verify batches of a token and 4 drafts from the engine's position:
    the first k drafts the true continuation (k cycles 0, 1, 2, 4), the rest
    random ids. Returns the tokens written. Checks every batch's logits are
    finite and, with want_logits (the sequential logits of each position
    after the start), that each kept row's logits are within 1e-3 of them."""
    total = total or len(truth)
    written, ks = [], (0, 1, 2, 4)
    it = 0
    while len(written) < total:
        k = ks[it % len(ks)]
        it += 1
        nxt = truth[len(written):len(written) + 4]
        drafts = nxt[:k] + _prompt(rng, 4 - len(nxt[:k]), eng.shape.vocab)
        rows = eng.forward([token] + drafts, draft=True).cpu().numpy()
        assert _finite(eng.logits[:5])
        kept = 1
        for i in range(4):
            if rows[i] != drafts[i]:
                break
            kept += 1
        if want_logits is not None:
            for j in range(kept):
                n = len(written) + j
                if n < len(want_logits):
                    got = eng.logits[j].cpu().numpy()
                    assert rel_l2(got, want_logits[n]) <= 1e-3, (n, j)
        eng.accept(kept)
        new = [int(x) for x in rows[:kept]]
        written += new
        token = new[-1]
    return written


# --------------------------------------------------------------- Qwen2-0.5B

def test_qwen2_05b_prompt_512_and_decode_past_520(hip):
    from webgllm_amd import engine as E
    w = E.Weights(E.QWEN2_05B, seed=5)
    eng = E.Engine(w, 1024)
    orc = OracleModel(w, 1024)
    rng = np.random.default_rng(12)
    prompt = _prompt(rng, 512, E.QWEN2_05B.vocab)
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok(), batch=128)
    got = eng.logits[:8].cpu().numpy()
    assert _finite(eng.logits[:8])
    assert rel_l2(got, logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    # greedy decode by graph replay, positions 512 .. 535
    first = int(picks[-1])
    toks = eng.decode(first, 24)
    last_logits = eng.logits[0].cpu().numpy()
    want, t = [], first
    for _ in range(24):
        lo, p = orc.forward_rows([t])
        t = p[0]
        want.append(t)
    assert eng.position == 536 and orc.position == 536
    assert toks == want
    assert rel_l2(last_logits, lo[0]) <= 1e-3


# ---------------------------------------------------------------- Llama-3-8B

P0_8B = 4070  # prompt length: the checks run at positions 4070 .. 4095


@pytest.fixture(scope="module")
def llama8b(hip):
    """The 8B-shape model in a 4096-token cache after a 4070-token prompt
    (GEMM batches): (engine, weights, the prompt's pick). Tests start from
    position 4070 with that token; rows before it are never rewritten."""
    from webgllm_amd import engine as E
    w = E.Weights(E.LLAMA3_8B, seed=31)
    eng = E.Engine(w, 4096)
    rng = np.random.default_rng(41)
    prompt = _prompt(rng, P0_8B, E.LLAMA3_8B.vocab)
    first = int(eng.forward(prompt).cpu()[-1])
    assert _finite(eng.logits[:6])
    yield eng, w, first
    del eng, w
    torch.cuda.empty_cache()


def _at_start(eng):
    eng.position = P0_8B
    eng.draft = None


def test_llama8b_layers_at_4070_against_oracle(llama8b):
    """One token at position 4070 run layer by layer: layers 0, 15 and 31
    (and the K, V rows they write) against the oracle given the engine's
    input h and the engine's cache rows 0..4069; the head's logits and
    pick against the oracle's over the engine's final h."""
    eng, w, first = llama8b
    _at_start(eng)
    checked = (0, 15, 31)
    orc = OracleModel(w, eng.ctx, layers=checked)
    p0 = eng.position
    for i in checked:
        orc.k[i][:p0] = eng.k_cache[i][:p0].cpu().numpy().view(np.uint16)
        orc.v[i][:p0] = eng.v_cache[i][:p0].cpu().numpy().view(np.uint16)
    eng.ids[0] = first
    eng.pos.fill_(p0)
    eng._embed_rows(1)
    for i in range(eng.shape.layers):
        h_in = eng.h[:1].cpu().numpy().copy()
        eng._layer_rows(i, 1, False)
        if i not in checked:
            continue
        h_out = eng.h[:1].cpu().numpy()
        want = orc.layer_rows(i, h_in, p0)
        assert np.isfinite(h_out).all()
        # the layer's own contribution (attention + FFN), not the residual
        assert rel_l2(h_out - h_in, want - h_in) <= 1e-3, i
        for got_c, want_c in ((eng.k_cache[i][p0], orc.k[i][p0]),
                              (eng.v_cache[i][p0], orc.v[i][p0])):
            got16 = got_c.cpu().numpy().view(np.float16).astype(np.float64)
            assert rel_l2(got16, want_c.view(np.float16).astype(np.float64)) <= 1e-3, i
    eng._head_rows(1)
    logits = eng.logits[:1].cpu().numpy()
    want_l, want_p = orc.head_rows(eng.h[:1].cpu().numpy())
    assert np.isfinite(logits).all()
    assert rel_l2(logits, want_l) <= 1e-3
    assert int(eng.next_ids[0]) == want_p[0]


def test_llama8b_graph_replay_equals_eager_near_4096(llama8b):
    """Eight tokens from position 4070 by graph replay, then the same eight
    steps eagerly through the per-op path from the same state: identical
    tokens, and the last step's logits bit for bit."""
    eng, _, first = llama8b
    _at_start(eng)
    eng.graph = None
    toks = eng.decode(first, 8)
    logits_graph = eng.logits[0].clone()
    assert _finite(logits_graph)
    _at_start(eng)
    t, eager = first, []
    for _ in range(8):
        t = int(eng.forward([t]).cpu()[0])
        eager.append(t)
    assert toks == eager
    assert torch.equal(logits_graph, eng.logits[0])


def test_llama8b_verify_equals_sequential_near_4096(llama8b):
    """From position 4070: 20 sequential greedy steps (their logits kept),
    then, from the same state, verify batches of 5 write the same tokens,
    and each kept row's logits are the sequential step's within 1e-3."""
    eng, _, first = llama8b
    _at_start(eng)
    seq, seq_logits, t = [], [], first
    for _ in range(20):
        t = int(eng.forward([t]).cpu()[0])
        assert _finite(eng.logits[:1])
        seq.append(t)
        seq_logits.append(eng.logits[0].cpu().numpy().copy())
    _at_start(eng)
    rng = np.random.default_rng(3)
    written = _verify_loop(eng, first, seq, rng, want_logits=seq_logits, total=20)
    assert written[:20] == seq
    assert eng.position <= eng.ctx


# ---------------------------------------------------------------- LFM2-1.2B

def test_lfm2_12b_verify_with_rollback_against_oracle(hip):
    """All 16 layers at full width: a 40-token prompt, then verify batches
    of 5 with mostly random drafts (each rejected draft rolls the KV
    position and the 10 conv states back) write the oracle's sequential
    greedy tokens; every kept row's logits are the oracle's."""
    from webgllm_amd import engine as E
    s = E.LFM2_12B
    w = E.Weights(s, seed=17)
    eng = E.Engine(w, 512)
    orc = OracleModel(w, 512)
    rng = np.random.default_rng(23)
    prompt = _prompt(rng, 40, s.vocab)
    picks = eng.forward(prompt).cpu().numpy()
    logits_o, picks_o = orc.forward(prompt, f16_weights=eng._prefill_ok(), batch=40)
    assert rel_l2(eng.logits[:8].cpu().numpy(), logits_o) <= 1e-3
    assert list(picks) == list(picks_o)
    first = int(picks[-1])
    truth, truth_logits, t = [], [], first
    for _ in range(24):
        lo, p = orc.forward_rows([t])
        t = p[0]
        truth.append(t)
        truth_logits.append(lo[0])
    written = _verify_loop(eng, first, truth, rng, want_logits=truth_logits, total=24)
    assert written[:24] == truth


def test_lfm2_12b_graph_verify_equals_oracle(hip):
    """All 16 layers at full width, every verify step one graph on the
    device (4 drafts from a table, mostly random, some the true
    continuation; accept and the 10 conv states' rollback on the device):
    the tokens written are the oracle's sequential greedy tokens."""
    from webgllm_amd import engine as E
    s = E.LFM2_12B
    w = E.Weights(s, seed=17)
    eng = E.Engine(w, 512)
    orc = OracleModel(w, 512)
    rng = np.random.default_rng(23)
    prompt = _prompt(rng, 40, s.vocab)
    first = int(eng.forward(prompt).cpu()[-1])
    orc.forward(prompt, f16_weights=eng._prefill_ok(), batch=40)
    truth = orc.decode(first, 40)
    # drafts: step s agrees for s % 3 tokens where the truth is known ahead
    # (assuming one token kept a step before), random after; 12 steps keep
    # at most 3 tokens each, within the 40 known
    drafts = []
    for st in range(12):
        k = st % 3
        nxt = truth[st:st + 4]
        drafts.append(nxt[:k] + _prompt(rng, 4 - len(nxt[:k]), s.vocab))
    tokens, kept = eng.verify_drafts(first, drafts)
    assert len(kept) == 12 and all(1 <= k <= 5 for k in kept)
    assert tokens == truth[:len(tokens)]
    assert eng.position == 40 + sum(kept)


def test_lfm2_12b_graph_decode_equals_verify_batches(hip):
    """The full model, no oracle: 30 tokens by graph replay from the
    prompt's state, then the same 30 from the same state (position and conv
    states restored) by verify batches with rollback: identical tokens."""
    from webgllm_amd import engine as E
    s = E.LFM2_12B
    w = E.Weights(s, seed=29)
    eng = E.Engine(w, 1024)
    rng = np.random.default_rng(31)
    prompt = _prompt(rng, 300, s.vocab)
    first = int(eng.forward(prompt).cpu()[-1])
    p0 = eng.position
    saved = {i: st.clone() for i, st in eng.state.items()}
    toks = eng.decode(first, 30)
    assert _finite(eng.logits[:1])
    eng.position = p0
    for i, st in saved.items():
        eng.state[i].copy_(st)
    written = _verify_loop(eng, first, toks, rng, total=30)
    assert written[:30] == toks


def test_lfm2_width_verify_layerwise_and_rollback(hip):
    """LFM2-1.2B width, 4 layers (conv, conv, attention, conv), verify
    batches of 5 at positions 9 onwards, run layer by layer: each layer's
    contribution for the 5 rows is the oracle's given the same input rows,
    conv state and cache rows (rel-L2 <= 1e-3); after accept(kept), kept
    cycling 1..5, every conv state equals bit for bit the oracle's state
    after the batch's first kept rows of the engine's own B | C | x rows,
    and the next batch continues from there. (An end-to-end float64
    comparison is not a kernel check on this model: the oracle's own
    float32 run differs from its float64 run by 1e-2 at position 9, where
    its residual grows from 0.9 to 470 over the four layers.)"""
    from oracle import oracle as O
    from webgllm_amd import engine as E
    s = dataclasses.replace(E.LFM2_12B, layers=4, conv_layers=(0, 1, 3))
    w = E.Weights(s, seed=43)
    eng, orc = E.Engine(w, 256), OracleModel(w, 256, head=False)
    eng.fuse_conv = False  # (the B | C | x rows stay in eng.bcx)
    rng = np.random.default_rng(47)
    prompt = _prompt(rng, 9, s.vocab)
    token = int(eng.forward(prompt).cpu()[-1])
    D, W = s.hidden, s.conv_kernel
    for rnd, kept in enumerate((1, 3, 5, 2, 4, 1)):
        p0 = eng.position
        for i in orc.state:
            orc.state[i] = eng.state[i].cpu().numpy().copy()
        for i in orc.k:
            orc.k[i][:p0] = eng.k_cache[i][:p0].cpu().numpy().view(np.uint16)
            orc.v[i][:p0] = eng.v_cache[i][:p0].cpu().numpy().view(np.uint16)
        before = {i: st.cpu().numpy().copy() for i, st in eng.state.items()}
        drafts = _prompt(rng, 4, s.vocab)
        eng.ids[:5].copy_(torch.tensor([token] + drafts, dtype=torch.int32))
        eng.pos.fill_(p0)
        eng._embed_rows(5)
        bcx = {}
        for i in range(s.layers):
            h_in = eng.h[:5].cpu().numpy().copy()
            eng._layer_rows(i, 5, keep_prefixes=True)
            if s.layer_type(i) == "conv":
                bcx[i] = eng.bcx[:5].cpu().numpy().copy()
            h_out = eng.h[:5].cpu().numpy()
            want = orc.layer_rows(i, h_in, p0)
            assert np.isfinite(h_out).all()
            assert rel_l2(h_out - h_in, want - h_in) <= 1e-3, (rnd, i)
        eng._head_rows(5)
        rows = eng.next_ids[:5].cpu().numpy()
        assert _finite(eng.logits[:5])
        eng.position = p0 + 5
        eng.draft = (p0, 5)
        eng.accept(kept)
        assert eng.position == p0 + kept
        for i, st in eng.state.items():
            _, want_state = O.short_conv(bcx[i][:kept], D, W, w.layers[i]["taps"].cpu().numpy(),
                                         before[i])
            assert np.array_equal(st.cpu().numpy(), want_state), (rnd, i, kept)
        token = int(rows[kept - 1])


def test_lfm2_conv_epilogue_equals_gemv_then_conv(hip):
    """The short convs in in_proj's epilogue against in_proj into the
    B | C | x rows then the conv kernel (which the layerwise test above
    checks against the oracle): the same logits, conv states and prefixes,
    bit for bit, over a prompt, verify batches with rollback and decode
    steps at LFM2-1.2B width."""
    from webgllm_amd import engine as E
    s = dataclasses.replace(E.LFM2_12B, layers=4, conv_layers=(0, 1, 3))
    w = E.Weights(s, seed=5)
    fused, plain = E.Engine(w, 256), E.Engine(w, 256)
    plain.fuse_conv = False
    rng = np.random.default_rng(9)
    prompt = _prompt(rng, 11, s.vocab)

    def same(step):
        assert torch.equal(fused.logits[:5].view(torch.int32),
                           plain.logits[:5].view(torch.int32)), step
        for i in fused.state:
            assert torch.equal(fused.state[i].view(torch.int32),
                               plain.state[i].view(torch.int32)), (step, i)

    ta, tb = fused.forward(prompt).cpu(), plain.forward(prompt).cpu()
    assert torch.equal(ta, tb)
    same("prompt")
    token = int(ta[-1])
    for step, kept in enumerate((1, 4, 2, 5, 3)):
        drafts = _prompt(rng, 4, s.vocab)
        ra = fused.forward([token] + drafts, draft=True).cpu()
        rb = plain.forward([token] + drafts, draft=True).cpu()
        assert torch.equal(ra, rb)
        for i in fused.prefixes:
            assert torch.equal(fused.prefixes[i][:5].view(torch.int32),
                               plain.prefixes[i][:5].view(torch.int32)), (step, i)
        same(step)
        fused.accept(kept)
        plain.accept(kept)
        same((step, kept))
        token = int(ra[kept - 1])
    for step in range(3):
        ta, tb = fused.forward([token]).cpu(), plain.forward([token]).cpu()
        assert torch.equal(ta, tb)
        same(("decode", step))
        token = int(ta[-1])
