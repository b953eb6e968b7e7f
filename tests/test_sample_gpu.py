"""Sampling candidates on the GPU (wg_pick_candidates) against the oracle's
restatement of the reference's PENALIZED + CHUNK_MAX / RANK / GATHER, bit
for bit, and the host sampler over them against the same sampler over the
full penalized vocabulary."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _case(rng, M, V):
    logits = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    logits[:, rng.integers(0, V, 50)] = 9.0                       # ties across chunks
    mask = rng.choice([0, 0, 0, 1, 2, 3], V).astype(np.uint8)     # prompt, never, written
    seen = [[int(rng.integers(0, V)), int(rng.choice([0, 1, 3])), int(rng.integers(0, M)),
             int(rng.integers(1, M + 1))] for _ in range(10)]
    seen.append([int(np.argmax(logits[0])), 3, 0, M])              # the top token, seen
    return logits, mask, seen


@pytest.mark.parametrize("M,V,count", [(1, 128256, 64), (5, 1000, 3), (3, 65536, 8),
                                       (2, 513, 3), (1, 131072, 64), (2, 262144, 64)])
@pytest.mark.parametrize("allow", [False, True])
def test_candidates_match_oracle(hip, M, V, count, allow):
    from webgllm_amd import ops
    rng = np.random.default_rng(V + M + allow)
    logits, mask, seen = _case(rng, M, V)
    allowed = None
    if allow:  # a token bitmap per row; row M - 1 allows only a few tokens
        words = (V + 31) // 32
        allowed = rng.integers(0, 2 ** 32, (M, words), dtype=np.uint64).astype(np.uint32)
        allowed[M - 1] = 0
        allowed[M - 1, 3] = 0x0F0F0F0F
    row0 = 2
    kw = dict(mask=mask, seen_rows=seen, row0=row0, penalty=1.3, presence=0.7,
              allowed=allowed)
    want_c, want_v = O.pick_candidates(logits, count, **kw)
    got_c, got_v = ops.pick_candidates(
        _t(logits), count, mask=_t(mask), seen_rows=seen, row0=row0, penalty=1.3,
        presence_penalty=0.7, allowed=None if allowed is None else _t(allowed.view(np.int32)))
    assert np.array_equal(got_c.cpu().numpy(), want_c)
    assert np.array_equal(got_v.cpu().numpy().view(np.uint32), want_v.view(np.uint32))


@pytest.mark.parametrize("settings", [dict(temperature=0.8, top_k=40, top_p=0.9),
                                      dict(temperature=1.0, top_k=64, min_p=0.05),
                                      dict(temperature=0.0, top_k=50)])
def test_sampling_from_candidates_equals_full_vocabulary(hip, settings):
    """The reference's pick: the GPU penalizes and keeps the top chunks, the
    host samples with penalize = false. For top_k <= count (each of the k
    largest tokens lies in a chunk whose maximum is among the k largest)
    the kept tokens, their probabilities and a uniform draw's token equal
    those of the sampler over the whole penalized vocabulary (as ids
    ascend)."""
    from webgllm_amd import ops
    from webgllm_amd.sampler import Sampler, draw_at
    rng = np.random.default_rng(5)
    V = 128256
    logits = (rng.standard_normal((1, V)) * 2).astype(np.float32)
    window = [int(t) for t in rng.integers(0, V, 64)]
    s = Sampler(repetition_penalty=1.2, presence_penalty=0.3, **settings)
    s.see(window[:40])
    s.see(window[40:], True)
    mask = np.zeros(V, np.uint8)
    for t, st in s.window.entries():
        mask[t] = st
    chunks, cand = ops.pick_candidates(_t(logits), 64, mask=_t(mask), penalty=1.2,
                                       presence_penalty=0.3)
    d = s.candidates(chunks.cpu().numpy()[0], cand.cpu().numpy()[0])
    full = logits[0].copy()
    dfull = s.distribution(full)  # the host penalizes, over every token
    o1, o2 = np.argsort(d.ids), np.argsort(dfull.ids)
    assert np.array_equal(d.ids[o1], dfull.ids[o2])
    assert np.array_equal(d.p[o1], dfull.p[o2])
    for u in (0.0, 0.3, 0.77, 0.999):
        assert draw_at(d, u) == draw_at(dfull, u)
