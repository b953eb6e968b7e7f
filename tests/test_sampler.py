"""The host sampler and penalty window against the reference's own sampler
and penalty-window tests (src/sampler.test.ts, src/penalty-window.test.ts):
their cases and expected values, and their second, rescanning
implementation of the selection, which the sampler must match bit for bit.
CPU only."""
import math

import numpy as np
import pytest

from webgllm_amd.sampler import (DEFAULT_REPEAT_LAST_N, MAX_SEEN_ROWS, Distribution,
                                 PenaltyWindow, Sampler, draw, verify)


def lcg(seed):
    """src/sampler.test.ts:6-12: s = s * 1664525 + 1013904223 (mod 2^32), s / 2^32."""
    s = [seed & 0xFFFFFFFF]

    def r():
        s[0] = (s[0] * 1664525 + 1013904223) & 0xFFFFFFFF
        return s[0] / 2 ** 32
    return r


def f32(*v):
    return np.array(v, dtype=np.float32)


def test_temperature_zero_is_argmax():
    d = Sampler(0, 0).distribution(f32(0.1, 3, -1, 2.9))
    assert list(d.ids) == [1] and list(d.p) == [1]


def test_repetition_penalty():
    s = Sampler(0, 0, repetition_penalty=2)
    s.see([1, 2])
    logits = f32(0, 3, -1, 2)
    assert list(s.distribution(logits).ids) == [3]
    assert logits[1] == 1.5 and logits[2] == -2


def test_presence_penalty_on_the_whole_window():
    s = Sampler(0, 0, repetition_penalty=2, presence_penalty=1.5)
    s.see([0, 1])
    s.see([1, 1, 2], True)
    logits = f32(4, 6, -1, 1)
    s.distribution(logits)
    assert list(logits) == [0.5, 1.5, -3.5, 1]
    fresh = Sampler(0, 0, presence_penalty=2)
    nxt = f32(4, 6, -1, 1)
    fresh.distribution(nxt)
    assert list(nxt) == [4, 6, -1, 1]


def test_frequency_penalty_per_occurrence():
    s = Sampler(0, 0, presence_penalty=0.5, frequency_penalty=1)
    s.see([0, 1])
    s.see([1, 1, 2], True)
    logits = f32(4, 6, -1, 1)
    s.distribution(logits)
    assert list(logits) == [2.5, 2.5, -2.5, 1]


def test_top_p_then_min_p():
    d = Sampler(1, 0, min_p=0.5, top_p=0.9).distribution(f32(0, math.log(0.6), math.log(0.1)))
    assert d.p[2] == 0
    assert abs(d.p[0] - 0.625) < 1e-6 and abs(d.p.sum() - 1) < 1e-6


def test_top_k_keeps_the_k_likeliest():
    d = Sampler(1, 2).distribution(f32(1, 4, 2, 3))
    assert sorted(d.ids) == [1, 3]
    p4 = d.p[list(d.ids).index(1)]
    assert abs(p4 - math.exp(4) / (math.exp(4) + math.exp(3))) < 1e-6


def test_top_p_drops_the_tail():
    d = Sampler(1, 0, top_p=0.5).distribution(f32(5, 0, 0, 0))
    assert [i for i, p in zip(d.ids, d.p) if p > 0] == [0]


def test_temperature_after_top_p():
    d = Sampler(0.1, 0, top_p=0.85).distribution(f32(math.log(0.5), math.log(0.4), math.log(0.1)))
    assert d.p[1] > 0 and d.p[2] == 0


def test_unpenalized_distribution():
    s = Sampler(0, 1, repetition_penalty=10, presence_penalty=5)
    s.see([0], True)
    assert list(s.distribution(f32(2, 1.9)).ids) == [1]
    assert list(s.distribution(f32(2, 1.9), penalize=False).ids) == [0]


D = Distribution(np.array([10, 11, 12, 13], np.int32), f32(0.5, 0.25, 0.15, 0.1))


@pytest.mark.parametrize("drafted", [10, 11, 13, 99])
def test_verify_keeps_the_distribution(drafted):
    rnd = lcg(42)
    n = 40000
    counts = {}
    for _ in range(n):
        kept, tok = verify(D, drafted, rnd)
        counts[tok] = counts.get(tok, 0) + 1
    for i, t in enumerate(D.ids):
        assert abs(counts.get(int(t), 0) / n - D.p[i]) < 0.01
    assert 99 not in counts


def test_verify_edges_and_draw():
    one = Distribution(np.array([5], np.int32), f32(1))
    assert verify(one, 5, lambda: 0.999) == (True, 5)
    assert verify(one, 6, lambda: 0.5) == (False, 5)
    d = Distribution(np.array([1, 2, 3], np.int32), f32(0, 1, 0))
    for x in (0, 0.5, 0.999999):
        assert draw(d, lambda: x) == 2
    d = Distribution(np.array([1, 2, 3], np.int32), f32(0.2, 0.3, 0.5))
    rnd = lcg(1)
    counts = [0, 0, 0]
    for _ in range(30000):
        counts[draw(d, rnd) - 1] += 1
    assert all(abs(counts[i] / 30000 - d.p[i]) < 0.01 for i in range(3))


def _rescanning(temperature, top_k, top_p, min_p, logits):
    """The reference test's second implementation of the selection
    (src/sampler.test.ts:144-190): k largest by rescanning for the smallest
    kept, top-p by a comparator sort; float32 stores where it has them."""
    n = logits.size
    k = max(1, min(top_k if top_k > 0 else n, n))
    if k >= n:
        ids = np.arange(n, dtype=np.int32)
        kept = logits.copy()
    else:
        ids = np.zeros(k, np.int32)
        kept = np.full(k, -np.inf, np.float32)
        smallest = 0
        for i in range(n):
            x = logits[i]
            if not (x > kept[smallest]):
                continue
            kept[smallest] = x
            ids[smallest] = i
            smallest = 0
            for j in range(1, k):
                if kept[j] < kept[smallest]:
                    smallest = j
    best = 0
    for j in range(1, k):
        if kept[j] > kept[best]:
            best = j
    mx = float(kept[best])
    weight = [math.exp(float(x) - mx) for x in kept]  # a plain array: doubles
    total = sum(weight)
    if top_p < 1:
        order = sorted(range(k), key=lambda j: -weight[j])
        share, cut = 0.0, False
        for j in order:
            if cut:
                weight[j] = 0
            else:
                share += weight[j] / total
                cut = share >= top_p
    for j in range(k):
        if weight[j] < min_p:
            weight[j] = 0
    left = 0.0
    for j in range(k):
        kept[j] = math.exp((float(kept[j]) - mx) / temperature) if weight[j] > 0 else 0
        left += float(kept[j])
    for j in range(k):
        kept[j] = float(kept[j]) / left
    return ids, kept


def test_selection_matches_the_rescanning_reference():
    """src/sampler.test.ts:192-218 (its generator and settings, smaller
    rounds): the same ids, in the same slots, and the same probabilities,
    bit for bit."""
    rnd = lcg(7)
    for rnd_i in range(30):
        n = 50 + int(rnd() * 800)
        step = 0.5 if rnd_i % 3 == 0 else 0
        logits = np.empty(n, np.float32)
        for i in range(n):
            x = (rnd() - 0.5) * 12
            logits[i] = -np.inf if rnd() < 0.05 else (round(x / step) * step if step else x)
        temperature = 0.3 + rnd() * 1.5
        top_k = [0, 1, 7, 40, 512, n, n + 3][rnd_i % 7]
        top_p = [1, 0.9, 0.5, 0, 0.99][rnd_i % 5]
        min_p = [0, 0, 0.05][rnd_i % 3]
        got = Sampler(temperature, top_k, top_p=top_p, min_p=min_p).distribution(logits.copy())
        ids, p = _rescanning(temperature, top_k, top_p, min_p, logits.copy())
        assert np.array_equal(got.ids, ids), rnd_i
        assert np.array_equal(got.p, p), rnd_i


def test_window_states():
    w = PenaltyWindow(3)
    assert w.push([1, 2, 2]) == [(1, 1), (2, 1)]
    assert dict(w.push([3, 4])) == {3: 1, 1: 0, 4: 1}
    assert dict(w.entries()) == {2: 1, 3: 1, 4: 1}
    assert dict(w.push([3], True)) == {3: 3, 2: 0}
    assert dict(w.push([5, 6, 7])) == {5: 1, 3: 0, 4: 0, 6: 1, 7: 1}
    assert DEFAULT_REPEAT_LAST_N == 64
    assert PenaltyWindow(0).push([1, 2, 3]) == []
    every = PenaltyWindow(-1)
    every.push(range(500))
    assert len(every.entries()) == 500


def test_sampler_penalizes_only_the_window():
    s = Sampler(0, 0, repetition_penalty=2, repeat_last_n=2)
    s.see([0, 1, 2])
    logits = f32(4, 4, 4, 3.9)
    assert s.distribution(logits).ids[0] == 0
    assert list(logits) == [4, 2, 2, np.float32(3.9)]


def _sequential(size, prompt, written, drafts):
    w = PenaltyWindow(size)
    w.push(prompt)
    w.push(written, True)
    rows = [dict(w.entries())]
    for d in drafts:
        w.push([d], True)
        rows.append(dict(w.entries()))
    return rows


def _ahead(size, prompt, written, drafts):
    w = PenaltyWindow(size)
    w.push(prompt)
    w.push(written, True)
    base = dict(w.entries())
    segs = w.ahead(drafts)
    assert len(segs) <= MAX_SEEN_ROWS
    assert dict(w.entries()) == base
    out = []
    for r in range(len(drafts) + 1):
        row = dict(base)
        for t, st, a, b in segs:
            if a <= r < b:
                row[t] = st
        out.append({t: st for t, st in row.items() if st != 0})
    return out


def test_ahead_equals_pushing_drafts_one_by_one():
    """src/penalty-window.test.ts:60-72 (its generator and window sizes)."""
    seed = [7]

    def rand(n):
        seed[0] = (seed[0] * 1103515245 + 12345) % 2 ** 31
        return seed[0] % n
    for size in (0, 1, 3, 8, 64, -1):
        for _ in range(150):
            prompt = [rand(6) for _ in range(rand(12))]
            written = [rand(6) for _ in range(rand(5))]
            drafts = [rand(6) for _ in range(1 + rand(8))]
            assert _ahead(size, prompt, written, drafts) == _sequential(size, prompt, written,
                                                                       drafts)


def test_ahead_examples():
    none = PenaltyWindow(0)
    none.push([1, 2])
    assert none.ahead([5, 6]) == []
    w = PenaltyWindow(2)
    w.push([1, 2])
    assert w.ahead([5, 6]) == [[5, 3, 1, 3], [1, 0, 1, 3], [6, 3, 2, 3], [2, 0, 2, 3]]
