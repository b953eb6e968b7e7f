"""The self-check's float64 recomputation (webgllm_amd/self_check.py) against
what the mathematics fixes: one visible key gives its value row, equal keys
the mean of the values, a dominant key its own row; query heads read their
own KV head; a row never sees the keys after its position; the relative
error of a row and the check's tokens (src/engine.ts:866)."""
import math

import numpy as np
import pytest

from webgllm_amd import self_check as S


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_one_key_gives_its_value_row():
    H, KV, hd = 4, 2, 8
    q = _rand((1, H * hd), 0)
    k, v = _rand((1, KV * hd), 1), _rand((1, KV * hd), 2)
    out = S.attention_rows(q, k, v, 0, H, KV, hd)
    for h in range(H):
        kh = h // (H // KV)
        np.testing.assert_allclose(out[0, h * hd:(h + 1) * hd], v[0, kh * hd:(kh + 1) * hd],
                                   rtol=0, atol=1e-6)


def test_equal_keys_average_the_values():
    H, KV, hd, n = 2, 1, 4, 7
    q = _rand((1, H * hd), 3)
    k = np.tile(_rand((1, KV * hd), 4), (n, 1))
    v = _rand((n, KV * hd), 5)
    out = S.attention_rows(q, k, v, n - 1, H, KV, hd)
    for h in range(H):
        np.testing.assert_allclose(out[0, h * hd:(h + 1) * hd], v.astype(np.float64).mean(0),
                                   rtol=1e-12, atol=1e-12)


def test_a_dominant_key_wins():
    H, KV, hd, n = 1, 1, 4, 5
    k = np.zeros((n, hd), np.float32)
    k[3] = [1, 0, 0, 0]
    q = np.array([[200.0, 0, 0, 0]], np.float32)
    v = _rand((n, hd), 6)
    out = S.attention_rows(q, k, v, n - 1, H, KV, hd)
    np.testing.assert_allclose(out[0], v[3], rtol=0, atol=1e-12)


def test_query_heads_read_their_kv_head():
    # KV head j's values are all j + 1: every query head h of group j gets j + 1
    H, KV, hd, n = 8, 2, 4, 3
    q = _rand((1, H * hd), 7)
    k = _rand((n, KV * hd), 8)
    v = np.repeat(np.arange(1, KV + 1, dtype=np.float32), hd)[None].repeat(n, 0)
    out = S.attention_rows(q, k, v, n - 1, H, KV, hd)
    want = np.repeat(np.arange(H) // (H // KV) + 1.0, hd)
    np.testing.assert_allclose(out[0], want, rtol=1e-12)


def test_rows_do_not_see_later_keys():
    # rows at positions 2 and 3 over 6 cached rows: rows 4 and 5 hold NaN
    H, KV, hd = 2, 2, 4
    q = _rand((2, H * hd), 9)
    k, v = _rand((6, KV * hd), 10), _rand((6, KV * hd), 11)
    k[4:], v[4:] = np.nan, np.nan
    out = S.attention_rows(q, k, v, 2, H, KV, hd)
    assert np.isfinite(out).all()
    # and row 0 (position 2) equals the same query over only rows 0..2
    alone = S.attention_rows(q[:1], k[:3], v[:3], 2, H, KV, hd)
    np.testing.assert_array_equal(out[0], alone[0])


def test_relative_error():
    w = np.array([3.0, 4.0])
    assert S.relative_error(w, w) == 0.0
    assert S.relative_error(np.array([3.0, 4.5]), w) == pytest.approx(0.1)
    assert S.relative_error(np.array([3.0, np.nan]), w) == math.inf
    assert S.relative_error(np.array([3.0, np.inf]), w) == math.inf


def test_check_tokens_follow_the_reference_formula():
    # checkToken(i, vocab) = (i * 7919 + 13) % vocab
    assert [S.check_token(i, 65536) for i in range(3)] == [13, 7932, 15851]
    assert S.check_token(9, 1000) == (9 * 7919 + 13) % 1000
    assert S.SELF_CHECK_MAX == 1e-2
