"""The oracle pinned against the reference's own known-answer tests and
against closed forms (CPU only). Each test names the reference test or the
mathematical fact it rests on."""
import math

import numpy as np
import pytest

from oracle import oracle as O


# --- src/half.test.ts -------------------------------------------------------

def test_half_round_trips_exact_values():
    # src/half.test.ts:6-10
    for v in [0, 1, -1, 0.5, 2, 65504, -65504, 6.103515625e-5, 5.960464477539063e-8,
              0.333251953125]:
        assert O.from_half(O.to_half(v)) == v


def test_half_rounds_to_nearest_even():
    # src/half.test.ts:12-15
    assert O.from_half(O.to_half(1 + 2 ** -11)) == 1
    assert O.from_half(O.to_half(1 + 3 * 2 ** -12)) == 1 + 2 ** -10


def test_half_overflow_nan_signed_zero():
    # src/half.test.ts:17-22
    assert O.from_half(O.to_half(1e6)) == math.inf
    assert O.from_half(O.to_half(-1e6)) == -math.inf
    assert math.isnan(O.from_half(O.to_half(math.nan)))
    z = O.from_half(O.to_half(-0.0))
    assert z == 0 and math.copysign(1, z) < 0


def test_half_table_values():
    # src/half.test.ts:24-31
    want = {0: 0.0, 1: 2 ** -24, 0x3C00: 1.0, 0x7BFF: 65504.0, 0x8001: -(2 ** -24),
            0xC000: -2.0, 0x7C00: math.inf, 0x0400: 2 ** -14}
    for h, v in want.items():
        assert O.from_half(h) == v
    assert list(O.halves_to_f32(np.array([0x3C00, 0xC000, 0x3800]))) == [1, -2, 0.5]


def test_half_matches_numpy_rne_on_float32_grid():
    # toHalf stores the value as a float32 first, then rounds to nearest
    # even: for float32 inputs that is IEEE float16 conversion (numpy's).
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s
                        for s in (1e-7, 1e-5, 1e-3, 1.0, 1e3, 6e4)])
    got = np.array([O.to_half(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# --- src/q4k-pack.test.ts ------------------------------------------------------

def _worst(m, want, rows, K, src_rows=None):
    err = scale = 0.0
    for r in range(rows):
        got = m.row(r)
        frm = (src_rows[r] if src_rows is not None else r)
        err = max(err, float(np.max(np.abs(got - want[frm]))))
        scale = max(scale, float(np.max(np.abs(want[frm]))))
    return err / scale


def test_q4k_packed_rows_are_the_files_weights():
    # src/q4k-pack.test.ts:55-68
    rows, K = 8, 512
    b = O.q4k_blocks(1, rows * K // 256)
    want = O.dequantize_q4_k(b, rows, K)
    m = O.QuantMatrix(rows, K, "halves")
    O.pack_q4_k(m, 0, b, rows)
    assert m.zeros is None and m.zero_halves is not None
    assert _worst(m, want, rows, K) < 1e-3


def test_q4k_rows_land_at_offset_in_order():
    # src/q4k-pack.test.ts:70-82
    rows, K = 4, 256
    b = O.q4k_blocks(2, rows)
    want = O.dequantize_q4_k(b, rows, K)
    m = O.QuantMatrix(8, K, "halves")
    order = [2, 0, 3, 1]
    O.pack_q4_k(m, 4, b, rows, order)
    for r in range(4):
        assert np.all(m.row(r) == 0)
    err = scale = 0.0
    for r in range(4):
        got = m.row(4 + r)
        err = max(err, float(np.max(np.abs(got - want[order[r]]))))
        scale = max(scale, float(np.max(np.abs(want[order[r]]))))
    assert err / scale < 1e-3


def test_q4k_zero_scale_subblock_keeps_constant():
    # src/q4k-pack.test.ts:84-97
    rows, K = 4, 256
    b = O.q4k_blocks(3, rows, zero_scale=True)
    want = O.dequantize_q4_k(b, rows, K)
    for r in range(rows):
        at = (r % 8) * 32
        assert np.all(want[r, at:at + 32] == want[r, at])
    m = O.QuantMatrix(rows, K, "halves")
    O.pack_q4_k(m, 0, b, rows)
    assert _worst(m, want, rows, K) < 1e-3
    # The constant sub-block is q = 15 with z' = 0 (repack.ts:156-161).
    for r in range(rows):
        at = (r % 8) * 32
        row = m.row(r)
        assert np.all(row[at:at + 32] == row[at])


def test_q4k_needs_fractional_zero_points():
    # src/q4k-pack.test.ts:99-101
    with pytest.raises(ValueError, match="fractional zero points"):
        O.pack_q4_k(O.QuantMatrix(4, 256, True), 0, O.q4k_blocks(4, 4), 4)


def test_q4k_scale_chain_by_hand():
    # repack.ts:149-163 on one hand-built sub-block: d = 1/64, sc = 5,
    # dmin = 1/128, m = 3 -> d' = 5/64 and z' = half(3/128 / (5/64)) = half(0.3).
    b = np.zeros(144, dtype=np.uint8)
    d, dm = O.to_half(1 / 64), O.to_half(1 / 128)
    b[0], b[1], b[2], b[3] = d & 255, d >> 8, dm & 255, dm >> 8
    b[4] = 5          # sub-block 0 scale
    b[8] = 3          # sub-block 0 min
    b[16:16 + 32] = 0x21  # low nibble 1 (sub-block 0), high nibble 2 (sub-block 1)
    m = O.QuantMatrix(4, 256, "halves")
    O.pack_q4_k(m, 0, np.tile(b, 4), 4)
    assert m.scales[0] == O.to_half(5 / 64)
    assert m.zero_halves[0] == O.to_half(0.3)
    assert O.from_half(m.zero_halves[0]) == np.float16(0.3)
    row = m.row(0)
    assert row[0] == np.float32(np.float64(5 / 64) * (1 - float(np.float16(0.3))))
    # sub-block 1 has scale 0 -> q = 15, d' = half(-0/15) = -0, z' = 0.
    assert m.scales[4] == 0x8000 and m.zero_halves[4] == 0
    assert np.all(row[32:64] == 0)


# --- src/repack-words.test.ts -------------------------------------------------

def test_q4_0_word_copies_offsets_and_permutations():
    # src/repack-words.test.ts:5-29 (4-bit)
    nbytes, stride = 16, 18
    for offset in [0, 1, 2, 3]:
        raw = np.array([(i * 71 + 19) & 255 for i in range(offset + 4 * 2 * stride)],
                       dtype=np.uint8)
        src = raw[offset:]
        perm = [3, 0, 2, 1]
        actual = O.QuantMatrix(12, 64, False)
        want = O.QuantMatrix(12, 64, False)
        target = want.quants.view(np.uint8)
        for i in range(4):
            for b in range(2):
                at = ((((4 + i) >> 2) * 2 + b) * 4 + ((4 + i) & 3))
                frm = (perm[i] * 2 + b) * stride
                want.scales[at] = int(src[frm]) | (int(src[frm + 1]) << 8)
                target[at * nbytes:(at + 1) * nbytes] = src[frm + 2:frm + stride]
        O.pack_q4_0(actual, 4, src, 4, perm)
        assert np.array_equal(actual.quants, want.quants)
        assert np.array_equal(actual.scales, want.scales)


# --- src/q4-repacker.test.ts --------------------------------------------------

@pytest.mark.parametrize("N,K", [(4, 32), (12, 2048), (64, 7680), (8, 64)])
def test_quants_from_raw_matches_byte_packer(N, K):
    # src/q4-repacker.test.ts:5-13 pins the word repack to quantsFromRaw; here
    # quantsFromRaw (words) and packMatMulNBits (bytes) pin each other.
    i = np.arange(N * K // 2, dtype=np.uint64)
    raw = (((i + 1) * 2654435761) & 0xFFFFFFFF) >> 24
    raw = raw.astype(np.uint8)
    words = O.quants_from_raw(raw, N, K)
    m = O.QuantMatrix(N, K, True)
    O.pack_nbits(m, 0, raw, np.zeros(N * K // 32, np.uint16), None, N)
    assert np.array_equal(words, m.quants)


def test_nbits_dequant_paths_agree():
    # dequantizeNBitsRow (load-onnx.ts:471-501) and matrixRow over packed and
    # raw rows (repack.ts:865-891) are three statements of one dequant.
    rng = np.random.default_rng(5)
    N, K = 8, 96
    blocks = K // 32
    quant = rng.integers(0, 256, N * blocks * 16, dtype=np.uint8)
    scales = np.array([O.to_half(v) for v in rng.uniform(-0.1, 0.1, N * blocks)], np.uint16)
    zp = rng.integers(0, 256, N * ((blocks + 1) // 2), dtype=np.uint8)
    packed = O.QuantMatrix(N, K, True)
    O.pack_nbits(packed, 0, quant, scales, zp, N)
    raw = O.QuantMatrix(N, K, True)
    raw.raw = quant
    O.pack_nbits_scales(raw, 0, scales, zp, N)
    for n in range(N):
        want = O.dequantize_nbits_row(K, quant, scales, zp, n)
        assert np.array_equal(packed.row(n), want)
        assert np.array_equal(raw.row(n), want)
    # Closed form: scale * (nibble - zero point), element 2i low nibble of byte i.
    n, b = 3, 1
    byte = quant[(n * blocks + b) * 16 + 2]
    z = (zp[n * ((blocks + 1) // 2) + (b >> 1)] >> ((b & 1) * 4)) & 15
    s = O.from_half(scales[n * blocks + b])
    assert packed.row(n)[b * 32 + 4] == np.float32(s * ((byte & 15) - z))
    assert packed.row(n)[b * 32 + 5] == np.float32(s * ((byte >> 4) - z))


def test_gguf_q4_0_zero_block_is_zero():
    # src/lfm2-gguf.test.ts:17: d = 1.0 (0x3C00), nibbles 0x88 -> weights 0.
    blk = np.array([0x00, 0x3C] + [0x88] * 16, dtype=np.uint8)
    m = O.QuantMatrix(4, 64, False)
    O.pack_q4_0(m, 0, np.tile(blk, 8), 4)
    assert np.all(m.dense() == 0)


def test_q4_0_dequant_closed_form():
    rng = np.random.default_rng(1)
    N, K = 4, 64
    src = rng.integers(0, 256, N * (K // 32) * 18, dtype=np.uint8)
    for b in range(N * K // 32):
        h = O.to_half(rng.uniform(-1, 1))
        src[b * 18], src[b * 18 + 1] = h & 255, h >> 8
    m = O.QuantMatrix(N, K, False)
    O.pack_q4_0(m, 0, src, N)
    for n in range(N):
        for b in range(K // 32):
            p = (n * (K // 32) + b) * 18
            d = O.from_half(int(src[p]) | (int(src[p + 1]) << 8))
            for j in range(16):
                byte = int(src[p + 2 + j])
                assert m.row(n)[b * 32 + j] == np.float32(d * ((byte & 15) - 8))
                assert m.row(n)[b * 32 + 16 + j] == np.float32(d * ((byte >> 4) - 8))


def test_quantize_q4_0_roundtrip_error_bounded():
    # ggml's Q4_0 maps the largest-magnitude weight m to q = 0 (d = m / -8):
    # in-range weights round to within |d| / 2, and weights near -m (q = 16)
    # clamp to 15, so |w - deq(w)| <= |d| = |m| / 8 (plus d's half rounding).
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    m = O.QuantMatrix(8, 256, False)
    O.pack_q4_0(m, 0, O.quantize_q4_0(w), 8)
    deq = m.dense()
    amax = np.abs(w.reshape(8, -1, 32)).max(-1)
    err = np.abs(deq - w).reshape(8, -1, 32).max(-1)
    assert np.all(err <= amax / 8 * 1.001 + 1e-7)
    assert np.mean(np.abs(deq - w)) < np.mean(amax) / 16


# --- matmul -------------------------------------------------------------------

def _random_q4_0(rng, N, K):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    m = O.QuantMatrix(N, K, False)
    O.pack_q4_0(m, 0, O.quantize_q4_0(w), N)
    return m


def test_gemv_f64_matches_dense_product():
    rng = np.random.default_rng(3)
    m = _random_q4_0(rng, 32, 256)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    want = x.astype(np.float64) @ m.dense().astype(np.float64).T
    assert np.allclose(O.gemv_f64(m, x), want, rtol=1e-12, atol=1e-12)


def test_gemv_special_cases():
    rng = np.random.default_rng(4)
    m = _random_q4_0(rng, 16, 128)
    # one-hot x -> a column of W, exactly
    x = np.zeros((1, 128), np.float32)
    x[0, 37] = 1
    assert np.array_equal(O.gemv_f64(m, x)[0], m.dense()[:, 37].astype(np.float64))
    # all nibbles at the zero point -> 0
    z = O.QuantMatrix(16, 128, False)
    z.quants[:] = 0x88888888
    z.scales[:] = O.to_half(0.5)
    assert np.all(O.gemv_f64(z, rng.standard_normal((1, 128))) == 0)
    assert np.all(O.matmul_split(z, O.f32_to_h2(rng.standard_normal((1, 128)))) == 0)


@pytest.mark.parametrize("M", [1, 5])
def test_matmul_split_block_form_matches_f64(M):
    # sum_b d_b (sum q a - z sum a) = sum w a: the shader's block form equals
    # the dense product up to float32 rounding.
    rng = np.random.default_rng(10 + M)
    m = _random_q4_0(rng, 64, 512)
    x16 = O.f32_to_h2(rng.standard_normal((M, 512)).astype(np.float32))
    want = O.gemv_f64(m, O.halves_to_f32(x16))
    got = O.matmul_split(m, x16)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-5
    # A planted mistake in the oracle's input (W transposed within a block
    # row: nibbles read high-first) must fail the bar.
    bad = O.QuantMatrix(64, 512, False)
    bad.scales[:] = m.scales
    qb = m.quants.view(np.uint8)
    bad.quants.view(np.uint8)[:] = ((qb & 15) << 4) | (qb >> 4)
    relbad = np.linalg.norm(O.matmul_split(bad, x16) - want) / np.linalg.norm(want)
    assert relbad > 1e-1


# --- attention, RoPE, norms -----------------------------------------------------

def test_attention_closed_forms():
    rng = np.random.default_rng(6)
    hd, heads, kvh = 8, 4, 2
    stride = kvh * hd
    q = rng.standard_normal(heads * hd).astype(np.float32)
    kc = O.f32_to_h2(rng.standard_normal((5, stride)).astype(np.float32))
    vc = O.f32_to_h2(rng.standard_normal((5, stride)).astype(np.float32))
    # one key -> out = v
    out = O.attention_f64(q, kc, vc, heads, kvh, hd, 1, stride)
    for h in range(heads):
        kh = h // 2
        assert np.allclose(out[h * hd:(h + 1) * hd], O.halves_to_f32(vc[0, kh * hd:(kh + 1) * hd]))
    # equal scores (q = 0) -> mean of V
    out = O.attention_f64(np.zeros_like(q), kc, vc, heads, kvh, hd, 5, stride)
    vf = O.halves_to_f32(vc).astype(np.float64)
    assert np.allclose(out[:hd], vf[:, :hd].mean(0))
    # equal keys: any shift of the scores leaves the output unchanged
    kc2 = np.tile(kc[:1], (5, 1))
    a = O.attention_f64(q, kc2, vc, heads, kvh, hd, 5, stride)
    assert np.allclose(a[:hd], vf[:, :hd].mean(0))
    # shift invariance: adding one vector c to every key adds q.c to every
    # score of a head. Keys on a 1/8 grid stay exact halves after the shift.
    kg = (rng.integers(-16, 16, (5, stride)) / 8).astype(np.float32)
    c = (rng.integers(-8, 8, stride) / 8).astype(np.float32)
    base = O.attention_f64(q, O.f32_to_h2(kg), vc, heads, kvh, hd, 5, stride)
    shifted = O.attention_f64(q, O.f32_to_h2(kg + c), vc, heads, kvh, hd, 5, stride)
    assert np.allclose(base, shifted, rtol=1e-9, atol=1e-12)
    # the softmax weights really depend on the scores (a wrong sign fails)
    assert not np.allclose(base, O.attention_f64(-q, O.f32_to_h2(kg), vc, heads, kvh, hd, 5,
                                                 stride))
    # causal: keys past the count are never read
    kc3, vc3 = kc.copy(), vc.copy()
    kc3[3:] = O.f32_to_h2(np.full((2, stride), 50.0, np.float32))
    vc3[3:] = O.f32_to_h2(np.full((2, stride), -7.0, np.float32))
    assert np.array_equal(O.attention_f64(q, kc, vc, heads, kvh, hd, 3, stride),
                          O.attention_f64(q, kc3, vc3, heads, kvh, hd, 3, stride))
    # a brute-force softmax for one head on the CPU
    kf = O.halves_to_f32(kc).astype(np.float64)
    s_ = kf[:, :hd] @ q[:hd].astype(np.float64)
    wts = np.exp(s_ - s_.max())
    wts /= wts.sum()
    full = O.attention_f64(q, kc, vc, heads, kvh, hd, 5, stride)
    assert np.allclose(full[:hd], wts @ vf[:, :hd], rtol=1e-12, atol=1e-12)


def test_attention_f32_closed_forms_and_f64():
    """The float32 attention (the CPU baseline's): one key gives v exactly,
    q = 0 the mean of V, causal keys unread, and 4096 keys of 8 heads
    within 1e-5 of the float64 form, single- and multi-threaded alike."""
    rng = np.random.default_rng(16)
    hd, heads, kvh = 128, 8, 2
    stride = kvh * hd
    q = (rng.standard_normal(heads * hd) / np.sqrt(hd)).astype(np.float32)
    kc = O.f32_to_h2(rng.standard_normal((4096, stride)).astype(np.float32))
    vc = O.f32_to_h2(rng.standard_normal((4096, stride)).astype(np.float32))
    vf = O.halves_to_f32(vc).astype(np.float64)
    one = O.attention_f32(q, kc, vc, heads, kvh, hd, 1, stride)
    for h in range(heads):
        kh = h // (heads // kvh)
        assert np.array_equal(one[h * hd:(h + 1) * hd],
                              O.halves_to_f32(vc[0, kh * hd:(kh + 1) * hd]))
    mean = O.attention_f32(np.zeros_like(q), kc, vc, heads, kvh, hd, 7, stride)
    assert np.allclose(mean[:hd], vf[:7, :hd].mean(0), rtol=1e-6, atol=1e-6)
    kc3, vc3 = kc.copy(), vc.copy()
    kc3[9:] = O.f32_to_h2(np.full((4096 - 9, stride), 50.0, np.float32))
    vc3[9:] = O.f32_to_h2(np.full((4096 - 9, stride), -7.0, np.float32))
    assert np.array_equal(O.attention_f32(q, kc, vc, heads, kvh, hd, 9, stride),
                          O.attention_f32(q, kc3, vc3, heads, kvh, hd, 9, stride))
    want = O.attention_f64(q, kc, vc, heads, kvh, hd, 4096, stride)
    a1 = O.attention_f32(q, kc, vc, heads, kvh, hd, 4096, stride, threads=1)
    a4 = O.attention_f32(q, kc, vc, heads, kvh, hd, 4096, stride, threads=4)
    assert np.array_equal(a1, a4)
    assert np.linalg.norm(a1 - want) / np.linalg.norm(want) <= 1e-5
    # a dropped max subtraction or a wrong GQA head map would fail here
    wrong = O.attention_f32(q, kc[:, ::-1].copy(), vc, heads, kvh, hd, 4096, stride)
    assert np.linalg.norm(wrong - want) / np.linalg.norm(want) > 1e-2


def test_rope_and_norm_closed_forms():
    hd, R = 64, 64
    rope = O.rope_table(1e6, hd, R, 4096)
    rng = np.random.default_rng(7)
    x = rng.standard_normal(hd).astype(np.float32)
    # position 0 is the identity
    assert np.allclose(O.head_prep(x, None, rope, hd, R, 0, 1e-6, 1.0, False), x, atol=1e-7)
    # a unit vector with unit weights normalizes to sqrt(hd) * v / |v|
    v = np.zeros(hd, np.float32)
    v[3] = 2.0
    got = O.head_prep(v, np.ones(hd), rope, hd, R, 0, 0.0, 1.0, True)
    assert np.allclose(got, v / 2 * math.sqrt(hd), atol=1e-5)
    # rotation keeps each pair's norm; the angle of pair 0 is pos radians
    for pos in (1, 1023, 1024, 3000):
        y = O.head_prep(x, None, rope, hd, R, pos, 0.0, 1.0, False)
        for j in range(R // 2):
            a = math.hypot(x[j], x[j + R // 2])
            b = math.hypot(y[j], y[j + R // 2])
            assert abs(a - b) < 1e-5 * max(1, a)
        # pair j turns by pos * theta^(-2j/hd)
        for j in (0, 1, 7, R // 2 - 1):
            ang = math.atan2(y[j + R // 2], y[j]) - math.atan2(x[j + R // 2], x[j])
            want = pos * 1e6 ** (-2 * j / hd)
            assert abs(math.remainder(ang - want, 2 * math.pi)) < 1e-4


def test_rms_norm_and_swiglu():
    x = np.array([[3.0, 4.0]], np.float32)
    out = O.rms_norm(x, np.array([1.0, 2.0]), 0.0)
    r = math.sqrt((9 + 16) / 2)
    assert np.allclose(out, [[3 / r, 8 / r]])
    gu = np.array([[0.0, 2.0, 5.0, 7.0]], np.float32)
    assert np.allclose(O.swiglu(gu), [[0.0, 2 / (1 + math.exp(-2)) * 7]])
    # silu(g) -> g for large g and -> 0 for very negative g
    big = O.swiglu(np.array([[40.0, -40.0, 3.0, 3.0]], np.float32))
    assert big[0, 0] == np.float32(120.0) and abs(big[0, 1]) < 1e-15


# --- short convolution -----------------------------------------------------------

def test_short_conv_closed_forms():
    rng = np.random.default_rng(8)
    D, W, M = 16, 3, 5
    bcx = rng.standard_normal((M, 3 * D)).astype(np.float32)
    state = rng.standard_normal((W - 1, D)).astype(np.float32)
    taps = np.zeros((D, W), np.float32)
    taps[:, W - 1] = 1
    out, new_state, pre = O.short_conv(bcx, D, W, taps, state, prefixes=True)
    B, Cm, X = bcx[:, :D], bcx[:, D:2 * D], bcx[:, 2 * D:]
    assert np.allclose(out, Cm * B * X)
    assert np.allclose(new_state, (B * X)[-(W - 1):])
    # prefix p's state equals a fresh run on the first p tokens
    for p in range(1, M + 1):
        _, st = O.short_conv(bcx[:p], D, W, taps, state)
        assert np.array_equal(pre[p - 1], st)
    # taps on the oldest position read the state for the first token
    taps2 = np.zeros((D, W), np.float32)
    taps2[:, 0] = 1
    out2, _ = O.short_conv(bcx[:1], D, W, taps2, state)
    assert np.allclose(out2[0], Cm[0] * state[0])


# --- greedy pick -------------------------------------------------------------------

def test_argmax_ties_lowest_id_and_nan():
    v = np.zeros(1000, np.float32)
    v[300] = 5
    v[700] = 5
    assert O.argmax(v) == (300, 5.0)
    v[10] = np.nan
    assert O.argmax(v)[0] == 300
    w = np.full(513, -1.0, np.float32)
    w[255] = 2.0
    w[256] = 2.0  # chunk boundary: the earlier chunk wins the tie
    assert O.argmax(w)[0] == 255
    assert O.argmax(np.full(10, -np.inf, np.float32))[0] == 0


# ------------------------------------------------- 8-bit and Q6_K matrices

def test_q8_0_dequant_known_answer():
    """src/q4k-pack.test.ts:103-118: d = 0.5 with codes j - 16, d = 0.25 with
    codes 4 j - 64."""
    b = np.zeros(68, np.uint8)
    for p, d in ((0, 0.5), (34, 0.25)):
        h = O.to_half(d)
        b[p], b[p + 1] = h & 255, h >> 8
    for j in range(32):
        b[2 + j] = (j - 16) & 255
        b[36 + j] = (4 * j - 64) & 255
    out = O.dequantize_q8_0(b, 2, 32)
    assert np.array_equal(out[0], 0.5 * (np.arange(32) - 16))
    assert np.array_equal(out[1], 0.25 * (4 * np.arange(32) - 64))


def test_pack_q8_0_rows_are_the_files_weights():
    """An 8-bit matrix's rows (matrixRow) equal dequantizeQ8_0 of the rows
    the packer took, at an offset and through a row permutation."""
    from tests.helpers import imul_bytes
    N, K = 12, 96
    src = imul_bytes(16 * (K // 32) * 34, 5).astype(np.uint8)
    for b in range(16 * K // 32):  # sane halves for d
        src[b * 34], src[b * 34 + 1] = 0x66, 0x1e
    want = O.dequantize_q8_0(src, 16, K)
    m = O.WideMatrix(N, K, 8)
    perm = [7, 0, 15, 3]
    O.pack_q8_0(m, 4, src, 4, src_rows=perm)
    O.pack_q8_0(m, 0, src, 4)
    for i, r in enumerate(perm):
        assert np.array_equal(m.row(4 + i), want[r])
    for n in range(4):
        assert np.array_equal(m.row(n), want[n])
    assert not m.quants[8 * K:].any()  # rows 8..11 untouched


def _q6k_reference_matrix(kind):
    from tests.helpers import imul_bytes, lcg_bytes
    if kind == "expanded":  # src/q6-expanded.test.ts:8-20
        rows, K = 12, 512
        raw = lcg_bytes(rows * (K // 256) * 210, 7)
        raw.reshape(-1, 210)[:, 208] = 0x00
        raw.reshape(-1, 210)[:, 209] = 0x24
    else:  # src/q6-split.test.ts:6-8
        rows, K = 8, 512
        raw = imul_bytes(rows * K // 256 * 210, 11).astype(np.uint8)
        raw.reshape(-1, 210)[:, 208] = 0x66
        raw.reshape(-1, 210)[:, 209] = 0x1e
    return rows, K, raw


@pytest.mark.parametrize("kind", ["expanded", "split"])
def test_q6_k_packed_rows_equal_dequantize_q6_k(kind):
    """The reference's Q6_K layout tests: a packQ6_K matrix read as its
    shaders index it gives dequantizeQ6_K's weights exactly
    (src/q6-expanded.test.ts:7-46, src/q6-split.test.ts:6-28)."""
    rows, K, raw = _q6k_reference_matrix(kind)
    want = O.dequantize_q6_k(raw, rows, K)
    m = O.WideMatrix(rows, K, 6)
    O.pack_q6_k(m, 0, raw, rows)
    got = m.dense()
    assert np.array_equal(got, want)
    # and the scales texture holds each super-block's d
    d = raw.reshape(rows, K // 256, 210)[:, :, 208:210].copy().view(np.uint16)[..., 0]
    g = np.arange(rows) // 4
    r = np.arange(rows) % 4
    for s in range(K // 256):
        at = (g * (K // 256) + s) * 4 + r
        assert np.array_equal(m.scales[at], d[:, s])


def test_q6_k_decode_inverts_ggml_packing():
    """Codes, scales and d packed by ggml's Q6_K packing loop (an encoder
    independent of the decoder) come back as d * sc[k / 16] * (q - 32), at
    every position."""
    from tests.helpers import encode_q6_k
    rng = np.random.default_rng(9)
    supers = 6
    q = rng.integers(0, 64, (supers, 256))
    q[0, :] = np.arange(256) % 64  # every code at every position class
    sc = rng.integers(-128, 128, (supers, 16))
    sc[1, :] = [-128, 127, 0, 1, -1, 64, -64, 2, 3, 5, 7, 11, 13, 17, 19, 23]
    d_bits = np.array([O.to_half(v) for v in (0.001, 0.5, 2.0 ** -20, 3.0, 1e-3, 65504.0)])
    raw = encode_q6_k(q, sc, d_bits)
    got = O.dequantize_q6_k(raw, 1, supers * 256).reshape(supers, 256)
    d = np.array([O.from_half(int(h)) for h in d_bits], np.float64)
    want = (d[:, None] * np.repeat(sc, 16, axis=1) * (q - 32)).astype(np.float32)
    assert np.array_equal(got, want)


def test_quantize_q8_hand_cases():
    """quantizeQ8 (src/repack.ts:634-704) on blocks worked out by hand:
    ties round up (floor(x + 0.5)), the clamp is +-127, a zero or NaN scale
    gives zeros, an infinite scale maps an infinity to -127 (NaN quotient ->
    ToInt32 0) and finite values to 0, a subnormal scale clamps."""
    K = 32 * 6
    v = np.zeros((4, K), np.float32)
    # block 0: max 127 -> scale exactly 1
    v[0, :8] = [127, 2.5, -2.5, 0.49, -0.5, 126.6, -127, 3.0]
    # block 1: all zero; block 2: a NaN; block 3: +inf; block 4: subnormal scale
    v[0, 64] = np.nan
    v[0, 65] = 1.0
    v[0, 96] = np.inf
    v[0, 97] = 5.0
    tiny = np.float32(127 * 1.25 * 2.0 ** -24)
    v[0, 128:131] = [tiny, -tiny, tiny / 2]
    # block 5: max 63.5 -> scale half(0.5) = 0.5
    v[0, 160:164] = [63.5, 0.25, -0.25, 0.75]
    v[1:] = np.random.default_rng(1).standard_normal((3, K)).astype(np.float32)
    m = O.WideMatrix(4, K, 8)
    O.quantize_q8(m, 0, v)
    q = m.quants.view(np.int8)

    def block(b):  # row 0's block b: si = b * 4
        return q[b * 4 * 32:(b * 4 + 1) * 32], int(m.scales[b * 4])

    c, s = block(0)
    assert s == O.to_half(1.0)
    assert list(c[:8]) == [127, 3, -2, 0, 0, 127, -127, 3] and not c[8:].any()
    c, s = block(1)
    assert s == 0 and not c.any()
    c, s = block(2)
    assert (s & 0x7C00) == 0x7C00 and (s & 0x3FF) and not c.any()
    c, s = block(3)
    assert s == 0x7C00 and c[0] == -127 and not c[1:].any()
    c, s = block(4)
    assert s == 1  # 2^-24
    assert list(c[:3]) == [127, -127, 79]  # 158.75 -> clamp; 79.375 -> 79
    c, s = block(5)
    assert s == O.to_half(0.5)
    assert list(c[:4]) == [127, 1, 0, 2]  # 0.5 + 0.5 -> 1; -0.5 + 0.5 -> 0; 1.5 + .5 -> 2


def test_quantize_q8_error_bound_and_layout():
    """Every code is the nearest to v / scale (within half a step, ties up)
    and sits at the layout's index; the max maps to +-127."""
    rng = np.random.default_rng(3)
    N, K = 8, 256
    v = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    m = O.WideMatrix(N, K, 8)
    O.quantize_q8(m, 0, v)
    dense = m.dense()
    for n in range(N):
        for b in range(K // 32):
            blk = v[n, 32 * b:32 * b + 32].astype(np.float64)
            s = O.from_half(int(m.scales[(n // 4 * (K // 32) + b) * 4 + n % 4]))
            assert s > 0
            err = np.abs(dense[n, 32 * b:32 * b + 32] - blk)
            assert np.all(err <= s / 2 * (1 + 1e-6))
            assert np.abs(np.round(np.abs(blk).max() / s)) >= 126


@pytest.mark.parametrize("bits", [8, 6])
def test_wide_matmul_block_form_matches_f64(bits):
    """The reference's float32 block forms (the 8-bit split matmul, the Q6_K
    head) against a float64 product of the pinned dequant."""
    from tests.helpers import encode_q6_k
    rng = np.random.default_rng(bits)
    N, K, M = 16, 512, 3
    m = O.WideMatrix(N, K, bits)
    if bits == 8:
        O.quantize_q8(m, 0, rng.standard_normal((N, K)).astype(np.float32) * 0.1)
    else:
        supers = N * K // 256
        raw = encode_q6_k(rng.integers(0, 64, (supers, 256)),
                          rng.integers(-128, 128, (supers, 16)),
                          [O.to_half(v) for v in rng.uniform(1e-4, 1e-3, supers)])
        O.pack_q6_k(m, 0, raw, N)
    x16 = O.f32_to_h2(rng.standard_normal((M, K)).astype(np.float32))
    got = m.matmul(x16)
    want = O.halves_to_f32(x16).astype(np.float64) @ m.dense().astype(np.float64).T
    assert np.max(np.abs(got - want)) <= 1e-5 * np.abs(want).max()


def test_q4_1_dequant_closed_form():
    """dequantizeQ4_1 (src/repack.ts:447-466): w = q d + m, weight j in byte
    j's low nibble and j + 16 in its high one."""
    b = np.zeros(40, np.uint8)
    for p, d, m in ((0, 0.5, -2.0), (20, 0.25, 1.5)):
        hd, hm = O.to_half(d), O.to_half(m)
        b[p:p + 4] = [hd & 255, hd >> 8, hm & 255, hm >> 8]
        b[p + 4:p + 20] = [(j & 15) | ((15 - j) << 4) for j in range(16)]
    out = O.dequantize_q4_1(b, 1, 64)[0]
    j = np.arange(16)
    assert np.array_equal(out[:16], j * 0.5 - 2.0)
    assert np.array_equal(out[16:32], (15 - j) * 0.5 - 2.0)
    assert np.array_equal(out[32:48], j * 0.25 + 1.5)
    assert np.array_equal(out[48:64], (15 - j) * 0.25 + 1.5)


def test_q5_k_decode_inverts_ggml_packing():
    """Codes, 6-bit scales and mins packed by ggml's Q5_K packing (an
    encoder independent of the decoder) come back as d sc q - dmin m at
    every position; the Q4_K decode of the same scale bytes agrees."""
    from tests.helpers import encode_q5_k
    rng = np.random.default_rng(11)
    supers = 5
    q = rng.integers(0, 32, (supers, 256))
    q[0] = np.arange(256) % 32
    sc = rng.integers(0, 64, (supers, 8))
    mn = rng.integers(0, 64, (supers, 8))
    sc[1] = [63, 0, 1, 62, 32, 31, 17, 48]
    d = [O.to_half(v) for v in rng.uniform(1e-3, 1e-2, supers)]
    dm = [O.to_half(v) for v in rng.uniform(1e-3, 1e-2, supers)]
    got = O.dequantize_q5_k(encode_q5_k(q, sc, mn, d, dm), 1, supers * 256).reshape(supers, 256)
    dd = np.array([O.from_half(h) for h in d], np.float64)[:, None]
    dmm = np.array([O.from_half(h) for h in dm], np.float64)[:, None]
    want = (dd * np.repeat(sc, 32, axis=1) * q - dmm * np.repeat(mn, 32, axis=1))
    assert np.array_equal(got, want.astype(np.float32))


# --- sampling candidates (src/gpu/kernels.ts:3085-3163, :3265-3323) ---------

def test_pick_candidates_hand_cases():
    """Hand-worked penalties: a logit 2.0 under penalty 2 and presence 0.5
    becomes 2/2 - 0.5 = 0.5, a logit -1.0 becomes -1*2 - 0.5 = -2.5; mask
    byte 2, a cleared allowed bit and ids past the vocabulary become -1e30;
    a seen row's state replaces the mask's only on its rows (state 0 lifts
    the penalty; only the mask byte forbids); chunks rank by maximum, ties
    to the lower chunk."""
    V = 600  # three chunks, the last one 88 ids long
    logits = np.zeros((3, V), np.float32)
    logits[:, 5] = 2.0     # chunk 0
    logits[:, 6] = -1.0
    logits[:, 300] = 2.0   # chunk 1
    logits[:, 520] = 1.0   # chunk 2
    logits[:, 530] = 5.0   # chunk 2, never drawn
    mask = np.zeros(V, np.uint8)
    mask[5], mask[6], mask[530] = 3, 1, 2
    # rows 1-2 see token 300 as written; row 2 no longer sees token 5
    seen = [[300, 3, 1, 3], [5, 0, 2, 3]]
    chunks, cand = O.pick_candidates(logits, 3, mask=mask, seen_rows=seen, row0=0,
                                     penalty=2.0, presence=0.5)
    # row 0: chunk 1 keeps 2.0, chunk 2 has 1.0, chunk 0 has 0.5
    assert list(chunks[0]) == [1, 2, 0]
    assert cand[0, 2, 5] == np.float32(0.5) and cand[0, 2, 6] == np.float32(-2.5)
    assert cand[0, 1, 530 - 512] == np.float32(-1e30)
    assert np.all(cand[0, 1, V - 512:] == np.float32(-1e30))
    # row 1: token 300 falls to 0.5 and ties chunk 0: chunk 2 first, then 0, then 1
    assert list(chunks[1]) == [2, 0, 1] and cand[1, 2, 300 - 256] == np.float32(0.5)
    # row 2: token 5 is unpenalized again (2.0); token 6 keeps its penalty
    assert list(chunks[2]) == [0, 2, 1]
    assert cand[2, 0, 5] == np.float32(2.0) and cand[2, 0, 6] == np.float32(-2.5)
    # the same rows picked one at a time (row0 names the batch row)
    c1, v1 = O.pick_candidates(logits[1:2], 3, mask=mask, seen_rows=seen, row0=1,
                               penalty=2.0, presence=0.5)
    assert np.array_equal(c1[0], chunks[1]) and np.array_equal(v1[0], cand[1])
    # an allowed bitmap with token 300's bit cleared
    allowed = np.full((1, (V + 31) // 32), 0xFFFFFFFF, np.uint32)
    allowed[0, 300 // 32] &= ~np.uint32(1 << (300 % 32))
    chunks, cand = O.pick_candidates(logits[:1], 3, allowed=allowed)
    assert list(chunks[0]) == [2, 0, 1] and cand[0, 2, 300 - 256] == np.float32(-1e30)


def test_pick_candidates_hold_the_top_k():
    """For k <= count, the k largest penalized logits all lie in the kept
    chunks (each lies in a chunk whose maximum is among the k largest):
    checked against a sort of the whole penalized row."""
    rng = np.random.default_rng(3)
    V, count = 5000, 6
    logits = rng.standard_normal((2, V)).astype(np.float32)
    chunks, cand = O.pick_candidates(logits, count)
    for m in range(2):
        top = np.argsort(-logits[m], kind="stable")[:count]
        kept = set(int(c) for c in chunks[m])
        assert all(int(t) // 256 in kept for t in top)
        got = np.sort(cand[m].reshape(-1))[::-1][:count]
        assert np.array_equal(got, np.sort(logits[m])[::-1][:count])


# --- Gated DeltaNet (src/delta-rule.test.ts) ----------------------------------

def _delta_inputs(seed, dk, dv, tokens, similar=0.0, decay=0.2):
    """src/delta-rule.test.ts:23-53: unit q (over sqrt(dk)) and k, beta in
    (0, 1), log-decays -decay * softplus(normal), from mulberry32."""
    rand = O.Mulberry32(seed)

    def normal():
        u = max(rand(), 1e-12)
        return math.sqrt(-2 * math.log(u)) * math.cos(2 * math.pi * rand())
    shared = [normal() for _ in range(dk)]

    def unit(scale):
        x = np.array([similar * shared[i] + normal() for i in range(dk)])
        return x / math.hypot(*x) * scale
    q = np.zeros((tokens, dk))
    k = np.zeros((tokens, dk))
    v = np.zeros((tokens, dv))
    beta = np.zeros(tokens)
    g = np.zeros(tokens)
    for t in range(tokens):
        q[t] = unit(1 / math.sqrt(dk))
        k[t] = unit(1)
        v[t] = [normal() for _ in range(dv)]
        beta[t] = 1 / (1 + math.exp(-2 * normal()))
        g[t] = -decay * math.log(1 + math.exp(normal()))
    return q, k, v, beta, g


def _random_state(seed, dk, dv):
    rand = O.Mulberry32(seed)
    return np.array([rand() - 0.5 for _ in range(dk * dv)]).reshape(dk, dv)


def _rel(a, b):
    return np.max(np.abs(a - b)) / np.max(np.abs(b))


@pytest.mark.parametrize("tokens,chunk", [(64, 16), (64, 32), (50, 16), (37, 32), (5, 16),
                                          (1, 16), (96, 64)])
def test_delta_chunked_matches_sequential(tokens, chunk):
    # src/delta-rule.test.ts:70-92
    x = _delta_inputs(tokens * 31 + chunk, 16, 12, tokens)
    s0 = _random_state(tokens + chunk, 16, 12)
    o1, s1 = O.delta_sequential(*x, s0)
    o2, s2, _ = O.delta_chunked(*x, s0, chunk)
    assert _rel(o2, o1) < 1e-10 and _rel(s2, s1) < 1e-10


def test_delta_collinear_keys_and_fast_decay():
    # src/delta-rule.test.ts:94-113
    x = _delta_inputs(7, 32, 8, 64, similar=6, decay=0.01)
    s0 = _random_state(8, 32, 8)
    o1, s1 = O.delta_sequential(*x, s0)
    o2, s2, _ = O.delta_chunked(*x, s0, 32)
    assert _rel(o2, o1) < 1e-8 and _rel(s2, s1) < 1e-8
    x = _delta_inputs(9, 16, 8, 48, decay=20)
    s0 = _random_state(10, 16, 8)
    o1, s1 = O.delta_sequential(*x, s0)
    o2, s2, _ = O.delta_chunked(*x, s0, 16)
    assert np.all(np.isfinite(o2)) and _rel(o2, o1) < 1e-10 and _rel(s2, s1) < 1e-10


@pytest.mark.parametrize("tokens,save_at", [(50, 7), (50, 39), (64, 1), (37, 31), (5, 3)])
def test_delta_chunk_ends_at_the_snapshot(tokens, save_at):
    # src/delta-rule.test.ts:115-141: a shorter first chunk so that one ends at save_at
    first = save_at % 16 or 16
    x = _delta_inputs(tokens * 7 + save_at, 16, 12, tokens)
    s0 = _random_state(tokens + save_at, 16, 12)
    o1, s1 = O.delta_sequential(*x, s0)
    o2, s2, snap = O.delta_chunked(*x, s0, 16, first=first, save_at=save_at)
    assert _rel(o2, o1) < 1e-10 and _rel(s2, s1) < 1e-10
    _, prefix = O.delta_sequential(*(a[:save_at] for a in x), s0)
    assert _rel(snap, prefix) < 1e-10


def test_delta_chunked_then_token_steps():
    # src/delta-rule.test.ts:143-165
    x = _delta_inputs(11, 16, 16, 40)
    s0 = _random_state(12, 16, 16)
    _, after, _ = O.delta_chunked(*(a[:33] for a in x), s0, 16)
    o_rest, s_rest = O.delta_sequential(*(a[33:] for a in x), after)
    o_all, s_all = O.delta_sequential(*x, s0)
    assert _rel(o_rest, o_all[33:]) < 1e-10 and _rel(s_rest, s_all) < 1e-10


def test_delta_rule_closed_forms():
    """The delta rule's defining facts: with a = 1, beta = 1 and a unit key,
    the new state reads v back (S'^T k = v); the output is the new state
    read by q (o = S'^T q); with beta = 0 the state only decays."""
    rng = np.random.default_rng(0)
    dk, dv = 8, 5
    S = rng.standard_normal((dk, dv))
    k = rng.standard_normal(dk)
    k /= np.linalg.norm(k)
    q = rng.standard_normal(dk)
    v = rng.standard_normal(dv)
    o, S1 = O.delta_sequential(q[None], k[None], v[None], [1.0], [0.0], S)
    assert np.allclose(S1.T @ k, v, atol=1e-12)
    assert np.allclose(o[0], S1.T @ q, atol=1e-12)
    o, S2 = O.delta_sequential(q[None], k[None], v[None], [0.0], [math.log(0.25)], S)
    assert np.allclose(S2, 0.25 * S, atol=1e-15) and np.allclose(o[0], 0.25 * S.T @ q)


def test_delta_layer_gates_prep_conv_norm():
    """LIN_GATES: sigmoid(0) = 1/2, softplus(0) = ln 2, softplus(t) -> t for
    large t, the log-decay A * softplus. LIN_PREP: unit k, q of norm
    1/sqrt(dk) (up to the 1e-6 inside the root). orc_delta_rule composes
    these with the sequential rule head by head. LIN_CONV: taps
    (0, ..., 0, 1) give silu(x); a batch split in two through the carried
    state equals the whole batch. LIN_NORM: a constant head output c gives
    c / sqrt(c^2 + eps) * w * silu(z)."""
    H, dk, dv = 2, 4, 3
    ba = np.array([[0.0, 3.0, 0.0, 40.0]], np.float32)
    A = np.array([-0.5, -2.0], np.float32)
    dt = np.zeros(2, np.float32)
    rng = np.random.default_rng(1)
    qkv = rng.standard_normal((1, 2 * H * dk + H * dv)).astype(np.float32)
    S0 = rng.standard_normal((H, dk, dv))
    out, S1, _ = O.delta_rule(qkv, ba, A, dt, H, dk, dv, S0)
    betas = [0.5, 1 / (1 + math.exp(-3.0))]
    logs = [-0.5 * math.log(2.0), -2.0 * 40.0]
    for h in range(H):
        q = qkv[0, h * dk:(h + 1) * dk].astype(np.float64)
        k = qkv[0, H * dk + h * dk:H * dk + (h + 1) * dk].astype(np.float64)
        v = qkv[0, 2 * H * dk + h * dv:2 * H * dk + (h + 1) * dv]
        qh = q / math.sqrt(q @ q + 1e-6) / math.sqrt(dk)
        kh = k / math.sqrt(k @ k + 1e-6)
        assert abs(np.linalg.norm(kh) - 1) < 1e-5
        o, S = O.delta_sequential(qh[None], kh[None], v[None], [betas[h]], [logs[h]], S0[h])
        assert np.allclose(out[0, h * dv:(h + 1) * dv], o[0], rtol=1e-12, atol=1e-12)
        assert np.allclose(S1[h], S, rtol=1e-12, atol=1e-12)
    # the convolution
    M, C, W = 6, 5, 4
    x = rng.standard_normal((M, C + 3)).astype(np.float32)
    st = rng.standard_normal((W - 1, C)).astype(np.float32)
    taps = np.zeros((C, W), np.float32)
    taps[:, -1] = 1
    y, _ = O.delta_conv(x, C, taps, st)
    xs = x[:, :C].astype(np.float64)
    assert np.allclose(y, xs / (1 + np.exp(-xs)), rtol=1e-14)
    taps = rng.standard_normal((C, W)).astype(np.float32)
    y, s_all = O.delta_conv(x, C, taps, st)
    y1, s1 = O.delta_conv(x[:2], C, taps, st)
    y2, s2 = O.delta_conv(x[2:], C, taps, s1)
    assert np.array_equal(np.vstack([y1, y2]), y) and np.array_equal(s2, s_all)
    assert np.array_equal(s_all, x[M - 3:, :C])
    # the gated norm
    o = np.full((1, H * dv), 0.75, np.float32)
    z = rng.standard_normal((1, H * dv)).astype(np.float32)
    w = rng.standard_normal(dv).astype(np.float32)
    got = O.delta_norm(o, H, dv, z, w, 1e-6)
    zz = z[0].astype(np.float64)
    want = 0.75 / math.sqrt(0.75 ** 2 + float(np.float32(1e-6))) * np.tile(w, H) * zz / (1 + np.exp(-zz))
    assert np.allclose(got[0], want, rtol=1e-12)
