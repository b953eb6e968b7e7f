"""Synthetic inputs shared by the tests (numpy, seeded)."""
import numpy as np

from oracle import oracle as O


def halves(rng, n, lo, hi):
    return np.array([O.to_half(v) for v in rng.uniform(lo, hi, n)], dtype=np.uint16) \
        if n < 4096 else rng.uniform(lo, hi, n).astype(np.float16).view(np.uint16)


def gguf_q4_0(rng, N, K, sigma=0.02):
    """GGUF Q4_0 bytes of an N(0, sigma) matrix, by ggml's reference quantizer."""
    w = (rng.standard_normal((N, K)) * sigma).astype(np.float32)
    return O.quantize_q4_0(w)


def random_q4_0_bytes(rng, N, K):
    """Arbitrary Q4_0 blocks: any nibbles, scales over a wide half range."""
    blocks = N * K // 32
    b = rng.integers(0, 256, blocks * 18, dtype=np.uint8).reshape(blocks, 18)
    d = halves(rng, blocks, -0.5, 0.5)
    b[:, 0] = d & 255
    b[:, 1] = d >> 8
    return b.reshape(-1)


def nbits(rng, N, K, sigma=0.02, with_zp=True):
    """MatMulNBits (quant, scale bytes, zp) of an N(0, sigma) matrix, zp ~ U{0..15}."""
    w = (rng.standard_normal((N, K)) * sigma).astype(np.float32)
    zpb = rng.integers(0, 16, N * (K // 32), dtype=np.uint8) if with_zp else \
        np.full(N * (K // 32), 8, np.uint8)
    quant, scales, zp = O.quantize_nbits(w, zpb)
    return quant, scales, (zp if with_zp else None)


def random_q4_k_bytes(rng, N, K, zero_scale_every=0, extreme=False):
    """Q4_K super-blocks with random nibbles and 6-bit scales/mins; d, dmin
    halves in a realistic range (or anywhere finite with `extreme`)."""
    supers = N * K // 256
    b = rng.integers(0, 256, supers * 144, dtype=np.uint8).reshape(supers, 144)
    if extreme:
        d = rng.integers(0, 0x7C00, supers).astype(np.uint16)
        dm = rng.integers(0, 0x7C00, supers).astype(np.uint16)
    else:
        d = rng.uniform(0.0005, 0.004, supers).astype(np.float16).view(np.uint16)
        dm = rng.uniform(0.0005, 0.006, supers).astype(np.float16).view(np.uint16)
    b[:, 0], b[:, 1] = d & 255, d >> 8
    b[:, 2], b[:, 3] = dm & 255, dm >> 8
    if zero_scale_every:
        # Zero the 6-bit scale of sub-block (s % 8) for every k-th super-block.
        for s in range(0, supers, zero_scale_every):
            j = s % 8
            if j < 4:
                b[s, 4 + j] &= 0xC0
            else:
                b[s, 4 + j + 4] &= 0xF0
                b[s, 4 + j - 4] &= 0x3F
    return b.reshape(-1)


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


def lcg_bytes(n, seed):
    """src/q6-expanded.test.ts:11-16: seed = seed * 1664525 + 1013904223
    (mod 2^32), byte = seed >> 24."""
    out = np.empty(n, dtype=np.uint8)
    for i in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = seed >> 24
    return out


def imul_bytes(n, offset):
    """src/q6-split.test.ts:7 and q8-converter.test.ts:5: Math.imul(i +
    offset, 2654435761) >>> 24."""
    i = np.arange(n, dtype=np.uint64) + np.uint64(offset)
    return ((i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)) >> np.uint64(24)


def encode_q6_k(q, sc, d_bits):
    """GGUF Q6_K super-blocks from 6-bit codes q [supers, 256] (0..63), int8
    sub-block scales sc [supers, 16] and half d bits [supers]: the packing
    loop of ggml's quantize_row_q6_K (per 128 weights j, l = 0..31: ql[l] =
    q[j+l] & 15 | (q[j+l+64] & 15) << 4, ql[l+32] = q[j+l+32] & 15 |
    (q[j+l+96] & 15) << 4, qh[l] = q[j+l] >> 4 | q[j+l+32] >> 4 << 2 |
    q[j+l+64] >> 4 << 4 | q[j+l+96] >> 4 << 6), ql then qh then scales then
    d, 210 bytes each."""
    q = np.asarray(q, dtype=np.int64)
    supers = q.shape[0]
    out = np.zeros((supers, 210), dtype=np.uint8)
    for s in range(supers):
        ql = np.zeros(128, np.int64)
        qh = np.zeros(64, np.int64)
        for half in range(2):
            L = q[s, 128 * half:128 * half + 128]
            for l in range(32):
                ql[64 * half + l] = (L[l] & 15) | ((L[l + 64] & 15) << 4)
                ql[64 * half + l + 32] = (L[l + 32] & 15) | ((L[l + 96] & 15) << 4)
                qh[32 * half + l] = ((L[l] >> 4) | ((L[l + 32] >> 4) << 2) |
                                     ((L[l + 64] >> 4) << 4) | ((L[l + 96] >> 4) << 6))
        out[s, :128] = ql
        out[s, 128:192] = qh
        out[s, 192:208] = np.asarray(sc[s], dtype=np.int8).view(np.uint8)
        out[s, 208] = int(d_bits[s]) & 255
        out[s, 209] = int(d_bits[s]) >> 8
    return out.reshape(-1)


def encode_q5_k(q, sc, mn, d_bits, dmin_bits):
    """GGUF Q5_K super-blocks from 5-bit codes q [supers, 256] (0..31), 6-bit
    sub-block scales sc and mins mn [supers, 8] and half d, dmin bits: the
    packing of ggml's quantize_row_q5_K (the scales and mins as Q4_K packs
    them: sub-blocks 0..3 in the low 6 bits of bytes j and j + 4, 4..7 split
    over the nibbles of bytes j + 8 and the top 2 bits of bytes j - 4 and j;
    per 64 weights, ql[l] = q[l] & 15 | (q[l + 32] & 15) << 4 and bits 2j,
    2j + 1 of qh[l] their fifth bits), 176 bytes each."""
    q = np.asarray(q, dtype=np.int64)
    supers = q.shape[0]
    out = np.zeros((supers, 176), dtype=np.uint8)
    for s in range(supers):
        out[s, 0], out[s, 1] = int(d_bits[s]) & 255, int(d_bits[s]) >> 8
        out[s, 2], out[s, 3] = int(dmin_bits[s]) & 255, int(dmin_bits[s]) >> 8
        scales = out[s, 4:16]
        for j in range(4):
            scales[j] = (sc[s][j] & 63) | ((sc[s][j + 4] >> 4) << 6)
            scales[j + 4] = (mn[s][j] & 63) | ((mn[s][j + 4] >> 4) << 6)
            scales[j + 8] = (sc[s][j + 4] & 15) | ((mn[s][j + 4] & 15) << 4)
        qh = np.zeros(32, np.int64)
        ql = np.zeros(128, np.int64)
        for pair in range(4):
            lo, hi = q[s, 64 * pair:64 * pair + 32], q[s, 64 * pair + 32:64 * pair + 64]
            ql[32 * pair:32 * pair + 32] = (lo & 15) | ((hi & 15) << 4)
            qh |= ((lo >> 4) & 1) << (2 * pair)
            qh |= ((hi >> 4) & 1) << (2 * pair + 1)
        out[s, 16:48] = qh
        out[s, 48:176] = ql
    return out.reshape(-1)
