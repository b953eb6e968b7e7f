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
