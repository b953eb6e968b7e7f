"""Decode attention that prepares its own heads (wg_attn_decode_prep) against
head preparation then the MFMA decode attention (wg_head_prep +
wg_attn_decode with attn_mfma 2), which test_kernels_gpu checks against the
oracle: the output, the prepared queries and both caches bit for bit, with
and without the q/k norm, new rows across chunk and split edges, at the
cache's first and last rows, grouped by XCD or not."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


class _Knobs:
    def __init__(self, **knobs):
        self.knobs = knobs

    def __enter__(self):
        from webgllm_amd import lib as L
        self.old = {k: L.tuning_get(k) for k in self.knobs}
        for k, v in self.knobs.items():
            L.tuning_set(k, v)

    def __exit__(self, *exc):
        from webgllm_amd import lib as L
        for k, v in self.old.items():
            L.tuning_set(k, v)


def _case(H, KV, hd, M, pos0, norm, ctx, xcd, seed=0):
    from webgllm_amd import ops
    rng = np.random.default_rng(seed + 7 * M + pos0)
    qkv = _t(rng.standard_normal((M, (H + 2 * KV) * hd)).astype(np.float32))
    qn = _t(rng.uniform(0.5, 1.5, hd).astype(np.float32)) if norm else None
    kn = _t(rng.uniform(0.5, 1.5, hd).astype(np.float32)) if norm else None
    rope = _t(O.rope_table(1e6, hd, hd, ctx))
    shape = ops.attn_shape(H, KV, hd, hd, 1e-5, norm)
    pos = _t(np.array([pos0], np.int32))
    base_k = _t(O.f32_to_h2(rng.standard_normal((ctx, KV * hd)).astype(np.float32) * 0.5)
                .view(np.int16))
    base_v = _t(O.f32_to_h2(rng.standard_normal((ctx, KV * hd)).astype(np.float32))
                .view(np.int16))
    with _Knobs(attn_mfma=2, attn_xcd=xcd):
        ka, va = base_k.clone(), base_v.clone()
        qa = torch.full((M, H * hd), 7.0, device="cuda")
        ops.head_prep(qkv, shape, rope, pos, ka, va, qn, kn, q_out=qa)
        oa = ops.attn_decode(qa, shape, ka, va, pos)
        kb, vb = base_k.clone(), base_v.clone()
        qb = torch.full((M, H * hd), 7.0, device="cuda")
        ob = ops.attn_decode_prep(qkv, shape, rope, pos, kb, vb, qn, kn, q_out=qb)
    torch.cuda.synchronize()
    assert ob is not None
    return (oa, qa, ka, va), (ob, qb, kb, vb)


def _same(a, b):
    ia = a.view(torch.int16) if a.element_size() == 2 else a.view(torch.int32)
    ib = b.view(torch.int16) if b.element_size() == 2 else b.view(torch.int32)
    return torch.equal(ia, ib)


@pytest.mark.parametrize("xcd", [1, 0])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("H,KV,hd", [(32, 8, 64), (32, 8, 128), (14, 2, 64)])
@pytest.mark.parametrize("M,pos0", [(1, 0), (5, 0), (5, 30), (5, 1021), (8, 3000), (2, 2046)])
def test_attn_prep_matches_head_prep_then_attention(hip, xcd, norm, H, KV, hd, M, pos0):
    ctx = 4096
    want, got = _case(H, KV, hd, M, pos0, norm, ctx, xcd)
    for name, a, b in zip(("out", "q", "k_cache", "v_cache"), want, got):
        assert _same(a, b), name


@pytest.mark.parametrize("M,pos0", [(16, 100), (16, 4090), (3, 4094)])
def test_attn_prep_many_rows_and_the_cache_end(hip, M, pos0):
    # 16 rows (a lane group's new key each); rows past the cache store
    # nothing and their queries are zero, as head preparation does
    ctx = 4096
    want, got = _case(32, 8, 64, M, pos0, True, ctx, 1, seed=3)
    for name, a, b in zip(("out", "q", "k_cache", "v_cache"), want, got):
        assert _same(a, b), name


def test_attn_prep_refuses_what_it_does_not_take(hip):
    from webgllm_amd import ops
    H, KV, hd, ctx = 8, 2, 128, 2048
    qkv = torch.zeros((2, (H + 2 * KV) * hd), device="cuda")
    rope = _t(O.rope_table(1e6, hd, 64, ctx))
    kc = torch.zeros((ctx, KV * hd), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    pos = _t(np.array([5], np.int32))
    # half the dims rotated: not taken, nothing launched
    shape = ops.attn_shape(H, KV, hd, 64, 1e-5, False)
    assert ops.attn_decode_prep(qkv, shape, rope, pos, kc, vc) is None
    # 17 rows: not taken
    shape = ops.attn_shape(H, KV, hd, hd, 1e-5, False)
    qkv17 = torch.zeros((17, 24 * hd), device="cuda")
    assert ops.attn_decode_prep(qkv17, ops.attn_shape(8, 8, hd, hd, 1e-5, False), rope, pos,
                                torch.zeros((ctx, 8 * hd), dtype=torch.int16, device="cuda"),
                                torch.zeros((ctx, 8 * hd), dtype=torch.int16, device="cuda"),
                                ) is None
    with pytest.raises(Exception, match="norm weights"):
        ops.attn_decode_prep(qkv, ops.attn_shape(H, KV, hd, hd, 1e-5, True), rope, pos, kc, vc)
    assert not kc.any() and not vc.any()
