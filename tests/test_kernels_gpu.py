"""Norm, SwiGLU, embedding, headPrep, decode attention, short convolution and
greedy pick on the GPU against the oracle."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gguf_q4_0, nbits, random_q4_k_bytes, rel_l2

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def _h(t):
    return O.halves_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("M,D", [(1, 896), (5, 2048), (1, 4096), (3, 14336)])
def test_rms_norm(hip, M, D):
    from webgllm_amd import ops
    rng = np.random.default_rng(D + M)
    x = (rng.standard_normal((M, D)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    rs = torch.empty(M, device="cuda")
    out = ops.rms_norm(_t(x), _t(w), 1e-5, rs_out=rs)
    want = O.rms_norm(x, w, 1e-5)
    got = _h(out)
    # half outputs: within half rounding of the float64 norm
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -10 + 1e-7)
    assert np.allclose(rs.cpu().numpy(), 1 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + 1e-5),
                       rtol=1e-5)


def test_swiglu(hip):
    from webgllm_amd import ops
    rng = np.random.default_rng(1)
    gu = (rng.standard_normal((3, 2 * 4864)) * 2).astype(np.float32)
    got = _h(ops.swiglu(_t(gu)))
    want = O.swiglu(gu)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -10 + 1e-6)


@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k", "q4_k_native"])
def test_embed_bit_exact(hip, fmt):
    from webgllm_amd import ops
    rng = np.random.default_rng(11)
    N, K = 512, 512
    if fmt == "q4_0":
        src = gguf_q4_0(rng, N, K)
        want = O.QuantMatrix(N, K, False)
        O.pack_q4_0(want, 0, src, N)
        m = ops.Q4Matrix.from_q4_0(ops.to_device_bytes(src), N, K)
    elif fmt == "nbits":
        q, s, z = nbits(rng, N, K)
        want = O.QuantMatrix(N, K, True)
        O.pack_nbits(want, 0, q, s, z, N)
        m = ops.Q4Matrix.from_nbits(ops.to_device_bytes(q), ops.to_device_bytes(s),
                                    ops.to_device_bytes(z), N, K)
    else:
        src = random_q4_k_bytes(rng, N, K, zero_scale_every=3)
        want = O.QuantMatrix(N, K, "halves")
        O.pack_q4_k(want, 0, src, N)
        m = ops.Q4Matrix.from_q4_k(ops.to_device_bytes(src), N, K, native=fmt == "q4_k_native")
    ids = np.array([0, 5, 511, 300, 7, 1000, -1], np.int32)
    got = ops.embed(m, _t(ids)).cpu().numpy()
    for i, n in enumerate(ids):
        if 0 <= n < N:
            assert np.array_equal(got[i].view(np.uint32), want.row(int(n)).view(np.uint32))
        else:
            assert np.all(got[i] == 0)


def _cache_rows(k_cache, rows):
    return k_cache[:rows].view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("H,KV,hd,R,norm", [(14, 2, 64, 64, False), (32, 8, 128, 128, False),
                                            (32, 8, 64, 64, True), (8, 2, 128, 64, True)])
@pytest.mark.parametrize("pos0", [0, 1021, 3000])
def test_head_prep(hip, H, KV, hd, R, norm, pos0):
    from webgllm_amd import ops
    rng = np.random.default_rng(H * hd + pos0)
    M, ctx = 3, 4096
    rope = O.rope_table(1e6, hd, R, ctx)
    qkv = rng.standard_normal((M, (H + 2 * KV) * hd)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    shape = ops.attn_shape(H, KV, hd, R, 1e-6, norm)
    kc = torch.zeros((ctx, KV * hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    q = ops.head_prep(_t(qkv), shape, _t(rope), _t(np.array([pos0], np.int32)), kc, vc,
                      _t(qn) if norm else None, _t(kn) if norm else None).cpu().numpy()
    kcn = _cache_rows(kc, ctx)
    vcn = _cache_rows(vc, ctx)
    for m in range(M):
        pos = pos0 + m
        for h in range(H):
            x = qkv[m, h * hd:(h + 1) * hd]
            want = O.head_prep(x, qn, rope, hd, R, pos, 1e-6, 1 / math.sqrt(hd), norm)
            assert np.allclose(q[m, h * hd:(h + 1) * hd], want, rtol=1e-5, atol=1e-6)
        for h in range(KV):
            x = qkv[m, (H + h) * hd:(H + h + 1) * hd]
            want = O.f32_to_h2(O.head_prep(x, kn, rope, hd, R, pos, 1e-6, 1.0, norm))
            got = kcn[pos, h * hd:(h + 1) * hd]
            # halves of float32 values that agree to ~1e-6: at most one half ulp apart
            assert np.max(np.abs(got.astype(np.int32) - want.astype(np.int32))) <= 1
            v = qkv[m, (H + KV + h) * hd:(H + KV + h + 1) * hd]
            assert np.array_equal(vcn[pos, h * hd:(h + 1) * hd], O.f32_to_h2(v))
    # rows outside the written positions stay untouched
    assert not np.any(kcn[pos0 + M:])


@pytest.fixture(params=["mfma", "mfma-xcd", "xcd", "xcd-1", "xcd-4", "one-launch",
                        "one-launch-1", "one-launch-2", "one-launch-4", "two-launch"])
def decode_path(request):
    """wg_attn_decode's forms: one launch on MFMA, its splits exchanged
    through memory or (KV heads x query groups a multiple of 8) within each
    XCD; one launch combined within each XCD (KV heads a multiple of 8;
    elsewhere the default form); one launch on vector units (chunks a
    workgroup chosen, or 1, 2, 4); or chunks then a combine."""
    from webgllm_amd import lib as L
    knobs = ("attn_mfma", "attn_fused", "attn_split_chunks", "attn_xcd")
    old = [L.tuning_get(k) for k in knobs]
    name = request.param
    L.tuning_set("attn_mfma", 2 if name.startswith("mfma") else 0)
    L.tuning_set("attn_xcd", 2 if name.startswith("xcd") else 1 if name == "mfma-xcd" else 0)
    L.tuning_set("attn_fused", 0 if name == "two-launch" else 2)
    L.tuning_set("attn_split_chunks", int(name[-1]) if name[-1].isdigit() else 0)
    yield name
    for k, v in zip(knobs, old):
        L.tuning_set(k, v)


@pytest.mark.parametrize("H,KV,hd", [(14, 2, 64), (32, 8, 128), (32, 8, 64)])
@pytest.mark.parametrize("M,pos0", [(1, 0), (1, 63), (1, 64), (1, 127), (1, 128), (1, 4095),
                                    (2, 129), (2, 4000), (5, 200), (5, 1500)])
def test_attn_decode(hip, decode_path, H, KV, hd, M, pos0):
    from webgllm_amd import ops
    rng = np.random.default_rng(H + hd + M + pos0)
    ctx = 4096 + 8
    shape = ops.attn_shape(H, KV, hd)
    kd = KV * hd
    nkeys = pos0 + M
    k = O.f32_to_h2((rng.standard_normal((nkeys, kd))).astype(np.float32))
    v = O.f32_to_h2(rng.standard_normal((nkeys, kd)).astype(np.float32))
    q = (rng.standard_normal((M, H * hd)) / math.sqrt(hd) * 2).astype(np.float32)
    kc = torch.zeros((ctx, kd), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:nkeys] = _t(k.view(np.int16))
    vc[:nkeys] = _t(v.view(np.int16))
    out = ops.attn_decode(_t(q), shape, kc, vc, _t(np.array([pos0], np.int32)))
    got = _h(out)
    for m in range(M):
        want = O.attention_f64(q[m], k, v, H, KV, hd, pos0 + m + 1, kd)
        err = rel_l2(got[m], want)
        assert err <= 1e-3, (m, err)


@pytest.mark.parametrize("H,KV,hd,M", [(32, 8, 128, 1), (14, 2, 64, 1), (32, 8, 64, 5)])
def test_attn_decode_ignores_rows_past_the_position(hip, decode_path, H, KV, hd, M):
    """Cache rows past the position and a scratch that hold NaN bits (the
    kernels load them before they know the position) never reach the
    output; only the counters at the scratch's start are zero."""
    from webgllm_amd import ops
    rng = np.random.default_rng(H + M)
    ctx, pos0 = 1024, 300
    shape = ops.attn_shape(H, KV, hd)
    kd = KV * hd
    k = O.f32_to_h2(rng.standard_normal((ctx, kd)).astype(np.float32))
    v = O.f32_to_h2(rng.standard_normal((ctx, kd)).astype(np.float32))
    k[pos0 + M:] = 0x7e00
    v[pos0 + M:] = 0x7e00
    q = (rng.standard_normal((M, H * hd)) / math.sqrt(hd) * 2).astype(np.float32)
    scratch = ops.attn_scratch(M, shape, ctx)
    scratch.fill_(0xff)
    # the counters: the scratch of no rows and no keys
    from webgllm_amd import lib as L
    scratch[:L.load().wg_attn_scratch_bytes(0, H, hd, 0)].zero_()
    got = _h(ops.attn_decode(_t(q), shape, _t(k.view(np.int16)), _t(v.view(np.int16)),
                             _t(np.array([pos0], np.int32)), scratch=scratch))
    assert np.isfinite(got).all()
    for m in range(M):
        want = O.attention_f64(q[m], k, v, H, KV, hd, pos0 + m + 1, kd)
        assert rel_l2(got[m], want) <= 1e-3


def test_attn_decode_reuses_its_scratch(hip, decode_path):
    """One scratch across calls at changing positions and row counts (both
    chunk kernels and the combine, or the one-launch form whose counters
    each call leaves at zero): every call matches the oracle."""
    from webgllm_amd import ops
    H, KV, hd, ctx = 32, 8, 128, 2048
    shape = ops.attn_shape(H, KV, hd)
    rng = np.random.default_rng(12)
    kd = KV * hd
    k = O.f32_to_h2(rng.standard_normal((ctx, kd)).astype(np.float32))
    v = O.f32_to_h2(rng.standard_normal((ctx, kd)).astype(np.float32))
    kc, vc = _t(k.view(np.int16)), _t(v.view(np.int16))
    scratch = ops.attn_scratch(8, shape, ctx)
    for pos0, M in [(5, 1), (700, 2), (129, 1), (2000, 5), (1500, 1), (31, 2), (2040, 8),
                    (64, 1)]:
        q = (rng.standard_normal((M, H * hd)) / math.sqrt(hd) * 2).astype(np.float32)
        got = _h(ops.attn_decode(_t(q), shape, kc, vc, _t(np.array([pos0], np.int32)),
                                 scratch=scratch))
        for m in range(M):
            want = O.attention_f64(q[m], k, v, H, KV, hd, pos0 + m + 1, kd)
            assert rel_l2(got[m], want) <= 1e-3, (pos0, M, m)


@pytest.mark.parametrize("form,H,KV,hd,M,keys", [("xcd", 32, 8, 128, 1, 4096),
                                                 ("xcd", 32, 8, 64, 2, 2048),
                                                 ("mfma-xcd", 32, 8, 64, 5, 1024),
                                                 ("mfma-xcd", 32, 8, 128, 3, 8192)])
def test_attn_decode_xcd_exchange_over_many_launches(hip, form, H, KV, hd, M, keys):
    """The forms whose partials, count and combine stay in one XCD's L2,
    over 160 launches of changing queries and positions back to back in a
    graph (4 layers' caches, one scratch), replayed 3 times: every launch
    agrees with the two-launch form run eagerly on the same inputs (a stale
    partial, from the launch before, would be off by far more)."""
    from webgllm_amd import lib as L
    from webgllm_amd import ops
    knobs = ("attn_mfma", "attn_fused", "attn_split_chunks", "attn_xcd")
    old = [L.tuning_get(k) for k in knobs]
    g = torch.Generator(device="cuda").manual_seed(hd + M)
    shape = ops.attn_shape(H, KV, hd)
    caches = [(torch.randn((keys, KV * hd), device="cuda", generator=g).half(),
               torch.randn((keys, KV * hd), device="cuda", generator=g).half()) for _ in range(4)]
    qs = [torch.randn((M, H * hd), device="cuda", generator=g) / math.sqrt(hd) * 2
          for _ in range(5)]
    q = torch.empty_like(qs[0])
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    scratch = ops.attn_scratch(M, shape, keys)
    iters = 40
    positions = [keys - M - (i * 37) % (keys // 2) for i in range(iters)]
    out = torch.zeros((iters, 4, M, H * hd), dtype=torch.float16, device="cuda")
    want = torch.zeros_like(out)

    def run(dst):
        for i in range(iters):
            q.copy_(qs[i % 5])
            pos.fill_(positions[i])
            for layer, (kc, vc) in enumerate(caches):
                ops.attn_decode(q, shape, kc, vc, pos, scratch=scratch, out=dst[i, layer])
    try:
        for k, v in zip(knobs, (0, 0, 0, 0)):
            L.tuning_set(k, v)
        run(want)
        L.tuning_set("attn_mfma", 2 if form == "mfma-xcd" else 0)
        L.tuning_set("attn_fused", 1)
        L.tuning_set("attn_xcd", 1 if form == "mfma-xcd" else 2)
        run(out)  # the first-call set-up outside the capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                run(out)
        torch.cuda.current_stream().wait_stream(stream)
        for replay in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            d = (out.float() - want.float()).flatten(2)
            err = d.norm(dim=2) / want.float().flatten(2).norm(dim=2)
            assert float(err.max()) <= 1e-3, (replay, float(err.max()))
    finally:
        for k, v in zip(knobs, old):
            L.tuning_set(k, v)


@pytest.mark.parametrize("keys,M", [(32768, 1), (20000, 2), (65536, 1)])
def test_attn_decode_long_context(hip, keys, M):
    """Past the two-launch form's 16,384 keys: 8B-shape heads (32 over 8 of
    128) over 20,000 to 65,536 cached keys in one launch, against the
    float64 oracle; a second call at a smaller position with the same
    scratch agrees too."""
    from webgllm_amd import ops
    H, KV, hd = 32, 8, 128
    shape = ops.attn_shape(H, KV, hd)
    rng = np.random.default_rng(keys + M)
    kd = KV * hd
    k = O.f32_to_h2(rng.standard_normal((keys, kd)).astype(np.float32))
    v = O.f32_to_h2(rng.standard_normal((keys, kd)).astype(np.float32))
    kc, vc = _t(k.view(np.int16)), _t(v.view(np.int16))
    scratch = ops.attn_scratch(M, shape, keys)
    for pos0 in (keys - M, keys // 3):
        q = (rng.standard_normal((M, H * hd)) / math.sqrt(hd) * 2).astype(np.float32)
        got = _h(ops.attn_decode(_t(q), shape, kc, vc, _t(np.array([pos0], np.int32)),
                                 scratch=scratch))
        for m in range(M):
            want = O.attention_f64(q[m], k, v, H, KV, hd, pos0 + m + 1, kd)
            assert rel_l2(got[m], want) <= 1e-3, (pos0, m)


def test_attn_decode_single_key_and_uniform(hip):
    from webgllm_amd import ops
    H, KV, hd = 4, 2, 64
    shape = ops.attn_shape(H, KV, hd)
    rng = np.random.default_rng(2)
    v = O.f32_to_h2(rng.standard_normal((300, KV * hd)).astype(np.float32))
    kc = torch.zeros((300, KV * hd), dtype=torch.int16, device="cuda")
    vc = _t(v.view(np.int16))
    # one key: out = v[0] exactly (weight 1)
    q = _t(rng.standard_normal((1, H * hd)).astype(np.float32))
    got = _h(ops.attn_decode(q, shape, kc, vc, _t(np.array([0], np.int32))))
    vf = O.halves_to_f32(v)
    assert np.array_equal(got[0, :hd], vf[0, :hd])
    # equal scores (zero keys): the mean of the values
    got = _h(ops.attn_decode(q, shape, kc, vc, _t(np.array([299], np.int32))))
    assert rel_l2(got[0, :hd], vf[:300, :hd].astype(np.float64).mean(0)) < 1e-3


def _prefill_case(H, KV, hd, M, pos0, seed, ctx=None, nan_past=False):
    from webgllm_amd import ops
    rng = np.random.default_rng(seed)
    kd = KV * hd
    nkeys = pos0 + M
    ctx = ctx or nkeys + 8
    k = O.f32_to_h2(rng.standard_normal((ctx, kd)).astype(np.float32))
    v = O.f32_to_h2(rng.standard_normal((ctx, kd)).astype(np.float32))
    if nan_past:
        k[nkeys:] = 0x7e00
        v[nkeys:] = 0x7e00
    q = (rng.standard_normal((M, H * hd)) / math.sqrt(hd) * 2).astype(np.float32)
    out = ops.attn_prefill(_t(q), ops.attn_shape(H, KV, hd), _t(k.view(np.int16)),
                           _t(v.view(np.int16)), _t(np.array([pos0], np.int32)))
    return q, k, v, _h(out)


@pytest.fixture(params=[4, 1, 0], ids=["mfma4", "mfma1", "valu"])
def prefill_kernel(request):
    """wg_attn_prefill's kernel: MFMA with 4 or 1 waves a workgroup, or VALU."""
    from webgllm_amd import lib as L
    old = L.tuning_get("attn_prefill_mfma")
    L.tuning_set("attn_prefill_mfma", request.param)
    yield request.param
    L.tuning_set("attn_prefill_mfma", old)


@pytest.mark.parametrize("H,KV,hd", [(14, 2, 64), (32, 8, 128), (32, 8, 64), (4, 2, 64)])
@pytest.mark.parametrize("M,pos0", [(1, 0), (37, 0), (64, 1000), (200, 63), (130, 3000)])
def test_attn_prefill(hip, prefill_kernel, H, KV, hd, M, pos0):
    """Prompt-batch attention (row m at position pos0 + m sees keys up to
    it) against the float64 oracle, on the first and last rows, the rows at
    block and chunk edges and a few random ones."""
    q, k, v, got = _prefill_case(H, KV, hd, M, pos0, seed=H + hd + M + pos0)
    kd = KV * hd
    rng = np.random.default_rng(M)
    rows = sorted({0, M - 1, min(M - 1, 7), min(M - 1, 8), min(M - 1, 63 - pos0 % 64)} |
                  set(rng.integers(0, M, 4).tolist()))
    assert np.isfinite(got).all()
    for m in rows:
        want = O.attention_f64(q[m], k, v, H, KV, hd, pos0 + m + 1, kd)
        assert rel_l2(got[m], want) <= 1e-3, (m, rel_l2(got[m], want))


def test_attn_prefill_ignores_rows_past_the_position(hip, prefill_kernel):
    """Cache rows past the batch's last position hold NaN bits: they never
    reach the output (masked scores, zero-read values)."""
    H, KV, hd, M, pos0 = 32, 8, 128, 45, 100
    q, k, v, got = _prefill_case(H, KV, hd, M, pos0, seed=5, ctx=1024, nan_past=True)
    assert np.isfinite(got).all()
    for m in (0, 20, M - 1):
        want = O.attention_f64(q[m], k, v, H, KV, hd, pos0 + m + 1, KV * hd)
        assert rel_l2(got[m], want) <= 1e-3


def test_attn_prefill_matches_decode_rows(hip, prefill_kernel):
    """A batch's row m equals the decode kernel's answer for that row alone
    at position pos0 + m (both against the same cache), to f32 rounding."""
    from webgllm_amd import ops
    H, KV, hd, M, pos0 = 32, 8, 128, 24, 777
    q, k, v, got = _prefill_case(H, KV, hd, M, pos0, seed=9)
    shape = ops.attn_shape(H, KV, hd)
    kc, vc = _t(k.view(np.int16)), _t(v.view(np.int16))
    for m in (0, 11, 23):
        one = _h(ops.attn_decode(_t(q[m:m + 1]), shape, kc, vc,
                                 _t(np.array([pos0 + m], np.int32))))
        assert rel_l2(got[m], one[0]) <= 1e-4


@pytest.mark.parametrize("M,D,W", [(1, 2048, 3), (5, 2048, 3), (8, 1024, 4), (40, 512, 3)])
def test_short_conv_and_accept(hip, M, D, W):
    from webgllm_amd import ops
    rng = np.random.default_rng(M * D + W)
    bcx = rng.standard_normal((M, 3 * D)).astype(np.float32)
    taps = rng.standard_normal((D, W)).astype(np.float32)
    state = rng.standard_normal((W - 1, D)).astype(np.float32)
    st = _t(state)
    pre = torch.empty((M, W - 1, D), device="cuda")
    out = ops.short_conv(_t(bcx), D, W, _t(taps), st, prefixes=pre)
    want, want_state, want_pre = O.short_conv(bcx, D, W, taps, state, prefixes=True)
    got = _h(out)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -10 + 1e-5)
    assert np.allclose(st.cpu().numpy(), want_state, rtol=1e-6, atol=1e-6)
    assert np.allclose(pre.cpu().numpy(), want_pre, rtol=1e-6, atol=1e-6)
    for kept in range(1, M + 1):
        ops.conv_accept(pre, kept, M, D, W, st)
        assert np.array_equal(st.cpu().numpy(), want_pre[kept - 1])
    with pytest.raises(Exception, match="can't keep"):
        ops.conv_accept(pre, M + 1, M, D, W, st)


@pytest.mark.parametrize("V", [1000, 65536, 128256, 151936])
def test_argmax(hip, V):
    from webgllm_amd import ops
    rng = np.random.default_rng(V)
    x = rng.standard_normal((3, V)).astype(np.float32)
    x[1, V // 3] = 50
    x[1, V // 2] = 50          # tie: lower id
    x[2, :] = -np.inf
    x[2, 17] = np.nan
    ids = ops.argmax_rows(_t(x)).cpu().numpy()
    for m in range(3):
        assert ids[m] == O.argmax(x[m])[0]
    assert ids[1] == V // 3 and ids[2] == 0
    # chunk boundary ties (256-logit chunks in the reference; 1024-logit
    # workgroups and 256-logit thread strides here)
    for b in (256, 1024, 4096):
        y = np.full((1, V), -1.0, np.float32)
        y[0, min(V - 1, b)] = 3
        y[0, min(V - 1, b - 1)] = 3
        assert ops.argmax_rows(_t(y)).cpu().numpy()[0] == O.argmax(y[0])[0]


@pytest.mark.parametrize("V", [1000, 128256])
def test_argmax_advance(hip, V):
    """The decode step's pick and advance: ids[0] = the pick, hist[pos + 1]
    = the pick, pos + 1; at the history's end the pick is not stored."""
    import torch
    from webgllm_amd import ops
    rng = np.random.default_rng(V + 1)
    x = rng.standard_normal(V).astype(np.float32)
    x[V // 5] = 9.0
    x[V // 2] = 9.0  # tie: lower id
    ids = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    pos = torch.tensor([5], dtype=torch.int32, device="cuda")
    hist = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    tops = torch.zeros(1, device="cuda")
    ops.argmax_advance(_t(x), ids, pos, hist=hist, tops=tops)
    want = O.argmax(x)[0]
    assert want == V // 5
    assert ids.cpu().tolist() == [want] + [-1] * 7
    assert pos.item() == 6
    assert hist.cpu().tolist() == [-1] * 6 + [want, -1]
    assert tops.item() == 9.0
    # twice more: pos 6 -> hist[7], then pos 7 -> hist[8] is past the end
    x[3] = 20.0
    ops.argmax_advance(_t(x), ids, pos, hist=hist)
    ops.argmax_advance(_t(x), ids, pos, hist=hist)
    assert pos.item() == 8 and ids[0].item() == 3
    assert hist.cpu().tolist() == [-1] * 6 + [want, 3]
    # no history
    ops.argmax_advance(_t(x), ids, pos)
    assert pos.item() == 9
