"""The short convolution in the in_proj GEMV's epilogue (EPI_SHORT_CONV)
against the same GEMV storing the B | C | x rows followed by the short-conv
kernel, which the oracle pins (test_kernels_gpu): the gated halves, the new
state and the per-token prefixes bit for bit, for each kernel form that
takes the epilogue, with and without the input norm, the state updated in
place or into another buffer, and under graph replay."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

# the kernel forms: streaming GEMVs for every row count, MFMA for every one
FORMS = {"stream": {"gemv_mfma": 0, "gemv_few_stream": 1}, "mfma": {"gemv_mfma": 2}}
ROWGROUP_FMTS = ["q4_0", "nbits", "q4_k_rowgroup", "q4_k_records"]


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _matrix(fmt, N, K, seed):
    from webgllm_amd import engine as E
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.__new__(E.Weights)
    w.shape = shape
    w.device = "cuda"
    w.g = torch.Generator(device="cuda")
    w.g.manual_seed(seed)
    return w.matrix(N, K)


class _Form:
    """Sets a kernel form's knobs, restoring the old values on exit."""

    def __init__(self, knobs):
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


def _inputs(M, D, K, W, norm, seed):
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    x = h * nw / np.float32(32) if norm else h / np.float32(4)
    x16 = _t(O.f32_to_h2(x).view(np.int16))
    parts = _t((h.reshape(M, K // 4, 4) ** 2).sum(-1).astype(np.float32))
    taps = _t(rng.standard_normal((D, W)).astype(np.float32))
    state = rng.standard_normal((W - 1, D)).astype(np.float32)
    return x16, parts, taps, state


def _norm(L, ep, parts, K, norm):
    if norm:
        ep.norm_parts = parts.data_ptr()
        ep.n_parts = ep.ld_parts_in = K // 4
        ep.norm_count = K
        ep.eps = 1e-5
        ep.norm_mult = 32.0
    return ep


def _unfused(m, x16, parts, taps, state, D, K, W, norm, keep):
    from webgllm_amd import lib as L, ops
    M = x16.shape[0]
    bcx = torch.zeros((M, 3 * D), dtype=torch.float32, device="cuda")
    ops.gemv(m, x16, out=bcx, epilogue=_norm(L, L.Epilogue(mode=L.EPI_STORE), parts, K, norm))
    st = _t(state)
    pre = torch.zeros((M, W - 1, D), device="cuda") if keep else None
    out = ops.short_conv(bcx, D, W, taps, st, prefixes=pre)
    return out, st, pre


def _fused(m, x16, parts, taps, state, D, K, W, norm, keep, in_place=True):
    from webgllm_amd import lib as L, ops
    M = x16.shape[0]
    out = torch.full((M, D), float("nan"), dtype=torch.float16, device="cuda")
    st = _t(state)
    st_out = st if in_place else torch.zeros_like(st)
    pre = torch.full((M, W - 1, D), float("nan"), device="cuda") if keep else None
    ep = _norm(L, L.Epilogue(mode=L.EPI_SHORT_CONV, out16=out.data_ptr(), ld_out16=D,
                             conv_taps=taps.data_ptr(), conv_state=st.data_ptr(),
                             conv_state_out=st_out.data_ptr(),
                             conv_prefixes=pre.data_ptr() if keep else None, conv_width=W),
               parts, K, norm)
    assert ops.gemv_short_conv(m, x16, ep)
    return out, st_out, pre


def _bits(t):
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16)


def _same(a, b):
    assert a.dtype == b.dtype
    assert torch.equal(_bits(a), _bits(b))


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("fmt", ROWGROUP_FMTS)
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_conv_epilogue_matches_gemv_then_conv(hip, form, fmt, M):
    D, K, W = 1024, 2048, 3
    m = _matrix(fmt, 3 * D, K, seed=M)
    for norm, keep in ((True, True), (False, False)):
        x16, parts, taps, state = _inputs(M, D, K, W, norm, seed=7 * M + norm)
        with _Form(FORMS[form]):
            want = _unfused(m, x16, parts, taps, state, D, K, W, norm, keep)
            got = _fused(m, x16, parts, taps, state, D, K, W, norm, keep)
        torch.cuda.synchronize()
        for g, w in zip(got, want):
            if w is not None:
                _same(g, w)


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("W", [2, 4])
@pytest.mark.parametrize("D,K", [(2048, 2048), (336, 1024)])
def test_conv_epilogue_widths_and_shapes(hip, form, W, D, K):
    M = 5
    m = _matrix("q4_0", 3 * D, K, seed=W + D)
    x16, parts, taps, state = _inputs(M, D, K, W, True, seed=W)
    with _Form(FORMS[form]):
        want = _unfused(m, x16, parts, taps, state, D, K, W, True, True)
        got = _fused(m, x16, parts, taps, state, D, K, W, True, True, in_place=False)
        one = _fused(m, x16[:1], parts[:1], taps, state, D, K, W, True, True)
        want1 = _unfused(m, x16[:1], parts[:1], taps, state, D, K, W, True, True)
    torch.cuda.synchronize()
    for g, w in zip(got + one, want + want1):
        _same(g, w)


def test_conv_epilogue_refusals(hip):
    from webgllm_amd import lib as L, ops
    D, K, W = 1024, 1024, 3
    x16, parts, taps, state = _inputs(2, D, K, W, False, seed=1)
    st = _t(state)
    out = torch.zeros((2, D), dtype=torch.int16, device="cuda")

    def ep(width=W, ld=D, state_out=None):
        return L.Epilogue(mode=L.EPI_SHORT_CONV, out16=out.data_ptr(), ld_out16=ld,
                          conv_taps=taps.data_ptr(), conv_state=st.data_ptr(),
                          conv_state_out=state_out or st.data_ptr(), conv_width=width)

    # other layouts: not taken (the caller runs the GEMV, then the conv)
    assert not ops.gemv_short_conv(_matrix("q8_0", 3 * D, K, seed=1), x16, ep())
    m = _matrix("q4_0", 3 * D, K, seed=1)
    with pytest.raises(Exception, match="width"):
        ops.gemv_short_conv(m, x16, ep(width=5))
    with pytest.raises(Exception, match="ld_out16"):
        ops.gemv_short_conv(m, x16, ep(ld=D - 1))
    with pytest.raises(Exception, match="overlap"):
        ops.gemv_short_conv(m, x16, ep(state_out=st.data_ptr() + 4))
    with pytest.raises(Exception, match="multiple of 16"):
        ops.gemv_short_conv(_matrix("q4_0", 3 * 1000, K, seed=1), x16, ep())


@pytest.mark.parametrize("form", sorted(FORMS))
def test_conv_epilogue_graph_replay(hip, form):
    """Captured once and replayed over fresh inputs: each replay matches the
    eager pair of launches."""
    M, D, K, W = 4, 1024, 2048, 3
    m = _matrix("nbits", 3 * D, K, seed=3)
    x16, parts, taps, state = _inputs(M, D, K, W, True, seed=3)
    from webgllm_amd import lib as L, ops
    out = torch.zeros((M, D), dtype=torch.float16, device="cuda")
    st = _t(state)
    pre = torch.zeros((M, W - 1, D), device="cuda")
    ep = _norm(L, L.Epilogue(mode=L.EPI_SHORT_CONV, out16=out.data_ptr(), ld_out16=D,
                             conv_taps=taps.data_ptr(), conv_state=st.data_ptr(),
                             conv_state_out=st.data_ptr(), conv_prefixes=pre.data_ptr(),
                             conv_width=W), parts, K, True)
    with _Form(FORMS[form]):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            assert ops.gemv_short_conv(m, x16, ep)  # warm-up (loads the kernels)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ops.gemv_short_conv(m, x16, ep)
        rng = np.random.default_rng(5)
        for _ in range(3):
            new = rng.standard_normal((W - 1, D)).astype(np.float32)
            st.copy_(_t(new))
            g.replay()
            torch.cuda.synchronize()
            got = (out.clone(), st.clone(), pre.clone())
            want = _unfused(m, x16, parts, taps, new, D, K, W, True, True)
            torch.cuda.synchronize()
            for a, b in zip(got, want):
                _same(a, b)
