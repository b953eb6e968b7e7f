"""The greedy pick's first stage run by the head GEMV (pick_parts) and
finished by wg_argmax_parts, against the two-stage pick over the logits the
same GEMV stores (wg_argmax_rows, which test_kernels_gpu checks against the
oracle's scan): ids and top logits bit for bit, on every GEMV form that
takes it; ties to the lowest id across workgroups; NaN never picked; the
decode advance; layouts that do not take it refused before any launch."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

FORMS = {"default": {}, "stream": {"gemv_mfma": 0, "gemv_few_stream": 1},
         "mfma": {"gemv_mfma": 2}}


def _matrix(fmt, N, K, seed, row_order=None):
    from webgllm_amd import engine as E
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.__new__(E.Weights)
    w.shape = shape
    w.device = "cuda"
    w.g = torch.Generator(device="cuda")
    w.g.manual_seed(seed)
    return w.matrix(N, K, row_order)


class _Form:
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


def _x16(M, K, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    return torch.from_numpy(O.f32_to_h2(x).view(np.int16)).cuda()


def _both(m, x16, N):
    """(ids, tops) through the GEMV's parts, then through the logits."""
    from webgllm_amd import ops
    M = x16.shape[0]
    logits = torch.full((M, N), float("nan"), device="cuda")
    parts = ops.pick_parts(M)
    assert ops.gemv_pick(m, x16, logits, parts)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    tops = torch.zeros(M, device="cuda")
    ops.argmax_parts(parts, M, ids, tops=tops)
    ids2 = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    tops2 = torch.zeros(M, device="cuda")
    ops.argmax_rows(logits, ids=ids2, tops=tops2)
    torch.cuda.synchronize()
    return ids, tops, ids2, tops2, logits


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k_rowgroup", "q4_k_records"])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("N,K", [(65536, 2048), (4004, 1024)])
def test_pick_parts_match_the_pick_over_the_logits(hip, form, fmt, M, N, K):
    m = _matrix(fmt, N, K, seed=N + M)
    x16 = _x16(M, K, seed=M)
    with _Form(FORMS[form]):
        ids, tops, ids2, tops2, logits = _both(m, x16, N)
    assert torch.equal(ids, ids2)
    assert torch.equal(tops.view(torch.int32), tops2.view(torch.int32))
    # and it is the logits' own argmax
    assert torch.equal(ids.long(), logits.argmax(dim=1))


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("M", [1, 5])
def test_pick_parts_ties_go_to_the_lowest_id(hip, form, M):
    # every stored row the same logical row: every logit of a token equal
    N, K = 20000, 1024
    m = _matrix("q4_0", N, K, seed=3, row_order=[7] * N)
    x16 = _x16(M, K, seed=4)
    with _Form(FORMS[form]):
        ids, tops, ids2, tops2, logits = _both(m, x16, N)
    assert torch.equal(ids, ids2)
    assert torch.equal(tops.view(torch.int32), tops2.view(torch.int32))
    assert (ids == 0).all()
    # rows 12345 and 19999 alone hold another logical row (a tie between two
    # workgroups' rows when it is the larger)
    order = [7] * N
    order[12345] = order[19999] = 1
    m2 = _matrix("q4_0", N, K, seed=3, row_order=order)
    with _Form(FORMS[form]):
        ids, tops, ids2, tops2, logits = _both(m2, x16, N)
    assert torch.equal(ids, ids2)
    want = logits.argmax(dim=1)
    assert torch.equal(ids.long(), want)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_pick_parts_never_pick_nan(hip, form):
    from webgllm_amd import ops
    N, K, M = 8192, 1024, 3
    m = _matrix("q4_0", N, K, seed=5)
    x16 = _x16(M, K, seed=6)
    x16[1, 100] = 0x7E00  # a NaN activation: every logit of row 1 is NaN
    with _Form(FORMS[form]):
        ids, tops, ids2, tops2, logits = _both(m, x16, N)
    assert torch.equal(ids, ids2)
    assert int(ids[1]) == 0
    assert torch.equal(tops.view(torch.int32), tops2.view(torch.int32))
    assert torch.isnan(logits[1]).all()


def test_pick_parts_advance(hip):
    from webgllm_amd import ops
    N, K = 32768, 2048
    m = _matrix("q4_0", N, K, seed=8)
    x16 = _x16(1, K, seed=9)
    logits = torch.zeros((1, N), device="cuda")
    parts = ops.pick_parts(1)
    ids = torch.zeros(4, dtype=torch.int32, device="cuda")
    pos = torch.tensor([10], dtype=torch.int32, device="cuda")
    hist = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    assert ops.gemv_pick(m, x16, logits, parts)
    ops.argmax_parts(parts, 1, ids, pos=pos, hist=hist)
    want = int(logits[0].argmax())
    assert int(ids[0]) == want and int(hist[11]) == want and int(pos[0]) == 11
    # at the end of the history: the pick and the position, no history entry
    pos.fill_(15)
    ops.argmax_parts(parts, 1, ids, pos=pos, hist=hist)
    assert int(pos[0]) == 16 and int(ids[0]) == want and int(hist[15]) == -1


def test_pick_parts_refusals(hip):
    from webgllm_amd import lib as L, ops
    N, K, M = 4096, 1024, 2
    x16 = _x16(M, K, seed=1)
    logits = torch.zeros((M, N), device="cuda")
    parts = ops.pick_parts(M)
    # other layouts: not taken, nothing launched
    assert not ops.gemv_pick(_matrix("q8_0", N, K, seed=1), x16, logits, parts)
    assert not ops.gemv_pick(_matrix("q4_k", N, K, seed=1), x16, logits, parts)
    m = _matrix("q4_0", N, K, seed=1)
    res = torch.zeros((M, N), device="cuda")
    with pytest.raises(Exception, match="residual"):
        ops.gemv_pick(m, x16, logits, parts,
                      L.Epilogue(mode=L.EPI_STORE, residual=res.data_ptr(), ld_residual=N))
    with pytest.raises(Exception, match="aligned"):
        ops.gemv_pick(m, x16, logits, parts[4:])
    with pytest.raises(Exception, match="one row"):
        ops.argmax_parts(parts, 2, torch.zeros(2, dtype=torch.int32, device="cuda"),
                         pos=torch.zeros(1, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("form", ["default", "mfma"])
def test_pick_parts_graph_replay(hip, form):
    """Captured once, replayed over changing activations: each replay's pick
    equals the eager pick over that replay's logits."""
    from webgllm_amd import ops
    N, K, M = 65536, 2048, 5
    m = _matrix("q4_0", N, K, seed=12)
    x16 = _x16(M, K, seed=13)
    logits = torch.zeros((M, N), device="cuda")
    parts = ops.pick_parts(M)
    ids = torch.zeros(M, dtype=torch.int32, device="cuda")
    with _Form(FORMS[form]):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            assert ops.gemv_pick(m, x16, logits, parts)
            ops.argmax_parts(parts, M, ids)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ops.gemv_pick(m, x16, logits, parts)
            ops.argmax_parts(parts, M, ids)
        for seed in range(3):
            x16.copy_(_x16(M, K, seed=100 + seed))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(ids.long(), logits.argmax(dim=1)), seed
