"""A device verify step's fused launches against the separate ones:
wg_embed_drafts = wg_verify_drafts then wg_embed, wg_verify_accept_parts =
wg_argmax_parts then wg_verify_accept (embeddings, ids, picks, kept counts,
history, position and rolled-back conv states bit for bit), and a whole
LFM2-shape verify run replayed with and without them."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _matrix(fmt, N, K, seed):
    from webgllm_amd import engine as E
    shape = E.ModelShape("t", K, 1, 1, 1, 4, 4, 4, fmt)
    w = E.Weights.__new__(E.Weights)
    w.shape = shape
    w.device = "cuda"
    w.g = torch.Generator(device="cuda")
    w.g.manual_seed(seed)
    return w.matrix(N, K)


@pytest.mark.parametrize("fmt", ["q4_0", "nbits", "q4_k_rowgroup", "q4_k_records", "q4_k",
                                 "q8_0", "q6_k"])
@pytest.mark.parametrize("cursor", [0, 2, 7, -3])
def test_embed_drafts_equals_drafts_then_embed(hip, fmt, cursor):
    from webgllm_amd import lib as L, ops
    N, K, rows, steps = 3000, 1024, 5, 4
    m = _matrix(fmt, N, K, seed=1)
    rng = np.random.default_rng(cursor + 10)
    table = torch.from_numpy(rng.integers(-5, N + 5, (steps, rows - 1)).astype(np.int32)).cuda()
    cur = torch.tensor([cursor], dtype=torch.int32, device="cuda")
    w16 = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).cuda()

    def run(fused):
        ids = torch.tensor([17, -1, -1, -1, -1], dtype=torch.int32, device="cuda")
        h = torch.full((rows, K), float("nan"), device="cuda")
        x16 = torch.zeros((rows, K), dtype=torch.float16, device="cuda")
        parts = torch.zeros((rows, K // 4), device="cuda")
        ep = L.Epilogue(mode=L.EPI_STORE, out16=x16.data_ptr(), ld_out16=K,
                        out16_w=w16.data_ptr(), norm_mult_out=32.0, parts_out=parts.data_ptr(),
                        ld_parts_out=K // 4)
        if fused:
            ops.embed_drafts(m, ids, rows, table, cur, out=h, epilogue=ep)
        else:
            ops.verify_drafts(ids, rows, table, cur)
            ops.embed(m, ids, out=h, epilogue=ep)
        torch.cuda.synchronize()
        return ids, h, x16, parts

    a, b = run(False), run(True)
    for name, x, y in zip(("ids", "h", "x16", "parts"), a, b):
        assert torch.equal(x.view(torch.int32) if x.element_size() == 4 else x.view(torch.int16),
                           y.view(torch.int32) if y.element_size() == 4 else y.view(torch.int16)), name


@pytest.mark.parametrize("agree", [0, 2, 4])
def test_verify_accept_parts_equals_pick_then_accept(hip, agree):
    from webgllm_amd import ops
    N, K, rows, D, W = 65536, 2048, 5, 2048, 3
    m = _matrix("q4_0", N, K, seed=2)
    rng = np.random.default_rng(agree)
    x = torch.from_numpy(rng.standard_normal((rows, K)).astype(np.float16)).cuda()
    logits = torch.zeros((rows, N), device="cuda")
    parts = ops.pick_parts(rows)
    assert ops.gemv_pick(m, x, logits, parts)
    picks = logits.argmax(dim=1).int()
    # drafts agreeing with the picks for `agree` rows, then not
    drafts = [int(picks[i]) for i in range(agree)] + [int(picks[i]) + 1 for i in range(agree, 4)]
    pre = [torch.from_numpy(rng.standard_normal((rows, W - 1, D)).astype(np.float32)).cuda()
           for _ in range(3)]

    def run(fused):
        states = [torch.zeros((W - 1, D), device="cuda") for _ in range(3)]
        convs = ops.conv_states(list(zip(pre, states)))
        ids = torch.tensor([9] + drafts, dtype=torch.int32, device="cuda")
        pos = torch.tensor([40], dtype=torch.int32, device="cuda")
        hist = torch.full((64,), -1, dtype=torch.int32, device="cuda")
        kept = torch.zeros(8, dtype=torch.int32, device="cuda")
        cursor = torch.tensor([3], dtype=torch.int32, device="cuda")
        out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
        if fused:
            ops.verify_accept_parts(parts, out, rows, convs, pos, ids, hist, kept, cursor)
        else:
            ops.argmax_parts(parts, rows, out)
            ops.verify_accept(out, rows, convs, pos, ids, hist, kept, cursor)
        torch.cuda.synchronize()
        return [out, ids, pos, hist, kept, cursor] + states

    a, b = run(False), run(True)
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), i
    assert torch.equal(a[0], picks)
    assert int(a[4][3]) == agree + 1


def test_graph_verify_run_fused_equals_separate(hip):
    """A run of device verify steps (LFM2 shape, 4 layers) with the fused
    launches and with the separate ones: the same tokens, kept counts,
    history, conv states and logits."""
    import dataclasses
    from webgllm_amd import engine as E
    s = dataclasses.replace(E.LFM2_12B, layers=4, conv_layers=(0, 1, 3))
    w = E.Weights(s, seed=21)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, s.vocab, 12).tolist()
    drafts = rng.integers(0, s.vocab, (20, 4)).tolist()
    out = []
    for fused in (False, True):
        eng = E.Engine(w, 256)
        eng.fuse_verify = fused
        token = int(eng.forward(prompt).cpu()[-1])
        tokens, kept = eng.verify_drafts(token, drafts)
        torch.cuda.synchronize()
        out.append((tokens, kept, eng.hist.clone(), {i: t.clone() for i, t in eng.state.items()},
                    eng.logits[:5].clone()))
    (t0, k0, h0, s0, l0), (t1, k1, h1, s1, l1) = out
    assert t0 == t1 and k0 == k1
    assert torch.equal(h0, h1)
    for i in s0:
        assert torch.equal(s0[i].view(torch.int32), s1[i].view(torch.int32)), i
    assert torch.equal(l0.view(torch.int32), l1.view(torch.int32))
