"""Gated DeltaNet on the GPU (wg_delta_rule, wg_delta_conv, wg_delta_norm)
against the oracle's float64 restatement of the reference's linear-attention
passes (src/gpu/kernels.ts:1544-1862, src/delta-rule.ts:38-62): outputs and
state within rel-L2 1e-4 (float32 sums of up to 256 products against
float64), the state copy of the convolution bit for bit, and properties
that hold at any size (a batch equals its rows one call at a time, bit for
bit; the snapshot equals the state of a shorter batch)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _layer(rng, H, dk, dv, M, pad=0):
    C = 2 * H * dk + H * dv
    qkv = rng.standard_normal((M, C + pad)).astype(np.float32)
    ba = rng.standard_normal((M, 2 * H + pad)).astype(np.float32)
    A = -np.exp(rng.standard_normal(H) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(H) * 0.5).astype(np.float32)
    state = (rng.standard_normal((H, dk, dv)) * 0.1).astype(np.float32)
    return qkv, ba, A, dt, state


@pytest.mark.parametrize("H,dk,dv,M", [(2, 16, 12, 5), (16, 128, 128, 1), (16, 128, 128, 8),
                                       (3, 64, 80, 37), (2, 256, 64, 4), (1, 5, 3, 3),
                                       (4, 128, 128, 256), (2, 200, 130, 9)])
def test_delta_rule_matches_oracle(hip, H, dk, dv, M):
    from webgllm_amd import ops
    rng = np.random.default_rng(H * 1000 + dk + M)
    qkv, ba, A, dt, state = _layer(rng, H, dk, dv, M, pad=3)
    want_o, want_s, _ = O.delta_rule(qkv, ba, A, dt, H, dk, dv, state)
    s = _t(state)
    out = ops.delta_rule(_t(qkv), _t(ba), _t(A), _t(dt), H, dk, dv, s)
    torch.cuda.synchronize()
    assert _rel(out.cpu().numpy(), want_o) < TOL
    assert _rel(s.cpu().numpy(), want_s) < TOL


def test_delta_rule_batch_equals_rows_and_snapshot(hip):
    """A batch of rows equals the rows one call at a time (the state between
    rows is float32 either way), and the snapshot after row 3 equals the
    state after the first 3 rows."""
    from webgllm_amd import ops
    rng = np.random.default_rng(7)
    H, dk, dv, M = 16, 128, 128, 8
    qkv, ba, A, dt, state = _layer(rng, H, dk, dv, M)
    q, b, a, d = _t(qkv), _t(ba), _t(A), _t(dt)
    s1 = _t(state)
    out1, snap = ops.delta_rule(q, b, a, d, H, dk, dv, s1, save_at=3)
    s2 = _t(state)
    rows = [ops.delta_rule(q[m:m + 1], b[m:m + 1], a, d, H, dk, dv, s2) for m in range(M)]
    s3 = _t(state)
    ops.delta_rule(q[:3], b[:3], a, d, H, dk, dv, s3)
    torch.cuda.synchronize()
    assert torch.equal(out1, torch.cat(rows))
    assert torch.equal(s1, s2)
    assert torch.equal(snap, s3)


def test_delta_rule_long_batch_stays_on_the_oracle(hip):
    """The layer shape (16 heads of 128) over a 512-row batch, against the
    float64 rule: the state stays within the tolerance however many rows
    the float32 recurrence carries it."""
    from webgllm_amd import ops
    rng = np.random.default_rng(11)
    H, dk, dv, M = 16, 128, 128, 512
    qkv, ba, A, dt, state = _layer(rng, H, dk, dv, M)
    want_o, want_s, _ = O.delta_rule(qkv, ba, A, dt, H, dk, dv, state)
    s = _t(state)
    out = ops.delta_rule(_t(qkv), _t(ba), _t(A), _t(dt), H, dk, dv, s)
    torch.cuda.synchronize()
    assert np.all(np.isfinite(out.cpu().numpy()))
    assert _rel(out.cpu().numpy(), want_o) < TOL and _rel(s.cpu().numpy(), want_s) < TOL


@pytest.mark.parametrize("H,dk,dv,M,save_at", [(16, 128, 128, 1, 0), (16, 128, 128, 64, 0),
                                               (16, 128, 128, 65, 0), (4, 128, 128, 300, 0),
                                               (3, 64, 80, 100, 37), (2, 16, 12, 37, 0),
                                               (2, 128, 100, 130, 64), (1, 4, 1, 5, 3),
                                               (2, 32, 128, 129, 128)])
def test_delta_chunked_matches_oracle(hip, H, dk, dv, M, save_at):
    """The chunked form (deltaChunked) against the float64 sequential rule:
    outputs, state, and the snapshot at a chunk end (the first chunk made
    shorter to end at save_at)."""
    from webgllm_amd import ops
    rng = np.random.default_rng(H * 100 + dk + M + save_at)
    qkv, ba, A, dt, state = _layer(rng, H, dk, dv, M, pad=2)
    want_o, want_s, want_snap = O.delta_rule(qkv, ba, A, dt, H, dk, dv, state, save_at=save_at)
    s = _t(state)
    got = ops.delta_rule_chunked(_t(qkv), _t(ba), _t(A), _t(dt), H, dk, dv, s, save_at=save_at)
    out, snap = got if save_at else (got, None)
    torch.cuda.synchronize()
    assert _rel(out.cpu().numpy(), want_o) < TOL
    assert _rel(s.cpu().numpy(), want_s) < TOL
    if save_at:
        assert _rel(snap.cpu().numpy(), want_snap) < TOL


def test_delta_chunked_equals_token_steps_at_prompt_size(hip):
    """A 2048-row batch at the layer shape: the chunked form and the
    row-at-a-time kernel agree (two float32 orders of the same sums), and a
    chunked batch continued by token steps equals the whole batch in chunks."""
    from webgllm_amd import ops
    rng = np.random.default_rng(21)
    H, dk, dv, M = 16, 128, 128, 2048
    qkv, ba, A, dt, state = _layer(rng, H, dk, dv, M)
    q, b, a, d = _t(qkv), _t(ba), _t(A), _t(dt)
    s1, s2, s3 = _t(state), _t(state), _t(state)
    o1 = ops.delta_rule_chunked(q, b, a, d, H, dk, dv, s1)
    o2 = ops.delta_rule(q, b, a, d, H, dk, dv, s2)
    o3 = ops.delta_rule_chunked(q[:2000], b[:2000], a, d, H, dk, dv, s3)
    o3b = ops.delta_rule(q[2000:], b[2000:], a, d, H, dk, dv, s3)
    torch.cuda.synchronize()
    assert torch.isfinite(o1).all()
    assert _rel(o1.cpu().numpy(), o2.cpu().numpy()) < TOL
    assert _rel(s1.cpu().numpy(), s2.cpu().numpy()) < TOL
    assert _rel(torch.cat([o3, o3b]).cpu().numpy(), o1.cpu().numpy()) < TOL
    assert _rel(s3.cpu().numpy(), s1.cpu().numpy()) < TOL


@pytest.mark.parametrize("M,C,W", [(1, 6144, 4), (7, 100, 4), (2, 33, 4), (5, 64, 1),
                                   (300, 6144, 4), (3, 10, 16)])
def test_delta_conv_matches_oracle(hip, M, C, W):
    from webgllm_amd import ops
    rng = np.random.default_rng(M * 7 + C + W)
    x = rng.standard_normal((M, C + 5)).astype(np.float32)
    taps = (rng.standard_normal((C, W)) * 0.5).astype(np.float32)
    st = rng.standard_normal((max(W - 1, 1), C)).astype(np.float32)
    want, want_state = O.delta_conv(x, C, taps, st[:W - 1])
    st_d = _t(st)
    st_out = torch.empty_like(st_d)
    out = ops.delta_conv(_t(x), C, _t(taps), st_d, st_out)
    torch.cuda.synchronize()
    assert _rel(out.cpu().numpy(), want) < 1e-6
    if W > 1:
        assert np.array_equal(st_out.cpu().numpy()[:W - 1], want_state)


@pytest.mark.parametrize("M,H,dv", [(1, 16, 128), (9, 3, 80), (4, 2, 256), (2, 5, 7)])
def test_delta_norm_matches_oracle(hip, M, H, dv):
    from webgllm_amd import ops
    rng = np.random.default_rng(M + H + dv)
    o = rng.standard_normal((M, H * dv + 2)).astype(np.float32)
    z = rng.standard_normal((M, H * dv + 1)).astype(np.float32)
    w = rng.standard_normal(dv).astype(np.float32)
    want = O.delta_norm(o, H, dv, z, w, 1e-6)
    got = ops.delta_norm(_t(o), H, dv, _t(z), _t(w), 1e-6)
    torch.cuda.synchronize()
    got = got.cpu().numpy().astype(np.float64)
    # halves: within one half-ulp of the float64 value, relative
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -11 * 1.01 + 2.0 ** -24)


def test_delta_rejections(hip):
    from webgllm_amd import lib as L, ops
    dev = "cuda"
    H, dk, dv = 2, 8, 4
    qkv = torch.zeros((2, 2 * H * dk + H * dv), device=dev)
    ba = torch.zeros((2, 2 * H), device=dev)
    A = torch.zeros(H, device=dev)
    s = torch.zeros((H, dk, dv), device=dev)
    with pytest.raises(L.WgError, match="key dims 1 to 256"):
        ops.delta_rule(torch.zeros((1, 2 * H * 300 + H * dv), device=dev), ba[:1], A, A, H, 300,
                       dv, torch.zeros((H, 300, dv), device=dev))
    with pytest.raises(L.WgError, match="save_at 3 of 2"):
        ops.delta_rule(qkv, ba, A, A, H, dk, dv, s, save_at=3)
    with pytest.raises(L.WgError, match="overlaps the state"):
        ops.delta_rule(qkv, ba, A, A, H, dk, dv, s, save_at=1, snapshot=s)
    with pytest.raises(L.WgError, match="strides too short"):
        ops.delta_rule(torch.zeros((2, 2 * H * dk + H * dv - 1), device=dev), ba, A, A, H, dk,
                       dv, s)
    st = torch.zeros((3, 8), device=dev)
    with pytest.raises(L.WgError, match="separate state_out"):
        ops.delta_conv(torch.zeros((2, 8), device=dev), 8, torch.zeros((8, 4), device=dev), st, st)
    with pytest.raises(L.WgError, match="1 to 16"):
        ops.delta_conv(torch.zeros((2, 8), device=dev), 8, torch.zeros((8, 17), device=dev),
                       torch.zeros((16, 8), device=dev), torch.zeros((16, 8), device=dev))
    with pytest.raises(L.WgError, match="a multiple of 4"):
        ops.delta_rule_chunked(torch.zeros((2, 2 * H * 6 + H * dv), device=dev), ba, A, A, H, 6,
                               dv, torch.zeros((H, 6, dv), device=dev))
    with pytest.raises(L.WgError, match="at most 128"):
        ops.delta_rule_chunked(torch.zeros((2, 2 * H * 256 + H * dv), device=dev), ba, A, A, H,
                               256, dv, torch.zeros((H, 256, dv), device=dev))
    with pytest.raises(L.WgError, match="needed"):
        ops.delta_rule_chunked(qkv, ba, A, A, H, dk, dv, s, scratch=torch.zeros(4, device=dev))
    with pytest.raises(L.WgError, match="1 to 256"):
        ops.delta_norm(torch.zeros((1, 300), device=dev), 1, 300, torch.zeros((1, 300), device=dev),
                       torch.zeros(300, device=dev), 1e-6)
