"""The backend objects of the C ABI on the GPU (the reference's Gpu /
PacedGpu contract, src/gpu/gl.ts:263-374, :448-461, :658-835;
src/gpu/paced.ts:11-22), driven through ctypes alone: no torch memory.

A context, buffers created, written, zeroed and read back behind fences;
cancelled reads; handles that report WG_ERR_DISPOSED after a delete, a
finished read or a destroyed context; the live-bytes count; the pinned
staging pool's bound; and the typed kernels (Q4_0 repack and GEMV) run on
the context's buffers and stream, checked against the oracle."""
import ctypes as C
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OK, INVALID, DISPOSED = 0, -1, -5


@pytest.fixture
def ctx(hip):
    c = C.c_void_p()
    assert hip.wg_ctx_create(0, C.byref(c)) == OK
    yield c
    hip.wg_ctx_destroy(c)  # may already be destroyed: then DISPOSED, ignored


def _buf(hip, ctx, nbytes, init=None):
    b = C.c_void_p()
    src = None if init is None else init.ctypes.data_as(C.c_void_p)
    assert hip.wg_buf_create(ctx, nbytes, src, C.byref(b)) == OK, hip.wg_last_error()
    return b


def _read(hip, ctx, b, offset, nbytes):
    out = np.empty(nbytes, np.uint8)
    assert hip.wg_read_now(ctx, b, offset, nbytes, out.ctypes.data_as(C.c_void_p)) == OK
    return out


def _wait(hip, fence, seconds=20.0):
    t0 = time.time()
    while True:
        r = hip.wg_fence_ready(fence)
        assert r >= 0, hip.wg_last_error()
        if r == 1:
            return
        assert time.time() - t0 < seconds, "fence never became ready"
        time.sleep(0.0005)


def test_limits_buffers_and_reads(hip, ctx):
    from webgllm_amd import lib as L
    lim = L.Limits()
    assert hip.wg_ctx_limits(ctx, C.byref(lim)) == OK
    assert lim.compute_units >= 1 and lim.wave_size == 64 and lim.global_bytes > 0
    rng = np.random.default_rng(0)
    init = rng.integers(0, 256, 1 << 20, dtype=np.uint8)
    before = hip.wg_bytes_live(ctx)
    b = _buf(hip, ctx, init.size, init)
    assert hip.wg_bytes_live(ctx) == before + init.size
    assert hip.wg_buf_size(b) == init.size and hip.wg_buf_ptr(b)
    assert np.array_equal(_read(hip, ctx, b, 0, init.size), init)
    # a write at an offset; the source is reusable as soon as the call returns
    patch = rng.integers(0, 256, 4096, dtype=np.uint8)
    assert hip.wg_buf_write(ctx, b, 1000, patch.ctypes.data_as(C.c_void_p), patch.size) == OK
    patch_copy = patch.copy()
    patch[:] = 0
    want = init.copy()
    want[1000:1000 + 4096] = patch_copy
    # a fenced read, polled, then finished
    fence = C.c_void_p()
    assert hip.wg_read_start(ctx, b, 0, init.size, C.byref(fence)) == OK
    _wait(hip, fence)
    out = np.empty(init.size, np.uint8)
    assert hip.wg_read_finish(fence, out.ctypes.data_as(C.c_void_p)) == OK
    assert np.array_equal(out, want)
    # the finished fence is gone
    assert hip.wg_fence_ready(fence) == DISPOSED
    assert hip.wg_read_finish(fence, None) == DISPOSED
    # zero
    assert hip.wg_buf_zero(ctx, b) == OK
    assert not _read(hip, ctx, b, 4096, 8192).any()
    # cancelled reads: the handle dies, later reads still work
    for _ in range(3):
        f = C.c_void_p()
        assert hip.wg_read_start(ctx, b, 0, 65536, C.byref(f)) == OK
        assert hip.wg_read_cancel(f) == OK
        assert hip.wg_read_cancel(f) == DISPOSED
    assert hip.wg_finish(ctx) == OK and hip.wg_flush(ctx) == OK
    # delete: the handle dies, the bytes leave the count
    assert hip.wg_buf_delete(ctx, b) == OK
    assert hip.wg_bytes_live(ctx) == before
    assert hip.wg_buf_write(ctx, b, 0, patch.ctypes.data_as(C.c_void_p), 16) == DISPOSED
    assert hip.wg_buf_delete(ctx, b) == DISPOSED
    assert hip.wg_buf_ptr(b) is None and hip.wg_buf_size(b) == 0


def test_rejections(hip, ctx):
    data = np.zeros(64, np.uint8)
    b = _buf(hip, ctx, 256)
    p = data.ctypes.data_as(C.c_void_p)
    assert hip.wg_buf_write(ctx, b, 200, p, 64) == INVALID
    assert "outside the 256-byte buffer" in hip.wg_last_error().decode()
    f = C.c_void_p()
    assert hip.wg_read_start(ctx, b, 250, 16, C.byref(f)) == INVALID
    assert hip.wg_read_start(ctx, b, 0, 0, C.byref(f)) == INVALID
    assert hip.wg_buf_create(ctx, 0, None, C.byref(f)) == INVALID
    other = C.c_void_p()
    assert hip.wg_ctx_create(0, C.byref(other)) == OK
    try:
        assert hip.wg_buf_write(other, b, 0, p, 16) == INVALID
        assert "another context" in hip.wg_last_error().decode()
    finally:
        assert hip.wg_ctx_destroy(other) == OK
    assert hip.wg_ctx_create(99, C.byref(other)) == INVALID


def test_many_writes_keep_their_order_and_a_bounded_pool(hip, ctx):
    """40 writes of 256 KiB into one buffer with no wait in between, each
    source overwritten right after its call: the last write wins, every
    earlier one landed in order, and the staging pool stays bounded."""
    n = 256 << 10
    b = _buf(hip, ctx, 2 * n)
    src = np.empty(n, np.uint8)
    for k in range(40):
        src[:] = k
        assert hip.wg_buf_write(ctx, b, (k % 2) * n, src.ctypes.data_as(C.c_void_p), n) == OK
        src[:] = 255  # the call already copied it
    out = _read(hip, ctx, b, 0, 2 * n)
    assert (out[:n] == 38).all() and (out[n:] == 39).all()
    slots, nbytes = C.c_int32(), C.c_size_t()
    assert hip.wg_ctx_staging(ctx, C.byref(slots), C.byref(nbytes)) == OK
    assert 1 <= slots.value <= 18, slots.value
    # reads reuse the pool
    for _ in range(20):
        _read(hip, ctx, b, 0, 4096)
    slots2 = C.c_int32()
    assert hip.wg_ctx_staging(ctx, C.byref(slots2), None) == OK
    assert slots2.value == slots.value


def test_destroy_cancels_reads_and_disposes_handles(hip):
    c = C.c_void_p()
    assert hip.wg_ctx_create(0, C.byref(c)) == OK
    b = _buf(hip, c, 1 << 16, np.arange(1 << 16, dtype=np.uint32).astype(np.uint8))
    f = C.c_void_p()
    assert hip.wg_read_start(c, b, 0, 1 << 16, C.byref(f)) == OK
    assert hip.wg_ctx_destroy(c) == OK
    assert hip.wg_fence_ready(f) == DISPOSED
    assert hip.wg_read_finish(f, None) == DISPOSED
    assert hip.wg_buf_zero(c, b) == DISPOSED
    assert hip.wg_bytes_live(c) == 0 and hip.wg_ctx_stream(c) is None
    assert hip.wg_finish(c) == DISPOSED
    assert hip.wg_ctx_destroy(c) == DISPOSED


def test_q4_0_gemv_on_context_buffers(hip, ctx):
    """GGUF Q4_0 bytes uploaded into a context buffer, repacked into the
    QuantMatrix layout in context buffers, a GEMV on the context's stream,
    the result read behind a fence: equal to the oracle's (dequant bit for
    bit; GEMV within rel-L2 1e-4 of float64)."""
    from oracle import oracle as O
    from tests.helpers import rel_l2
    from webgllm_amd import lib as L
    rng = np.random.default_rng(3)
    N, K = 512, 2048
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    src = O.quantize_q4_0(w)
    qb, sb, zb = C.c_size_t(), C.c_size_t(), C.c_size_t()
    assert hip.wg_q4_sizes(N, K, L.LAYOUT_ROWGROUP, L.ZERO_8, C.byref(qb), C.byref(sb),
                           C.byref(zb)) == OK
    bsrc = _buf(hip, ctx, src.nbytes, np.ascontiguousarray(src).view(np.uint8).reshape(-1))
    bq, bs = _buf(hip, ctx, qb.value), _buf(hip, ctx, sb.value)
    desc = L.Q4MatrixDesc(N, K, L.LAYOUT_ROWGROUP, L.ZERO_8, hip.wg_buf_ptr(bq),
                          hip.wg_buf_ptr(bs), None)
    stream = hip.wg_ctx_stream(ctx)
    assert hip.wg_repack_q4_0(C.byref(desc), 0, N, hip.wg_buf_ptr(bsrc), None, stream) == OK
    x = rng.standard_normal((1, K)).astype(np.float32)
    x16 = O.f32_to_h2(x)
    bx = _buf(hip, ctx, x16.nbytes, np.ascontiguousarray(x16).view(np.uint8).reshape(-1))
    by = _buf(hip, ctx, N * 4)
    assert hip.wg_q4_gemv(C.byref(desc), hip.wg_buf_ptr(bx), 1, K, hip.wg_buf_ptr(by), N, None,
                          stream) == OK, hip.wg_last_error()
    f = C.c_void_p()
    assert hip.wg_read_start(ctx, by, 0, N * 4, C.byref(f)) == OK
    y = np.empty(N, np.float32)
    _wait(hip, f)
    assert hip.wg_read_finish(f, y.ctypes.data_as(C.c_void_p)) == OK
    want_m = O.QuantMatrix(N, K, False)
    O.pack_q4_0(want_m, 0, src, N)
    quants = _read(hip, ctx, bq, 0, qb.value).view(np.uint32)
    assert np.array_equal(quants, want_m.quants)
    want = O.gemv_f64(want_m, O.halves_to_f32(x16))[0]
    assert rel_l2(y, want) <= 1e-4
