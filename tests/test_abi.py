"""The C ABI on the CPU: the library loads, exports what the header
declares, and rejects bad arguments before any device work."""
import ctypes as C

import pytest

from webgllm_amd import lib as L


def test_library_exports_every_declared_symbol():
    lib = L.load()
    names = L.header_functions()
    assert len(names) > 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_no_error_initially():
    lib = L.load()
    assert b"gfx950" in lib.wg_version()


def test_sizes():
    lib = L.load()
    q, s, z = C.c_size_t(), C.c_size_t(), C.c_size_t()
    L.check(lib.wg_q4_sizes(2048, 2048, L.LAYOUT_ROWGROUP, L.ZERO_8, C.byref(q), C.byref(s),
                            C.byref(z)))
    # src/weights.ts:153-178: 2048 x 2048 Q4_0 = 524,288 words and 131,072 halves.
    assert (q.value, s.value, z.value) == (2048 * 2048 // 2, 131072 * 2, 0)
    L.check(lib.wg_q4_sizes(4096, 4096, L.LAYOUT_ROWGROUP, L.ZERO_U8, C.byref(q), C.byref(s),
                            C.byref(z)))
    assert z.value == 4096 * 128
    L.check(lib.wg_q4_sizes(4096, 4096, L.LAYOUT_Q4K, 0, C.byref(q), C.byref(s), C.byref(z)))
    assert q.value == 4096 * 16 * 144
    # Q4_K records: the file's 144 bytes a super-block row, as 128 nibble
    # bytes and a 64-byte record a row group (16 a row), no zeros array
    L.check(lib.wg_q4_sizes(4096, 4096, L.LAYOUT_ROWGROUP, L.ZERO_Q4K, C.byref(q), C.byref(s),
                            C.byref(z)))
    assert (q.value, s.value, z.value) == (4096 * 16 * 128, 4096 * 16 * 16, 0)
    assert q.value + s.value == 4096 * 16 * 144
    with pytest.raises(L.WgError, match="multiple of 256"):
        L.check(lib.wg_q4_sizes(4, 32, L.LAYOUT_ROWGROUP, L.ZERO_Q4K, None, None, None))
    with pytest.raises(L.WgError, match="multiple of 4"):
        L.check(lib.wg_q4_sizes(6, 32, 0, 0, None, None, None))
    with pytest.raises(L.WgError, match="multiple of 256"):
        L.check(lib.wg_q4_sizes(4, 32, L.LAYOUT_Q4K, 0, None, None, None))


def _desc(N=8, K=64, layout=L.LAYOUT_ROWGROUP, zero=L.ZERO_8):
    # Fake device addresses: these calls must fail validation before any launch.
    return L.Q4MatrixDesc(N, K, layout, zero, 0x1000, 0x2000, 0x3000 if zero else 0)


@pytest.mark.parametrize("desc,M,msg", [
    (_desc(N=6), 1, "multiple of 4"),
    (_desc(K=48), 1, "multiple of 32"),
    (_desc(), 0, "1 to 8"),
    (_desc(), 9, "1 to 8"),
    (_desc(zero=7), 1, "zero-point kind"),
    (_desc(layout=5), 1, "layout"),
])
def test_gemv_rejects_bad_shapes(desc, M, msg):
    lib = L.load()
    rc = lib.wg_q4_gemv(C.byref(desc), 0x10000, M, 64, 0x20000, 8, None, None)
    assert rc != 0 and msg in L.last_error()


def test_gemv_rejects_overlap_and_alignment():
    lib = L.load()
    d = _desc()
    rc = lib.wg_q4_gemv(C.byref(d), 0x10000, 1, 64, 0x10000 + 8, 8, None, None)
    assert rc == -1 and "overlap" in L.last_error()
    rc = lib.wg_q4_gemv(C.byref(d), 0x10002, 1, 64, 0x20000, 8, None, None)
    assert rc == -1 and "aligned" in L.last_error()
    ep = L.Epilogue(mode=L.EPI_STORE, residual=0x20004, ld_residual=8)
    rc = lib.wg_q4_gemv(C.byref(d), 0x10000, 1, 64, 0x20000, 8, C.byref(ep), None)
    assert rc == -1 and "residual overlaps" in L.last_error()


@pytest.mark.parametrize("fields,msg", [
    (dict(mode=7), "epilogue mode"),
    (dict(mode=L.EPI_STORE, norm_parts=0x5000, n_parts=0), "input norm"),
    (dict(mode=L.EPI_STORE, out16=0x6000, ld_out16=8), "prescaled half output"),
    (dict(mode=L.EPI_SWIGLU), "SwiGLU"),
    (dict(mode=L.EPI_ROPE_KV, heads=1, kv_heads=1, head_dim=4), "RoPE epilogue"),
])
def test_gemv_rejects_bad_epilogues(fields, msg):
    lib = L.load()
    d = _desc(N=12, K=64)
    ep = L.Epilogue(**fields)
    rc = lib.wg_q4_gemv(C.byref(d), 0x10000, 1, 64, 0x20000, 12, C.byref(ep), None)
    assert rc == -1 and msg in L.last_error(), L.last_error()


def test_repack_rejects_mismatched_layouts():
    lib = L.load()
    d = _desc(zero=L.ZERO_U8)
    assert lib.wg_repack_q4_0(C.byref(d), 0, 8, 0x1000, None, None) == -1
    assert "without zero points" in L.last_error()
    d = _desc(zero=L.ZERO_8)
    assert lib.wg_repack_q4_k(C.byref(d), 0, 8, 0x1000, None, None) == -1
    assert "half zero points or Q4_K records" in L.last_error()
    assert lib.wg_repack_q4_0(C.byref(d), 4, 8, 0x1000, None, None) == -1
    assert "outside the matrix" in L.last_error()
    d = _desc(zero=L.ZERO_8)
    assert lib.wg_repack_nbits(C.byref(d), 0, 8, 0x1, 0x2, 0x3, None, None) == -1
    assert "without them" in L.last_error()


def test_tuning_knobs():
    assert L.tuning_get("gemv_min_waves") >= 0
    old = L.tuning_get("gemv_wg_per_cu")
    L.tuning_set("gemv_wg_per_cu", 4)
    assert L.tuning_get("gemv_wg_per_cu") == 4
    L.tuning_set("gemv_wg_per_cu", old)
    with pytest.raises(L.WgError, match="outside"):
        L.tuning_set("gemv_wg_per_cu", 0)
    with pytest.raises(L.WgError, match="no knob"):
        L.tuning_set("nope", 1)


def test_argmax_advance_rejects_before_any_device_work():
    lib = L.load()
    f = 0x1000  # fake device addresses: validation fails before a launch
    with pytest.raises(L.WgError, match="null argument"):
        L.check(lib.wg_argmax_advance(f, 100, f, None, None, 0, None, f, 4096, None))
    with pytest.raises(L.WgError, match="history of 4 entries"):
        L.check(lib.wg_argmax_advance(f, 100, f, f, None, 4, None, f, 4096, None))
    need = lib.wg_argmax_scratch_bytes(1, 128256)
    assert need == 2 * 4 * ((128256 + 1023) // 1024)
    with pytest.raises(L.WgError, match="scratch of"):
        L.check(lib.wg_argmax_advance(f, 128256, f, f, None, 0, None, f, need - 1, None))


def test_attn_prefill_rejects_before_any_device_work():
    lib = L.load()
    f = 0x1000
    sh = L.AttnShape(32, 8, 96, 96, 1e-6, 0)
    with pytest.raises(L.WgError, match="head_dim 96"):
        L.check(lib.wg_attn_prefill(f, 4, 4096, C.byref(sh), f, f, f, 64, f, 4096, None))
    sh = L.AttnShape(32, 8, 128, 128, 1e-6, 0)
    with pytest.raises(L.WgError, match="null argument"):
        L.check(lib.wg_attn_prefill(None, 4, 4096, C.byref(sh), f, f, f, 64, f, 4096, None))
    with pytest.raises(L.WgError, match="16-byte aligned"):
        L.check(lib.wg_attn_prefill(f + 4, 4, 4096, C.byref(sh), f, f, f, 64, f, 4096, None))


def test_wide_sizes_and_rejections():
    """8-bit and Q6_K matrices: sizes as newQuantMatrix (src/repack.ts:14-35)
    makes them; packers refuse the wrong destination; the GEMM takes 4-bit
    row groups only."""
    lib = L.load()
    q, s, z = C.c_size_t(), C.c_size_t(), C.c_size_t()
    L.check(lib.wg_q4_sizes(128, 4096, L.LAYOUT_Q8, 0, C.byref(q), C.byref(s), C.byref(z)))
    assert (q.value, s.value, z.value) == (128 * 4096, 128 * 128 * 2, 0)
    L.check(lib.wg_q4_sizes(128, 4096, L.LAYOUT_Q6K, 0, C.byref(q), C.byref(s), C.byref(z)))
    assert (q.value, s.value, z.value) == (128 * 16 * 208, 128 * 16 * 2, 0)
    with pytest.raises(L.WgError, match="multiple of 256"):
        L.check(lib.wg_q4_sizes(4, 512 + 32, L.LAYOUT_Q6K, 0, None, None, None))
    q4 = _desc()
    q8 = _desc(layout=L.LAYOUT_Q8)
    q6 = _desc(K=256, layout=L.LAYOUT_Q6K)
    for fn, d, msg in ((lib.wg_repack_q8_0, q4, "8-bit"), (lib.wg_repack_q6_k, q8, "Q6_K"),
                       (lib.wg_repack_q4_0, q8, "row-group")):
        rc = fn(C.byref(d), 0, 4, 0x5000, None, None)
        assert rc == -1 and msg in L.last_error()
    rc = lib.wg_quantize_q8(C.byref(q6), 0, 4, 0x5000, None)
    assert rc == -1 and "8-bit" in L.last_error()
    rc = lib.wg_repack_q8_0(C.byref(q8), 4, 8, 0x5000, None, None)
    assert rc == -1 and "outside" in L.last_error()
    rc = lib.wg_q4_gemm(C.byref(q8), 0x10000, 64, 64, 0x20000, 8, None, 0, None, None, None)
    assert rc != 0
