"""wg_attn_decode_noalloc (decode attention with the library's built-in
scratch, no allocation) against wg_attn_decode with a caller's scratch:
the same kernels, so the same halves bit for bit. Two calls in a row, the
second smaller than the first (the built-in scratch keeps the first call's
partials, which the second must not read), then a request larger than the
built-in scratch, refused before anything runs."""
import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(g, M, H, KV, hd, max_keys, pos0):
    q = (torch.randn((M, H * hd), generator=g, device="cuda") / hd ** 0.5).contiguous()
    k = torch.randn((max_keys, KV * hd), generator=g, device="cuda").half().contiguous()
    v = torch.randn((max_keys, KV * hd), generator=g, device="cuda").half().contiguous()
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda")
    return q, k, v, pos


def _noalloc(hip, q, shape, k, v, pos, max_keys, out):
    return hip.wg_attn_decode_noalloc(q.data_ptr(), q.shape[0], q.shape[1], C.byref(shape),
                                      k.data_ptr(), v.data_ptr(), pos.data_ptr(), max_keys,
                                      out.data_ptr(), out.shape[1],
                                      torch.cuda.current_stream().cuda_stream)


def test_noalloc_attention_equals_the_scratch_entry_point(hip):
    from webgllm_amd import ops
    g = torch.Generator(device="cuda").manual_seed(5)
    # (rows, query heads, KV heads, head_dim, cache rows, position): a verify
    # batch of 8 at the 8B shape near 4096 keys, then one Qwen2-shape row
    for M, H, KV, hd, max_keys, pos0 in [(8, 32, 8, 128, 4096, 4080), (1, 14, 2, 64, 1024, 700)]:
        q, k, v, pos = _inputs(g, M, H, KV, hd, max_keys, pos0)
        shape = ops.attn_shape(H, KV, hd)
        want = ops.attn_decode(q, shape, k, v, pos)
        got = torch.full_like(want, 7)
        assert _noalloc(hip, q, shape, k, v, pos, max_keys, got) == 0, \
            hip.wg_last_error().decode()
        torch.cuda.synchronize()
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got, want), (M, H, max_keys)


def test_noalloc_attention_refuses_more_than_its_scratch(hip):
    from webgllm_amd import ops
    g = torch.Generator(device="cuda").manual_seed(6)
    M, H, KV, hd, max_keys = 8, 32, 8, 128, 8192  # 17 MB of partials > 16 MiB
    q, k, v, pos = _inputs(g, M, H, KV, hd, max_keys, 100)
    out = torch.full((M, H * hd), 3, dtype=torch.float16, device="cuda")
    shape = ops.attn_shape(H, KV, hd)
    assert _noalloc(hip, q, shape, k, v, pos, max_keys, out) == -1
    assert "built-in scratch holds" in hip.wg_last_error().decode()
    torch.cuda.synchronize()
    assert (out == 3).all()  # nothing ran
