"""The GGUF reader (wg_gguf_*, the library's host code) on files written
from the format: every metadata value type, lazy arrays, tensor infos,
offsets under both alignments, the data view, and the errors
readGgufHeader raises (src/gguf.ts:276-328). CPU only."""
import struct

import numpy as np
import pytest

from tests import gguf_writer as W


def _meta():
    return [("general.architecture", W.STRING, "lfm2"),
            ("t.u8", W.U8, 250), ("t.i8", W.I8, -5), ("t.u16", W.U16, 65000),
            ("t.i16", W.I16, -30000), ("t.u32", W.U32, 4000000000), ("t.i32", W.I32, -7),
            ("t.f32", W.F32, 1e-5), ("t.bool", W.BOOL, True), ("t.u64", W.U64, 2 ** 40),
            ("t.i64", W.I64, -2 ** 40), ("t.f64", W.F64, 0.1),
            ("t.ints", W.ARRAY, (W.I32, [0, 4, 0, 4])),
            ("t.strs", W.ARRAY, (W.STRING, ["a", "", "héllo"])),
            ("t.long", W.ARRAY, (W.STRING, [f"tok{i}" for i in range(1500)])),
            ("t.empty", W.STRING, "")]


def _tensors(rng):
    return [("a.weight", (64, 2), 0, rng.standard_normal(128).astype(np.float32)),
            ("b.weight", (32, 3), 2, rng.integers(0, 256, 3 * 18, dtype=np.uint8)),
            ("c.weight", (7,), 1, rng.standard_normal(7).astype(np.float16))]


@pytest.mark.parametrize("alignment", [None, 64])
@pytest.mark.parametrize("version", [2, 3])
def test_reader_round_trip(tmp_path, alignment, version):
    from webgllm_amd import gguf as G
    rng = np.random.default_rng(0)
    tensors = _tensors(rng)
    path = tmp_path / "t.gguf"
    data_offset = W.write_gguf(path, _meta(), tensors, version=version, alignment=alignment)
    with G.GgufFile(path) as f:
        assert f.version == version and f.data_offset == data_offset
        assert data_offset % (alignment or 32) == 0
        m = f.metadata
        assert m["general.architecture"] == "lfm2"
        assert (m["t.u8"], m["t.i8"], m["t.u16"], m["t.i16"]) == (250, -5, 65000, -30000)
        assert (m["t.u32"], m["t.i32"], m["t.u64"], m["t.i64"]) == (4000000000, -7, 2 ** 40,
                                                                      -2 ** 40)
        assert m["t.f32"] == float(np.float32(1e-5)) and m["t.f64"] == 0.1
        assert m["t.bool"] is True and m["t.empty"] == ""
        assert m["t.ints"] == [0, 4, 0, 4] and m["t.strs"] == ["a", "", "héllo"]
        lazy = m["t.long"]
        assert isinstance(lazy, G.LazyArray) and lazy.length == 1500
        assert f.read_array("t.long")[1499] == "tok1499"
        off = data_offset
        for name, dims, t, data in tensors:
            info = f.tensors[name]
            assert info.dims == dims and info.type == t and info.offset == off
            raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            assert info.nbytes == raw.size
            assert np.array_equal(f.data(name), raw)
            off += -(-raw.size // (alignment or 32)) * (alignment or 32)


def test_reader_errors(tmp_path):
    from webgllm_amd import gguf as G, lib as L
    rng = np.random.default_rng(1)
    good = tmp_path / "good.gguf"
    W.write_gguf(good, _meta(), _tensors(rng))
    raw = good.read_bytes()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 1) + raw[8:],
        "truncated header": raw[:200],
        "truncated data": raw[:-40],
    }
    msgs = {"magic": "not a GGUF file", "version": "version 1",
            "truncated header": "GGUF", "truncated data": "past the end"}
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        with pytest.raises(L.WgError, match=msgs[name]):
            G.GgufFile(p)
    with pytest.raises(L.WgError, match="No such file"):
        G.GgufFile(tmp_path / "missing.gguf")


def test_lfm2_config_from_metadata(tmp_path):
    """ggufConfig (src/load-gguf.ts:600-752) for LFM2: layer kinds from the
    per-layer KV head counts, float32 settings as their decimals, and the
    cases the engine refuses."""
    from tests.test_gguf_gpu import lfm2_file
    from webgllm_amd import gguf as G, load_gguf as LG
    path = lfm2_file(tmp_path / "m.gguf", layers=3, kv=[0, 2, 0])
    with G.GgufFile(path) as f:
        s = LG.gguf_shape(f)
    assert s.conv_layers == (0, 2) and s.layer_type(1) == "attn"
    assert (s.hidden, s.heads, s.kv_heads, s.head_dim, s.intermediate, s.vocab) == \
        (256, 4, 2, 64, 512, 1024)
    assert s.eps == 1e-5 and s.rope_theta == 1e6 and s.conv_kernel == 3 and s.qk_norm
    for kw, msg in ((dict(arch="lfm3"), "architecture lfm3 is not one this engine runs"),
                    (dict(sliding=4), "sliding-window"),
                    (dict(output_head=True), "its own output.weight"),
                    (dict(kv=[0, 2, 1]), r"differ in KV heads \(\[1, 2\]\)"),
                    (dict(kv=[0, 0, 0]), "no attention layer")):
        p = lfm2_file(tmp_path / "bad.gguf", layers=3, **{"kv": [0, 2, 0], **kw})
        with G.GgufFile(p) as f, pytest.raises(ValueError, match=msg):
            LG.gguf_shape(f)
