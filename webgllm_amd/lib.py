"""ctypes binding of libwebgllm_hip.so (the C ABI in include/webgllm_hip.h).

torch supplies device memory and the current stream; every computation runs
in the HIP library. There is no CPU fallback: if the library is missing the
import of an op fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwebgllm_hip.so")
HEADER = os.path.join(os.path.dirname(_HERE), "include", "webgllm_hip.h")

WG_OK = 0
ERR_UNSUPPORTED = -6
STATUS = {-1: "invalid", -2: "out-of-memory", -3: "device", -4: "aliased", -5: "disposed",
          -6: "unsupported"}

LAYOUT_ROWGROUP, LAYOUT_Q4K, LAYOUT_Q8, LAYOUT_Q6K = 0, 1, 2, 3
ZERO_8, ZERO_U8, ZERO_F16, ZERO_Q4K = 0, 1, 2, 3


class WgError(RuntimeError):
    """A failed call; `kind` as the reference's GpuError kinds (src/gpu/gl.ts)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.kind = STATUS.get(status, "unknown")


class Q4MatrixDesc(C.Structure):
    _fields_ = [("N", C.c_int32), ("K", C.c_int32), ("layout", C.c_int32), ("zero", C.c_int32),
                ("quants", C.c_void_p), ("scales", C.c_void_p), ("zeros", C.c_void_p)]


EPI_STORE, EPI_SWIGLU, EPI_ROPE_KV, EPI_SHORT_CONV = 0, 1, 2, 3


class ConvState(C.Structure):
    """wg_conv_state (include/webgllm_hip.h): a conv layer's rollback operands."""
    _fields_ = [("prefixes", C.c_void_p), ("state", C.c_void_p), ("dim", C.c_int32),
                ("width", C.c_int32)]


class Epilogue(C.Structure):
    """wg_epilogue (include/webgllm_hip.h)."""
    _fields_ = [("mode", C.c_int32),
                ("norm_parts", C.c_void_p), ("n_parts", C.c_int32), ("ld_parts_in", C.c_int32),
                ("norm_count", C.c_int32), ("eps", C.c_float), ("norm_mult", C.c_float),
                ("row_scale", C.c_void_p),
                ("residual", C.c_void_p), ("ld_residual", C.c_int32),
                ("out16", C.c_void_p), ("ld_out16", C.c_int32), ("out16_w", C.c_void_p),
                ("norm_mult_out", C.c_float),
                ("parts_out", C.c_void_p), ("ld_parts_out", C.c_int32),
                ("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("ctx", C.c_int32), ("rope_rows", C.c_int32),
                ("rope", C.c_void_p), ("pos0", C.c_void_p),
                ("q_out", C.c_void_p), ("ld_q_out", C.c_int32),
                ("k_cache", C.c_void_p), ("v_cache", C.c_void_p),
                ("conv_taps", C.c_void_p), ("conv_state", C.c_void_p),
                ("conv_state_out", C.c_void_p), ("conv_prefixes", C.c_void_p),
                ("conv_width", C.c_int32), ("pick_parts", C.c_void_p)]


class AttnShape(C.Structure):
    _fields_ = [("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("rotated_dims", C.c_int32), ("eps", C.c_float), ("use_norm", C.c_int32)]


class DeltaShape(C.Structure):
    """wg_delta_shape."""
    _fields_ = [("heads", C.c_int32), ("key_dim", C.c_int32), ("value_dim", C.c_int32)]


class OnnxTensorInfo(C.Structure):
    """wg_onnx_tensor_info."""
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int32), ("dims", C.c_int64 * 8),
                ("data_type", C.c_int32), ("raw", C.c_void_p), ("raw_bytes", C.c_uint64),
                ("location", C.c_char_p), ("offset", C.c_int64), ("length", C.c_int64),
                ("int64_data", C.POINTER(C.c_int64)), ("n_int64", C.c_int64),
                ("float_data", C.POINTER(C.c_float)), ("n_float", C.c_int64)]


class OnnxNodeInfo(C.Structure):
    """wg_onnx_node_info."""
    _fields_ = [("name", C.c_char_p), ("op_type", C.c_char_p), ("domain", C.c_char_p),
                ("n_inputs", C.c_int32), ("n_outputs", C.c_int32), ("n_attrs", C.c_int32)]


class OnnxAttr(C.Structure):
    """wg_onnx_attr."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("f", C.c_float), ("i", C.c_int64),
                ("s", C.c_void_p), ("s_len", C.c_uint64), ("ints", C.POINTER(C.c_int64)),
                ("n_ints", C.c_int64), ("floats", C.POINTER(C.c_float)), ("n_floats", C.c_int64),
                ("n_strings", C.c_int64), ("tensor", C.c_int64)]


class GgufTensorInfo(C.Structure):
    """wg_gguf_tensor_info."""
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int32), ("dims", C.c_int64 * 4),
                ("type", C.c_int32), ("offset", C.c_uint64), ("bytes", C.c_uint64),
                ("data", C.c_void_p)]


class GgufValue(C.Structure):
    """wg_gguf_value."""
    _fields_ = [("key", C.c_char_p), ("type", C.c_int32), ("elem_type", C.c_int32),
                ("length", C.c_uint64), ("i", C.c_int64), ("f", C.c_double),
                ("s", C.c_void_p), ("offset", C.c_uint64)]


class Limits(C.Structure):
    _fields_ = [("device", C.c_int32), ("compute_units", C.c_int32),
                ("global_bytes", C.c_int64), ("max_alloc_bytes", C.c_int64),
                ("lds_bytes_per_block", C.c_int32), ("wave_size", C.c_int32)]


_lib = None


def header_functions() -> list[str]:
    """Every function include/webgllm_hip.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wg_[a-z0-9_]+)\s*\(", text)))


def load():
    """The loaded library; raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it first (python -c "
                          "'import __graft_entry__ as g; g.build()')")
    # torch brings its own HIP runtime; loaded first, it is the one the
    # library binds to (two runtimes in one process do not share devices).
    import torch  # noqa: F401
    lib = C.CDLL(LIB_PATH)
    P, I32, I64, SZ = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t
    sig = {
        "wg_last_error": (C.c_char_p, []),
        "wg_tuning_set": (C.c_int, [C.c_char_p, I32]),
        "wg_tuning_get": (C.c_int, [C.c_char_p, C.POINTER(I32)]),
        "wg_version": (C.c_char_p, []),
        "wg_ctx_create": (C.c_int, [C.c_int, C.POINTER(P)]),
        "wg_ctx_destroy": (C.c_int, [P]),
        "wg_ctx_limits": (C.c_int, [P, C.POINTER(Limits)]),
        "wg_ctx_stream": (P, [P]),
        "wg_buf_create": (C.c_int, [P, SZ, P, C.POINTER(P)]),
        "wg_buf_write": (C.c_int, [P, P, SZ, P, SZ]),
        "wg_buf_zero": (C.c_int, [P, P]),
        "wg_buf_delete": (C.c_int, [P, P]),
        "wg_buf_ptr": (P, [P]),
        "wg_buf_size": (SZ, [P]),
        "wg_bytes_live": (SZ, [P]),
        "wg_read_start": (C.c_int, [P, P, SZ, SZ, C.POINTER(P)]),
        "wg_fence_ready": (C.c_int, [P]),
        "wg_read_finish": (C.c_int, [P, P]),
        "wg_read_cancel": (C.c_int, [P]),
        "wg_read_now": (C.c_int, [P, P, SZ, SZ, P]),
        "wg_flush": (C.c_int, [P]),
        "wg_finish": (C.c_int, [P]),
        "wg_ctx_staging": (C.c_int, [P, C.POINTER(I32), C.POINTER(SZ)]),
        "wg_q4_sizes": (C.c_int, [I32, I32, I32, I32, C.POINTER(SZ), C.POINTER(SZ),
                                  C.POINTER(SZ)]),
        "wg_repack_q4_0": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P, P]),
        "wg_repack_q4_k": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P, P]),
        "wg_q4k_record_halves": (C.c_int, [C.POINTER(Q4MatrixDesc), P, P, P]),
        "wg_repack_q4_k_native": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P, P]),
        "wg_repack_nbits": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P, P, P, P]),
        "wg_repack_q8_0": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P, P]),
        "wg_quantize_q8": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P]),
        "wg_repack_q6_k": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P, P]),
        "wg_q4_dequant": (C.c_int, [C.POINTER(Q4MatrixDesc), I32, I32, P, P]),
        "wg_q4_gemv": (C.c_int, [C.POINTER(Q4MatrixDesc), P, I32, I32, P, I32,
                                 C.POINTER(Epilogue), P]),
        "wg_f32_to_f16": (C.c_int, [P, P, I64, P]),
        "wg_q4_gemm": (C.c_int, [C.POINTER(Q4MatrixDesc), P, I32, I32, P, I32, P, I32, P, P, P]),
        "wg_q4_gemm_swiglu": (C.c_int, [C.POINTER(Q4MatrixDesc), P, I32, I32, P, I32, P, P]),
        "wg_rms_norm": (C.c_int, [P, I32, I32, I32, P, C.c_float, P, I32, P, P]),
        "wg_norm_to_h2": (C.c_int, [P, I32, I32, I32, P, C.c_float, P, I32, P, P]),
        "wg_swiglu": (C.c_int, [P, I32, I32, I32, P, I32, P]),
        "wg_embed": (C.c_int, [C.POINTER(Q4MatrixDesc), P, I32, P, I32, C.POINTER(Epilogue),
                               P]),
        "wg_head_prep": (C.c_int, [P, I32, I32, C.POINTER(AttnShape), P, P, P, I32, P, P, I32,
                                   P, P, I32, P]),
        "wg_attn_scratch_bytes": (SZ, [I32, I32, I32, I32]),
        "wg_attn_prefill": (C.c_int, [P, I32, I32, C.POINTER(AttnShape), P, P, P, I32, P, I32, P]),
        "wg_attn_decode": (C.c_int, [P, I32, I32, C.POINTER(AttnShape), P, P, P, I32, P, I32,
                                     P, SZ, P]),
        "wg_attn_decode_prep": (C.c_int, [P, I32, I32, C.POINTER(AttnShape), P, P, P, I32, I32,
                                          P, P, P, I32, P, I32, P, I32, P, SZ, P]),
        "wg_attn_decode_noalloc": (C.c_int, [P, I32, I32, C.POINTER(AttnShape), P, P, P, I32,
                                             P, I32, P]),
        "wg_verify_accept": (C.c_int, [P, I32, P, I32, I32, P, P, P, I32, P, I32, P, P]),
        "wg_verify_accept_parts": (C.c_int, [P, P, I32, P, I32, I32, P, P, P, I32, P, I32, P, P]),
        "wg_embed_drafts": (C.c_int, [C.POINTER(Q4MatrixDesc), P, I32, P, I32, P, P, I32,
                                      C.POINTER(Epilogue), P]),
        "wg_verify_drafts": (C.c_int, [P, I32, P, I32, P, P]),
        "wg_short_conv": (C.c_int, [P, I32, I32, I32, I32, P, P, P, P, P, I32, P]),
        "wg_conv_accept": (C.c_int, [P, I32, I32, I32, I32, P, P]),
        "wg_argmax_scratch_bytes": (SZ, [I32, I32]),
        "wg_argmax_rows": (C.c_int, [P, I32, I32, I32, P, P, P, SZ, P]),
        "wg_argmax_advance": (C.c_int, [P, I32, P, P, P, I32, P, P, SZ, P]),
        "wg_pick_parts_bytes": (SZ, [I32]),
        "wg_argmax_parts": (C.c_int, [P, I32, P, P, P, P, I32, P]),
        "wg_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
        "wg_gguf_close": (C.c_int, [P]),
        "wg_gguf_version": (I32, [P]),
        "wg_gguf_data_offset": (I64, [P]),
        "wg_gguf_tensor_count": (I64, [P]),
        "wg_gguf_meta_count": (I64, [P]),
        "wg_gguf_find_tensor": (I64, [P, C.c_char_p]),
        "wg_gguf_find_meta": (I64, [P, C.c_char_p]),
        "wg_gguf_tensor": (C.c_int, [P, I64, C.POINTER(GgufTensorInfo)]),
        "wg_gguf_meta": (C.c_int, [P, I64, C.POINTER(GgufValue)]),
        "wg_gguf_meta_element": (C.c_int, [P, I64, C.c_uint64, C.POINTER(GgufValue)]),
        "wg_onnx_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
        "wg_onnx_close": (C.c_int, [P]),
        "wg_onnx_graph_name": (C.c_char_p, [P]),
        "wg_onnx_node_count": (I64, [P]),
        "wg_onnx_tensor_count": (I64, [P]),
        "wg_onnx_init_count": (I64, [P]),
        "wg_onnx_find_init": (I64, [P, C.c_char_p]),
        "wg_onnx_tensor": (C.c_int, [P, I64, C.POINTER(OnnxTensorInfo)]),
        "wg_onnx_node": (C.c_int, [P, I64, C.POINTER(OnnxNodeInfo)]),
        "wg_onnx_node_input": (C.c_char_p, [P, I64, I32]),
        "wg_onnx_node_output": (C.c_char_p, [P, I64, I32]),
        "wg_onnx_node_attr": (C.c_int, [P, I64, I32, C.POINTER(OnnxAttr)]),
        "wg_rows_to_floats": (C.c_int, [I32, P, I32, I32, P, P]),
        "wg_pick_scratch_bytes": (SZ, [I32, I32]),
        "wg_pick_candidates": (C.c_int, [P, I32, I32, I32, P, P, I32, I32, C.c_float,
                                         C.c_float, P, I32, I32, I32, P, P, P, SZ, P]),
        "wg_delta_rule": (C.c_int, [P, I32, I32, P, I32, P, P, C.POINTER(DeltaShape), P, P, I32,
                                    P, I32, P]),
        "wg_delta_chunk_scratch_bytes": (SZ, [I32, C.POINTER(DeltaShape), I32]),
        "wg_delta_rule_chunked": (C.c_int, [P, I32, I32, P, I32, P, P, C.POINTER(DeltaShape),
                                            P, P, I32, P, I32, P, SZ, P]),
        "wg_delta_conv": (C.c_int, [P, I32, I32, I32, I32, P, P, P, P, I32, P]),
        "wg_delta_norm": (C.c_int, [P, I32, I32, C.POINTER(DeltaShape), P, I32, P, C.c_float, P,
                                    I32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != WG_OK:
        raise WgError(rc, load().wg_last_error().decode())


def last_error() -> str:
    return load().wg_last_error().decode()


def tuning_set(name: str, value: int) -> None:
    check(load().wg_tuning_set(name.encode(), int(value)))


def tuning_get(name: str) -> int:
    v = C.c_int32()
    check(load().wg_tuning_get(name.encode(), C.byref(v)))
    return v.value
