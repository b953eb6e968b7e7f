"""MI355X (gfx950) backend for webgllm's Q4 decode/prefill hot path.

The kernels are hand-written HIP in webgllm_amd/csrc, built into
libwebgllm_hip.so with the C ABI of include/webgllm_hip.h. This package is
the host-side mirror of the reference's GPU-backend contract over that ABI.
"""
from . import lib  # noqa: F401

__all__ = ["lib"]
