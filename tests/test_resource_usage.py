"""Compile-time guards on the GEMV epilogue (CPU: hipcc cross-compiles for
gfx950, no GPU needed): a probe kernel that runs the epilogue's input
scales and finish for 5 tokens must use exactly the LDS it declares and no
scratch. An array of the M tokens indexed by a loop variable is moved into
LDS by the compiler (256 threads x M floats) before the loop is unrolled;
in the few-token GEMVs that cost about 11 us a launch."""
import os
import re
import shutil
import subprocess

import pytest

HIPCC = "/opt/rocm/bin/hipcc"
CSRC = os.path.join(os.path.dirname(__file__), "..", "webgllm_amd", "csrc")

PROBE = r'''
#include "epilogue.h"
namespace wg {
template <int M, int MODE>
__global__ __launch_bounds__(256) void probe(const wg_epilogue e, float *y, int ldy, int G) {
  __shared__ float nred[4 * M];
  float scale[M], tot[M];
  input_scales_wg<M, 4>(e, scale, nred);
  for (int m = 0; m < M; m++) tot[m] = y[threadIdx.x * M + m];
  EpiPre pre = {};
  finish<M, MODE>(e, blockIdx.x, G, tot, scale, y, ldy, pre, 0);
}
template __global__ void probe<5, WG_EPI_STORE>(const wg_epilogue, float *, int, int);
template __global__ void probe<5, WG_EPI_SWIGLU>(const wg_epilogue, float *, int, int);
template __global__ void probe<8, WG_EPI_STORE>(const wg_epilogue, float *, int, int);
}
'''


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="no hipcc")
def test_epilogue_keeps_token_arrays_in_registers(tmp_path):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    r = subprocess.run([HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", CSRC,
                        "--cuda-device-only", "-c", "-Rpass-analysis=kernel-resource-usage",
                        str(src), "-o", str(tmp_path / "probe.o")],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    kernels = re.findall(r"Function Name: (\S+).*?ScratchSize \[bytes/lane\]: (\d+).*?"
                         r"LDS Size \[bytes/block\]: (\d+)", r.stderr, re.S)
    assert len(kernels) == 3
    for name, scratch, lds in kernels:
        m = 8 if "ILi8E" in name else 5
        assert int(scratch) == 0, name
        assert int(lds) == 4 * m * 4, (name, lds)  # nred only
