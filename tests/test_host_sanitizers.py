"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

The host-sanitized build (sunshape_amd/build.py: build_host_sanitized; device code built plainly) is
loaded in a child process with the sanitizer runtime preloaded and no GPU visible, and
tests/host_abi_fuzz.py drives every argument check, kernel choice, launch plan and workspace
size of ssq_decode / ssq_attention_scores / ssq_decode_noalloc / ssq_encode / the grid build /
ssq_dequantize / ssq_pack_codes with hypothesis-generated arguments (valid, edge and invalid
shapes, strides, dtypes, code widths, masks and pointers).  Any sanitizer report aborts the child.
"""

import os
import subprocess
import sys

import pytest

from sunshape_amd import build as B

HERE = os.path.dirname(os.path.abspath(__file__))


def _gpu_visible() -> bool:
    import torch

    return torch.cuda.device_count() > 0


@pytest.mark.skipif(B.asan_runtime() is None, reason="no shared AddressSanitizer runtime in this toolchain")
def test_host_code_under_asan_and_ubsan():
    if _gpu_visible():
        pytest.skip("runs where no GPU is visible (the driver's CPU suite)")
    lib = B.build_host_sanitized()
    env = dict(os.environ)
    env.update(LD_PRELOAD=B.asan_runtime(), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="-1",
               ROCR_VISIBLE_DEVICES="-1", CUDA_VISIBLE_DEVICES="-1", PYTHONHASHSEED="0")
    r = subprocess.run([sys.executable, os.path.join(HERE, "host_abi_fuzz.py"), lib, "1500"], env=env,
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    assert "no sanitizer report" in r.stdout
