"""The quantizers' FP8 encode (the hardware e4m3fn conversion in quant.hip) equals the
spec's software encode on every fp32 value of [-448, 448]: tests/gpu_checks/
fp8_encode_check.hip compares the two over all 2,277,507,074 of them on the GPU. The
quantizer itself is held to the numpy spec by tests/test_quant_gpu.py, including the e4m3
midpoints (test_quantizer_rounding_ties). Needs a GPU and the binary that
kvq_decode_amd.build compiles."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gpu_checks", "fp8_encode_check")


def test_fp8_encode_matches_spec_exhaustively():
    assert os.path.exists(BIN), f"{BIN} missing: build with python -m kvq_decode_amd.build"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
