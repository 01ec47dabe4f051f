"""The INT8 quantizer's quotient (reciprocal + two fused-multiply-add corrections, q8 in tcq_device.h) against IEEE division,
on the host (tests/native/quotient_check.c built with gcc): the same rounded integer for every checked v of the quantizer's
domain at scales in [2^-90, 2^90], and the correctly rounded quotient wherever |v / s| >= 2^-12. A full sweep of every FP32
pattern at six scales (run once with STEP 1) found no rounded-integer difference; this test runs a strided sweep."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which('gcc') is None, reason='needs gcc')
def test_quotient_scheme_matches_division(tmp_path):
    exe = tmp_path / 'quotient_check'
    subprocess.run(['gcc', '-O2', '-o', str(exe), str(HERE / 'native' / 'quotient_check.c'), '-lm'], check=True)
    out = subprocess.run([str(exe), '2000000', '1021'], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert 'round-mismatches 0 quotient-mismatches 0' in out.stdout
