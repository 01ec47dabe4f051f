"""CPU checks of the C ABI: the built library loads and exports every function include/tcq_api.h declares, and the ctypes
table covers exactly those functions. No compute calls (there is no GPU here)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'tcq_api.h'
LIB = ROOT / 'yanlongvla_amd' / 'libtcq.so'


def declared():
    src = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r'^\s*(?:const\s+)?[\w\s\*]+?\b(tcq_\w+)\s*\(', src, flags=re.M)))


def test_header_declares_functions():
    names = declared()
    assert 'tcq_version' in names and 'tcq_gemv_f16' in names and len(names) >= 10


@pytest.mark.skipif(not LIB.exists(), reason='libtcq.so not built (run python -m yanlongvla_amd.build)')
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    from yanlongvla_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared()


@pytest.mark.skipif(not LIB.exists(), reason='libtcq.so not built')
def test_version_and_limits_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    lib.tcq_version.restype = ctypes.c_char_p
    assert b'gfx950' in lib.tcq_version()
    assert lib.tcq_max_width() == 16384
    lib.tcq_repack_words.restype = ctypes.c_int64
    assert lib.tcq_repack_words(2048, 2048) == 128 * 8 * 256
    assert lib.tcq_repack_words(48, 80) == 3 * 1 * 256
    assert lib.tcq_repack_words(40, 80) == -2


@pytest.mark.skipif(not LIB.exists(), reason='libtcq.so not built')
def test_argument_errors_are_reported_before_launch():
    """Null pointers and bad shapes are rejected on the host with the documented status codes (no device work)."""
    lib = ctypes.CDLL(str(LIB))
    P = ctypes.c_void_p
    assert lib.tcq_decode_i8(None, None, None, 16, 16, None) == -1
    assert lib.tcq_decode_i8(P(16), P(16), P(16), 24, 16, None) == -2
    assert lib.tcq_decode_i8(P(16), P(16), P(8), 16, 16, None) == -5
    assert lib.tcq_rht(P(16), 7, 16, None, P(16), 0, 16, 1, 16, None) == -3
    assert lib.tcq_rht(P(16), 0, 32768, None, P(16), 0, 32768, 1, 32768, None) == -2
    assert lib.tcq_pre(P(16), 1, None, P(16), None, 0, P(16), 1, 18, None) == -2
    assert lib.tcq_gemv_f16(P(16), 1, P(16), P(16), 17, 16, 16, None) == -4
    assert lib.tcq_pre_h(P(16), 1, None, None, None, 0, 1, 16, None) == -1          # neither h nor hT
    assert lib.tcq_pre_h(P(16), 1, None, None, P(16), 1, 2, 16, None) == -1         # ldh < M
    assert lib.tcq_gemmf_w8_hT(P(16), P(16), 1, P(16), P(16), 2, 16, 16, None) == -1
    assert lib.tcq_gemmf_tcq_hT(P(16), P(16), P(16), 1, P(16), P(16), 1, 24, 16, 0, 0, None) == -2
    assert lib.tcq_gemmf_tcq_hT(P(16), P(16), P(16), 1, P(16), P(8), 1, 16, 16, 0, 0, None) == -5
    assert lib.tcq_gemmf_tcq(P(16), 1, P(16), 1, 16, 3, 16, None) == -3               # int32 out: not a float product
    # one-layer entry points: tcq_pre_gemv_f16(x, x_dtype, su, wdev, tlut, row_scale, M, m, n, z, stream)
    assert lib.tcq_pre_gemv_f16(None, 2, P(16), P(16), P(16), P(16), 1, 2048, 2048, P(16), None) == -1
    assert lib.tcq_pre_gemv_f16(P(16), 2, P(16), P(16), P(16), P(16), 17, 2048, 2048, P(16), None) == -4   # M > 16
    assert lib.tcq_pre_gemv_f16(P(16), 2, P(16), P(16), P(16), P(16), 1, 2056, 2048, P(16), None) == -2   # m % 16
    assert lib.tcq_pre_gemv_f16(P(16), 2, P(16), P(16), P(16), P(16), 1, 2048, 2048, P(8), None) == -5    # z alignment
    assert lib.tcq_pre_gemv_f16(P(16), 2, P(16), P(16), P(16), P(4), 1, 2048, 2048, P(16), None) == -5    # row scales
    assert lib.tcq_pre_gemv_f16(P(16), 7, P(16), P(16), P(16), P(16), 1, 2048, 2048, P(16), None) == -3   # x dtype
    # tcq_layer_f16 needs its counter and output
    assert lib.tcq_layer_f16(P(16), 2, P(16), P(16), P(16), P(16), P(16), None, P(16), 2, 1, 2048, 2048, P(16), None,
                             None) == -1


@pytest.mark.skipif(not LIB.exists(), reason='libtcq.so not built')
def test_mid2_available_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    assert [lib.tcq_mid2_available(n) for n in (1024, 4096, 4304, 16384, 16400, 24, 0)] == [1, 1, 1, 1, 0, 0, 0]
