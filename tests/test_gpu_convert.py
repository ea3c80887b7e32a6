"""The kernels' binary16 conversions (sc_convert.hpp) against the CPU oracle, over every input.

f16_bits_rne runs on the conversion instruction with a NaN select; here it converts all 2^32 binary32 patterns on the
device (tests/hip/convert_probe.hip includes the same header) and every result must equal the oracle's sco_f16_bits
(pinned by the reference's own vectors and numpy).  f32_of_f16 converts all 2^16 binary16 patterns and must equal
numpy's exact widening (NaNs: any NaN).  Every f16 the carves write (K/V rows, int8 scales, q4_0 d) and every f32
the int8 quantizer reads back from its scale comes from these two functions.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PROBE = Path(__file__).resolve().parent / "hip" / "bin" / "libconvert_probe.so"
CHUNK = 1 << 28


@pytest.fixture(scope="module")
def probe(cuda):
    assert PROBE.exists(), "tests/hip/bin/libconvert_probe.so is missing: run __graft_entry__.build()"
    lib = C.CDLL(str(PROBE))
    lib.probe_f16_of_f32.argtypes = [C.c_uint32, C.c_uint64, C.c_void_p]
    lib.probe_f16_of_f32.restype = C.c_int
    lib.probe_f32_of_f16.argtypes = [C.c_void_p]
    lib.probe_f32_of_f16.restype = C.c_int
    return lib


def test_f16_of_every_f32(probe, oracle):
    got = np.empty(CHUNK, np.uint16)
    for c in range((1 << 32) // CHUNK):
        lo = c * CHUNK
        assert probe.probe_f16_of_f32(lo, CHUNK, got.ctypes.data) == 0
        src = np.arange(lo, lo + CHUNK, dtype=np.uint64).astype(np.uint32).view(np.float32)
        want = oracle.f16_bits(src)
        if not np.array_equal(got, want):
            i = int(np.argmax(got != want))
            raise AssertionError(f"f32 0x{lo + i:08x}: device 0x{int(got[i]):04x}, oracle 0x{int(want[i]):04x}")


def test_f32_of_every_f16(probe):
    got = np.empty(65536, np.uint32)
    assert probe.probe_f32_of_f16(got.ctypes.data) == 0
    want = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    g = got.view(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(got[~nan], want.view(np.uint32)[~nan])
