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


@pytest.fixture(scope="module")
def arith(probe):
    probe.probe_arith_mismatches.argtypes = [C.c_uint32, C.c_uint64, C.c_int, C.POINTER(C.c_ulonglong),
                                             C.POINTER(C.c_uint32)]
    probe.probe_arith_mismatches.restype = C.c_int
    probe.probe_recip.argtypes = [C.c_uint32, C.c_uint64, C.c_void_p]
    probe.probe_recip.restype = C.c_int
    return probe


def _mismatches(arith, mode, lo, n):
    total, first = 0, []
    step = 1 << 30
    for s in range(lo, lo + n, step):
        cnt, f = C.c_ulonglong(), (C.c_uint32 * 8)()
        assert arith.probe_arith_mismatches(s, min(step, lo + n - s), mode, C.byref(cnt), f) == 0
        total += cnt.value
        first += [f[i] for i in range(min(8, cnt.value))]
    return total, first


def test_recip_normal_is_the_ieee_reciprocal_over_its_range(arith):
    """sc_arith.hpp's recip_normal (v_rcp_f32 + one fused Newton step), used by the quantizers for 1/scale, equals
    the IEEE division 1.0f / d for every binary32 d with 2^-126 <= |d| < 2^126 (counted on the device), and agrees
    with numpy's division on a random sample (checked here on the CPU)."""
    total, first = _mismatches(arith, 0, 0, 1 << 32)
    assert total == 0, [hex(x) for x in first]
    rng = np.random.default_rng(11)
    lo = int(rng.integers(0x00800000, 0x7E000000))   # a window of consecutive normal patterns
    n = 1 << 24
    got = np.empty(n, np.uint32)
    assert arith.probe_recip(lo, n, got.ctypes.data) == 0
    d = np.arange(lo, lo + n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = (np.float32(1.0) / d).view(np.uint32)
    ok = (np.abs(d) >= np.float32(2.0 ** -126)) & (np.abs(d) < np.float32(2.0 ** 126))
    assert np.array_equal(got[ok], want[ok])


def test_div127_is_the_ieee_quotient_for_every_non_negative_input(arith):
    """div127 (one product with RN(1/127) and one fused correction), the int8 scale's division, equals a / 127.0f for
    every non-negative binary32 a including +0, subnormals and +inf (counted on the device)."""
    total, first = _mismatches(arith, 1, 0, 1 << 31)
    assert total == 0, [hex(x) for x in first]
