"""The int8 quantizer's quotient (q8_code in sc_kernels.hip) equals the IEEE quotient, checked exhaustively.

tests/cpp/quotient_check.c runs the kernel's sequence (y = 1/b once, q0 = a*y, one fused correction) over every
binary32 significand against every binary16 significand, 2^33 pairs, and counts mismatches with a / b.  A sequence
without the correction step fails about a quarter of the pairs, so the check has teeth.
"""
import subprocess
from pathlib import Path

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "quotient_check"


def test_quotient_matches_ieee_division_exhaustively():
    assert BIN.exists(), "tests/cpp/bin/quotient_check is missing: run __graft_entry__.build()"
    proc = subprocess.run([str(BIN)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    assert proc.returncode == 0, proc.stdout
    assert "8589934592 pairs, 0 mismatches" in proc.stdout
