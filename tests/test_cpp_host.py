"""The C++ host layer (the engine interface: conversation_kv_*, conversation_checkpoint_*, conversation_snapshot_*)
through its own test programs in tests/cpp, built by __graft_entry__.build(), and through the reference's own tests
of that interface compiled unmodified against this library (oracle/_ref, built where the reference's sources are):
src/core/conversation_validation_test.cpp on the host layer (CPU, copies linked to memcpy as the reference's host-only
build does) and src/core/conversation_snapshot_test.cpp on the device."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "bin"
REF = ROOT / "oracle" / "_ref"


def _run(name: str, timeout: int, where: Path = BIN) -> str:
    exe = where / name
    assert exe.exists(), f"{exe} is not built (run __graft_entry__.build())"
    proc = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    assert proc.returncode == 0, proc.stdout[-4000:]
    return proc.stdout


def test_validation_refuses_before_any_write():
    """Host-only: malformed images are refused with no copy and intact sentinels; late failures are
    transfer_failed (the reference's conversation_validation_test matrix)."""
    out = _run("conversation_validation_test", 120)
    assert "checks passed" in out


@pytest.mark.skipif(not (REF / "ref_validation_test_on_ours").exists(),
                    reason="the reference test builds (oracle/_ref) are not here")
def test_reference_validation_test_against_this_library():
    """src/core/conversation_validation_test.cpp, unmodified, on this library's host layer: all its checks pass."""
    out = _run("ref_validation_test_on_ours", 120, REF)
    assert "FAIL" not in out and "checks passed" in out
    print(out.strip().splitlines()[-1])


@pytest.mark.gpu
@pytest.mark.skipif(not (REF / "ref_snapshot_test_on_ours").exists(),
                    reason="the reference test builds (oracle/_ref) did not travel with the tree")
def test_reference_snapshot_test_against_this_library(cuda):
    """src/core/conversation_snapshot_test.cpp, unmodified, on this library with device pools: every format x
    resident/streamed mode x expert count, A/B/A, incremental reuse, split stages, the draft ring."""
    print("case reference conversation_snapshot_test", flush=True)
    out = _run("ref_snapshot_test_on_ours", 240, REF)
    assert "FAIL" not in out and "checks passed" in out
    print(out.strip().splitlines()[-1])
