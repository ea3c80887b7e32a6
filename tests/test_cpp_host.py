"""The C++ host layer (the engine interface: conversation_kv_*, conversation_checkpoint_*, conversation_snapshot_*)
through its own test programs in tests/cpp, built by __graft_entry__.build()."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "bin"


def _run(name: str, timeout: int) -> str:
    exe = BIN / name
    assert exe.exists(), f"{exe} is not built (run __graft_entry__.build())"
    proc = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    assert proc.returncode == 0, proc.stdout[-4000:]
    return proc.stdout


def test_validation_refuses_before_any_write():
    """Host-only: malformed images are refused with no copy and intact sentinels; late failures are
    transfer_failed (the reference's conversation_validation_test matrix)."""
    out = _run("conversation_validation_test", 120)
    assert "checks passed" in out


@pytest.mark.gpu
def test_snapshot_aba_on_device(cuda):
    """Device pools in f16/int8/q4/K8V4 x resident/streamed/ring: A/B/A exactness, refusals, incremental capture,
    checkpoint spare-row rebuild, layer split."""
    out = _run("conversation_snapshot_test", 240)
    assert "checks passed" in out
    print(out.strip().splitlines()[-1])
