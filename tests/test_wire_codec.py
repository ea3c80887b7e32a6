"""The product's payload codec (host/src/conversation_wire.cpp, in libsc_core) against the reference codec's output.

tests/cpp/bin/wire_driver is oracle/ref_wire_driver.cpp - the program that produced the golden vectors from the
reference's codec - compiled against this library's codec instead.  Every spec must encode to the same bytes and hash
the reference produced, and every corrupted payload must be accepted or refused exactly as the reference decided.
conversation_wire_test restates the reference's own codec test scenarios in C++ (host only), and where the
reference's sources are at hand, oracle/_ref/ref_wire_test_on_ours is the reference's own codec test
(src/core/saved_conv_wire_test.cpp) compiled unmodified against this library's codec header and library.
"""
import json
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = ROOT / "tests" / "golden"
BIN = ROOT / "tests" / "cpp" / "bin"
MANIFEST = json.loads((GOLDEN / "wire_manifest.json").read_text())


REF_TEST = ROOT / "oracle" / "_ref" / "ref_wire_test"
REF_TEST_ON_OURS = ROOT / "oracle" / "_ref" / "ref_wire_test_on_ours"


def _run_ref_test(exe: Path) -> str:
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0 and "FAIL" not in out, "\n".join(l for l in out.splitlines() if "FAIL" in l) or out
    return out


@pytest.mark.skipif(not REF_TEST_ON_OURS.exists(), reason="the reference codec test build (oracle/_ref) is not here")
def test_reference_codec_test_against_this_library():
    """src/core/saved_conv_wire_test.cpp, unmodified, on this library's codec: every one of its checks passes, and it
    counts as many checks as it does on the reference's own codec."""
    out = _run_ref_test(REF_TEST_ON_OURS)
    assert "checks passed" in out
    if REF_TEST.exists():
        assert out.split()[-3:] == _run_ref_test(REF_TEST).split()[-3:]


def _driver(*args) -> str:
    exe = BIN / "wire_driver"
    assert exe.exists(), f"{exe} is not built (run __graft_entry__.build())"
    return subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True, check=True,
                          timeout=120).stdout.strip()


@pytest.mark.parametrize("name", sorted(MANIFEST["specs"]))
def test_encode_matches_reference(tmp_path, name):
    entry = MANIFEST["specs"][name]
    out = tmp_path / "p.bin"
    size, h = _driver("encode", GOLDEN / "wire" / f"{name}.spec", out).split()
    assert int(size) == entry["bytes"]
    assert int(h, 16) == int(entry["payload_hash"], 16)
    if "payload" in entry:
        assert out.read_bytes() == (GOLDEN / entry["payload"]).read_bytes()


@pytest.mark.parametrize("case", MANIFEST["mutations"], ids=[m["case"] for m in MANIFEST["mutations"]])
def test_decode_verdicts_match_reference(tmp_path, case):
    from oracle import sc_wire
    import importlib.util
    spec = importlib.util.spec_from_file_location("mwv", GOLDEN / "make_wire_vectors.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    name = case["of"]
    image, geom, pack = sc_wire.image_from_spec((GOLDEN / "wire" / f"{name}.spec").read_text())
    good = (GOLDEN / "wire" / f"{name}.bin").read_bytes()
    payload, exp = next((p, e) for label, p, e in mod.mutations(name, image, good, geom, pack) if label == case["case"])
    path = tmp_path / "m.bin"
    path.write_bytes(payload)
    h = sc_wire.payload_hash(good) if exp.get("hash") == "original" else sc_wire.payload_hash(payload)
    verdict = _driver("decode", path, geom & (2**64 - 1), pack & (2**64 - 1), h, exp.get("stage_parts", -1),
                      exp.get("max_payload", 0))
    assert verdict.startswith("refused") == case["refused"], (verdict, case["reason"])
    if case["case"].endswith(":valid"):
        assert verdict == "ok 1", "a valid payload re-encodes to the same bytes"


def test_codec_scenarios():
    exe = BIN / "conversation_wire_test"
    assert exe.exists(), f"{exe} is not built"
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert "checks passed" in proc.stdout
