"""The codec oracle (oracle/sc_wire.py) against the reference codec's own output.

tests/golden/wire_manifest.json holds, for every spec under tests/golden/wire/, the payload length and FNV-1a payload
hash that the reference's conversation_wire_encode produced (oracle/_ref/ref_wire, built from
src/core/conversation_wire.cpp), the payload bytes for the small ones, and the reference decoder's accept / refuse
verdict on 78 corrupted payloads.  The oracle must reproduce every byte, every hash and every verdict.  When the
reference build is present (this container), a few specs are also re-encoded live to show the fixtures are current.
"""
import json
import struct
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = ROOT / "tests" / "golden"
MANIFEST = json.loads((GOLDEN / "wire_manifest.json").read_text())
REF = ROOT / "oracle" / "_ref" / "ref_wire"


@pytest.fixture(scope="module")
def wire():
    from oracle import sc_wire
    return sc_wire


@pytest.mark.parametrize("name", sorted(MANIFEST["specs"]))
def test_oracle_encode_matches_reference(wire, name):
    entry = MANIFEST["specs"][name]
    image, geom, pack = wire.image_from_spec((GOLDEN / "wire" / f"{name}.spec").read_text())
    payload = wire.encode(image, geom & (2**64 - 1), pack & (2**64 - 1))
    assert len(payload) == entry["bytes"]
    assert wire.payload_hash(payload) == int(entry["payload_hash"], 16)
    if "payload" in entry:
        assert payload == (GOLDEN / entry["payload"]).read_bytes()


@pytest.mark.parametrize("name", sorted(n for n, e in MANIFEST["specs"].items() if "payload" in e))
def test_oracle_decodes_reference_payload(wire, name):
    payload = (GOLDEN / MANIFEST["specs"][name]["payload"]).read_bytes()
    image, geom, pack = wire.image_from_spec((GOLDEN / "wire" / f"{name}.spec").read_text())
    got = wire.decode(payload, geom & (2**64 - 1), pack & (2**64 - 1), wire.payload_hash(payload),
                      geometry=image["geometry"])
    assert wire.images_equal(image, got)
    assert wire.encode(got, geom & (2**64 - 1), pack & (2**64 - 1)) == payload


def _mutated(wire, case):
    """Rebuild a corrupted payload from its label (the same edits tests/golden/make_wire_vectors.py made)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("mwv", GOLDEN / "make_wire_vectors.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    name = case["of"]
    image, geom, pack = wire.image_from_spec((GOLDEN / "wire" / f"{name}.spec").read_text())
    good = (GOLDEN / "wire" / f"{name}.bin").read_bytes()
    for label, payload, exp in mod.mutations(name, image, good, geom, pack):
        if label == case["case"]:
            return image, geom, pack, good, payload, exp
    raise KeyError(case["case"])


@pytest.mark.parametrize("case", MANIFEST["mutations"], ids=[m["case"] for m in MANIFEST["mutations"]])
def test_oracle_refuses_what_reference_refuses(wire, case):
    image, geom, pack, good, payload, exp = _mutated(wire, case)
    h = wire.payload_hash(good) if exp.get("hash") == "original" else wire.payload_hash(payload)
    try:
        wire.decode(payload, geom & (2**64 - 1), pack & (2**64 - 1), h, stage_parts=exp.get("stage_parts", -1),
                    max_payload_bytes=exp.get("max_payload", 0))
        refused = False
    except wire.WireRefusal:
        refused = True
    assert refused == case["refused"], case["reason"]


def test_layout_facts(wire):
    """Fixed facts of the format (conversation_wire.hpp:33-60): header record 256 bytes, magic 'SR4H', the pool
    64-aligned, the END record spelling 'END!'."""
    payload = (GOLDEN / "wire" / "handoff_shape.bin").read_bytes()
    assert payload[:4] == b"SR4H"
    pool_off, pool_bytes = struct.unpack_from("<QQ", payload, 200)
    assert pool_off % 64 == 0 and pool_off + pool_bytes == len(payload)
    assert payload.find(b"END!") == pool_off - 16 or payload[pool_off - 16 - 48:pool_off].count(b"END!") == 1


@pytest.mark.skipif(not REF.exists(), reason="the reference codec build (oracle/_ref) is not present")
@pytest.mark.parametrize("name", ["empty", "handoff_shape", "layer_split"])
def test_fixtures_are_current(tmp_path, name):
    out = tmp_path / "p.bin"
    size, h = subprocess.run([str(REF), "encode", str(GOLDEN / "wire" / f"{name}.spec"), str(out)],
                             capture_output=True, text=True, check=True).stdout.split()
    assert int(size) == MANIFEST["specs"][name]["bytes"]
    assert int(h, 16) == int(MANIFEST["specs"][name]["payload_hash"], 16)
