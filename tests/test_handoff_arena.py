"""The hand-off arena (strata-concurrent_amd/host/src/handoff.cpp) on the CPU: this library's test program, the
reference's own arena test compiled against this library, and the two implementations on the same arena files.

* tests/cpp/bin/handoff_arena_test - this library's test of every scenario (always runs).
* oracle/_ref/ref_arena_test_on_ours - src/core/handoff_arena_test.cpp, the reference's test, compiled in place
  against this library's handoff.hpp and libsc_core.so (where the reference is mounted: this container).
* interop - the same driver (oracle/ref_arena_driver.cpp) built against each implementation: one writes and publishes,
  the other reads and refuses; files created by either are byte-identical outside the creator's pid and start time;
  a claim made through one is exclusive against the other.
* the oracle (oracle/sc_arena.py) - sizing, split spec, geometry hash and path - equals both implementations.
"""
import os
import random
import shutil
import struct
import subprocess
from pathlib import Path

import pytest

from oracle import sc_arena

ROOT = Path(__file__).resolve().parent.parent
OURS = ROOT / "tests" / "cpp" / "bin" / "arena_driver"
REF = ROOT / "oracle" / "_ref" / "ref_arena"
OUR_TEST = ROOT / "tests" / "cpp" / "bin" / "handoff_arena_test"
REF_TEST_ON_OURS = ROOT / "oracle" / "_ref" / "ref_arena_test_on_ours"
needs_ref = pytest.mark.skipif(not REF.exists(), reason="the reference arena build (oracle/_ref) is not here")

PACK, GEOM = 0x0123456789ABCDEF, 0x1F2E3D4C5B6A7988
TIERS = "1024:2,4096:1,16384:2"
PRICED = "1048576,2097152,4194309"


def run(binary, *args, stdin=None):
    # the window and big-slot cases commit several GiB of arena pages: a minute alone, longer beside other tests
    proc = subprocess.run([str(binary), *map(str, args)], capture_output=True, text=True, timeout=600, input=stdin)
    assert proc.returncode == 0, proc.stderr + proc.stdout
    return proc.stdout


def fields(line):
    return dict(w.split("=", 1) for w in line.split() if "=" in w)


def last(out, word):
    lines = [l for l in out.splitlines() if l.startswith(word)]
    assert lines, out
    return fields(lines[-1])


@pytest.fixture
def shm(tmp_path_factory):
    d = Path(f"/dev/shm/sc-arena-interop-{os.getpid()}-{random.randrange(1 << 30)}")
    d.mkdir(parents=True)
    yield d
    shutil.rmtree(d, ignore_errors=True)


def test_our_arena_test_program():
    out = run(OUR_TEST)
    assert out.strip().endswith("0 failed"), out[-3000:]


@pytest.mark.skipif(not REF_TEST_ON_OURS.exists(), reason="the reference arena test build (oracle/_ref) is not here")
def test_reference_arena_test_against_this_library():
    """src/core/handoff_arena_test.cpp, unmodified, on this library's arena: every one of its checks passes."""
    out = run(REF_TEST_ON_OURS)
    assert "FAIL" not in out, "\n".join(l for l in out.splitlines() if "FAIL" in l)
    assert out.strip().splitlines()[-1].endswith("checks, OK")


@pytest.mark.parametrize("impl", ["ours", pytest.param("ref", marks=needs_ref)])
@pytest.mark.parametrize("tiers,priced", [([(1024, 2), (4096, 1), (16384, 2)], [1 << 20, 2 << 20, (4 << 20) + 5]),
                                          ([(131072, 3)], [3_300_000_007]),
                                          ([(i * 1000, i) for i in range(1, 9)], [i * 77777 for i in range(1, 9)])])
def test_sizing_equals_the_oracle(impl, tiers, priced):
    binary = OURS if impl == "ours" else REF
    out = run(binary, "size", ",".join(f"{t}:{c}" for t, c in tiers), ",".join(map(str, priced)))
    want = sc_arena.size_arena(tiers, priced)
    rows = [fields(l) for l in out.splitlines() if l.startswith("tier=")]
    assert [int(r["slot_bytes"]) for r in rows] == want["slot_bytes"]
    assert [int(r["slot_off"]) for r in rows] == want["slot_off"]
    s = last(out, "SIZE")
    assert int(s["arena"]) == want["arena_bytes"] and int(s["total"]) == want["slot_total"]
    assert int(s["max"]) == want["max_tokens"]


@pytest.mark.parametrize("impl", ["ours", pytest.param("ref", marks=needs_ref)])
def test_identity_equals_the_oracle(impl):
    binary = OURS if impl == "ours" else REF
    rng = random.Random(5)
    splits = [(0, 48, [], True), (0, 16, [(16, 34), (34, 48)], True), (0, 16, [(16, 34), (34, 48)], False),
              (4, 20, [(20, 48)], True)]
    for lo, hi, stages, last_ in splits:
        args = [lo, hi, int(last_)] + [x for st in stages for x in st]
        spec = last(run(binary, "split-spec", *args), "spec")["spec"]
        assert spec == sc_arena.split_spec(lo, hi, stages, last_)
        for _ in range(3):
            geo = [rng.randrange(-5, 1 << 40) for _ in range(18)]
            got = int(last(run(binary, "geom-hash", spec, *geo), "hash")["hash"], 16)
            assert got == sc_arena.geom_hash(geo, spec)
    path = last(run(binary, "path", "/dev/shm/x", "00000000000abcde", "main=0..48||n=1|draft=main", "pf"), "path")
    assert path["path"] == sc_arena.arena_path("/dev/shm/x", 0xABCDE, "main=0..48||n=1|draft=main", "pf")


def pattern(n, seed):
    i = __import__("numpy").arange(n, dtype="uint64")
    return ((i * 131 + seed * 17 + (i >> 9)) & 0xFF).astype("uint8").tobytes()


@needs_ref
@pytest.mark.parametrize("writer,reader", [(OURS, REF), (REF, OURS)], ids=["ours-to-ref", "ref-to-ours"])
@pytest.mark.parametrize("nbytes,tier", [(0, 0), (1, 0), (4099, 1), (5_000_003, 2)])
def test_one_implementation_writes_the_other_reads(shm, writer, reader, nbytes, tier):
    path = shm / "pair" / "arena"
    out = run(writer, "write", path, f"{PACK:016x}", f"{GEOM:016x}", TIERS, PRICED, tier, 4242, 77, nbytes, 9, 1234, 0)
    c, p = last(out, "CLAIM"), last(out, "PUBLISH")
    assert c["ok"] == "1" and p["ok"] == "1", out
    slot, nonce = int(c["slot"]), c["nonce"]
    assert int(p["hash"], 16) == sc_arena.sc_oracle.fnv1a64(pattern(nbytes, 9), sc_arena.SEED)
    r = last(run(reader, "read", path, f"{PACK:016x}", f"{GEOM:016x}", slot, nonce, 4242, 9), "READ")
    assert r["ok"] == "1" and r["pattern"] == "1" and int(r["bytes"]) == nbytes and int(r["tokens"]) == 1234
    assert r["hash"] == r["recorded"] == p["hash"] and int(r["request"]) == 77 and int(r["tier"]) == tier
    for args, word in (((slot, f"{int(nonce, 16) ^ 1:016x}", 4242), "nonce"), ((slot, nonce, 4243), "addressed"),
                       (((slot + 1) % 5, nonce, 4242), "not READY")):
        bad = last(run(reader, "read", path, f"{PACK:016x}", f"{GEOM:016x}", *args, 9), "READ")
        assert bad["ok"] == "0"
    bad = last(run(reader, "read", path, f"{PACK ^ 1:016x}", f"{GEOM:016x}", slot, nonce, 4242, 9), "OPEN")
    assert bad["ok"] == "0"
    # and both implementations describe the published slot the same way
    a = last(run(OURS, "info", path, f"{PACK:016x}", f"{GEOM:016x}", slot), "INFO")
    b = last(run(REF, "info", path, f"{PACK:016x}", f"{GEOM:016x}", slot), "INFO")
    assert a == b and a["state"] == "2" and int(a["bytes"]) == nbytes and a["seq"] == "1"


@needs_ref
def test_files_are_byte_identical_outside_the_creator(shm):
    paths = {}
    for name, binary in (("ours", OURS), ("ref", REF)):
        paths[name] = shm / name / "arena"
        assert last(run(binary, "create", paths[name], f"{PACK:016x}", f"{GEOM:016x}", TIERS, PRICED), "OPEN")["ok"] == "1"
    a, b = paths["ours"].read_bytes(), paths["ref"].read_bytes()
    assert len(a) == len(b)
    tiers = [(1024, 2), (4096, 1), (16384, 2)]
    layout = sc_arena.size_arena(tiers, [1048576, 2097152, 4194309])
    assert len(a) == layout["arena_bytes"]
    ha, hb = sc_arena.parse(a, sc_arena.ARENA_FIELDS), sc_arena.parse(b, sc_arena.ARENA_FIELDS)
    for h in (ha, hb):
        assert h["magic"] == sc_arena.ARENA_MAGIC and h["version"] == 1 and h["header_bytes"] == 4096
        assert h["tier_slot_off"][:3] == layout["slot_off"] and h["tier_slot_bytes"][:3] == layout["slot_bytes"]
        assert h["pack_hash"] == PACK and h["geom_hash"] == GEOM and h["created_pid"] != 0
    assert a[:64] == b[:64] and a[80:4096] == b[80:4096]       # everything but created_pid / created_start
    for base, _ in sc_arena.slot_bases(layout, tiers):
        assert a[base:base + 4096] == b[base:base + 4096]
        s = sc_arena.parse(a[base:base + 4096], sc_arena.SLOT_FIELDS)
        assert s["magic"] == sc_arena.SLOT_MAGIC and s["state"] == 0
    import numpy as np
    diff = np.flatnonzero(np.frombuffer(a, np.uint8) != np.frombuffer(b, np.uint8))
    assert ((diff >= 64) & (diff < 80)).all(), diff[:10]


@needs_ref
def test_slot_headers_written_by_either_are_the_same_record(shm):
    """A claim+publish through each implementation with the same inputs: every field the protocol fixes is equal
    (nonce, owner and times are per process)."""
    recs = []
    for binary in (OURS, REF):
        path = shm / binary.name / "arena"
        out = run(binary, "write", path, f"{PACK:016x}", f"{GEOM:016x}", TIERS, PRICED, 1, 99, 5, 70000, 3, 4321, 0)
        c = last(out, "CLAIM")
        raw = path.read_bytes()[int(c["base"]):int(c["base"]) + 4096]
        s = sc_arena.parse(raw, sc_arena.SLOT_FIELDS)
        assert s["nonce"] == int(c["nonce"], 16) and s["owner_pid"] != 0 and s["published_ms"] >= s["claimed_ms"] > 0
        for k in ("nonce", "owner_pid", "owner_start", "claimed_ms", "published_ms"):
            s.pop(k)
        recs.append((s, raw[144:]))
    assert recs[0] == recs[1]
    s = recs[0][0]
    assert s["state"] == 2 and s["flags"] == 0 and s["tier"] == 1 and s["client_id"] == 99 and s["request_id"] == 5
    assert s["tokens"] == 4321 and s["payload_bytes"] == 70000 and s["seq"] == 1
    assert s["payload_hash"] == sc_arena.sc_oracle.fnv1a64(pattern(70000, 3), sc_arena.SEED)


@needs_ref
@pytest.mark.parametrize("holder,first,second", [(OURS, REF, OURS), (REF, OURS, REF)], ids=["ours-holds", "ref-holds"])
def test_a_claim_is_exclusive_across_implementations(shm, holder, first, second):
    """One process of one implementation creates a one-slot arena and stays alive; a writer of the other implementation
    takes the slot and publishes; a third writer (of the first implementation) is told there is no free slot; a reader
    of the holder's implementation reads what was published."""
    path = shm / "x" / "arena"
    proc = subprocess.Popen([str(holder), "hold", str(path), f"{PACK:016x}", f"{GEOM:016x}", "1024:1", "4096"],
                            stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True)
    try:
        line = proc.stdout.readline()
        while line and not line.startswith("HELD"):
            line = proc.stdout.readline()
        assert line.startswith("HELD")
        w1 = run(first, "write", path, f"{PACK:016x}", f"{GEOM:016x}", "1024:1", "4096", 0, 7, 1, 3000, 4, 11, 1)
        assert last(w1, "PUBLISH")["ok"] == "1", w1
        w2 = run(second, "write", path, f"{PACK:016x}", f"{GEOM:016x}", "1024:1", "4096", 0, 7, 2, 3000, 5, 11, 1)
        c2 = last(w2, "CLAIM")
        assert c2["ok"] == "0" and "no free handoff slot" in w2, w2
        # without the test-only flag the live holder's arena is refused outright
        w3 = run(second, "write", path, f"{PACK:016x}", f"{GEOM:016x}", "1024:1", "4096", 0, 7, 3, 3000, 5, 11, 0)
        assert last(w3, "OPEN")["ok"] == "0" and "one arena per prefill instance" in w3
        r = last(run(holder, "read", path, f"{PACK:016x}", f"{GEOM:016x}", 0, last(w1, "CLAIM")["nonce"], 7, 4), "READ")
        assert r["ok"] == "1" and r["pattern"] == "1" and int(r["bytes"]) == 3000
    finally:
        proc.communicate("done\n", timeout=30)


@needs_ref
def test_a_restarted_writer_of_either_implementation_rebuilds_the_table(shm):
    path = shm / "restart" / "arena"
    out = run(REF, "write", path, f"{PACK:016x}", f"{GEOM:016x}", TIERS, PRICED, 2, 1, 1, 100, 1, 1, 0)
    nonce = last(out, "CLAIM")["nonce"]
    slot = last(out, "CLAIM")["slot"]
    assert last(run(OURS, "read", path, f"{PACK:016x}", f"{GEOM:016x}", slot, nonce, 1, 1), "READ")["ok"] == "1"
    o = last(run(OURS, "create", path, f"{PACK:016x}", f"{GEOM:016x}", TIERS, PRICED), "OPEN")
    assert o["ok"] == "1" and o["free"] == "5/5"
    assert last(run(REF, "read", path, f"{PACK:016x}", f"{GEOM:016x}", slot, nonce, 1, 1), "READ")["ok"] == "0"
    h = sc_arena.parse(path.read_bytes()[:4096], sc_arena.ARENA_FIELDS)
    assert h["created_pid"] != 0
