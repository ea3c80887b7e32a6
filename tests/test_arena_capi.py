"""The arena's C-ABI (include/sc_arena.h) on the CPU: sizing and the geometry hash equal the oracle, and a host-side
hand-off through the C-ABI (claim, write, publish, read with the CPU hash check, release) works and refuses the way
the C++ API does.  The device movers are tested on the GPU (tests/test_gpu_arena.py)."""
import os
import random
import shutil
from pathlib import Path

import numpy as np
import pytest

from oracle import sc_arena as oracle_arena

PACK, GEOM = 0x5EEDF00D12345678, 0x0BADC0DE87654321


@pytest.fixture(scope="module")
def arena_abi():
    import sc_arena
    return sc_arena


@pytest.fixture
def shm():
    d = Path(f"/dev/shm/sc-arena-capi-{os.getpid()}-{random.randrange(1 << 30)}")
    d.mkdir(parents=True)
    yield d
    shutil.rmtree(d, ignore_errors=True)


def test_size_and_hash_equal_the_oracle(arena_abi):
    tiers, priced = [(1024, 2), (16384, 3), (131072, 1)], [12345, 700_000_001, 3_300_000_000]
    sb, so, total, desc = arena_abi.size(tiers, priced)
    want = oracle_arena.size_arena(tiers, priced)
    assert sb == want["slot_bytes"] and so == want["slot_off"] and total == want["arena_bytes"]
    assert desc.startswith("slots 2,3,1 (tiers 1024,16384,131072), max 131072 tokens")
    geo = list(range(-3, 15))
    spec = oracle_arena.split_spec(0, 16, [(16, 48)], True)
    assert arena_abi.geom_hash(geo, spec) == oracle_arena.geom_hash(geo, spec)
    with pytest.raises(arena_abi.ArenaError):
        arena_abi.size([(4096, 1), (1024, 1)], [1, 1])


def test_host_handoff_through_the_c_abi(arena_abi, shm):
    path = shm / "a" / "arena"
    tiers, priced = [(1024, 1), (4096, 1)], [1 << 20, 4 << 20]
    w = arena_abi.Arena.writer(path, tiers, priced, PACK, GEOM)
    r = arena_abi.Arena.reader(path, PACK, GEOM)
    body = np.random.default_rng(1).integers(0, 256, 3_000_001, dtype=np.uint8).tobytes()
    c = w.claim(0, 77, 5)
    assert c.index == 0 and c.tier == 0
    w.abort(c.index, c.nonce)
    assert w.slot(0).flags & arena_abi.FLAG_PARTIAL
    c = w.claim(1, 77, 5)
    assert c.tier == 1 and c.capacity == oracle_arena.size_arena(tiers, priced)["slot_bytes"][1]
    with pytest.raises(arena_abi.ArenaError) as e:
        w.claim(1, 77, 6)
    assert e.value.code == arena_abi.SC_EBUSY and "no free handoff slot" in str(e.value)
    w.write(c, 0, body[:1000])
    w.write(c, 1000, body[1000:])
    h = oracle_arena.sc_oracle.fnv1a64(body, oracle_arena.SEED)
    with pytest.raises(arena_abi.ArenaError):
        r.read_host(c.index, c.nonce, 77, len(body))     # CLAIMED, not READY
    w.publish(c, 99, len(body), h)
    got, s = r.read_host(c.index, c.nonce, 77, len(body))
    assert got.tobytes() == body and s.state == arena_abi.READY and s.payload_hash == h and s.tokens == 99
    with pytest.raises(arena_abi.ArenaError) as e:
        r.read_host(c.index, c.nonce, 78, len(body))
    assert "addressed to client" in str(e.value)
    with pytest.raises(arena_abi.ArenaError):
        r.read_host(c.index, c.nonce, 77, len(body) - 1)   # the buffer is too small
    # a byte changed in the file after publish fails the reader's hash check
    with open(path, "r+b") as f:
        f.seek(c.payload_off + 12345)
        f.write(bytes([body[12345] ^ 0xFF]))
    with pytest.raises(arena_abi.ArenaError) as e:
        r.read_host(c.index, c.nonce, 77, len(body))
    assert e.value.code == arena_abi.SC_ESTALE
    w.release(c.index, c.nonce)
    assert w.slot(c.index).state == arena_abi.FREE
    w.close()
    r.close()
