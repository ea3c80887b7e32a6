"""Hand-off payloads between HBM and the arena (sc_mover_*, strata/core/handoff_device.hpp) on the GPU.

The device writer's slot must read back through the reference's own reader path: HandoffArena::read_slot plus the
byte-serial payload_hash_of (sc_arena_read_host here, and oracle/_ref/ref_arena - the reference's handoff.cpp - where
that build travelled with the tree).  The device reader must restore exactly the slot's bytes, verify the hash on the
device, and refuse before writing device memory when the slot does not qualify.  End to end: a slot's payload written
on the device, handed through the arena, read into another device buffer and mounted into fresh pools with the
payload hash checked.
"""
import os
import random
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
REF = ROOT / "oracle" / "_ref" / "ref_arena"
PACK, GEOM = 0x0123456789ABCDEF, 0x1F2E3D4C5B6A7988
TIERS = [(1024, 2), (131072, 2)]
PRICED = [8 << 20, 160 << 20]
SEED = 1469598103934665603


@pytest.fixture(scope="module")
def ar():
    import sc_arena
    return sc_arena


@pytest.fixture(scope="module")
def mover(ar, cuda):
    m = ar.Mover(chunk_bytes=8 << 20, depth=3, threads=4)
    yield m
    m.destroy()


@pytest.fixture
def shm():
    """A fresh directory on /dev/shm when it has room for these arenas (1 GiB), else under the temp directory."""
    st = os.statvfs("/dev/shm") if os.path.isdir("/dev/shm") else None
    base = "/dev/shm" if st and st.f_bavail * st.f_frsize > (1 << 30) else os.environ.get("TMPDIR", "/tmp")
    d = Path(base) / f"sc-arena-gpu-{os.getpid()}-{random.randrange(1 << 30)}"
    d.mkdir(parents=True)
    yield d
    shutil.rmtree(d, ignore_errors=True)


def ref_pattern(n, seed):
    i = np.arange(n, dtype=np.uint64)
    return ((i * 131 + seed * 17 + (i >> 9)) & 0xFF).astype(np.uint8)


def device_bytes(sc, data: np.ndarray):
    buf = sc.DeviceBuffer(max(len(data), 1), "uint8")
    buf.upload(data)
    return buf


@pytest.mark.parametrize("nbytes", [0, 1, 4097, 8 << 20, (24 << 20) + 5, 150_000_013])
def test_device_write_reads_back_through_the_host_reader(sc, oracle, ar, mover, shm, nbytes):
    print(f"case device write {nbytes} B", flush=True)
    data = np.random.default_rng(nbytes).integers(0, 256, nbytes, dtype=np.uint8)
    src = device_bytes(sc, data)
    w = ar.Arena.writer(shm / "a" / "arena", TIERS, PRICED, PACK, GEOM)
    r = ar.Arena.reader(shm / "a" / "arena", PACK, GEOM)
    c = w.claim(0 if nbytes < (8 << 20) else 1, 42, 7)
    h = mover.write(w, c, src.ptr, nbytes)
    assert h == oracle.fnv1a64(data.tobytes(), SEED)          # the device hash of the payload
    assert w.slot(c.index).state == ar.CLAIMED                 # writing does not publish
    w.publish(c, 1234, nbytes, h)
    got, s = r.read_host(c.index, c.nonce, 42, nbytes, check_hash=True)
    assert got.tobytes() == data.tobytes() and s.payload_hash == h and s.tokens == 1234
    # and the device reader restores it, verified on the device
    dst = sc.DeviceBuffer(nbytes + 64, "uint8")
    dst.fill(0xAB)
    s2 = mover.read(r, c.index, c.nonce, 42, dst.ptr, nbytes + 64, verify=True)
    back = dst.numpy()
    assert back[:nbytes].tobytes() == data.tobytes() and (back[nbytes:] == 0xAB).all()
    assert s2.payload_bytes == nbytes and s2.nonce == c.nonce
    w.release(c.index, c.nonce)
    w.close()
    r.close()


def test_publish_from_device_and_reserve(sc, oracle, ar, mover, shm):
    data = np.random.default_rng(3).integers(0, 256, 50_000_000, dtype=np.uint8)
    src = device_bytes(sc, data)
    w = ar.Arena.writer(shm / "b" / "arena", TIERS, PRICED, PACK, GEOM, reserve=True)
    r = ar.Arena.reader(shm / "b" / "arena", PACK, GEOM)
    for rep in range(3):    # the same slot again and again (pages and page tables already in place)
        c = w.claim(1, 5, rep)
        mover.publish(w, c, src.ptr, data.size, 777 + rep)
        s = w.slot(c.index)
        assert s.state == ar.READY and s.payload_hash == oracle.fnv1a64(data.tobytes(), SEED) and s.tokens == 777 + rep
        got, _ = r.read_host(c.index, c.nonce, 5, data.size)
        assert got.tobytes() == data.tobytes()
        w.release(c.index, c.nonce)


@pytest.mark.skipif(not REF.exists(), reason="the reference arena build (oracle/_ref) did not travel with the tree")
@pytest.mark.parametrize("nbytes", [1, 5_000_003])
def test_reference_reader_reads_a_device_publish(sc, ar, mover, shm, nbytes):
    data = ref_pattern(nbytes, 9)
    src = device_bytes(sc, data)
    path = shm / "c" / "arena"
    w = ar.Arena.writer(path, [(1024, 2), (4096, 1), (16384, 2)], [1048576, 2097152, 4194309], PACK, GEOM)
    c = w.claim(2, 4242, 77)
    mover.publish(w, c, src.ptr, nbytes, 1234)
    out = subprocess.run([str(REF), "read", str(path), f"{PACK:016x}", f"{GEOM:016x}", str(c.index), f"{c.nonce:016x}",
                          "4242", "9"], capture_output=True, text=True, timeout=120).stdout
    words = dict(x.split("=", 1) for x in out.split() if "=" in x)
    assert words.get("ok") == "1" and words["pattern"] == "1" and words["hash"] == words["recorded"], out
    assert int(words["bytes"]) == nbytes and int(words["request"]) == 77


@pytest.mark.skipif(not REF.exists(), reason="the reference arena build (oracle/_ref) did not travel with the tree")
def test_device_reader_reads_a_reference_publish(sc, ar, mover, shm):
    path = shm / "d" / "arena"
    nbytes = 3_000_017
    out = subprocess.run([str(REF), "write", str(path), f"{PACK:016x}", f"{GEOM:016x}", "1024:2,4096:1,16384:2",
                          "1048576,2097152,4194309", "1", "31", "32", str(nbytes), "5", "999", "0"],
                         capture_output=True, text=True, timeout=120).stdout
    claim = dict(x.split("=", 1) for x in out.splitlines()[1].split() if "=" in x)
    assert claim["ok"] == "1", out
    r = ar.Arena.reader(path, PACK, GEOM)
    dst = sc.DeviceBuffer(nbytes, "uint8")
    s = mover.read(r, int(claim["slot"]), int(claim["nonce"], 16), 31, dst.ptr, nbytes, verify=True)
    assert s.tokens == 999 and s.request_id == 32
    assert dst.numpy().tobytes() == ref_pattern(nbytes, 5).tobytes()


def test_refusals_leave_device_memory_alone(sc, ar, mover, shm):
    data = np.random.default_rng(9).integers(0, 256, 1 << 20, dtype=np.uint8)
    src = device_bytes(sc, data)
    path = shm / "e" / "arena"
    w = ar.Arena.writer(path, TIERS, PRICED, PACK, GEOM)
    r = ar.Arena.reader(path, PACK, GEOM)
    c = w.claim(0, 8, 8)
    dst = sc.DeviceBuffer(2 << 20, "uint8")
    dst.fill(0x3C)

    def refused(index, nonce, client, capacity, code=None, word=None):
        with pytest.raises(ar.ArenaError) as e:
            mover.read(r, index, nonce, client, dst.ptr, capacity)
        assert (dst.numpy() == 0x3C).all(), "a refused read wrote device memory"
        if code is not None:
            assert e.value.code == code
        if word:
            assert word in str(e.value), str(e.value)

    mover.write(w, c, src.ptr, data.size)
    refused(c.index, c.nonce, 8, 2 << 20, sc.SC_EINVAL, "CLAIMED")           # written, not published
    w.publish(c, 1, data.size, mover.write(w, c, src.ptr, data.size))
    refused(c.index, c.nonce ^ 1, 8, 2 << 20, sc.SC_EINVAL, "nonce")
    refused(c.index, c.nonce, 9, 2 << 20, sc.SC_EINVAL, "addressed to client")
    refused(c.index, c.nonce, 8, data.size - 1, sc.SC_EINVAL, "room for")
    refused(c.index + 1, c.nonce, 8, 2 << 20, sc.SC_EINVAL, "FREE")
    with pytest.raises(ar.ArenaError):
        mover.write(r, c, src.ptr, data.size)                                  # a reader never writes
    big = w.claim(0, 8, 9)
    with pytest.raises(ar.ArenaError) as e:
        mover.write(w, big, src.ptr, big.capacity + 1)                         # past the slot
    assert "holds" in str(e.value)
    # a byte changed in the slot after publish: copied, then refused by the device hash (SC_ESTALE)
    with open(path, "r+b") as f:
        f.seek(c.payload_off + 777)
        f.write(bytes([data[777] ^ 1]))
    with pytest.raises(ar.ArenaError) as e:
        mover.read(r, c.index, c.nonce, 8, dst.ptr, 2 << 20, verify=True)
    assert e.value.code == ar.SC_ESTALE and "payload hash" in str(e.value)
    # without verification the same bytes arrive as they are in the file
    mover.read(r, c.index, c.nonce, 8, dst.ptr, 2 << 20, verify=False)
    got = dst.numpy(data.size)
    assert got[777] == data[777] ^ 1 and np.array_equal(np.delete(got, 777), np.delete(data, 777))


def test_verified_read_refuses_a_change_in_a_later_chunk(sc, oracle, ar, mover, shm):
    """The device reader hashes each 8 MiB chunk as it lands (the running hash chained on the device): a byte changed
    in the slot's third chunk or in its last byte is caught, and the unchanged payload passes."""
    nbytes = (20 << 20) + 3
    data = np.random.default_rng(21).integers(0, 256, nbytes, dtype=np.uint8)
    src = device_bytes(sc, data)
    path = shm / "g" / "arena"
    w = ar.Arena.writer(path, TIERS, PRICED, PACK, GEOM)
    r = ar.Arena.reader(path, PACK, GEOM)
    c = w.claim(1, 8, 1)
    mover.publish(w, c, src.ptr, nbytes, 5)
    dst = sc.DeviceBuffer(nbytes, "uint8")
    s = mover.read(r, c.index, c.nonce, 8, dst.ptr, nbytes, verify=True)
    assert s.payload_hash == oracle.fnv1a64(data.tobytes(), SEED)
    assert dst.numpy().tobytes() == data.tobytes()
    for at in ((16 << 20) + 12345, nbytes - 1):
        print(f"case tampered byte {at}", flush=True)
        with open(path, "r+b") as f:
            f.seek(c.payload_off + at)
            f.write(bytes([data[at] ^ 0x80]))
        with pytest.raises(ar.ArenaError) as e:
            mover.read(r, c.index, c.nonce, 8, dst.ptr, nbytes, verify=True)
        assert e.value.code == ar.SC_ESTALE and "payload hash" in str(e.value)
        with open(path, "r+b") as f:
            f.seek(c.payload_off + at)
            f.write(bytes([data[at]]))
    mover.read(r, c.index, c.nonce, 8, dst.ptr, nbytes, verify=True)   # restored: accepted again
    w.close()
    r.close()


SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
GEOKEY = [2560, 8, 4, 32, 4, 8, 4, 520, 256, 24, 2, 256, 128, 4, 4, 3, 1, 0]


@pytest.mark.parametrize("fmt", [0, 1, 3])
def test_slot_to_arena_to_slot(sc, ar, mover, shm, fmt):
    """Prefill side: a slot's payload encoded on the device and published through the arena.  Decode side: the slot
    read into device memory and mounted into fresh pools with the payload hash checked."""
    import sc_wire as wire
    geo = sc.geometry(**SMALL)
    tokens = 333
    pools = sc.LayerPools(geo, fmt, 352, True)
    pools.randomize(0xA11CE + fmt)
    ids = (np.arange(tokens, dtype=np.int64) * 7919 % 151_000).astype(np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128, imgs=[(3, 0xFEED)], used=tokens,
                                small=(b"ple!", b"", b"dead", bytes(range(16))))
    enc = wire.Encoder(geo, pools, tokens, live, GEOM, PACK)
    payload = sc.DeviceBuffer(enc.bytes, "uint8")
    enc.encode(payload.ptr, enc.bytes)
    h = enc.hash()
    path = shm / "f" / "arena"
    w = ar.Arena.writer(path, TIERS, [enc.bytes, 160 << 20], PACK, GEOM)
    c = w.claim(0, 0xDEC0DE, 11)
    assert mover.write(w, c, payload.ptr, enc.bytes) == h     # the mover's device hash is the encoder's
    w.publish(c, tokens, enc.bytes, h)
    r = ar.Arena.reader(path, PACK, GEOM)
    arrived = sc.DeviceBuffer(c.capacity, "uint8")
    s = mover.read(r, c.index, c.nonce, 0xDEC0DE, arrived.ptr, c.capacity, verify=False)
    dst = sc.LayerPools(geo, fmt, 352, True)
    dst.fill(0x5A)
    dec = wire.Decoder(arrived.ptr, s.payload_bytes, geo, dst, geometry=GEOKEY, geom_hash=GEOM, pack_hash=PACK,
                       check_identity=True, payload_hash=s.payload_hash, check_hash=True)
    assert dec.tokens == tokens
    dec.restore()
    a, b = pools.host(), dst.host()
    sizes = sc.layer_blob_bytes(geo, fmt, True, tokens)
    for key in a:
        if key == "gdn":
            assert np.array_equal(a[key], b[key])
        else:
            n = sizes[key[0]]
            assert np.array_equal(a[key][:n], b[key][:n]) and (b[key][n:] == 0x5A).all(), key
    assert np.array_equal(dec.live_ids(), ids) and dec.small(0) == b"ple!" and dec.small(3) == bytes(range(16))
    w.release(c.index, c.nonce)


def test_publish_overlapping_the_encoder_hash(sc, oracle, ar, mover, shm):
    """The writer's fast order: the mover's D2H on a second stream waits only for the encoder's gather (its
    `gathered` event), the encoder's FNV-1a runs beside the copy, the mover does not hash, and the arena publishes the
    encoder's hash.  The slot must hold exactly the payload and pass the device reader's chunk-by-chunk check."""
    import sc_wire as wire
    geo = sc.geometry(**SMALL)
    tokens = 1501
    pools = sc.LayerPools(geo, 1, 1520, True)
    pools.randomize(0xBEE)
    ids = (np.arange(tokens, dtype=np.int64) * 31 % 151_000).astype(np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128, used=tokens)
    enc = wire.Encoder(geo, pools, tokens, live, GEOM, PACK)
    payload = sc.DeviceBuffer(enc.bytes, "uint8")
    payload.fill(0x77)
    path = shm / "h" / "arena"
    w = ar.Arena.writer(path, TIERS, [enc.bytes, 160 << 20], PACK, GEOM)
    r = ar.Arena.reader(path, PACK, GEOM)
    stream, side, gathered = sc.Stream(), sc.Stream(), sc.Event()
    c = w.claim(0, 5, 1)
    enc.encode(payload.ptr, enc.bytes, stream, gathered=gathered)
    side.wait(gathered)
    assert mover.write(w, c, payload.ptr, enc.bytes, side.handle, want_hash=False) is None
    h = enc.hash()
    w.publish(c, tokens, enc.bytes, h)
    got, s = r.read_host(c.index, c.nonce, 5, enc.bytes, check_hash=True)
    stream.sync()
    assert got.tobytes() == payload.numpy().tobytes() and s.payload_hash == h == oracle.fnv1a64(got.tobytes())
    arrived = sc.DeviceBuffer(enc.bytes, "uint8")
    mover.read(r, c.index, c.nonce, 5, arrived.ptr, enc.bytes, verify=True)
    assert arrived.numpy().tobytes() == got.tobytes()
    w.release(c.index, c.nonce)
    w.close()
    r.close()
