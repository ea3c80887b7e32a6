"""Hand-off payloads shipped with their carries (sc_wire_encoder_set_carry, sc_wire_decoder_set_carry).

An encoder told where to put them writes, beside the payload, the low byte of the running payload hash after every
64 KiB; a decoder given them checks the payload hash without the look-back across the payload.  Here: the carries are
the byte loop's low bytes at every 64 KiB boundary of the payload (contiguous, into segments, and through the gather
that a checked park uses); the hash is the one written without carries; mounting with them reproduces the source
slot byte for byte, contiguous and from segments; a flipped payload byte or a flipped carry is refused with nothing
mounted, the carry case saying so; and the intact payload then mounts.
"""
import numpy as np
import pytest

import sc_synthetic as synth
from test_gpu_wire import GEOKEY, GEOM_HASH, PACK_HASH, SMALL, _live

pytestmark = pytest.mark.gpu

GROUP = 64 << 10


@pytest.fixture(scope="module")
def wire():
    import sc_wire
    return sc_wire


def oracle_carries(oracle, data, seed):
    out, h = [], seed
    for k in range((len(data) - 1) // GROUP if len(data) else 0):
        h = oracle.fnv1a64(data[k * GROUP:(k + 1) * GROUP], h)
        out.append(h & 0xFF)
    return np.array(out, dtype=np.uint8)


def _source(sc, geo, tokens, seed):
    case = synth.SyntheticCase(geo, tokens, seed=seed)
    src = case.new_slot(max_cells=tokens + 16)
    case.carve_into(src)
    return src


def _same_slot(geo, tokens, src, dst):
    got, want = dst.host_state(), src.host_state()
    n = geo.cells(tokens) * geo.n_head_kv * geo.head_dim
    for j in range(geo.n_qsa):
        for name in (f"k{j}", f"v{j}"):
            if not np.array_equal(got[name].reshape(-1)[:n], want[name].reshape(-1)[:n]):
                return False
    return np.array_equal(got["gdn"], want["gdn"])


def test_encode_writes_carries_and_mount_checks_with_them(sc, oracle, wire, cuda):
    geo = sc.geometry(**SMALL)
    tokens = 333
    print(f"case wire carries {tokens} tokens", flush=True)
    src = _source(sc, geo, tokens, 0xC0)
    live, keep, ids = _live(wire, tokens)
    enc = wire.Encoder(geo, src, tokens, live, GEOM_HASH, PACK_HASH)
    n = enc.bytes
    nc = sc.carry_bytes(n)
    assert nc >= 8
    buf = sc.DeviceBuffer(n + 64, "uint8")
    carry = sc.DeviceBuffer(nc, "uint8")
    enc.encode(buf.ptr, n)
    h_plain = enc.hash()
    enc.set_carry(carry.ptr)
    carry.fill(0)
    enc.encode(buf.ptr, n)
    h = enc.hash()
    assert h == h_plain
    data = buf.numpy(n).copy()
    assert h == oracle.fnv1a64(data)
    want_carry = oracle_carries(oracle, data, sc.REFERENCE_FNV_SEED)
    assert np.array_equal(carry.numpy(nc), want_carry)
    # the gather-then-hash form (a checked park's) writes the same carries
    carry.fill(0)
    ev = sc.Event()
    enc.encode(buf.ptr, n, gathered=ev)
    assert enc.hash() == h and np.array_equal(carry.numpy(nc), want_carry)
    # mounted with them: the source slot, byte for byte
    dst = sc.new_slot(geo, tokens + 16, fill=0xAB)
    dec = wire.Decoder(buf.ptr, n, geo, dst, geometry=GEOKEY, geom_hash=GEOM_HASH, pack_hash=PACK_HASH,
                       check_identity=True, payload_hash=h, check_hash=True, carry=carry.ptr)
    dec.restore()
    assert _same_slot(geo, tokens, src, dst)
    assert np.array_equal(dec.live_ids(), ids)

    # refusals leave a slot untouched
    dst2 = sc.new_slot(geo, tokens + 16, fill=0xCD)
    before = {k: v.copy() for k, v in dst2.host_state().items()}

    def untouched():
        after = dst2.host_state()
        return all(np.array_equal(before[k], after[k]) for k in before)

    # a carry flipped: refused, and the message says the carries do not match
    bad = want_carry.copy()
    bad[nc // 2] ^= 0x10
    carry.upload(bad)
    with pytest.raises(wire.WireError) as e:
        wire.Decoder(buf.ptr, n, geo, dst2, payload_hash=h, check_hash=True, carry=carry.ptr).restore()
    assert e.value.code == sc.SC_EINVAL and "carries" in str(e.value)
    assert untouched()
    carry.upload(want_carry)
    # a payload byte flipped, with the carries of the intact payload: refused
    at = enc.pool_offset + 3 * GROUP + 5
    orig = buf.numpy(1, start=at)
    buf.upload(orig ^ 0x20, start=at)
    with pytest.raises(wire.WireError) as e:
        wire.Decoder(buf.ptr, n, geo, dst2, payload_hash=h, check_hash=True, carry=carry.ptr).restore()
    assert e.value.code == sc.SC_EINVAL
    assert untouched()
    buf.upload(orig, start=at)
    # the intact payload with its carries mounts
    wire.Decoder(buf.ptr, n, geo, dst2, payload_hash=h, check_hash=True, carry=carry.ptr).restore()
    assert _same_slot(geo, tokens, src, dst2)
    for b in (buf, carry):
        b.free()


def test_segments_with_carries(sc, oracle, wire, cuda):
    geo = sc.geometry(**SMALL)
    tokens = 301
    print(f"case wire carries in segments {tokens} tokens", flush=True)
    src = _source(sc, geo, tokens, 0xC1)
    live, keep, ids = _live(wire, tokens)
    enc = wire.Encoder(geo, src, tokens, live, GEOM_HASH, PACK_HASH)
    n = enc.bytes
    nc = sc.carry_bytes(n)
    seg = 3 * GROUP
    segs = [sc.DeviceBuffer(seg, "uint8") for _ in range((n + seg - 1) // seg)]
    ptrs = [s.ptr for s in segs]
    carry = sc.DeviceBuffer(nc, "uint8")
    enc.set_carry(carry.ptr)
    enc.encode_segments(ptrs, seg)
    h = enc.hash()
    data = np.concatenate([s.numpy(seg) for s in segs])[:n]
    assert h == oracle.fnv1a64(data)
    assert np.array_equal(carry.numpy(nc), oracle_carries(oracle, data, sc.REFERENCE_FNV_SEED))
    dst = sc.new_slot(geo, tokens + 16, fill=0x11)
    wire.Decoder(0, n, geo, dst, payload_hash=h, check_hash=True, segments=(ptrs, seg), carry=carry.ptr).restore()
    assert _same_slot(geo, tokens, src, dst)
    bad = carry.numpy(nc).copy()
    bad[0] ^= 1
    carry.upload(bad)
    dst2 = sc.new_slot(geo, tokens + 16, fill=0x22)
    before = dst2.host_state()
    with pytest.raises(wire.WireError) as e:
        wire.Decoder(0, n, geo, dst2, payload_hash=h, check_hash=True, segments=(ptrs, seg), carry=carry.ptr).restore()
    assert "carries" in str(e.value)
    after = dst2.host_state()
    assert all(np.array_equal(before[k], after[k]) for k in before)
    for b in segs + [carry]:
        b.free()
