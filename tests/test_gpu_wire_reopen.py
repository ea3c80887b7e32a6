"""A wire decoder opened again for the next payload (sc_wire_decoder_reopen): same slot, next payload.

A serving engine holds one decoder per slot and re-opens it per hand-off, keeping its buffers and - when the payload's
place, the slot and the blob offsets are unchanged - its scatter plan.  Here every mount after a re-open must be the
mount a fresh decoder makes: the next payload of another conversation of the same length in the same buffer (the plan
kept), one of another length (the plan rebuilt), the same from segments, a slot in int8 with the indexer's rows, a
wrong hash refused with the slot untouched and the decoder usable afterwards, a refused re-open (corrupted head) after
which a restore is refused with the slot untouched, and the refusals of the call itself.
"""
import numpy as np
import pytest

import sc_synthetic as synth
from test_gpu_wire import GEOM_HASH, PACK_HASH, SMALL, _live

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def wire():
    import sc_wire
    return sc_wire


def _slot_equal(geo, tokens, src, dst):
    got, want = dst.host_state(), src.host_state()
    n = geo.cells(tokens) * geo.n_head_kv * geo.head_dim
    for j in range(geo.n_qsa):
        for name in (f"k{j}", f"v{j}"):
            if not np.array_equal(got[name].reshape(-1)[:n], want[name].reshape(-1)[:n]):
                return False
    return np.array_equal(got["gdn"], want["gdn"])


def _source(geo, tokens, seed, cells):
    case = synth.SyntheticCase(geo, tokens, seed=seed)
    src = case.new_slot(max_cells=cells)
    case.carve_into(src)
    return src


def test_reopen_contiguous(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    cells = 320
    print("case reopen contiguous", flush=True)
    buf = sc.DeviceBuffer(8 << 20, "uint8")
    dst = sc.new_slot(geo, cells, fill=0)
    dec = None
    for i, tokens in enumerate((200, 200, 200, 57, 57, 301)):
        src = _source(geo, tokens, 0x50 + i, cells)
        live, keep, ids = _live(wire, tokens)
        enc = wire.Encoder(geo, src, tokens, live, GEOM_HASH, PACK_HASH)
        n = enc.bytes
        enc.encode(buf.ptr, n)
        h = enc.hash()
        if dec is None:
            dec = wire.Decoder(buf.ptr, n, geo, dst, payload_hash=h, check_hash=True)
        else:
            dec.reopen(buf.ptr, n, h)
        assert dec.tokens == tokens
        dec.restore()
        assert _slot_equal(geo, tokens, src, dst), (i, tokens)
        assert np.array_equal(dec.live_ids(), ids)
        enc.destroy()
    # a wrong expected hash: refused with the slot untouched, and the decoder opens again afterwards
    before = dst.host_state()
    dec.reopen(buf.ptr, n, h ^ 1)
    with pytest.raises(wire.WireError):
        dec.restore()
    after = dst.host_state()
    assert all(np.array_equal(before[k], after[k]) for k in before)
    dec.reopen(buf.ptr, n, h)
    dec.restore()
    # a refused re-open (a corrupted head) leaves nothing to restore: the restore is refused with the slot untouched,
    # though the decoder keeps its scatter plan for the next open, which then mounts
    magic = buf.numpy(1, start=0)
    buf.upload(magic ^ 0xFF, start=0)
    with pytest.raises(wire.WireError):
        dec.reopen(buf.ptr, n, h)
    before = dst.host_state()
    with pytest.raises(wire.WireError):
        dec.restore()
    after = dst.host_state()
    assert all(np.array_equal(before[k], after[k]) for k in before)
    buf.upload(magic, start=0)
    dec.reopen(buf.ptr, n, h)
    dec.restore()
    assert _slot_equal(geo, tokens, src, dst)
    # the call's own refusals: a contiguous decoder needs a payload
    with pytest.raises(wire.WireError):
        dec.reopen(None, n, h)
    dec.destroy()
    buf.free()


def test_reopen_segments_and_carries(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    cells, tokens = 320, 250
    print("case reopen segments", flush=True)
    seg = 4 << 16
    segs = [sc.DeviceBuffer(seg, "uint8") for _ in range(24)]
    ptrs = [s.ptr for s in segs]
    dst = sc.new_slot(geo, cells, fill=0)
    carry = sc.DeviceBuffer(1024, "uint8")
    dec = None
    for i in range(3):
        src = _source(geo, tokens, 0x70 + i, cells)
        live, keep, ids = _live(wire, tokens)
        enc = wire.Encoder(geo, src, tokens, live, GEOM_HASH, PACK_HASH)
        n = enc.bytes
        assert sc.carry_bytes(n) <= 1024
        enc.set_carry(carry.ptr)
        enc.encode_segments(ptrs, seg)
        h = enc.hash()
        if dec is None:
            dec = wire.Decoder(0, n, geo, dst, payload_hash=h, check_hash=True, segments=(ptrs, seg), carry=carry.ptr)
        else:
            dec.reopen(None, n, h, carry=carry.ptr)
        dec.restore()
        assert _slot_equal(geo, tokens, src, dst), i
        enc.destroy()
    with pytest.raises(wire.WireError):   # a segmented decoder takes its payload from its segments
        dec.reopen(ptrs[0], n, h)
    dec.destroy()
    for b in segs + [carry]:
        b.free()


def test_reopen_int8_with_index(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    print("case reopen int8 layers", flush=True)
    cells = 256
    buf = sc.DeviceBuffer(8 << 20, "uint8")
    dst = sc.LayerPools(geo, sc.SC_KV_INT8, cells, True)
    dst.fill(0)
    dec = None
    for i, tokens in enumerate((190, 190, 33)):
        src = sc.LayerPools(geo, sc.SC_KV_INT8, cells, True)
        src.randomize(0x90 + i)
        live, keep, ids = _live(wire, tokens)
        enc = wire.Encoder(geo, src, tokens, live, GEOM_HASH, PACK_HASH)
        n = enc.bytes
        enc.encode(buf.ptr, n)
        h = enc.hash()
        if dec is None:
            dec = wire.Decoder(buf.ptr, n, geo, dst, payload_hash=h, check_hash=True)
        else:
            dec.reopen(buf.ptr, n, h)
        dec.restore()
        # the mounted slot writes the same payload back
        enc2 = wire.Encoder(geo, dst, tokens, live, GEOM_HASH, PACK_HASH)
        other = sc.DeviceBuffer(n, "uint8")
        enc2.encode(other.ptr, n)
        assert enc2.hash() == h, i
        enc2.destroy()
        enc.destroy()
        other.free()
    dec.destroy()
    buf.free()
