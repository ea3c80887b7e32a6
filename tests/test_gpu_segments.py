"""A hand-off payload held in segments (sc_segments: byte o at ptr[o // segment_bytes] + o % segment_bytes), written
and mounted where it lies, against the same payload written and mounted contiguously.

sc_wire_encode_segments_async writes the payload straight into segments (the same-GPU hand-off's exported ones) and
sc_wire_decoder_open_segments / _open_layers_segments mount it from them (the imported ones); no contiguous copy of the
payload exists on either side.  For an f16 slot through identity and shuffled page tables and for slots in f16, int8
and q4_0 with the indexer's rows, with 64 KiB and 192 KiB segments (so that the head, blobs and single pages straddle
segment boundaries at many offsets) and with one segment larger than the payload:
  - the segments' bytes, joined, equal the contiguous encode's, and the two hashes are equal (and the byte loop's);
  - the mount from the segments, hash checked on the device over the segments, leaves the slot byte for byte as the
    mount of the contiguous payload does;
  - a wrong expected hash refuses and leaves the slot untouched;
  - with every page table in destination order, the first piece of each blob cut at a segment end is ordered and the
    later pieces keep the source order at their chunk offset, and the mount still equals the contiguous one;
  - at config 2's full depth (884 MB in 64 MiB segments) the segments equal the contiguous payload and the mount from
    them reproduces the source slot.
The contiguous path is itself held to the oracle by tests/test_gpu_wire.py and tests/test_gpu_wire_layers.py.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
GEOKEY = [2560, 8, 4, 32, 4, 8, 4, 520, 256, 24, 2, 256, 128, 4, 4, 3, 1, 0]
PACK, GEOM = 0x0123456789ABCDEF, 0x1F2E3D4C5B6A7988
SEED = 1469598103934665603
SEGS = [65536, 3 * 65536, 64 << 20]   # the last: one segment larger than the payload


def _segments(sc, n, seg, fill):
    bufs = [sc.DeviceBuffer(min(seg, n - o), "uint8") for o in range(0, n, seg)]
    for b in bufs:
        b.fill(fill)
    return bufs


def _joined(bufs):
    return np.concatenate([b.numpy() for b in bufs])


def _encode_both(sc, oracle, wire, enc, seg):
    n = enc.bytes
    buf = sc.DeviceBuffer(n, "uint8")
    enc.encode(buf.ptr, n)
    h = enc.hash()
    want = buf.numpy(n).copy()
    assert h == oracle.fnv1a64(want, SEED)
    segs = _segments(sc, n, seg, 0xCD)
    assert len(segs) >= 4 or seg > n
    enc.encode_segments([b.ptr for b in segs], seg)
    assert enc.hash() == h
    got = _joined(segs)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]
    return buf, segs, h


def _tables(sc, geo, n_pages, per, seed):
    tabs = [np.random.default_rng(seed + j).permutation(n_pages)[:per].astype(np.int32) for j in range(geo.n_qsa)]
    return sc.device_tables(tabs)


@pytest.fixture
def order_all(sc, request):
    """With request.param, every page table gets the destination order, however few pages it covers: the first piece
    of a blob cut at a segment end is then ordered and the later pieces keep the source order."""
    prev = sc.set_order_min_pages(1) if request.param else None
    yield request.param
    if prev is not None:
        sc.set_order_min_pages(prev)


@pytest.mark.parametrize("order_all", [False, True], indirect=True, ids=["default_order", "ordered"])
@pytest.mark.parametrize("seg", SEGS)
@pytest.mark.parametrize("table", ["identity", "shuffled"])
def test_f16_slot_through_segments(sc, oracle, cuda, seg, table, order_all):
    import sc_wire as wire
    geo = sc.geometry(**SMALL)
    tokens, max_cells = 301, 320
    print(f"case segments f16 {table} seg {seg} ordered {order_all}", flush=True)
    case = synth.SyntheticCase(geo, tokens, seed=0x5E6 + seg // 65536)
    n_pages = max_cells // geo.page_size + 5
    per = max_cells // geo.page_size

    def slot(seed, fill):
        if table == "identity":
            return case.new_slot(max_cells=max_cells, fill=fill)
        return case.new_slot(max_cells=max_cells, n_pages=n_pages, tables=_tables(sc, geo, n_pages, per, seed),
                             fill=fill)

    src = slot(1, 0x33)
    case.carve_into(src)
    ids = (np.arange(tokens, dtype=np.int64) * 7919 % 151_000).astype(np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128)
    enc = wire.Encoder(geo, src, tokens, live, GEOM, PACK)
    buf, segs, h = _encode_both(sc, oracle, wire, enc, seg)
    n = enc.bytes
    ptrs = [b.ptr for b in segs]
    da, db = slot(2, 0x6B), slot(2, 0x6B)          # the same tables: a destination order unlike the source's
    wire.Decoder(buf.ptr, n, geo, da, payload_hash=h, check_hash=True).restore()
    with pytest.raises(wire.WireError):
        wire.Decoder(0, n, geo, db, payload_hash=h ^ 1, check_hash=True, segments=(ptrs, seg)).restore()
    assert all(np.all(v.view(np.uint8) == 0x6B) for v in db.host_state().values())
    dec = wire.Decoder(0, n, geo, db, payload_hash=h, check_hash=True, segments=(ptrs, seg))
    assert dec.tokens == tokens
    dec.restore()
    assert np.array_equal(dec.live_ids(), ids)
    a, b = da.host_state(), db.host_state()
    for key in a:
        assert np.array_equal(a[key].view(np.uint8), b[key].view(np.uint8)), key
    enc.destroy()


@pytest.mark.parametrize("seg", SEGS)
@pytest.mark.parametrize("fmt", [0, 1, 3])
def test_layer_slot_through_segments(sc, oracle, cuda, seg, fmt):
    import sc_wire as wire
    geo = sc.geometry(**SMALL)
    tokens = 517
    cap = (tokens + 3) // 4 * 4 + 16
    print(f"case segments format {fmt} seg {seg}", flush=True)
    src = sc.LayerPools(geo, fmt, cap, True)
    src.randomize(0xA11 + fmt)
    ids = (np.arange(tokens, dtype=np.int64) * 31 % 151_000).astype(np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128, imgs=[(5, 77)], used=tokens,
                                small=(b"ple", b"tails", b"", b"bp"))
    enc = wire.Encoder(geo, src, tokens, live, GEOM, PACK)
    buf, segs, h = _encode_both(sc, oracle, wire, enc, seg)
    n = enc.bytes
    ptrs = [b.ptr for b in segs]
    da, db = sc.LayerPools(geo, fmt, cap, True), sc.LayerPools(geo, fmt, cap, True)
    da.fill(0x99)
    db.fill(0x99)
    wire.Decoder(buf.ptr, n, geo, da, payload_hash=h, check_hash=True).restore()
    with pytest.raises(wire.WireError):
        wire.Decoder(0, n, geo, db, payload_hash=h ^ 1, check_hash=True, segments=(ptrs, seg)).restore()
    assert all((v == 0x99).all() for v in db.host().values())
    dec = wire.Decoder(0, n, geo, db, geom_hash=GEOM, pack_hash=PACK, check_identity=True, payload_hash=h,
                       check_hash=True, segments=(ptrs, seg))
    dec.restore()
    assert dec.small(0) == b"ple" and dec.small(1) == b"tails" and dec.small(3) == b"bp"
    a, b = da.host(), db.host()
    for key in a:
        assert np.array_equal(a[key], b[key]), key
    enc.destroy()


def test_segment_refusals(sc, cuda):
    import sc_wire as wire
    geo = sc.geometry(**SMALL)
    tokens = 301
    pools = sc.LayerPools(geo, 1, 320, True)
    pools.randomize(3)
    ids = np.zeros(tokens, dtype=np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128)
    enc = wire.Encoder(geo, pools, tokens, live, GEOM, PACK)
    n = enc.bytes
    seg = 65536
    segs = _segments(sc, n, seg, 0)
    ptrs = [b.ptr for b in segs]
    with pytest.raises(wire.WireError):
        enc.encode_segments(ptrs[:-1], seg)                    # the segments do not cover the payload
    with pytest.raises(wire.WireError):
        enc.encode_segments(ptrs, seg + 4096)                  # not a whole multiple of 64 KiB
    with pytest.raises(wire.WireError):
        enc.encode_segments([ptrs[0] + 8] + ptrs[1:], seg)     # a segment that is not 16-byte aligned
    big = sc.DeviceBuffer(65 * seg, "uint8")
    with pytest.raises(wire.WireError):                        # more than SC_IPC_MAX_SEGMENTS segments
        enc.encode_segments([big.ptr + k * seg for k in range(65)], seg)
    enc.encode_segments(ptrs, seg)
    h = enc.hash()
    dst = sc.LayerPools(geo, 1, 320, True)
    with pytest.raises(wire.WireError):
        wire.Decoder(0, n, geo, dst, payload_hash=h, check_hash=True, segments=(ptrs[:-1], seg))
    with pytest.raises(wire.WireError):
        wire.Decoder(0, n, geo, dst, payload_hash=h, check_hash=True, segments=(ptrs, seg + 4096))
    enc.destroy()


def test_full_depth_through_segments(sc, oracle, cuda):
    """Config 2 (48 layers, 32K tokens): the 884 MB payload encoded into 64 MiB segments equals the contiguous encode
    byte for byte with the same hash, and its mount from the segments reproduces every buffer of the source slot."""
    import sc_wire as wire
    geo = sc.geometry()
    tokens = 32768
    print(f"case full-depth segments {tokens} tokens", flush=True)
    case = synth.SyntheticCase(geo, tokens, seed=0x5E9)
    src = case.new_slot(max_cells=tokens)
    case.carve_into(src)
    del case
    ids = (np.arange(tokens, dtype=np.int64) % 151_000).astype(np.int32)
    geokey = [2560, 48, 4, 128, 16, 32, 4, 8192, 4096, 24, 2, 256, 128, 4, 4, 3, 1, 0]
    live, keep = wire.make_live(geokey, ids, layer_hi=48, idx_dim=128)
    enc = wire.Encoder(geo, src, tokens, live, GEOM, PACK)
    n, seg = enc.bytes, 64 << 20
    buf = sc.DeviceBuffer(n, "uint8")
    enc.encode(buf.ptr, n)
    h = enc.hash()
    segs = _segments(sc, n, seg, 0xCD)
    assert len(segs) >= 13
    enc.encode_segments([b.ptr for b in segs], seg)
    assert enc.hash() == h
    assert sc.fnv1a64_device(buf.ptr, n) == h
    want = buf.numpy(n)
    at = 0
    for b in segs:
        got = b.numpy()
        assert np.array_equal(got, want[at:at + b.nbytes]), at
        at += b.nbytes
    del want
    buf.free()
    dst = sc.new_slot(geo, tokens, fill=0)
    wire.Decoder(0, n, geo, dst, payload_hash=h, check_hash=True, segments=([b.ptr for b in segs], seg)).restore()
    for a, b in zip(src.buffers(), dst.buffers()):
        assert sc.fnv1a64_device(a.ptr, a.nbytes) == sc.fnv1a64_device(b.ptr, b.nbytes)
    enc.destroy()
