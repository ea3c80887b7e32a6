"""Device hand-off payloads (include/sc_wire.h, libsc_core.so) against the codec oracle, bit for bit.

The oracle codec (oracle/sc_wire.py) is pinned to the reference codec's own payloads and verdicts
(tests/test_wire_oracle.py).  Here a payload written on the device straight from a decode slot must equal, byte for
byte, the oracle's encode of the same conversation (the slot's K/V prefix and GDN rows from the CPU carve oracle, plus
the host-side live checkpoint); its device hash must equal the byte loop's; mounting it into a fresh slot must
reproduce the slot and the host fields; and every refusal must leave the target slot untouched.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
GEOKEY = [2560, 8, 4, 32, 4, 8, 4, 520, 256, 24, 2, 256, 128, 4, 4, 3, 1, 0]
GEOM_HASH, PACK_HASH = 0x1122334455667788, 0x0AABBCCDDEEFF001
SMALL_BUFS = (bytes(range(40)), bytes(range(7, 19)), b"", bytes(range(200, 208)))
IMGS = [(4, 0xDEADBEEF), (12, 0xFEEDFACE12345678)]


@pytest.fixture(scope="module")
def wire():
    import sc_wire
    return sc_wire


@pytest.fixture(scope="module")
def codec():
    from oracle import sc_wire as codec
    return codec


def _live(wire, tokens, **kw):
    ids = (np.arange(tokens, dtype=np.int64) * 7919 % 151_000).astype(np.int32)
    args = dict(layer_lo=0, layer_hi=8, idx_dim=128, imgs=IMGS, used=tokens * 3, small=SMALL_BUFS)
    args.update(kw)
    live, keep = wire.make_live(GEOKEY, ids, **args)
    return live, keep, ids


def _expected_image(geo, state, tokens, ids, draft=True):
    cells = geo.cells(tokens)
    kvb = cells * geo.n_head_kv * geo.head_dim * 2
    kv = []
    for j in range(geo.n_qsa):
        kv.append({"format": 0, "cells": cells, "heads": geo.n_head_kv, "head_dim": geo.head_dim,
                   "page_size": geo.page_size, "pooled_rows": 0, "idx_dim": 128,
                   "k": state[f"k{j}"].tobytes()[:kvb], "v": state[f"v{j}"].tobytes()[:kvb],
                   "k_scale": b"", "v_scale": b"", "pooled": b""})
    if draft:
        kv.append({"format": 0, "cells": 0, "heads": 0, "head_dim": 0, "page_size": 0, "pooled_rows": 0, "idx_dim": 0,
                   "k": b"", "v": b"", "k_scale": b"", "v_scale": b"", "pooled": b""})
    live = {"ids": ids, "imgs": IMGS, "gdn": state["gdn"].tobytes() if "gdn" in state else b"",
            "ple": SMALL_BUFS[0], "tails": SMALL_BUFS[1], "dead": SMALL_BUFS[2], "block_pos": SMALL_BUFS[3],
            "used": tokens * 3, "stage_parts": []}
    return {"geometry": GEOKEY, "layer_lo": 0, "layer_hi": 8, "cvec": True, "kv": kv, "live": live,
            "checkpoints": [], "stage_parts": []}


def _encode(sc, wire, geo, slot, tokens, live):
    enc = wire.Encoder(geo, slot, tokens, live, GEOM_HASH, PACK_HASH)
    buf = sc.DeviceBuffer(enc.bytes + 64, "uint8")
    buf.fill(0x5A)   # the encode must define every byte of the payload
    enc.encode(buf.ptr, enc.bytes)
    return enc, buf, enc.hash()


@pytest.mark.parametrize("tokens", [77, 80, 1, 0])
def test_device_payload_equals_oracle_encode(sc, oracle, wire, codec, cuda, tokens):
    geo = sc.geometry(**SMALL)
    case = synth.SyntheticCase(geo, tokens, seed=0x5EED + tokens)
    slot = case.new_slot(max_cells=128)
    case.carve_into(slot)
    live, keep, ids = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, slot, tokens, live)
    payload = buf.numpy(enc.bytes).tobytes()
    state = oracle.expected_slot(geo, case.host_inputs(), slot_cells=128)
    want = codec.encode(_expected_image(geo, state, tokens, ids), GEOM_HASH, PACK_HASH)
    assert len(payload) == len(want)
    if payload != want:
        bad = next(i for i in range(len(want)) if payload[i] != want[i])
        raise AssertionError(f"payload differs from the oracle first at byte {bad} (pool at {enc.pool_offset})")
    assert h == codec.payload_hash(want)
    back = codec.decode(payload, GEOM_HASH, PACK_HASH, h, geometry=GEOKEY)
    assert back["live"]["used"] == tokens * 3


@pytest.mark.parametrize("table", ["reversed", "shuffled"])
def test_paged_slot_payload_equals_identity(sc, wire, cuda, table):
    """The capture reads through the page tables: a paged slot holding the same cells writes the same payload."""
    geo = sc.geometry(**SMALL)
    tokens = 77
    case = synth.SyntheticCase(geo, tokens, seed=99)
    flat = case.new_slot(max_cells=128)
    case.carve_into(flat)
    n_pages = 32
    t = np.arange(n_pages)[::-1].astype(np.int32) if table == "reversed" else \
        np.random.default_rng(5).permutation(n_pages).astype(np.int32)
    tables = sc.device_tables([t] * geo.n_qsa)
    paged = case.new_slot(max_cells=128, n_pages=n_pages, tables=tables)
    case.carve_into(paged)
    live, keep, ids = _live(wire, tokens)
    e1, b1, h1 = _encode(sc, wire, geo, flat, tokens, live)
    e2, b2, h2 = _encode(sc, wire, geo, paged, tokens, live)
    assert h1 == h2
    assert np.array_equal(b1.numpy(e1.bytes), b2.numpy(e2.bytes))


def test_mount_round_trip_and_host_fields(sc, oracle, wire, cuda):
    geo = sc.geometry(**SMALL)
    tokens = 77
    case = synth.SyntheticCase(geo, tokens, seed=7)
    src = case.new_slot(max_cells=128)
    case.carve_into(src)
    live, keep, ids = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, src, tokens, live)
    dst = sc.new_slot(geo, 128, fill=0xAB)
    dec = wire.Decoder(buf.ptr, enc.bytes, geo, dst, geometry=GEOKEY, geom_hash=GEOM_HASH, pack_hash=PACK_HASH,
                       check_identity=True, payload_hash=h, check_hash=True)
    assert dec.tokens == tokens
    dec.restore()
    got, want = dst.host_state(), src.host_state()
    cells = geo.cells(tokens)
    per_cell = geo.n_head_kv * geo.head_dim
    for j in range(geo.n_qsa):
        for name in (f"k{j}", f"v{j}"):
            w, g = want[name].reshape(-1), got[name].reshape(-1)
            assert np.array_equal(g[: cells * per_cell], w[: cells * per_cell]), name
            assert np.all(g[cells * per_cell:] == 0xABAB), f"{name}: cells past the image were written"
    assert np.array_equal(got["gdn"], want["gdn"])
    assert np.array_equal(dec.live_ids(), ids)
    for which, b in enumerate(SMALL_BUFS):
        assert dec.small(which) == b


def test_mount_into_paged_slot(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    tokens = 61
    case = synth.SyntheticCase(geo, tokens, seed=8)
    src = case.new_slot(max_cells=64)
    case.carve_into(src)
    live, keep, ids = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, src, tokens, live)
    n_pages = 24
    t = np.random.default_rng(11).permutation(n_pages).astype(np.int32)
    dst = sc.new_slot(geo, 64, n_pages=n_pages, tables=sc.device_tables([t] * geo.n_qsa), fill=0)
    dec = wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True)
    dec.restore()
    # read the paged slot back through its tables into a payload: it must be the same payload
    enc2, buf2, h2 = _encode(sc, wire, geo, dst, tokens, live)
    assert h2 == h


def test_refusals_leave_the_slot_untouched(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    tokens = 40
    case = synth.SyntheticCase(geo, tokens, seed=21)
    src = case.new_slot(max_cells=64)
    case.carve_into(src)
    live, keep, ids = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, src, tokens, live)
    dst = sc.new_slot(geo, 64, fill=0xCD)
    before = {k: v.copy() for k, v in dst.host_state().items()}

    def untouched():
        after = dst.host_state()
        return all(np.array_equal(before[k], after[k]) for k in before)

    # a flipped pool byte: the device hash refuses before the scatter
    pool_byte = enc.pool_offset + 1000
    orig = buf.numpy(1, start=pool_byte)
    buf.upload(orig ^ 0x40, start=pool_byte)
    dec = wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True)
    with pytest.raises(wire.WireError) as e:
        dec.restore()
    assert e.value.code == sc.SC_EINVAL and "hash" in str(e.value)
    assert untouched()
    buf.upload(orig, start=pool_byte)
    # head refusals at open: identity, geometry, a slot of another shape, a truncated buffer
    with pytest.raises(wire.WireError):
        wire.Decoder(buf.ptr, enc.bytes, geo, dst, geom_hash=1, pack_hash=PACK_HASH, check_identity=True)
    with pytest.raises(wire.WireError):
        wire.Decoder(buf.ptr, enc.bytes, geo, dst, geometry=[g + 1 for g in GEOKEY])
    other = sc.geometry(**dict(SMALL, head_dim=128))
    odst = sc.new_slot(other, 64, fill=0)
    with pytest.raises(wire.WireError):
        wire.Decoder(buf.ptr, enc.bytes, other, odst)
    with pytest.raises(wire.WireError):
        wire.Decoder(buf.ptr, enc.bytes - 64, geo, dst)
    # a corrupt header field (the payload_hash word must be zero)
    word = buf.numpy(8, start=240)
    buf.upload(np.frombuffer((1).to_bytes(8, "little"), np.uint8), start=240)
    with pytest.raises(wire.WireError):
        wire.Decoder(buf.ptr, enc.bytes, geo, dst)
    buf.upload(word, start=240)
    assert untouched()
    # and the intact payload still mounts
    wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True).restore()
    assert not untouched()


def test_encoder_refusals(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    slot = sc.new_slot(geo, 64, fill=0)
    live, keep, ids = _live(wire, 10)
    with pytest.raises(wire.WireError):
        wire.Encoder(geo, slot, 11, live)          # ids are not the token count
    with pytest.raises(wire.WireError):
        wire.Encoder(geo, slot, 10, live).encode(0, 1 << 20)   # no payload buffer
    enc = wire.Encoder(geo, slot, 10, live)
    small = sc.DeviceBuffer(enc.bytes - 64, "uint8")
    with pytest.raises(wire.WireError):
        enc.encode(small.ptr, enc.bytes - 64)


@pytest.mark.parametrize("tokens", [32768, 131072])
def test_full_depth_payload(sc, oracle, wire, cuda, tokens):
    """Configs 2 and 3: the device hash equals the byte loop over the payload read back, the pool equals the park image
    of the slot, and a mount into a fresh slot reproduces every pool byte (compared by device hash)."""
    geo = sc.geometry()
    case = synth.SyntheticCase(geo, tokens, seed=0x5EED)
    src = case.new_slot(max_cells=tokens)
    case.carve_into(src)
    del case
    live, keep, ids = _live(wire, tokens, layer_hi=48)
    enc, buf, h = _encode(sc, wire, geo, src, tokens, live)
    host = sc.PinnedBuffer(enc.bytes)
    sc.check(sc.lib.sc_copy_async(host.ptr, buf.ptr, enc.bytes, None), "copy")
    sc.device_sync()
    payload = host.numpy()
    assert h == oracle.fnv1a64(payload)
    # the pool's K/V + GDN entries are the park image's blobs at the same relative offsets
    _, total = sc.image_layout(geo, tokens)
    img = sc.DeviceBuffer(total, "uint8")
    cap = sc.plan_capture(geo, src, tokens, img.ptr, total)
    cap.launch()
    sc.device_sync()
    blobs, _ = sc.image_layout(geo, tokens)
    image = img.numpy()
    pool = enc.pool_offset
    kv_bytes = blobs[0].bytes
    for b in blobs:
        if b.kind in (sc.SC_BLOB_K, sc.SC_BLOB_V):
            at = pool + b.offset
            assert np.array_equal(payload[at:at + b.bytes], image[b.offset:b.offset + b.bytes]), (b.kind, b.layer)
    img.free()
    host.free()
    dst = sc.new_slot(geo, tokens, fill=0)
    wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True).restore()
    for a, b in zip(src.buffers(), dst.buffers()):
        assert sc.fnv1a64_device(a.ptr, a.nbytes) == sc.fnv1a64_device(b.ptr, b.nbytes)
    assert kv_bytes == geo.cells(tokens) * geo.n_head_kv * geo.head_dim * 2
