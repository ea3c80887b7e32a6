"""Device hand-off payloads of slots in every K/V format (sc_wire_encoder_create_layers / sc_wire_decoder_open_layers).

A payload written on the device from an int8, q4_0, K8V4 or f16 slot - with or without the indexer's pooled rows -
must equal, byte for byte, the oracle codec's encode of the same conversation (K/V records of the slot's format whose
buffers are the slot's blob prefixes; the oracle codec is pinned to the reference codec's own payloads, including
records with scales and indexer rows).  Mounting it restores exactly those prefixes and the host fields; a payload
whose records are not the slot's format is refused with the slot untouched.
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
IMGS = [(4, 0xDEADBEEF)]


@pytest.fixture(scope="module")
def wire():
    import sc_wire
    return sc_wire


@pytest.fixture(scope="module")
def codec():
    from oracle import sc_wire as codec
    return codec


def _live(wire, tokens):
    ids = (np.arange(tokens, dtype=np.int64) * 104729 % 151_000).astype(np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128, imgs=IMGS, used=tokens + 1,
                                small=SMALL_BUFS)
    return live, keep, ids


def _expected_image(oracle, geo, pools, fmt, index, tokens, ids):
    sizes = oracle.layer_blob_bytes(geo, fmt, index, tokens)
    host = pools.host()
    cells = (tokens + geo.page_size - 1) // geo.page_size * geo.page_size
    kv = []
    for j in range(geo.n_qsa):
        rec = {"format": fmt, "cells": cells, "heads": geo.n_head_kv, "head_dim": geo.head_dim,
               "page_size": geo.page_size, "pooled_rows": sizes[4] // (geo.idx_key_dim * 4), "idx_dim": 128}
        for b, name in enumerate(("k", "v", "k_scale", "v_scale", "pooled")):
            rec[name] = host[(b, j)][:sizes[b]].tobytes() if sizes[b] else b""
        kv.append(rec)
    kv.append({"format": 0, "cells": 0, "heads": 0, "head_dim": 0, "page_size": 0, "pooled_rows": 0, "idx_dim": 0,
               "k": b"", "v": b"", "k_scale": b"", "v_scale": b"", "pooled": b""})
    live = {"ids": ids, "imgs": IMGS, "gdn": host["gdn"].tobytes(), "ple": SMALL_BUFS[0], "tails": SMALL_BUFS[1],
            "dead": SMALL_BUFS[2], "block_pos": SMALL_BUFS[3], "used": tokens + 1, "stage_parts": []}
    return {"geometry": GEOKEY, "layer_lo": 0, "layer_hi": 8, "cvec": True, "kv": kv, "live": live,
            "checkpoints": [], "stage_parts": []}, sizes, host


def _encode(sc, wire, geo, pools, tokens, live):
    enc = wire.Encoder(geo, pools, tokens, live, GEOM_HASH, PACK_HASH)
    buf = sc.DeviceBuffer(enc.bytes + 64, "uint8")
    buf.fill(0x5A)   # the encode must define every byte of the payload
    enc.encode(buf.ptr, enc.bytes)
    return enc, buf, enc.hash()


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("index", [False, True])
@pytest.mark.parametrize("tokens", [1, 77])
def test_layered_payload_equals_oracle_encode(sc, oracle, wire, codec, cuda, fmt, index, tokens):
    geo = sc.geometry(**SMALL)
    pools = sc.LayerPools(geo, fmt, 96, index)
    pools.randomize(0xC0DE + 3 * fmt + tokens)
    live, keep, ids = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, pools, tokens, live)
    payload = buf.numpy(enc.bytes).tobytes()
    image, _, _ = _expected_image(oracle, geo, pools, fmt, index, tokens, ids)
    want = codec.encode(image, GEOM_HASH, PACK_HASH)
    assert len(payload) == len(want)
    if payload != want:
        bad = next(i for i in range(len(want)) if payload[i] != want[i])
        raise AssertionError(f"payload differs from the oracle first at byte {bad} (pool at {enc.pool_offset})")
    assert h == codec.payload_hash(want)


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_layered_mount_round_trip(sc, oracle, wire, cuda, fmt):
    geo = sc.geometry(**SMALL)
    tokens = 123
    pools = sc.LayerPools(geo, fmt, 160, True)
    pools.randomize(0xFACE + fmt)
    live, keep, ids = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, pools, tokens, live)
    _, sizes, host = _expected_image(oracle, geo, pools, fmt, True, tokens, ids)
    dst = sc.LayerPools(geo, fmt, 160, True)
    dst.fill(0x77)
    dec = wire.Decoder(buf.ptr, enc.bytes, geo, dst, geometry=GEOKEY, geom_hash=GEOM_HASH, pack_hash=PACK_HASH,
                       check_identity=True, payload_hash=h, check_hash=True)
    assert dec.tokens == tokens
    dec.restore()
    got = dst.host()
    for j in range(geo.n_qsa):
        for b in range(5):
            if (b, j) in got:
                assert np.array_equal(got[(b, j)][:sizes[b]], host[(b, j)][:sizes[b]]), (b, j)
                assert (got[(b, j)][sizes[b]:] == 0x77).all(), (b, j)
    assert np.array_equal(got["gdn"], host["gdn"])
    assert np.array_equal(dec.live_ids(), ids)
    assert [dec.small(i) for i in range(4)] == list(SMALL_BUFS)


def test_format_mismatch_is_refused_and_writes_nothing(sc, wire, cuda):
    geo = sc.geometry(**SMALL)
    tokens = 40
    pools = sc.LayerPools(geo, sc.SC_KV_INT8, 64, True)
    pools.randomize(5)
    live, keep, _ = _live(wire, tokens)
    enc, buf, h = _encode(sc, wire, geo, pools, tokens, live)
    for fmt, index in ((sc.SC_KV_Q4, True), (sc.SC_KV_K8V4, True), (sc.SC_KV_INT8, False), (sc.SC_KV_F16, True)):
        dst = sc.LayerPools(geo, fmt, 64, index)
        dst.fill(0x42)
        with pytest.raises(wire.WireError) as e:
            wire.Decoder(buf.ptr, enc.bytes, geo, dst)
        assert "conversation wire" in str(e.value)
        assert all((a == 0x42).all() for a in dst.host().values())


def test_quantized_carve_to_payload_and_back(sc, wire, cuda):
    """The quantizing carve's K8V4 pools with indexer rows, encoded on the device and mounted into fresh pools."""
    geo = sc.geometry(**SMALL)
    T = 257
    case = synth.SyntheticCase(geo, T, seed=0xAB, kv_dtype=sc.SC_DTYPE_F32)
    cap = 272
    slot = sc.new_quant_slot(geo, sc.SC_KV_K8V4, cap)
    sc.plan_carve_quant(geo, case.prefill, slot).launch()
    pooled = [sc.DeviceBuffer((cap // 4 + 1) * geo.idx_key_dim * 4, "uint8") for _ in range(geo.n_qsa)]
    for i, b in enumerate(pooled):
        b.fill(i + 1)
    sc.device_sync()
    src = sc.LayerPools.from_quant(slot, pooled)
    live, keep, ids = _live(wire, T)
    enc, buf, h = _encode(sc, wire, geo, src, T, live)
    fresh = sc.new_quant_slot(geo, sc.SC_KV_K8V4, cap, fill=0)
    fresh_pooled = [sc.DeviceBuffer(b.nbytes, "uint8") for b in pooled]
    for b in fresh_pooled:
        b.fill(0)
    dst = sc.LayerPools.from_quant(fresh, fresh_pooled)
    dec = wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True)
    dec.restore()
    a, b = src.host(), dst.host()
    cells = (T + 3) // 4 * 4
    for key in a:
        if key == "gdn":
            assert np.array_equal(a[key], b[key])
            continue
        k, j = key
        n = {0: cells * 2 * 256, 1: cells * 2 * 144, 2: cells * 2 * 8, 4: (T // 4 + 1) * 512}[k]
        assert np.array_equal(a[key][:n], b[key][:n]), key
