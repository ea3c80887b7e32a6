"""Layer-split hand-off payloads on the device (sc_wire_encoder_create_split / sc_wire_decoder_open_split).

When the model is split over stages the reference's snapshot keeps each later stage's state in a stage part: the
stage's layer range, its own K/V records (one per QSA layer the stage owns) and its running state (the live ids, its
GDN rows and its small index buffers), saved from and restored into that stage's session
(src/core/conversation_state.cpp:397-413, 497-509).  Here every stage is a decode slot of its own on the device; the
encoder gathers each part from its slot, the decoder scatters each part into its slot, and all scatters are gated by
the one device hash verdict.  The payload must equal, byte for byte, the oracle codec's encode (oracle/sc_wire.py,
pinned to the reference codec's payloads in tests/test_wire_oracle.py) of the image the CPU carve oracle gives.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

BASE = dict(qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32, ssm_k_heads=4, ssm_v_heads=8,
            ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
GEOKEY = [2560, 16, 4, 32, 4, 8, 4, 520, 256, 24, 2, 256, 128, 4, 4, 3, 1, 0]
GEOM_HASH, PACK_HASH = 0x1122334455667788, 0x0AABBCCDDEEFF001
MAIN_SMALL = (bytes(range(40)), bytes(range(7, 19)), b"", bytes(range(200, 208)))
IMGS = [(4, 0xDEADBEEF)]
# (layers the stage's slot holds, its layer range, its small buffers)
STAGES = [(4, (4, 8), (b"", bytes(range(30, 42)), bytes(range(3)), bytes(range(90, 98)))),
          (8, (8, 16), (b"", bytes(range(60, 84)), bytes(range(5, 11)), bytes(range(100, 116))))]
CELLS = 128


@pytest.fixture(scope="module")
def wire():
    import sc_wire
    return sc_wire


@pytest.fixture(scope="module")
def codec():
    from oracle import sc_wire as codec
    return codec


def _kv_records(geo, state, tokens):
    cells = geo.cells(tokens)
    kvb = cells * geo.n_head_kv * geo.head_dim * 2
    return [{"format": 0, "cells": cells, "heads": geo.n_head_kv, "head_dim": geo.head_dim,
             "page_size": geo.page_size, "pooled_rows": 0, "idx_dim": 128,
             "k": state[f"k{j}"].tobytes()[:kvb], "v": state[f"v{j}"].tobytes()[:kvb],
             "k_scale": b"", "v_scale": b"", "pooled": b""} for j in range(geo.n_qsa)]


class Split:
    """A main slot of 4 layers and two later stages, each carved from its own synthetic prefill."""

    def __init__(self, sc, tokens, seed):
        self.tokens = tokens
        self.geo = sc.geometry(n_layers=4, **BASE)
        self.case = synth.SyntheticCase(self.geo, tokens, seed=seed)
        self.slot = self.case.new_slot(max_cells=CELLS)
        self.case.carve_into(self.slot)
        self.stages = []
        for i, (layers, rng, small) in enumerate(STAGES):
            geo = sc.geometry(n_layers=layers, **BASE)
            case = synth.SyntheticCase(geo, tokens, seed=seed + 101 * (i + 1))
            slot = case.new_slot(max_cells=CELLS)
            case.carve_into(slot)
            self.stages.append((geo, case, slot, rng, small))
        self.ids = (np.arange(tokens, dtype=np.int64) * 7919 % 151_000).astype(np.int32)

    def live(self, wire):
        return wire.make_live(GEOKEY, self.ids, layer_lo=0, layer_hi=4, idx_dim=128, imgs=IMGS, used=self.tokens * 3,
                              small=MAIN_SMALL)

    def stage_array(self, wire, with_small=True, slots=None):
        slots = slots or [s[2] for s in self.stages]
        return wire.make_stages([(geo, slot, rng[0], rng[1], small if with_small else None)
                                 for (geo, _, _, rng, small), slot in zip(self.stages, slots)])

    def expected_image(self, oracle):
        state = oracle.expected_slot(self.geo, self.case.host_inputs(), slot_cells=CELLS)
        kv = _kv_records(self.geo, state, self.tokens)
        kv.append({"format": 0, "cells": 0, "heads": 0, "head_dim": 0, "page_size": 0, "pooled_rows": 0, "idx_dim": 0,
                   "k": b"", "v": b"", "k_scale": b"", "v_scale": b"", "pooled": b""})
        live = {"ids": self.ids, "imgs": IMGS, "gdn": state["gdn"].tobytes(), "ple": MAIN_SMALL[0],
                "tails": MAIN_SMALL[1], "dead": MAIN_SMALL[2], "block_pos": MAIN_SMALL[3], "used": self.tokens * 3,
                "stage_parts": []}
        parts = []
        for geo, case, _, (lo, hi), small in self.stages:
            st = oracle.expected_slot(geo, case.host_inputs(), slot_cells=CELLS)
            parts.append({"layer_lo": lo, "layer_hi": hi, "kv": _kv_records(geo, st, self.tokens),
                          "state": {"ids": self.ids, "imgs": [], "gdn": st["gdn"].tobytes(), "ple": small[0],
                                    "tails": small[1], "dead": small[2], "block_pos": small[3], "used": 0,
                                    "stage_parts": []}})
        return {"geometry": GEOKEY, "layer_lo": 0, "layer_hi": 4, "cvec": True, "kv": kv, "live": live,
                "checkpoints": [], "stage_parts": parts}


def _encode(sc, wire, split):
    live, keep = split.live(wire)
    arr, keep2 = split.stage_array(wire)
    enc = wire.Encoder(split.geo, split.slot, split.tokens, live, GEOM_HASH, PACK_HASH, stages=arr,
                       n_stages=len(split.stages))
    buf = sc.DeviceBuffer(enc.bytes + 64, "uint8")
    buf.fill(0x5A)   # the encode must define every byte of the payload
    enc.encode(buf.ptr, enc.bytes)
    return enc, buf, enc.hash()


def _fresh(sc, split, fill):
    main = sc.new_slot(split.geo, CELLS, fill=fill)
    stages = [sc.new_slot(geo, CELLS, fill=fill) for geo, *_ in split.stages]
    return main, stages


def _open(wire, split, buf, nbytes, main, stages, h=0, check=False, **kw):
    arr, keep = split.stage_array(wire, with_small=False, slots=stages)
    n = kw.pop("n_stages", len(stages))
    return wire.Decoder(buf.ptr, nbytes, split.geo, main, geometry=GEOKEY, geom_hash=GEOM_HASH, pack_hash=PACK_HASH,
                        check_identity=True, payload_hash=h, check_hash=check, stages=arr, n_stages=n, **kw)


@pytest.mark.parametrize("tokens", [77, 1, 0])
def test_split_payload_equals_oracle_encode(sc, oracle, wire, codec, cuda, tokens):
    print(f"case split payload tokens={tokens}", flush=True)
    split = Split(sc, tokens, seed=0x5100 + tokens)
    enc, buf, h = _encode(sc, wire, split)
    payload = buf.numpy(enc.bytes).tobytes()
    want = codec.encode(split.expected_image(oracle), GEOM_HASH, PACK_HASH)
    assert len(payload) == len(want)
    if payload != want:
        bad = next(i for i in range(len(want)) if payload[i] != want[i])
        raise AssertionError(f"payload differs from the oracle first at byte {bad} (pool at {enc.pool_offset})")
    assert h == codec.payload_hash(want)
    back = codec.decode(payload, GEOM_HASH, PACK_HASH, h, geometry=GEOKEY, stage_parts=2)
    assert [(p["layer_lo"], p["layer_hi"]) for p in back["stage_parts"]] == [s[1] for s in STAGES]


def test_split_mount_round_trip(sc, wire, cuda):
    print("case split mount round trip", flush=True)
    split = Split(sc, 77, seed=0x5200)
    enc, buf, h = _encode(sc, wire, split)
    main, stages = _fresh(sc, split, 0xAB)
    dec = _open(wire, split, buf, enc.bytes, main, stages, h, check=True)
    assert dec.tokens == 77
    dec.restore()
    cells = split.geo.cells(77)
    pairs = [(split.geo, split.slot, main)] + [(geo, src, dst) for (geo, _, src, _, _), dst in zip(split.stages, stages)]
    for geo, src, dst in pairs:
        got, want = dst.host_state(), src.host_state()
        per_cell = geo.n_head_kv * geo.head_dim
        for j in range(geo.n_qsa):
            for name in (f"k{j}", f"v{j}"):
                w, g = want[name].reshape(-1), got[name].reshape(-1)
                assert np.array_equal(g[: cells * per_cell], w[: cells * per_cell]), name
                assert np.all(g[cells * per_cell:] == 0xABAB), f"{name}: cells past the image were written"
        assert np.array_equal(got["gdn"], want["gdn"])
    assert np.array_equal(dec.live_ids(), split.ids)
    for which, b in enumerate(MAIN_SMALL):
        assert dec.small(which) == b
    for i, (_, _, _, _, small) in enumerate(split.stages):
        for which, b in enumerate(small):
            assert dec.stage_small(i, which) == b


def test_split_refusals_leave_every_slot_untouched(sc, oracle, wire, cuda):
    print("case split refusals", flush=True)
    split = Split(sc, 40, seed=0x5300)
    enc, buf, h = _encode(sc, wire, split)
    main, stages = _fresh(sc, split, 0xCD)
    slots = [main] + stages
    before = [{k: v.copy() for k, v in s.host_state().items()} for s in slots]

    def untouched():
        return all(all(np.array_equal(b[k], s.host_state()[k]) for k in b) for b, s in zip(before, slots))

    # a flipped byte in the last stage's K record: the one device verdict gates every scatter, the main slot's too
    geo, case, *_ = split.stages[-1]
    st = oracle.expected_slot(geo, case.host_inputs(), slot_cells=CELLS)
    payload = buf.numpy(enc.bytes).tobytes()
    at = payload.find(st["k1"].tobytes()[:512])
    assert at >= enc.pool_offset
    orig = buf.numpy(1, start=at + 100)
    buf.upload(orig ^ 0x10, start=at + 100)
    dec = _open(wire, split, buf, enc.bytes, main, stages, h, check=True)
    with pytest.raises(wire.WireError) as e:
        dec.restore()
    assert e.value.code == sc.SC_EINVAL and "hash" in str(e.value)
    sc.device_sync()
    assert untouched()
    buf.upload(orig, start=at + 100)
    # open refusals: stage count, a stage's layer range, a stage slot of another shape, a split payload without stages
    with pytest.raises(wire.WireError, match="stage parts"):
        _open(wire, split, buf, enc.bytes, main, stages[:1], n_stages=1)
    with pytest.raises(wire.WireError, match="2 stage parts"):
        wire.Decoder(buf.ptr, enc.bytes, split.geo, main)
    saved = split.stages[0]
    split.stages[0] = saved[:3] + ((4, 9),) + saved[4:]
    with pytest.raises(wire.WireError, match="covers layers"):
        _open(wire, split, buf, enc.bytes, main, stages)
    split.stages[0] = saved
    other_geo = sc.geometry(n_layers=8, **BASE)       # the first stage's slot with two QSA layers instead of one
    odst = sc.new_slot(other_geo, CELLS, fill=0)
    split.stages[0] = (other_geo,) + saved[1:]
    with pytest.raises(wire.WireError):
        _open(wire, split, buf, enc.bytes, main, [odst, stages[1]])
    split.stages[0] = saved
    assert untouched()
    # the intact payload still mounts, every slot
    _open(wire, split, buf, enc.bytes, main, stages, h, check=True).restore()
    sc.device_sync()
    after = [s.host_state() for s in slots]
    assert all(not np.array_equal(b["gdn"], a["gdn"]) for b, a in zip(before, after))


def test_split_encoder_refusals(sc, wire, cuda):
    """A stage slot read through page tables, or a negative stage count, is refused."""
    split = Split(sc, 12, seed=0x5400)
    live, keep = split.live(wire)
    geo, case, slot, rng, small = split.stages[0]
    t = np.arange(8)[::-1].astype(np.int32)
    paged = case.new_slot(max_cells=32, n_pages=8, tables=sc.device_tables([t] * geo.n_qsa))
    arr, keep2 = split.stage_array(wire, slots=[paged, split.stages[1][2]])
    with pytest.raises(wire.WireError, match="identity page tables"):
        wire.Encoder(split.geo, split.slot, split.tokens, live, stages=arr, n_stages=2)
    arr, keep2 = split.stage_array(wire)
    with pytest.raises(wire.WireError, match="invalid stage array"):
        wire.Encoder(split.geo, split.slot, split.tokens, live, stages=arr, n_stages=-1)
