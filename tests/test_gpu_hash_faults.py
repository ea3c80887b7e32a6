"""A device hash whose look-back wait ran out is never acted on: the callers of the hash refuse instead.

The hash kernel's waits are bounded; a wait that runs out ends the launch with the fault word set and a hash that is
not the payload's (sc_hash.hip).  SC_FNV_FORCE_FAULT makes every wait past the first workgroup run out at once, so
these tests force the condition from the host while every kernel still exits normally.  Under it:
  - the wire encoder's payload hash is refused (sc_wire_encoder_hash), not returned;
  - a mount with the hash checked refuses and writes nothing into the slot (the device verdict that gates the scatter
    includes the fault, and the host reads the same two words);
  - the arena mover's write does not return a hash, its publish leaves the slot unpublished, and its verified read
    refuses.
With the default bound the same calls succeed, with the hashes of the byte loop.
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


@pytest.fixture
def forced(sc, cuda):
    """Run the test body's forced part with every look-back wait running out; the default bound is restored after."""
    class Force:
        def __enter__(self):
            sc.check(sc.lib.sc_fnv1a64_set_spin_limit(sc.SC_FNV_FORCE_FAULT), "spin limit")

        def __exit__(self, *exc):
            sc.check(sc.lib.sc_fnv1a64_set_spin_limit(0), "spin limit")
    yield Force()
    sc.check(sc.lib.sc_fnv1a64_set_spin_limit(0), "spin limit")


def test_encode_and_mount_refuse_a_faulted_hash(sc, oracle, forced):
    import sc_wire as wire
    geo = sc.geometry(**SMALL)
    tokens = 300   # a payload of several 64 KiB workgroups
    case = synth.SyntheticCase(geo, tokens, seed=0xFA17)
    slot = case.new_slot(max_cells=320)
    case.carve_into(slot)
    ids = (np.arange(tokens, dtype=np.int64) * 7919 % 151_000).astype(np.int32)
    live, keep = wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128)
    enc = wire.Encoder(geo, slot, tokens, live, GEOM, PACK)
    assert enc.bytes > 4 * 65536
    buf = sc.DeviceBuffer(enc.bytes, "uint8")
    print(f"case forced encode of {enc.bytes} bytes", flush=True)
    with forced:
        enc.encode(buf.ptr, enc.bytes)
        with pytest.raises(wire.WireError, match="did not complete"):
            enc.hash()
    enc.encode(buf.ptr, enc.bytes)
    h = enc.hash()
    assert h == oracle.fnv1a64(buf.numpy(), SEED)
    # a mount with the hash checked: the faulted check mounts nothing and says so; then the real one mounts
    dst = case.new_slot(max_cells=320, fill=0x6B)
    print("case forced mount", flush=True)
    with forced:
        dec = wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True)
        with pytest.raises(wire.WireError, match="did not complete"):
            dec.restore()
    state = dst.host_state()
    assert all(np.all(v.view(np.uint8) == 0x6B) for v in state.values())
    wire.Decoder(buf.ptr, enc.bytes, geo, dst, payload_hash=h, check_hash=True).restore()
    want = slot.host_state()
    got = dst.host_state()
    pages = geo.cells(tokens) // geo.page_size   # the pools are [page][H][page_size][D]
    for j in range(geo.n_qsa):
        for x in ("k", "v"):
            assert np.array_equal(got[f"{x}{j}"][:pages], want[f"{x}{j}"][:pages])
    assert np.array_equal(got["gdn"], want["gdn"])


def test_mover_refuses_a_faulted_hash(sc, oracle, forced, tmp_path):
    import sc_arena as ar
    n = 20_000_003
    data = np.random.default_rng(17).integers(0, 256, n, dtype=np.uint8)
    src = sc.DeviceBuffer(n, "uint8")
    src.upload(data)
    want = oracle.fnv1a64(data.tobytes(), SEED)
    mover = ar.Mover(chunk_bytes=8 << 20, depth=3, threads=4)
    path = tmp_path / "arena"
    w = ar.Arena.writer(path, [(1024, 2), (131072, 2)], [8 << 20, 64 << 20], PACK, GEOM)
    r = ar.Arena.reader(path, PACK, GEOM)
    try:
        c = w.claim(1, 42, 7)
        print("case forced mover write and publish", flush=True)
        with forced:
            with pytest.raises(ar.ArenaError, match="did not complete"):
                mover.write(w, c, src.ptr, n)
            with pytest.raises(ar.ArenaError, match="did not complete"):
                mover.publish(w, c, src.ptr, n, 1234)
        assert w.slot(c.index).state == ar.CLAIMED   # nothing was published
        mover.publish(w, c, src.ptr, n, 1234)
        s = w.slot(c.index)
        assert s.state == ar.READY and s.payload_hash == want
        dst = sc.DeviceBuffer(n, "uint8")
        print("case forced verified read", flush=True)
        with forced:
            with pytest.raises(ar.ArenaError, match="did not complete"):
                mover.read(r, c.index, c.nonce, 42, dst.ptr, n, verify=True)
        dst.fill(0)
        mover.read(r, c.index, c.nonce, 42, dst.ptr, n, verify=True)
        assert dst.numpy().tobytes() == data.tobytes()
        w.release(c.index, c.nonce)
    finally:
        mover.destroy()
        w.close()
        r.close()
