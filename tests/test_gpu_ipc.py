"""The same-GPU hand-off between processes (sc_ipc_*, include/sc_handoff.h) on the GPU.

A second process (tests/ipc_peer.py) exports device segments and stages payloads into them; this process opens the
segments and fetches each payload into its own device memory.  Every fetched payload must equal, byte for byte, what
the exporter staged (regenerated here from the same seed) and carry the exporter's device FNV-1a; a slot's payload
fetched this way must mount into fresh pools equal to the exporter's (rebuilt here from the same seed).

The zero-copy hand-off: the exporter encodes the slot straight into its exported segments (no payload buffer, no
stage), and this process mounts the payload where it lies in the imported segments (no fetch), the hash checked on the
device over the segments before any byte reaches the slot.  The mounted pools must equal the exporter's, in f16, int8
and q4_0 with the indexer's rows; a wrong expected hash must leave the pools untouched.  Two processes use the GPU;
each shared allocation stays at or under 1 GiB.
"""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
PEER = ROOT / "tests" / "ipc_peer.py"


class Peer:
    def __init__(self, *args):
        print(f"case ipc peer {args}", flush=True)
        self.proc = subprocess.Popen([sys.executable, "-u", str(PEER), *map(str, args)], stdin=subprocess.PIPE,
                                     stdout=subprocess.PIPE, text=True)
        self.first = self.read()

    def read(self):
        line = self.proc.stdout.readline()
        assert line, f"the exporting process ended early (status {self.proc.poll()})"
        return json.loads(line)

    def ask(self, line):
        self.proc.stdin.write(line + "\n")
        self.proc.stdin.flush()
        return self.read()

    def segments(self):
        return [(bytes.fromhex(h), n) for h, n in self.first["segments"]]

    def finish(self):
        try:
            self.proc.stdin.write("done\n")
            self.proc.stdin.flush()
        except BrokenPipeError:
            pass
        assert self.proc.wait(timeout=60) == 0


def test_raw_payloads_cross_the_process_boundary(sc, cuda):
    cap, seg = (40 << 20) + 4096, 16 << 20          # three segments, the last one partly used
    peer = Peer("raw", cap, seg)
    imp = None
    try:
        segs = peer.segments()
        assert [n for _, n in segs] == [16 << 20, 16 << 20, (8 << 20) + 4096]
        imp = sc.IpcImport(segs)
        dst = sc.DeviceBuffer(cap + 64, "uint8")
        for n, seed in ((1, 1), (4099, 2), (16 << 20, 3), ((16 << 20) + 1, 4), (cap, 5), (cap - 3, 6)):
            h = peer.ask(f"stage {n} {seed}")["hash"]
            dst.fill(0xEE)
            imp.fetch(dst.ptr, n)
            sc.device_sync()
            want = np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)
            got = dst.numpy(n + 64)
            assert np.array_equal(got[:n], want), (n, seed)
            assert (got[n:] == 0xEE).all()
            assert sc.fnv1a64_device(dst.ptr, n) == h
        with pytest.raises(sc.ScError):
            imp.fetch(dst.ptr, cap + 4096 + 1)        # more than the segments hold
    finally:
        if imp:
            imp.close()
        peer.finish()


def _pools(sc, fmt, tokens, seed):
    geo = sc.geometry(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
                      ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
    cap = (tokens + 3) // 4 * 4 + 16
    src = sc.LayerPools(geo, fmt, cap, True)
    src.randomize(seed)                             # the exporter's pools, rebuilt from the same seed
    dst = sc.LayerPools(geo, fmt, cap, True)
    dst.fill(0x99)
    return geo, src, dst


def _assert_mounted(sc, geo, fmt, tokens, src, dst):
    a, b = src.host(), dst.host()
    sizes = sc.layer_blob_bytes(geo, fmt, True, tokens)
    for key in a:
        if key == "gdn":
            assert np.array_equal(a[key], b[key])
        else:
            k = sizes[key[0]]
            assert np.array_equal(a[key][:k], b[key][:k]) and (b[key][k:] == 0x99).all(), key


@pytest.mark.parametrize("fmt", [0, 1, 3])
def test_slot_payload_mounts_from_another_process(sc, cuda, fmt):
    import sc_wire
    tokens, seed = 301, 0xC0FFEE + fmt
    peer = Peer("slot", fmt, tokens, seed)
    imp = None
    try:
        n, h = peer.first["bytes"], peer.first["hash"]
        imp = sc.IpcImport(peer.segments())
        payload = sc.DeviceBuffer(n, "uint8")
        imp.fetch(payload.ptr, n)
        sc.device_sync()
        geo, src, dst = _pools(sc, fmt, tokens, seed)
        dec = sc_wire.Decoder(payload.ptr, n, geo, dst, geom_hash=0x1111, pack_hash=0x2222, check_identity=True,
                              payload_hash=h, check_hash=True)
        assert dec.tokens == tokens
        dec.restore()
        _assert_mounted(sc, geo, fmt, tokens, src, dst)
    finally:
        if imp:
            imp.close()
        peer.finish()


@pytest.mark.parametrize("fmt", [0, 1, 3])
def test_zero_copy_hand_off(sc, cuda, fmt):
    """Encode into the exported segments, mount from the imported ones: no stage, no fetch."""
    import sc_wire
    tokens, seed = 1203, 0xBEEF + fmt           # a payload over several 1 MiB segments
    peer = Peer("zerocopy", fmt, tokens, seed)
    imp = None
    try:
        n, h = peer.first["bytes"], peer.first["hash"]
        imp = sc.IpcImport(peer.segments())
        ptrs, seg_bytes = imp.layout()
        assert seg_bytes == 1 << 20 and len(ptrs) == (n + seg_bytes - 1) // seg_bytes >= 2
        # the exporter's hash is the hash of the bytes the segments hold, hashed here where they lie
        hp = sc.HashPlan(n)
        hmap = sc.HashMap.read(ptrs, seg_bytes, n)
        hmap.launch(hp)
        sc.device_sync()
        assert hp.result() == h
        hmap.destroy()
        hp.free()
        geo, src, dst = _pools(sc, fmt, tokens, seed)
        with pytest.raises(sc_wire.WireError):
            sc_wire.Decoder(0, n, geo, dst, geom_hash=0x1111, pack_hash=0x2222, check_identity=True,
                            payload_hash=h ^ 1, check_hash=True, segments=(ptrs, seg_bytes)).restore()
        assert all((v == 0x99).all() for v in dst.host().values())
        dec = sc_wire.Decoder(0, n, geo, dst, geom_hash=0x1111, pack_hash=0x2222, check_identity=True,
                              payload_hash=h, check_hash=True, segments=(ptrs, seg_bytes))
        assert dec.tokens == tokens
        dec.restore()
        assert dec.small(0) == b"ple" and dec.small(1) == b"tails" and dec.small(3) == b"bp"
        _assert_mounted(sc, geo, fmt, tokens, src, dst)
    finally:
        if imp:
            imp.close()
        peer.finish()


def test_refusals_before_any_handle_is_opened(sc, cuda):
    with pytest.raises(sc.ScError) as e:
        sc.IpcExport(1 << 20, (1 << 30) + 4096)
    assert e.value.code == sc.SC_ERANGE
    with pytest.raises(sc.ScError) as e:
        sc.IpcExport(1 << 20, 1000)
    assert e.value.code == sc.SC_ERANGE
    with pytest.raises(sc.ScError) as e:
        sc.IpcImport([(bytes(64), (1 << 30) + 1)])    # a segment over 1 GiB is never opened
    assert e.value.code == sc.SC_ERANGE
    with pytest.raises(sc.ScError) as e:
        sc.IpcImport([(bytes(64), 0)])
    assert e.value.code == sc.SC_ERANGE


def test_device_copy_kernel(sc, cuda):
    """sc_copy_device_async at every alignment pair and awkward sizes equals the source bytes."""
    src = sc.DeviceBuffer(1 << 20, "uint8")
    data = np.random.default_rng(7).integers(0, 256, 1 << 20, dtype=np.uint8)
    src.upload(data)
    dst = sc.DeviceBuffer((1 << 20) + 64, "uint8")
    for so, do, n in ((0, 0, 1 << 19), (3, 3, 100003), (5, 9, 77777), (16, 0, 4096), (1, 2, 15), (0, 0, 0)):
        dst.fill(0)
        sc.check(sc.lib.sc_copy_device_async(dst.ptr + do, src.ptr + so, n, None), "copy")
        sc.device_sync()
        got = dst.numpy()
        assert np.array_equal(got[do:do + n], data[so:so + n]), (so, do, n)
        assert not got[:do].any() and not got[do + n:].any()
