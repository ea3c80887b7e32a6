"""The exporting process of the same-GPU hand-off tests (tests/test_gpu_ipc.py starts it; pytest does not collect it).

    python tests/ipc_peer.py raw CAPACITY SEGMENT_BYTES
        reads commands on stdin, one per line, answers one JSON line each:
          stage NBYTES SEED   host random bytes of SEED uploaded and staged into the exported segments -> {"hash": ...}
          done                exits (after its importer closed the segments)
        the first line it prints lists the segments: {"segments": [[handle_hex, bytes], ...]}
    python tests/ipc_peer.py slot FORMAT TOKENS SEED
        a slot of LayerPools randomized with SEED, its payload encoded and staged ->
        {"segments": ..., "bytes": ..., "hash": ...}; then waits for "done"
    python tests/ipc_peer.py zerocopy FORMAT TOKENS SEED
        the same slot's payload encoded straight into the exported segments (no payload buffer, no stage copy)
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "strata-concurrent_amd"))
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

import sc_handoff as sc  # noqa: E402

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
GEOKEY = [2560, 8, 4, 32, 4, 8, 4, 520, 256, 24, 2, 256, 128, 4, 4, 3, 1, 0]


def say(obj):
    print(json.dumps(obj), flush=True)


def segments_json(ex):
    return [[h.hex(), n] for h, n in ex.segments()]


def raw(capacity, segment_bytes):
    ex = sc.IpcExport(capacity, segment_bytes)
    say({"segments": segments_json(ex)})
    buf = sc.DeviceBuffer(capacity, "uint8")
    for line in sys.stdin:
        cmd = line.split()
        if not cmd or cmd[0] == "done":
            break
        n, seed = int(cmd[1]), int(cmd[2])
        data = np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)
        buf.upload(data)
        ex.stage(buf.ptr, n)
        sc.device_sync()
        say({"hash": sc.fnv1a64_device(buf.ptr, n)})
    ex.destroy()


def slot(fmt, tokens, seed, zero_copy=False):
    import sc_wire
    geo = sc.geometry(**SMALL)
    pools = sc.LayerPools(geo, fmt, (tokens + 3) // 4 * 4 + 16, True)
    pools.randomize(seed)
    ids = (np.arange(tokens, dtype=np.int64) * 31 % 151_000).astype(np.int32)
    live, keep = sc_wire.make_live(GEOKEY, ids, layer_lo=0, layer_hi=8, idx_dim=128, imgs=[(5, 77)], used=tokens,
                                   small=(b"ple", b"tails", b"", b"bp"))
    enc = sc_wire.Encoder(geo, pools, tokens, live, 0x1111, 0x2222)
    ex = sc.IpcExport(enc.bytes, 1 << 20)      # 1 MiB segments: the payload spans several
    if zero_copy:
        enc.encode_segments(*ex.layout())
    else:
        payload = sc.DeviceBuffer(enc.bytes, "uint8")
        enc.encode(payload.ptr, enc.bytes)
        ex.stage(payload.ptr, enc.bytes)
    sc.device_sync()
    say({"segments": segments_json(ex), "bytes": enc.bytes, "hash": enc.hash()})
    sys.stdin.readline()
    ex.destroy()


if __name__ == "__main__":
    if sys.argv[1] == "raw":
        raw(int(sys.argv[2]), int(sys.argv[3]))
    else:
        slot(int(sys.argv[2]), int(sys.argv[3]), int(sys.argv[4]), zero_copy=sys.argv[1] == "zerocopy")
