"""Writes the hand-off payload codec's golden vectors from the REFERENCE's own codec.

Run in the build container, where /root/reference exists and `make -f oracle/Makefile.ref` has built
oracle/_ref/ref_wire from the reference's sources (src/core/conversation_wire.cpp and the files it links):

    python tests/golden/make_wire_vectors.py

For every spec below (the grammar and fill rule are in oracle/ref_wire_driver.cpp) it records the payload length and
FNV-1a payload hash the reference encoder produced, and keeps the payload itself under tests/golden/wire/ when it is
small.  For a set of corruptions of two fixture payloads (restating the refusal cases of the reference's
src/core/saved_conv_wire_test.cpp:661-960) it records whether the reference decoder accepts or refuses them.
Output: tests/golden/wire_manifest.json, tests/golden/wire/*.spec, tests/golden/wire/*.bin.
"""
from __future__ import annotations

import json
import struct
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
from oracle import sc_wire  # noqa: E402

REF = ROOT / "oracle" / "_ref" / "ref_wire"
OUT = HERE / "wire"
KEEP_BYTES = 64 * 1024   # payloads up to this size are committed byte for byte; larger ones by length and hash


def kv(fmt=0, cells=8, heads=2, head_dim=16, ps=4, pooled_rows=0, idx_dim=0, lk=None, lv=None, lks=0, lvs=0, lp=0):
    data = cells * heads * head_dim * (2 if fmt == 0 else 1)
    return [fmt, cells, heads, head_dim, ps, pooled_rows, idx_dim, data if lk is None else lk,
            data if lv is None else lv, lks, lvs, lp]


def cp(n_ids=0, n_imgs=0, gdn=0, ple=0, tails=0, dead=0, block_pos=0, used=0, parts=()):
    out = [n_ids, n_imgs, gdn, ple, tails, dead, block_pos, used, len(parts)]
    for p in parts:
        out += p
    return out


def spec(geom_hash, pack_hash, geometry, layer_lo, layer_hi, cvec, kvs, live, checkpoints=(), stages=()):
    out = [geom_hash, pack_hash, *geometry, layer_lo, layer_hi, int(cvec), len(kvs)]
    for k in kvs:
        out += k
    out += live
    out.append(len(checkpoints))
    for c in checkpoints:
        out += c
    out.append(len(stages))
    for lo, hi, state, skv in stages:
        out += [lo, hi, *state, len(skv)]
        for k in skv:
            out += k
    return " ".join(str(x) for x in out)


GEO = [2560, 16, 4, 32, 4, 8, 4, 520, 256, 24, 2, 256, 128, 4, 4, 3, 1, 0]
NEG_GEO = [-1, 2, -3, 4, -(1 << 62), 1 << 62, 0, 7, -7, 1, 1, 1, 1, 1, 1, 1, 1, -9]


def specs() -> dict[str, str]:
    s = {}
    s["empty"] = spec(0, 0, [0] * 18, 0, 0, False, [], cp())
    s["minimal_live"] = spec(11, 22, GEO, 0, 16, True, [], cp(n_ids=1, gdn=100))
    # the handoff's own shape: 4 QSA layers of f16 K/V + an empty draft layer; the live checkpoint holds the ids and
    # every GDN row (here 12 rows of 1024 bytes)
    s["handoff_shape"] = spec(0x1122334455667788, 0x0ABBCCDDEEFF0011, GEO, 0, 16, True,
                              [kv(cells=12, head_dim=64) for _ in range(4)] + [kv(cells=0, lk=0, lv=0)],
                              cp(n_ids=9, gdn=12 * 1024))
    s["single_gpu_full"] = spec(101, 202, GEO, 0, 16, True,
                                [kv(cells=8), kv(cells=8, pooled_rows=3, idx_dim=8, lp=96), kv(cells=0, lk=0, lv=0),
                                 kv(cells=4)],
                                cp(n_ids=37, n_imgs=3, gdn=1000, ple=400, tails=24, dead=36, block_pos=12, used=77),
                                checkpoints=[cp(n_ids=16, n_imgs=1, gdn=1000, ple=400, used=5),
                                             cp(n_ids=5, gdn=3, used=9, parts=[cp(n_ids=2, gdn=7)])])
    s["int8_scales"] = spec(3, 4, GEO, 0, 8, False,
                            [kv(fmt=1, cells=8, head_dim=128, lks=8 * 2 * 2 * 2, lvs=8 * 2 * 2 * 2, pooled_rows=3,
                                idx_dim=16, lp=3 * 16 * 4),
                             kv(fmt=2, cells=4, head_dim=64, lk=4 * 2 * 36, lv=4 * 2 * 36)],
                            cp(n_ids=8, gdn=64))
    s["layer_split"] = spec(-5, 6, GEO, 0, 8, True, [kv(cells=4), kv(cells=4)],
                            cp(n_ids=4, n_imgs=2, gdn=256, tails=8),
                            checkpoints=[cp(n_ids=2, gdn=256)],
                            stages=[(8, 12, cp(n_ids=0, gdn=128, tails=4, dead=4, block_pos=4), [kv(cells=4)]),
                                    (12, 16, cp(n_ids=0, gdn=128), [kv(cells=4), kv(cells=0, lk=0, lv=0)])])
    deep = cp(n_ids=3)
    for _ in range(3):
        deep = cp(n_ids=3, gdn=5, parts=[deep])
    s["nested_parts"] = spec(7, 8, GEO, 0, 4, True, [], cp(n_ids=2, gdn=16), checkpoints=[deep, cp(n_ids=1)])
    s["negative_fields"] = spec(-1, -2, NEG_GEO, -4, -2, True, [kv(fmt=-3, cells=-1, heads=-2, head_dim=0, ps=-4,
                                                                   pooled_rows=-5, idx_dim=-6, lk=10, lv=0)],
                                cp(n_ids=3, used=(1 << 63) - 1))
    s["odd_lengths"] = spec(1, 2, GEO, 0, 4, True, [kv(cells=1, lk=1, lv=63), kv(cells=1, lk=65, lv=127, lks=1)],
                            cp(n_ids=1, gdn=1, ple=2, tails=3, dead=5, block_pos=129))
    # a buffer larger than one 16 MiB ConversationBuffer segment (conversation_buffer.hpp:18)
    s["spanning_segments"] = spec(9, 10, GEO, 0, 4, True, [kv(cells=0, lk=20 * 1024 * 1024 + 3, lv=5 * 1024 * 1024)],
                                  cp(n_ids=4096, gdn=3 * 1024 * 1024 + 5))
    return s


def run(*args) -> str:
    return subprocess.run([str(REF), *map(str, args)], capture_output=True, text=True, check=True).stdout.strip()


def patch(p: bytearray, off: int, v: int, width: int = 8) -> None:
    p[off:off + width] = (v & ((1 << (8 * width)) - 1)).to_bytes(width, "little")


def landmarks(image: dict, payload: bytes) -> dict:
    """Offsets of records inside a payload: the live CHECKPOINT record, its id count, the first KV BLOBREF, the first
    STAGE record and the END record (walked with the record sizes, not guessed from the pool offset)."""
    n_kv = len(image["kv"])
    live = sc_wire.HEADER_BYTES + n_kv * (sc_wire.RECORD_HEADER_BYTES + sc_wire.KV_BODY_BYTES)
    at = live
    for c in [image["live"], *image["checkpoints"]]:
        at += sc_wire.RECORD_HEADER_BYTES + sc_wire._cp_body(c, 0, sc_wire.MAX_DEPTH)
    first_stage = at if image["stage_parts"] else None
    for st in image["stage_parts"]:
        at += sc_wire.RECORD_HEADER_BYTES + sc_wire._stage_body(st, sc_wire.MAX_DEPTH)
    return {"live_record": live, "live_ids": live + 16, "first_blobref": 256 + 16 + 56 if n_kv else None,
            "first_stage": first_stage, "end": at}


def mutations(name: str, image: dict, good: bytes, geom: int, pack: int) -> list[tuple[str, bytes, dict]]:
    """(label, payload, expectations) - restating the corruption cases of saved_conv_wire_test.cpp:661-960."""
    lm = landmarks(image, good)
    pool_off, pool_bytes = struct.unpack_from("<QQ", good, 200)
    out = [("valid", good, {})]
    for cut in (1, 64, 4096, len(good) - 1):
        if cut < len(good):
            out.append((f"truncated_{cut}", good[:cut], {}))
    for v in (0, 2, 65535):
        p = bytearray(good); patch(p, 4, v, 2); out.append((f"version_{v}", bytes(p), {}))
    p = bytearray(good); patch(p, 0, 0x44454144, 4); out.append(("magic", bytes(p), {}))
    for off in (216, 224):
        p = bytearray(good); patch(p, off, 0x0123456789ABCDEF); out.append((f"identity_{off}", bytes(p), {}))
    out.append(("over_slot", good, {"max_payload": len(good) - 1}))
    p = bytearray(good); patch(p, 232, (1 << 63) - 1); out.append(("absurd_size", bytes(p), {"max_payload": 1 << 20}))
    p = bytearray(good); patch(p, lm["live_ids"], 0x00007FFFFFFFFFFF); out.append(("huge_id_count", bytes(p), {}))
    p = bytearray(good); patch(p, lm["live_ids"], -1); out.append(("negative_id_count", bytes(p), {}))
    p = bytearray(good); patch(p, lm["end"], 0x11223344, 4); out.append(("no_end", bytes(p), {}))
    p = bytearray(good); patch(p, lm["end"] + 8, 8); out.append(("end_with_body", bytes(p), {}))
    p = bytearray(good); patch(p, 256, 99, 4); out.append(("first_kind", bytes(p), {}))
    p = bytearray(good); patch(p, 256 + 8, 1 << 40); out.append(("first_record_length", bytes(p), {}))
    p = bytearray(good); patch(p, lm["live_record"] + 8, 1 << 40); out.append(("live_record_length", bytes(p), {}))
    p = bytearray(good); patch(p, 256 + 4, 1, 4); out.append(("first_record_flags", bytes(p), {}))
    p = bytearray(good); patch(p, lm["live_record"], 7, 4); out.append(("live_kind", bytes(p), {}))
    p = bytearray(good); patch(p, lm["live_record"] + 4, 3, 4); out.append(("live_flags", bytes(p), {}))
    if lm["first_stage"] is not None:
        p = bytearray(good); patch(p, lm["first_stage"] + 8, 4); out.append(("stage_length", bytes(p), {}))
        p = bytearray(good); patch(p, lm["first_stage"], sc_wire.KIND_KV, 4); out.append(("stage_kind", bytes(p), {}))
    if lm["first_blobref"] is not None:
        fb = lm["first_blobref"]
        p = bytearray(good); patch(p, fb + 8, pool_off + pool_bytes + 64); out.append(("blob_outside", bytes(p), {}))
        p = bytearray(good); patch(p, fb + 8, pool_off + 3); out.append(("blob_misaligned", bytes(p), {}))
        p = bytearray(good); patch(p, fb, 0); out.append(("blob_zero_with_offset", bytes(p), {}))
        # the pool chopped with the header's numbers fixed to match (saved_conv_wire_test.cpp:686-700)
        p = bytearray(good[:-8]); patch(p, 232, len(p)); patch(p, 208, len(p) - pool_off)
        out.append(("pool_chopped", bytes(p), {}))
    for off in (240, 248):
        p = bytearray(good); patch(p, off, 7); out.append((f"reserved_{off}", bytes(p), {}))
    flags = struct.unpack_from("<H", good, 6)[0]
    p = bytearray(good); patch(p, 6, flags | 4, 2); out.append(("partial_flag", bytes(p), {}))
    p = bytearray(good); patch(p, 6, flags | (1 << 9), 2); out.append(("unknown_flag", bytes(p), {}))
    p = bytearray(good); patch(p, 6, flags ^ 2, 2); out.append(("stage_flag_flipped", bytes(p), {}))
    p = bytearray(good); patch(p, 200, pool_off + 8); out.append(("pool_unaligned", bytes(p), {}))
    p = bytearray(good); patch(p, 192, len(image["live"]["ids"]) + 1); out.append(("live_tokens", bytes(p), {}))
    p = bytearray(good); p[pool_off + min(100, pool_bytes - 1)] ^= 0x40
    out.append(("flipped_pool_byte", bytes(p), {"hash": "original"}))
    out.append(("split_into_single", good, {"stage_parts": 0}))
    out.append(("single_into_split", good, {"stage_parts": 1}))
    p = bytearray(good); patch(p, pool_off - 1, 1, 1)   # the END-to-pool padding must be zero
    out.append(("pad_byte", bytes(p), {}))
    return [(f"{name}:{label}", payload, exp) for label, payload, exp in out]


def main() -> int:
    if not REF.exists():
        print(f"{REF} is not built: run `make -f oracle/Makefile.ref` here first", file=sys.stderr)
        return 1
    OUT.mkdir(exist_ok=True)
    manifest = {"source": "oracle/_ref/ref_wire (the reference's src/core/conversation_wire.cpp)", "specs": {},
                "mutations": []}
    with tempfile.TemporaryDirectory() as tmp:
        for name, text in specs().items():
            (OUT / f"{name}.spec").write_text(text + "\n")
            out = Path(tmp) / f"{name}.bin"
            size, h = run("encode", OUT / f"{name}.spec", out).split()
            payload = out.read_bytes()
            entry = {"bytes": int(size), "payload_hash": f"0x{h}"}
            if len(payload) <= KEEP_BYTES:
                (OUT / f"{name}.bin").write_bytes(payload)
                entry["payload"] = f"wire/{name}.bin"
            manifest["specs"][name] = entry
        for name in ("single_gpu_full", "layer_split"):
            image, geom, pack = sc_wire.image_from_spec((OUT / f"{name}.spec").read_text())
            good = (OUT / f"{name}.bin").read_bytes()
            for label, payload, exp in mutations(name, image, good, geom, pack):
                path = Path(tmp) / "m.bin"
                path.write_bytes(payload)
                h = sc_wire.payload_hash(good) if exp.get("hash") == "original" else sc_wire.payload_hash(payload)
                verdict = run("decode", path, geom & 0xFFFFFFFFFFFFFFFF, pack & 0xFFFFFFFFFFFFFFFF, h,
                              exp.get("stage_parts", -1), exp.get("max_payload", 0))
                mut = {"case": label, "of": name, "expect": exp, "refused": verdict.startswith("refused"),
                       "reason": verdict.split(" ", 1)[1] if verdict.startswith("refused") else ""}
                if label.endswith(":valid"):
                    mut["reencodes_identically"] = verdict == "ok 1"
                manifest["mutations"].append(mut)
    (HERE / "wire_manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    n_ref = sum(m["refused"] for m in manifest["mutations"])
    print(f"{len(manifest['specs'])} specs, {len(manifest['mutations'])} corruption cases ({n_ref} refused)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
