"""CPU restatement of the hand-off arena's arithmetic and identity (TEST INFRASTRUCTURE ONLY: only tests/ use it).

Follows the reference's src/core/handoff.cpp:
  split_spec   115-130   "main=<lo>..<hi>|<lo>..<hi>,...|n=<stages>|draft=<last|main>"
  geom_hash    132-138   FNV-1a (engine seed) over "strata-handoff-geom-v1", 18 little-endian u64 words, the spec; 0 -> 1
  arena_path   140-149   "<dir>/<pack16>-<spec>[/<instance>]/arena"
  size_arena   164-231   slot = round_up_64(payload) + 64 MiB; groups laid out ascending after a 4 KiB header
and the header layouts of include/strata/core/handoff.hpp:26-68 (ARENA_FIELDS / SLOT_FIELDS).

Pinning: tests/test_handoff_arena.py checks every function here against the reference's own implementation
(oracle/_ref/ref_arena, compiled from src/core/handoff.cpp) and against the arena files it writes, and the geometry hash
against a byte-serial FNV-1a of the concatenated stream (sc_oracle.fnv1a64, pinned by the payload codec's fixtures).
"""
from __future__ import annotations

import struct

from . import sc_oracle

SEED = 1469598103934665603
HEADER_BYTES = 4096
SLACK_BYTES = 64 << 20
MAX_TIERS = 8

# (name, offset, struct format) of every field, from the protocol's description
ARENA_FIELDS = [("magic", 0, "16s"), ("version", 16, "<I"), ("header_bytes", 20, "<I"), ("tier_count", 24, "<I"),
                ("slot_total", 32, "<Q"), ("arena_bytes", 40, "<Q"), ("pack_hash", 48, "<Q"), ("geom_hash", 56, "<Q"),
                ("created_pid", 64, "<Q"), ("created_start", 72, "<Q"), ("tier_max_tokens", 80, "<8Q"),
                ("tier_slot_count", 144, "<8Q"), ("tier_slot_bytes", 208, "<8Q"), ("tier_slot_off", 272, "<8Q")]
SLOT_FIELDS = [("magic", 0, "16s"), ("version", 16, "<I"), ("header_bytes", 20, "<I"), ("state", 24, "<I"),
               ("flags", 28, "<I"), ("tier", 32, "<I"), ("owner_pid", 40, "<Q"), ("owner_start", 48, "<Q"),
               ("nonce", 56, "<Q"), ("client_id", 64, "<Q"), ("request_id", 72, "<Q"), ("pack_hash", 80, "<Q"),
               ("geom_hash", 88, "<Q"), ("tokens", 96, "<Q"), ("payload_bytes", 104, "<Q"),
               ("payload_hash", 112, "<Q"), ("claimed_ms", 120, "<Q"), ("published_ms", 128, "<Q"),
               ("seq", 136, "<Q")]
ARENA_MAGIC = b"STRATA-HARENA-V1"
SLOT_MAGIC = b"STRATA-HSLOT-V1\0"


def split_spec(main_lo: int, main_hi: int, stages=(), draft_on_last: bool = True) -> str:
    later = ",".join(f"{lo}..{hi}" for lo, hi in stages)
    draft = "last" if draft_on_last and stages else "main"
    return f"main={main_lo}..{main_hi}|{later}|n={len(stages) + 1}|draft={draft}"


def geom_hash(geometry, spec: str) -> int:
    assert len(geometry) == 18
    stream = b"strata-handoff-geom-v1" + struct.pack("<18Q", *[g & (2**64 - 1) for g in geometry]) + spec.encode()
    h = sc_oracle.fnv1a64(stream, SEED)
    return h or 1


def arena_path(directory: str, pack_hash: int, spec: str, instance: str) -> str:
    p = directory if not directory or directory.endswith("/") else directory + "/"
    p += f"{pack_hash:016x}-{spec}"
    if instance:
        p += "/" + instance
    return p + "/arena"


def size_arena(tiers, priced):
    """tiers: [(max_tokens, slot_count)], priced: payload bytes per tier -> dict of the layout (or ValueError)."""
    if not tiers:
        raise ValueError("no tiers")
    if len(tiers) > MAX_TIERS or len(priced) != len(tiers):
        raise ValueError("tiers")
    slot_bytes, slot_off, off = [], [], HEADER_BYTES
    for i, ((tokens, count), p) in enumerate(zip(tiers, priced)):
        if tokens == 0 or count == 0 or (i and tokens <= tiers[i - 1][0]):
            raise ValueError("tier")
        sb = (p + 63) // 64 * 64 + SLACK_BYTES
        slot_bytes.append(sb)
        slot_off.append(off)
        off += count * (HEADER_BYTES + sb)
    return {"slot_bytes": slot_bytes, "slot_off": slot_off, "arena_bytes": off,
            "slot_total": sum(c for _, c in tiers), "max_tokens": max(t for t, _ in tiers)}


def slot_bases(layout, tiers):
    bases = []
    for (tokens, count), sb, off in zip(tiers, layout["slot_bytes"], layout["slot_off"]):
        bases += [(off + k * (HEADER_BYTES + sb), sb) for k in range(count)]
    return bases


def parse(raw: bytes, fields) -> dict:
    out = {}
    for name, off, fmt in fields:
        v = struct.unpack_from(fmt, raw, off)
        out[name] = v[0] if len(v) == 1 else list(v)
    return out
