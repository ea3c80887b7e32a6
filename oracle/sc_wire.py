"""CPU restatement of the reference's hand-off payload codec (the "wire" format), for checking.

TEST INFRASTRUCTURE ONLY: imported by tests/ and tests/golden/make_wire_vectors.py as the checker; the product never
imports it.  It restates include/strata/core/conversation_wire.hpp:24-81 (the format) and
src/core/conversation_wire.cpp:118-480 (encode), :480-880 (decode) in plain Python, field by field.  It is pinned by
the payloads, hashes and refusal verdicts the reference's own codec produced for the same specs
(tests/golden/wire_manifest.json, written by tests/golden/make_wire_vectors.py from oracle/_ref/ref_wire).

An image is a dict tree mirroring SavedConversation (include/strata/core/conversation_cache.hpp:51-162):
    image      {geometry[18], layer_lo, layer_hi, cvec, kv[kv], live: cp, checkpoints[cp], stage_parts[stage]}
    kv         {format, cells, heads, head_dim, page_size, pooled_rows, idx_dim, k, v, k_scale, v_scale, pooled}
    cp         {ids[int32], imgs[(start, hash)], gdn, ple, tails, dead, block_pos, used, stage_parts[cp]}
    stage      {layer_lo, layer_hi, state: cp, kv[kv]}
Buffers are `bytes`.
"""
from __future__ import annotations

import struct

import numpy as np

from . import sc_oracle

MAGIC = 0x48345253            # 'S','R','4','H' read little-endian (conversation_wire.hpp:180)
VERSION = 1
HEADER_BYTES = 256
RECORD_HEADER_BYTES = 16
BLOB_ALIGN = 64
KV_BODY_BYTES = 136           # i32 format, i32 pad, 6 x i64, 5 BLOBREFs (conversation_wire.cpp:101)
KIND_KV, KIND_CHECKPOINT, KIND_STAGE, KIND_END = 1, 2, 3, 0x21444E45
FLAG_CVEC, FLAG_STAGE_PARTS, FLAG_PARTIAL = 1, 2, 4
FLAGS_KNOWN = FLAG_CVEC | FLAG_STAGE_PARTS | FLAG_PARTIAL
MAX_DEPTH = 8
MAX_KV, MAX_CHECKPOINTS, MAX_STAGE_PARTS, MAX_IMAGES = 4096, 1 << 20, 64, 1 << 16
SEED = sc_oracle.REFERENCE_FNV_SEED

KV_BUFFERS = ("k", "v", "k_scale", "v_scale", "pooled")
CP_BUFFERS = ("gdn", "ple", "tails", "dead", "block_pos")


class WireRefusal(Exception):
    """The codec refused a payload or an image; nothing was produced."""


def _up64(n: int) -> int:
    return (n + 63) // 64 * 64


def payload_hash(payload: bytes) -> int:
    return sc_oracle.fnv1a64(payload, SEED)


# ---- sizes (conversation_wire.cpp:104-130) ---------------------------------------------------------------------------

def _ids_pad(n_ids: int) -> int:
    return 4 if (n_ids * 4) % 8 else 0


def _cp_body(cp: dict, depth: int, max_depth: int) -> int:
    if depth > max_depth:
        raise WireRefusal("checkpoint stage_parts nesting exceeds the bound")
    n = 8 + 4 * len(cp["ids"]) + _ids_pad(len(cp["ids"])) + 8 + 16 * len(cp["imgs"]) + 5 * 16 + 8 + 8
    for part in cp["stage_parts"]:
        n += RECORD_HEADER_BYTES + _cp_body(part, depth + 1, max_depth)
    return n


def _stage_body(st: dict, max_depth: int) -> int:
    return 16 + RECORD_HEADER_BYTES + _cp_body(st["state"], 0, max_depth) + 8 + \
        len(st["kv"]) * (RECORD_HEADER_BYTES + KV_BODY_BYTES)


# ---- encode -------------------------------------------------------------------------------------------------------------

class _Pool:
    """Blob offsets assigned in emission order, each 64-aligned relative to the pool start (conversation_wire.cpp:211-226)."""

    def __init__(self):
        self.entries: list[tuple[int, bytes]] = []
        self.rel = 0

    def add(self, buf: bytes) -> int:
        if not buf:
            return -1
        at = _up64(self.rel)
        self.entries.append((at, buf))
        self.rel = at + len(buf)
        return at


def _records(image: dict, pool: _Pool, pool_off: int, max_depth: int) -> bytes:
    out = bytearray()

    def ref(buf: bytes) -> bytes:
        at = pool.add(buf)
        return struct.pack("<QQ", len(buf), 0 if at < 0 else pool_off + at)

    def kv(k: dict) -> None:
        out.extend(struct.pack("<IIQ", KIND_KV, 0, KV_BODY_BYTES))
        out.extend(struct.pack("<iI6q", k["format"], 0, k["cells"], k["heads"], k["head_dim"], k["page_size"],
                               k["pooled_rows"], k["idx_dim"]))
        for name in KV_BUFFERS:
            out.extend(ref(k[name]))

    def checkpoint(cp: dict, depth: int) -> None:
        out.extend(struct.pack("<IIQ", KIND_CHECKPOINT, 0, _cp_body(cp, depth, max_depth)))
        ids = np.asarray(cp["ids"], dtype=np.int32)
        out.extend(struct.pack("<q", ids.size))
        out.extend(ids.astype("<i4").tobytes())
        out.extend(b"\0" * _ids_pad(ids.size))
        out.extend(struct.pack("<q", len(cp["imgs"])))
        for start, h in cp["imgs"]:
            out.extend(struct.pack("<qQ", start, h))
        for name in CP_BUFFERS:
            out.extend(ref(cp[name]))
        out.extend(struct.pack("<Qq", cp["used"], len(cp["stage_parts"])))
        for part in cp["stage_parts"]:
            checkpoint(part, depth + 1)

    for k in image["kv"]:
        kv(k)
    checkpoint(image["live"], 0)
    for cp in image["checkpoints"]:
        checkpoint(cp, 0)
    for st in image["stage_parts"]:
        out.extend(struct.pack("<IIQ", KIND_STAGE, 0, _stage_body(st, max_depth)))
        out.extend(struct.pack("<qq", st["layer_lo"], st["layer_hi"]))
        checkpoint(st["state"], 0)
        out.extend(struct.pack("<q", len(st["kv"])))
        for k in st["kv"]:
            kv(k)
    out.extend(struct.pack("<IIQ", KIND_END, 0, 0))
    return bytes(out)


def encode(image: dict, geom_hash: int = 0, pack_hash: int = 0, max_depth: int = MAX_DEPTH) -> bytes:
    """The payload of `image` (conversation_wire_encode): header, records, zero pad to 64, blob pool."""
    if image["live"]["stage_parts"]:
        raise WireRefusal("a parked image must keep its stage state in stage_parts, not in live")
    # pass 1: the record stream's length does not depend on the offsets it carries
    records_len = len(_records(image, _Pool(), 0, max_depth))
    pool_off = _up64(HEADER_BYTES + records_len)
    pool = _Pool()
    records = _records(image, pool, pool_off, max_depth)
    pool_bytes = _up64(pool.rel) if pool.entries else 0
    total = pool_off + pool_bytes
    flags = (FLAG_CVEC if image["cvec"] else 0) | (FLAG_STAGE_PARTS if image["stage_parts"] else 0)
    header = struct.pack("<IHH18qqqqqqqQQQQQQQ", MAGIC, VERSION, flags, *image["geometry"], image["layer_lo"],
                         image["layer_hi"], len(image["kv"]), len(image["checkpoints"]), len(image["stage_parts"]),
                         len(image["live"]["ids"]), pool_off, pool_bytes, geom_hash, pack_hash, total, 0, 0)
    assert len(header) == HEADER_BYTES
    payload = bytearray(total)
    payload[:HEADER_BYTES] = header
    payload[HEADER_BYTES:HEADER_BYTES + len(records)] = records
    for at, buf in pool.entries:
        payload[pool_off + at:pool_off + at + len(buf)] = buf
    return bytes(payload)


# ---- decode (conversation_wire.cpp:480-880) ------------------------------------------------------------------------------

class _Cursor:
    def __init__(self, data: bytes, begin: int, end: int):
        self.d, self.pos, self.end = data, begin, end

    def take(self, n: int) -> bytes:
        if n > self.end - self.pos:
            raise WireRefusal("the payload is shorter than its records claim")
        b = self.d[self.pos:self.pos + n]
        self.pos += n
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def i64(self) -> int:
        return struct.unpack("<q", self.take(8))[0]

    def zeros(self, n: int) -> None:
        if any(self.take(n)):
            raise WireRefusal("a reserved field is not zero")


def _count(n: int, cap: int, what: str, room: int, element: int) -> None:
    if n < 0 or n > cap or (element and n > room // element):
        raise WireRefusal(f"{what} {n} is out of bounds")


def decode(payload: bytes, geom_hash: int | None = None, pack_hash: int | None = None,
           check_payload_hash: int | None = None, geometry: list | None = None, stage_parts: int = -1,
           max_payload_bytes: int = 0, max_depth: int = MAX_DEPTH) -> dict:
    """Parse a payload with the reference decoder's checks, in its order; raises WireRefusal."""
    if len(payload) < HEADER_BYTES:
        raise WireRefusal("the payload is shorter than the header record")
    h = struct.unpack("<IHH18QQQqqqqQQQQQQQ", payload[:HEADER_BYTES])
    magic, version, flags = h[0], h[1], h[2]
    geo = list(h[3:21])
    (layer_lo, layer_hi, n_kv, n_cp, n_stage, live_tokens, pool_off, pool_bytes, g_hash, p_hash, total, p_field,
     reserved) = h[21:]
    if magic != MAGIC:
        raise WireRefusal("not a hand-off payload")
    if version != VERSION:
        raise WireRefusal("payload format version mismatch")
    if flags & FLAG_PARTIAL:
        raise WireRefusal("the payload says it is partial")
    if flags & ~FLAGS_KNOWN & 0xFFFF:
        raise WireRefusal("unknown header flag bits")
    if p_field != 0 or reserved != 0:
        raise WireRefusal("a reserved header field is not zero")
    if total < HEADER_BYTES:
        raise WireRefusal("the declared payload size is absurd")
    if max_payload_bytes and total > max_payload_bytes:
        raise WireRefusal("the payload declares more bytes than its slot")
    if total > len(payload):
        raise WireRefusal("the payload is truncated")
    if pool_off < HEADER_BYTES or pool_off % BLOB_ALIGN:
        raise WireRefusal("the blob pool does not start on a 64-byte boundary")
    if pool_bytes > total - pool_off:
        raise WireRefusal("the blob pool runs past the end of the payload")
    if (n_stage <= 0) if (flags & FLAG_STAGE_PARTS) else (n_stage > 0):
        raise WireRefusal("the stage-parts flag and the stage-parts count disagree")
    if geometry is not None and [g & 0xFFFFFFFFFFFFFFFF for g in geometry] != geo:
        raise WireRefusal("incompatible runtime geometry")
    if geom_hash is not None and g_hash != geom_hash:
        raise WireRefusal("geometry hash mismatch")
    if pack_hash is not None and p_hash != pack_hash:
        raise WireRefusal("pack hash mismatch")
    if stage_parts >= 0 and n_stage != stage_parts:
        raise WireRefusal("stage-part count mismatch")
    _count(n_kv, MAX_KV, "n_kv", 0, 0)
    _count(n_cp, MAX_CHECKPOINTS, "n_checkpoints", 0, 0)
    _count(n_stage, MAX_STAGE_PARTS, "n_stage_parts", 0, 0)
    if live_tokens < 0:
        raise WireRefusal("live_tokens is negative")
    if check_payload_hash is not None and payload_hash(payload[:total]) != check_payload_hash:
        raise WireRefusal("payload hash mismatch")
    pool_end = pool_off + pool_bytes

    def blobref(c: _Cursor) -> bytes:
        n, off = c.u64(), c.u64()
        if n == 0:
            if off:
                raise WireRefusal("a zero-length blob must be referenced as {0,0}")
            return b""
        if off < pool_off or off % BLOB_ALIGN:
            raise WireRefusal("a blob reference is not on a 64-byte boundary inside the pool")
        if off > pool_end or n > pool_end - off:
            raise WireRefusal("a blob reference runs past the end of the pool")
        return bytes(payload[off:off + n])

    def kv_body(c: _Cursor) -> dict:
        fmt = c.u32()
        c.zeros(4)
        k = {"format": struct.unpack("<i", struct.pack("<I", fmt))[0]}
        for name in ("cells", "heads", "head_dim", "page_size", "pooled_rows", "idx_dim"):
            k[name] = c.i64()
        for name in KV_BUFFERS:
            k[name] = blobref(c)
        return k

    def kv_record(c: _Cursor, what: str) -> dict:
        kind, f, b = c.u32(), c.u32(), c.u64()
        if kind != KIND_KV or f != 0 or b != KV_BODY_BYTES:
            raise WireRefusal(f"the {what} does not hold plain KV records")
        return kv_body(c)

    def checkpoint(c: _Cursor, depth: int) -> dict:
        if depth > max_depth:
            raise WireRefusal("stage_parts nested past the bound")
        kind, f, b = c.u32(), c.u32(), c.u64()
        if kind != KIND_CHECKPOINT:
            raise WireRefusal("expected a CHECKPOINT record")
        if f:
            raise WireRefusal("a record's flags field is not zero")
        if b > c.end - c.pos:
            raise WireRefusal("a record declares more bytes than the payload has")
        body_end = c.pos + b
        n_ids = c.i64()
        _count(n_ids, (1 << 63) // 8 - 1, "n_ids", body_end - c.pos, 4)
        ids = np.frombuffer(c.take(4 * n_ids), dtype="<i4").astype(np.int32)
        if _ids_pad(n_ids):
            c.zeros(4)
        n_imgs = c.i64()
        _count(n_imgs, MAX_IMAGES, "n_imgs", body_end - c.pos, 16)
        imgs = [(c.i64(), c.u64()) for _ in range(n_imgs)]
        cp = {"ids": ids, "imgs": imgs}
        for name in CP_BUFFERS:
            cp[name] = blobref(c)
        cp["used"] = c.u64()
        n_parts = c.i64()
        _count(n_parts, MAX_STAGE_PARTS, "checkpoint stage_parts", body_end - c.pos, RECORD_HEADER_BYTES)
        cp["stage_parts"] = [checkpoint(c, depth + 1) for _ in range(n_parts)]
        if c.pos != body_end:
            raise WireRefusal("a CHECKPOINT record's body does not end where its header said")
        return cp

    def stage(c: _Cursor) -> dict:
        kind, f, b = c.u32(), c.u32(), c.u64()
        if kind != KIND_STAGE:
            raise WireRefusal("expected a STAGE record")
        if f:
            raise WireRefusal("a record's flags field is not zero")
        if b > c.end - c.pos:
            raise WireRefusal("a record declares more bytes than the payload has")
        body_end = c.pos + b
        st = {"layer_lo": c.i64(), "layer_hi": c.i64()}
        st["state"] = checkpoint(c, 0)
        n = c.i64()
        _count(n, MAX_KV, "stage n_kv", body_end - c.pos, RECORD_HEADER_BYTES + KV_BODY_BYTES)
        st["kv"] = [kv_record(c, "stage's K/V array") for _ in range(n)]
        if c.pos != body_end:
            raise WireRefusal("a STAGE record's body does not end where its header said")
        return st

    c = _Cursor(payload, HEADER_BYTES, pool_off)
    image = {"geometry": [int(np.int64(np.uint64(g))) for g in geo],
             "layer_lo": int(np.int64(np.uint64(layer_lo))), "layer_hi": int(np.int64(np.uint64(layer_hi))),
             "cvec": bool(flags & FLAG_CVEC)}
    image["kv"] = [kv_record(c, "KV array") for _ in range(n_kv)]
    image["live"] = checkpoint(c, 0)
    image["checkpoints"] = [checkpoint(c, 0) for _ in range(n_cp)]
    image["stage_parts"] = [stage(c) for _ in range(n_stage)]
    try:
        kind, f, b = c.u32(), c.u32(), c.u64()
    except WireRefusal:
        raise WireRefusal("the record stream has no END marker")
    if kind != KIND_END or f != 0 or b != 0:
        raise WireRefusal("the END marker is malformed")
    c.zeros(pool_off - c.pos)
    if live_tokens != len(image["live"]["ids"]):
        raise WireRefusal("live_tokens disagrees with the live checkpoint's id count")
    return image


# ---- specs: the deterministic synthetic images shared with the reference driver and the C++ test -------------------

def _pattern(salt: int, n: int) -> bytes:
    i = np.arange(n, dtype=np.uint64)
    s = np.uint64(salt)
    v = s * np.uint64(131) + i * np.uint64(31) + (i >> np.uint64(8)) * np.uint64(7) + (i >> np.uint64(16)) * np.uint64(3)
    return (v & np.uint64(0xFF)).astype(np.uint8).tobytes()


def _mix(z: int) -> int:
    return int(sc_oracle.lib.sco_mix64(z & 0xFFFFFFFFFFFFFFFF))


def image_from_spec(text: str) -> tuple[dict, int, int]:
    """Build (image, geom_hash, pack_hash) from a wire spec (grammar and fill rule: oracle/ref_wire_driver.cpp)."""
    vals = [int(x) for x in text.split()]
    pos = 0
    salt = 1

    def nxt() -> int:
        nonlocal pos
        v = vals[pos]
        pos += 1
        return v

    def take_salt() -> int:
        nonlocal salt
        s = salt
        salt += 1
        return s

    def kv() -> dict:
        k = {name: nxt() for name in ("format", "cells", "heads", "head_dim", "page_size", "pooled_rows", "idx_dim")}
        lens = [nxt() for _ in KV_BUFFERS]
        for name, n in zip(KV_BUFFERS, lens):
            k[name] = _pattern(take_salt(), n)
        return k

    def checkpoint() -> dict:
        n_ids, n_imgs = nxt(), nxt()
        lens = [nxt() for _ in CP_BUFFERS]
        used, n_parts = nxt(), nxt()
        s = take_salt()
        i = np.arange(n_ids, dtype=np.uint64)
        ids = (np.uint64(s) * np.uint64(2654435761) + i * np.uint64(40503)).astype(np.uint32).view(np.int32)
        s = take_salt()
        imgs = [(4 * i2 + s, _mix(s * 1000003 + i2)) for i2 in range(n_imgs)]
        cp = {"ids": ids, "imgs": imgs}
        for name, n in zip(CP_BUFFERS, lens):
            cp[name] = _pattern(take_salt(), n)
        cp["used"] = used & 0xFFFFFFFFFFFFFFFF
        cp["stage_parts"] = [checkpoint() for _ in range(n_parts)]
        return cp

    g_hash, p_hash = nxt() & 0xFFFFFFFFFFFFFFFF, nxt() & 0xFFFFFFFFFFFFFFFF
    image = {"geometry": [nxt() for _ in range(18)], "layer_lo": nxt(), "layer_hi": nxt(), "cvec": nxt() != 0}
    image["kv"] = [kv() for _ in range(nxt())]
    image["live"] = checkpoint()
    image["checkpoints"] = [checkpoint() for _ in range(nxt())]
    stages = []
    for _ in range(nxt()):
        st = {"layer_lo": nxt(), "layer_hi": nxt()}
        st["state"] = checkpoint()
        st["kv"] = [kv() for _ in range(nxt())]
        stages.append(st)
    image["stage_parts"] = stages
    return image, g_hash, p_hash


def images_equal(a: dict, b: dict) -> bool:
    def cp_eq(x, y) -> bool:
        return (np.array_equal(np.asarray(x["ids"], np.int32), np.asarray(y["ids"], np.int32)) and
                [tuple(t) for t in x["imgs"]] == [tuple(t) for t in y["imgs"]] and
                all(x[n] == y[n] for n in CP_BUFFERS) and x["used"] == y["used"] and
                len(x["stage_parts"]) == len(y["stage_parts"]) and
                all(cp_eq(p, q) for p, q in zip(x["stage_parts"], y["stage_parts"])))

    def kv_eq(x, y) -> bool:
        return all(x[n] == y[n] for n in x)

    return (a["geometry"] == b["geometry"] and a["layer_lo"] == b["layer_lo"] and a["layer_hi"] == b["layer_hi"] and
            a["cvec"] == b["cvec"] and len(a["kv"]) == len(b["kv"]) and
            all(kv_eq(x, y) for x, y in zip(a["kv"], b["kv"])) and cp_eq(a["live"], b["live"]) and
            len(a["checkpoints"]) == len(b["checkpoints"]) and
            all(cp_eq(x, y) for x, y in zip(a["checkpoints"], b["checkpoints"])) and
            len(a["stage_parts"]) == len(b["stage_parts"]) and
            all(x["layer_lo"] == y["layer_lo"] and x["layer_hi"] == y["layer_hi"] and cp_eq(x["state"], y["state"]) and
                len(x["kv"]) == len(y["kv"]) and all(kv_eq(p, q) for p, q in zip(x["kv"], y["kv"]))
                for x, y in zip(a["stage_parts"], b["stage_parts"])))
