"""Python binding of include/sc_arena.h (libsc_core.so): the hand-off arena (the reference's HandoffArena, same file
format) and the movers between HBM and its slots.  Device memory and streams come from sc_handoff."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import sc_handoff as sc

LIB_PATH = Path(sc.LIB_PATH).parent / "libsc_core.so"
if not LIB_PATH.exists():
    raise ImportError(f"libsc_core.so is not built ({LIB_PATH}); run __graft_entry__.build() first")
lib = C.CDLL(str(LIB_PATH))

SC_EBUSY, SC_ESTALE = 5, 6
FREE, CLAIMED, READY = 0, 1, 2
FLAG_CANCELLED, FLAG_ABANDONED, FLAG_PARTIAL = 1, 2, 4


class Claim(C.Structure):
    _fields_ = [("index", C.c_int32), ("tier", C.c_uint32), ("base", C.c_uint64), ("payload_off", C.c_uint64),
                ("capacity", C.c_uint64), ("nonce", C.c_uint64)]


class Slot(C.Structure):
    _fields_ = [("index", C.c_int32), ("state", C.c_uint32), ("flags", C.c_uint32), ("tier", C.c_uint32),
                *[(n, C.c_uint64) for n in ("base", "capacity", "owner_pid", "owner_start", "nonce", "client_id",
                                            "request_id", "pack_hash", "geom_hash", "tokens", "payload_bytes",
                                            "payload_hash", "claimed_ms", "published_ms", "seq")]]


_P, _U64, _I32, _U32 = C.c_void_p, C.c_uint64, C.c_int32, C.c_uint32
_PU64 = C.POINTER(C.c_uint64)
_SIGS = {
    "sc_arena_last_error": (C.c_char_p, []),
    "sc_arena_size": (C.c_int, [_I32, _PU64, _PU64, _PU64, _PU64, _PU64, _PU64, C.c_char_p, _U64]),
    "sc_arena_geom_hash": (_U64, [C.POINTER(C.c_int64), C.c_char_p]),
    "sc_arena_open_writer": (C.c_int, [C.c_char_p, _I32, _PU64, _PU64, _PU64, _U64, _U64, _I32, C.c_int64,
                                       C.POINTER(_P)]),
    "sc_arena_open_reader": (C.c_int, [C.c_char_p, _U64, _U64, C.POINTER(_P)]),
    "sc_arena_close": (C.c_int, [_P]),
    "sc_arena_reserve": (C.c_int, [_P]),
    "sc_arena_claim_slot": (C.c_int, [_P, _U32, _U64, _U64, C.POINTER(Claim)]),
    "sc_arena_write": (C.c_int, [_P, C.POINTER(Claim), _U64, _P, _U64]),
    "sc_arena_publish": (C.c_int, [_P, C.POINTER(Claim), _U64, _U64, _U64]),
    "sc_arena_release": (C.c_int, [_P, _I32, _U64]),
    "sc_arena_abort": (C.c_int, [_P, _I32, _U64]),
    "sc_arena_cancel": (C.c_int, [_P, _I32, _U64]),
    "sc_arena_slot_info": (C.c_int, [_P, _I32, C.POINTER(Slot)]),
    "sc_arena_read_host": (C.c_int, [_P, _I32, _U64, _U64, _P, _U64, _I32, C.POINTER(Slot)]),
    "sc_mover_create": (C.c_int, [_U64, _I32, _I32, C.POINTER(_P)]),
    "sc_mover_destroy": (C.c_int, [_P]),
    "sc_mover_write": (C.c_int, [_P, _P, C.POINTER(Claim), _P, _U64, _P, _PU64]),
    "sc_mover_publish": (C.c_int, [_P, _P, C.POINTER(Claim), _P, _U64, _U64, _P]),
    "sc_mover_read": (C.c_int, [_P, _P, _I32, _U64, _U64, _P, _U64, _P, _I32, C.POINTER(Slot)]),
    "sc_mover_last": (C.c_int, [_P, _PU64] + [C.POINTER(C.c_double)] * 4),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype, _fn.argtypes = _res, _args
EXPORTS = tuple(_SIGS)


class ArenaError(RuntimeError):
    def __init__(self, code: int, where: str):
        self.code = code
        super().__init__(f"{where}: status {code}: {lib.sc_arena_last_error().decode()}")


def _check(code: int, where: str) -> None:
    if code != sc.SC_OK:
        raise ArenaError(code, where)


def _u64s(values):
    return (C.c_uint64 * max(1, len(values)))(*values)


def size(tiers, priced):
    """handoff_size_arena: (slot_bytes, slot_off, arena_bytes, describe) of [(max_tokens, slots)] and priced bytes."""
    n = len(tiers)
    sb, so, total, desc = _u64s([0] * n), _u64s([0] * n), C.c_uint64(), C.create_string_buffer(256)
    _check(lib.sc_arena_size(n, _u64s([t for t, _ in tiers]), _u64s([c for _, c in tiers]), _u64s(priced), sb, so,
                             C.byref(total), desc, 256), "sc_arena_size")
    return list(sb)[:n], list(so)[:n], total.value, desc.value.decode()


def geom_hash(geometry, spec: str) -> int:
    g = (C.c_int64 * 18)(*geometry)
    return int(lib.sc_arena_geom_hash(g, spec.encode()))


class Arena:
    """One open arena (writer or reader)."""

    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def writer(cls, path, tiers, priced, pack_hash, geom_hash, reserve=False, lease_ms=-1):
        h = C.c_void_p()
        _check(lib.sc_arena_open_writer(str(path).encode(), len(tiers), _u64s([t for t, _ in tiers]),
                                        _u64s([c for _, c in tiers]), _u64s(priced), pack_hash, geom_hash, int(reserve),
                                        lease_ms, C.byref(h)), "sc_arena_open_writer")
        return cls(h)

    @classmethod
    def reader(cls, path, pack_hash, geom_hash):
        h = C.c_void_p()
        _check(lib.sc_arena_open_reader(str(path).encode(), pack_hash, geom_hash, C.byref(h)), "sc_arena_open_reader")
        return cls(h)

    def close(self):
        if self.handle:
            lib.sc_arena_close(self.handle)
            self.handle = None

    def reserve(self):
        """Writer: commit the file's pages and map them; reader: map the file read-only, populated."""
        _check(lib.sc_arena_reserve(self.handle), "sc_arena_reserve")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def claim(self, tier, client_id, request_id) -> Claim:
        c = Claim()
        _check(lib.sc_arena_claim_slot(self.handle, tier, client_id, request_id, C.byref(c)), "sc_arena_claim_slot")
        return c

    def write(self, claim, offset, data):
        """Host bytes (bytes or a contiguous numpy array, passed without a copy) into the claimed slot."""
        import numpy as np
        a = np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) else \
            np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        _check(lib.sc_arena_write(self.handle, C.byref(claim), offset, a.ctypes.data if a.size else None, a.size),
               "sc_arena_write")

    def publish(self, claim, tokens, payload_bytes, payload_hash):
        _check(lib.sc_arena_publish(self.handle, C.byref(claim), tokens, payload_bytes, payload_hash), "sc_arena_publish")

    def release(self, index, nonce):
        _check(lib.sc_arena_release(self.handle, index, nonce), "sc_arena_release")

    def abort(self, index, nonce):
        _check(lib.sc_arena_abort(self.handle, index, nonce), "sc_arena_abort")

    def cancel(self, index, nonce):
        _check(lib.sc_arena_cancel(self.handle, index, nonce), "sc_arena_cancel")

    def slot(self, index) -> Slot:
        s = Slot()
        _check(lib.sc_arena_slot_info(self.handle, index, C.byref(s)), "sc_arena_slot_info")
        return s

    def read_host(self, index, nonce, client_id, capacity, check_hash=True):
        """The reference's reader path on the host: (payload bytes, Slot)."""
        import numpy as np
        out = np.empty(max(1, capacity), np.uint8)
        s = Slot()
        _check(lib.sc_arena_read_host(self.handle, index, nonce, client_id, out.ctypes.data, capacity, int(check_hash),
                                      C.byref(s)), "sc_arena_read_host")
        return out[:s.payload_bytes], s


class Mover:
    """Pinned staging + host copy threads moving payloads between device memory and arena slots."""

    def __init__(self, chunk_bytes=64 << 20, depth=4, threads=8):
        self.handle = C.c_void_p()
        _check(lib.sc_mover_create(chunk_bytes, depth, threads, C.byref(self.handle)), "sc_mover_create")

    def destroy(self):
        if self.handle:
            lib.sc_mover_destroy(self.handle)
            self.handle = None

    def write(self, arena, claim, device_ptr, nbytes, stream=None, want_hash=True):
        h = C.c_uint64()
        _check(lib.sc_mover_write(self.handle, arena.handle, C.byref(claim), device_ptr, nbytes, stream,
                                  C.byref(h) if want_hash else None), "sc_mover_write")
        return h.value if want_hash else None

    def publish(self, arena, claim, device_ptr, nbytes, tokens, stream=None):
        _check(lib.sc_mover_publish(self.handle, arena.handle, C.byref(claim), device_ptr, nbytes, tokens, stream),
               "sc_mover_publish")

    def read(self, arena, index, nonce, client_id, device_ptr, capacity, stream=None, verify=True) -> Slot:
        s = Slot()
        _check(lib.sc_mover_read(self.handle, arena.handle, index, nonce, client_id, device_ptr, capacity, stream,
                                 int(verify), C.byref(s)), "sc_mover_read")
        return s

    def last(self):
        """(bytes, ms, hash_ms, copy_ms, wait_ms) of the last transfer."""
        b, ms, hms, cms, wms = C.c_uint64(), C.c_double(), C.c_double(), C.c_double(), C.c_double()
        _check(lib.sc_mover_last(self.handle, C.byref(b), C.byref(ms), C.byref(hms), C.byref(cms), C.byref(wms)),
               "sc_mover_last")
        return b.value, ms.value, hms.value, cms.value, wms.value
