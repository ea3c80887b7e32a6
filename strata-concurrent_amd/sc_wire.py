"""Python binding of include/sc_wire.h (libsc_core.so): hand-off payloads written from and mounted into a decode slot
on the device.  Device memory, streams and slots come from sc_handoff (the same HIP runtime)."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import sc_handoff as sc

LIB_PATH = Path(sc.LIB_PATH).parent / "libsc_core.so"
if not LIB_PATH.exists():
    raise ImportError(f"libsc_core.so is not built ({LIB_PATH}); run __graft_entry__.build() first")
lib = C.CDLL(str(LIB_PATH))


class Live(C.Structure):
    _fields_ = [("geometry", C.c_int64 * 18), ("layer_lo", C.c_int64), ("layer_hi", C.c_int64), ("cvec", C.c_int32),
                ("draft_record", C.c_int32), ("idx_dim", C.c_int64), ("ids", C.POINTER(C.c_int32)), ("n_ids", C.c_int64),
                ("img_start", C.POINTER(C.c_int64)), ("img_hash", C.POINTER(C.c_uint64)), ("n_imgs", C.c_int64),
                ("used", C.c_uint64), ("small", C.c_void_p * 4), ("small_bytes", C.c_uint64 * 4)]


class Stage(C.Structure):
    """One later stage of a layer split: its f16 slot, geometry, layer range and (encode) small host buffers."""
    _fields_ = [("geometry", sc.Geometry), ("slot", sc.DecodeSlot), ("layer_lo", C.c_int64), ("layer_hi", C.c_int64),
                ("small", C.c_void_p * 4), ("small_bytes", C.c_uint64 * 4)]


_P, _I64, _U64, _I32 = C.c_void_p, C.c_int64, C.c_uint64, C.c_int32
for _name, _res, _args in (
    ("sc_wire_last_error", C.c_char_p, []),
    ("sc_wire_encoder_create", C.c_int, [C.POINTER(sc.Geometry), C.POINTER(sc.DecodeSlot), _I64, C.POINTER(Live), _U64,
                                         _U64, C.POINTER(_P)]),
    ("sc_wire_encoder_create_split", C.c_int, [C.POINTER(sc.Geometry), C.POINTER(sc.DecodeSlot), _I64,
                                               C.POINTER(Live), C.POINTER(Stage), _I32, _U64, _U64, C.POINTER(_P)]),
    ("sc_wire_encoder_create_layers", C.c_int, [C.POINTER(sc.Geometry), C.POINTER(sc.SlotLayers), _I64,
                                                C.POINTER(Live), _U64, _U64, C.POINTER(_P)]),
    ("sc_wire_encoder_bytes", _U64, [_P]),
    ("sc_wire_encoder_pool_offset", _U64, [_P]),
    ("sc_wire_encode_async", C.c_int, [_P, _P, _U64, _P, _P]),
    ("sc_wire_encode_segments_async", C.c_int, [_P, C.POINTER(sc.Segments), _P]),
    ("sc_wire_encoder_hash", C.c_int, [_P, C.POINTER(_U64)]),
    ("sc_wire_encoder_set_carry", C.c_int, [_P, _P]),
    ("sc_wire_encoder_destroy", C.c_int, [_P]),
    ("sc_wire_decoder_open", C.c_int, [_P, _U64, C.POINTER(sc.Geometry), C.POINTER(sc.DecodeSlot), C.POINTER(C.c_int64),
                                       _U64, _U64, _I32, _U64, _I32, C.POINTER(_P)]),
    ("sc_wire_decoder_open_split", C.c_int, [_P, _U64, C.POINTER(sc.Geometry), C.POINTER(sc.DecodeSlot),
                                             C.POINTER(Stage), _I32, C.POINTER(C.c_int64), _U64, _U64, _I32, _U64, _I32,
                                             C.POINTER(_P)]),
    ("sc_wire_decoder_open_layers", C.c_int, [_P, _U64, C.POINTER(sc.Geometry), C.POINTER(sc.SlotLayers),
                                              C.POINTER(C.c_int64), _U64, _U64, _I32, _U64, _I32, C.POINTER(_P)]),
    ("sc_wire_decoder_open_segments", C.c_int, [C.POINTER(sc.Segments), _U64, C.POINTER(sc.Geometry),
                                                C.POINTER(sc.DecodeSlot), C.POINTER(C.c_int64), _U64, _U64, _I32, _U64,
                                                _I32, C.POINTER(_P)]),
    ("sc_wire_decoder_open_layers_segments", C.c_int, [C.POINTER(sc.Segments), _U64, C.POINTER(sc.Geometry),
                                                       C.POINTER(sc.SlotLayers), C.POINTER(C.c_int64), _U64, _U64, _I32,
                                                       _U64, _I32, C.POINTER(_P)]),
    ("sc_wire_decoder_tokens", _I64, [_P]),
    ("sc_wire_decoder_restore", C.c_int, [_P, _P]),
    ("sc_wire_decoder_set_carry", C.c_int, [_P, _P]),
    ("sc_wire_decoder_reopen", C.c_int, [_P, _P, _U64, _U64]),
    ("sc_wire_decoder_live_ids", C.c_int, [_P, C.POINTER(C.c_int32), _I64, C.POINTER(_I64)]),
    ("sc_wire_decoder_small", C.c_int, [_P, _I32, C.POINTER(C.c_uint8), _U64, C.POINTER(_U64)]),
    ("sc_wire_decoder_stage_small", C.c_int, [_P, _I32, _I32, C.POINTER(C.c_uint8), _U64, C.POINTER(_U64)]),
    ("sc_wire_decoder_destroy", C.c_int, [_P]),
):
    _fn = getattr(lib, _name)
    _fn.restype, _fn.argtypes = _res, _args

EXPORTS = ("sc_wire_last_error", "sc_wire_encoder_create", "sc_wire_encoder_create_split",
           "sc_wire_encoder_create_layers", "sc_wire_encoder_bytes", "sc_wire_encoder_pool_offset",
           "sc_wire_encode_async", "sc_wire_encode_segments_async", "sc_wire_encoder_hash", "sc_wire_encoder_set_carry",
           "sc_wire_encoder_destroy",
           "sc_wire_decoder_open", "sc_wire_decoder_open_split", "sc_wire_decoder_open_layers",
           "sc_wire_decoder_open_segments", "sc_wire_decoder_open_layers_segments", "sc_wire_decoder_tokens",
           "sc_wire_decoder_restore", "sc_wire_decoder_set_carry", "sc_wire_decoder_reopen", "sc_wire_decoder_live_ids", "sc_wire_decoder_small", "sc_wire_decoder_stage_small",
           "sc_wire_decoder_destroy")


class WireError(RuntimeError):
    def __init__(self, code: int, where: str):
        self.code = code
        super().__init__(f"{where}: status {code}: {lib.sc_wire_last_error().decode()}")


def _check(code: int, where: str) -> None:
    if code != sc.SC_OK:
        raise WireError(code, where)


def make_live(geometry, ids, layer_lo=0, layer_hi=0, cvec=True, draft_record=True, idx_dim=0, imgs=(), used=0,
              small=(b"", b"", b"", b"")) -> tuple[Live, tuple]:
    """A Live struct plus the host arrays it points into (keep both alive while the encoder is created)."""
    import numpy as np
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    starts = np.ascontiguousarray([s for s, _ in imgs] or [0], dtype=np.int64)
    hashes = np.ascontiguousarray([h for _, h in imgs] or [0], dtype=np.uint64)
    smalls = [np.frombuffer(bytes(b), dtype=np.uint8) if len(b) else np.zeros(1, np.uint8) for b in small]
    lv = Live()
    for i, g in enumerate(geometry):
        lv.geometry[i] = int(g)
    lv.layer_lo, lv.layer_hi, lv.cvec, lv.draft_record, lv.idx_dim = layer_lo, layer_hi, int(cvec), int(draft_record), idx_dim
    lv.ids = ids.ctypes.data_as(C.POINTER(C.c_int32))
    lv.n_ids = ids.size
    lv.img_start = starts.ctypes.data_as(C.POINTER(C.c_int64))
    lv.img_hash = hashes.ctypes.data_as(C.POINTER(C.c_uint64))
    lv.n_imgs = len(imgs)
    lv.used = used
    for i, (b, arr) in enumerate(zip(small, smalls)):
        lv.small[i] = arr.ctypes.data
        lv.small_bytes[i] = len(b)
    return lv, (ids, starts, hashes, smalls)


def make_stages(stages) -> tuple:
    """A Stage array from (geometry, slot, layer_lo, layer_hi, small) tuples (`small` the four byte strings, or None
    when decoding), plus the host arrays it points into (keep both alive while the encoder or decoder is created)."""
    import numpy as np
    arr = (Stage * max(len(stages), 1))()
    keep = []
    for i, (geo, slot, lo, hi, small) in enumerate(stages):
        st = arr[i]
        st.geometry = geo
        cs = slot.c_struct()
        keep.append(cs)
        st.slot = cs
        st.layer_lo, st.layer_hi = lo, hi
        for k, b in enumerate(small or (b"",) * 4):
            buf = np.frombuffer(bytes(b), dtype=np.uint8) if len(b) else np.zeros(1, np.uint8)
            keep.append(buf)
            st.small[k] = buf.ctypes.data
            st.small_bytes[k] = len(b)
    return arr, keep


class Encoder:
    """The device encoder of a slot: an f16 decode slot (sc_handoff.Slot) or a slot in any K/V format
    (sc_handoff.LayerPools); with `stages` (from make_stages) a layer-split payload of an f16 slot."""

    def __init__(self, geo, slot, tokens: int, live: Live, geom_hash: int = 0, pack_hash: int = 0, stages=None,
                 n_stages: int = 0):
        self._slot = slot.c_struct()
        h = C.c_void_p()
        if stages is not None:
            _check(lib.sc_wire_encoder_create_split(C.byref(geo), C.byref(self._slot), tokens, C.byref(live), stages,
                                                    n_stages, geom_hash, pack_hash, C.byref(h)),
                   "sc_wire_encoder_create_split")
        else:
            create = lib.sc_wire_encoder_create_layers if isinstance(slot, sc.LayerPools) else lib.sc_wire_encoder_create
            _check(create(C.byref(geo), C.byref(self._slot), tokens, C.byref(live), geom_hash, pack_hash, C.byref(h)),
                   "sc_wire_encoder_create")
        self.handle = h.value

    @property
    def bytes(self) -> int:
        return int(lib.sc_wire_encoder_bytes(self.handle))

    @property
    def pool_offset(self) -> int:
        return int(lib.sc_wire_encoder_pool_offset(self.handle))

    def encode(self, payload_ptr: int, capacity: int, stream=None, gathered=None) -> None:
        """Enqueue the encode; `gathered` (an sc_handoff.Event) is recorded once the payload bytes are in place."""
        _check(lib.sc_wire_encode_async(self.handle, payload_ptr, capacity, sc._stream(stream),
                                        gathered.handle if gathered is not None else None), "sc_wire_encode_async")

    def encode_segments(self, seg_ptrs, segment_bytes: int, stream=None) -> None:
        """Enqueue the encode straight into a payload held in segments (sc_wire_encode_segments_async)."""
        segs, keep = sc.segments_struct(seg_ptrs, segment_bytes)
        _check(lib.sc_wire_encode_segments_async(self.handle, C.byref(segs), sc._stream(stream)),
               "sc_wire_encode_segments_async")

    def set_carry(self, carry_ptr) -> None:
        """Later encodes also write the payload's carries at `carry_ptr` (None stops it; sc_wire_encoder_set_carry)."""
        _check(lib.sc_wire_encoder_set_carry(self.handle, carry_ptr), "sc_wire_encoder_set_carry")

    def hash(self) -> int:
        out = C.c_uint64(0)
        _check(lib.sc_wire_encoder_hash(self.handle, C.byref(out)), "sc_wire_encoder_hash")
        return int(out.value)

    def destroy(self) -> None:
        if self.handle:
            lib.sc_wire_encoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Decoder:
    """A payload opened for a slot.  `payload_ptr` is a contiguous device payload, or `segments` = (device pointers,
    segment_bytes) a payload held in segments (another process's imported ones), mounted where it lies."""

    def __init__(self, payload_ptr: int, nbytes: int, geo, slot, geometry=None, geom_hash=0, pack_hash=0,
                 check_identity=False, payload_hash=0, check_hash=False, stages=None, n_stages: int = 0,
                 segments=None, carry=None):
        self._slot = slot.c_struct()
        self._geo18 = (C.c_int64 * 18)(*geometry) if geometry is not None else None
        h = C.c_void_p()
        if segments is not None:
            if stages is not None:
                raise ValueError("a layer-split payload is not mounted from segments")
            segs, keep = sc.segments_struct(*segments)
            open_ = (lib.sc_wire_decoder_open_layers_segments if isinstance(slot, sc.LayerPools)
                     else lib.sc_wire_decoder_open_segments)
            _check(open_(C.byref(segs), nbytes, C.byref(geo), C.byref(self._slot), self._geo18, geom_hash, pack_hash,
                         int(check_identity), payload_hash, int(check_hash), C.byref(h)), "sc_wire_decoder_open_segments")
        elif stages is not None:
            _check(lib.sc_wire_decoder_open_split(payload_ptr, nbytes, C.byref(geo), C.byref(self._slot), stages,
                                                  n_stages, self._geo18, geom_hash, pack_hash, int(check_identity),
                                                  payload_hash, int(check_hash), C.byref(h)),
                   "sc_wire_decoder_open_split")
        else:
            open_ = lib.sc_wire_decoder_open_layers if isinstance(slot, sc.LayerPools) else lib.sc_wire_decoder_open
            _check(open_(payload_ptr, nbytes, C.byref(geo), C.byref(self._slot), self._geo18, geom_hash, pack_hash,
                         int(check_identity), payload_hash, int(check_hash), C.byref(h)), "sc_wire_decoder_open")
        self.handle = h.value
        if carry is not None:   # the payload's carries as its encoder wrote them (sc_wire_decoder_set_carry)
            _check(lib.sc_wire_decoder_set_carry(self.handle, carry), "sc_wire_decoder_set_carry")

    @property
    def tokens(self) -> int:
        return int(lib.sc_wire_decoder_tokens(self.handle))

    def restore(self, stream=None) -> None:
        _check(lib.sc_wire_decoder_restore(self.handle, sc._stream(stream)), "sc_wire_decoder_restore")

    def reopen(self, payload_ptr, nbytes: int, payload_hash: int = 0, carry=None) -> None:
        """Open this decoder again for the next payload (None: the same segments), keeping its buffers and, when the
        place, slot and blob offsets are unchanged, its scatter plan (sc_wire_decoder_reopen)."""
        _check(lib.sc_wire_decoder_reopen(self.handle, payload_ptr, nbytes, payload_hash), "sc_wire_decoder_reopen")
        if carry is not None:
            _check(lib.sc_wire_decoder_set_carry(self.handle, carry), "sc_wire_decoder_set_carry")

    def live_ids(self):
        import numpy as np
        out = np.zeros(max(self.tokens, 1), dtype=np.int32)
        n = C.c_int64(0)
        _check(lib.sc_wire_decoder_live_ids(self.handle, out.ctypes.data_as(C.POINTER(C.c_int32)), out.size, C.byref(n)),
               "sc_wire_decoder_live_ids")
        return out[: n.value]

    def small(self, which: int) -> bytes:
        import numpy as np
        n = C.c_uint64(0)
        lib.sc_wire_decoder_small(self.handle, which, None, 0, C.byref(n))
        out = np.zeros(max(n.value, 1), dtype=np.uint8)
        _check(lib.sc_wire_decoder_small(self.handle, which, out.ctypes.data_as(C.POINTER(C.c_uint8)), out.size,
                                         C.byref(n)), "sc_wire_decoder_small")
        return out[: n.value].tobytes()

    def stage_small(self, stage: int, which: int) -> bytes:
        import numpy as np
        n = C.c_uint64(0)
        lib.sc_wire_decoder_stage_small(self.handle, stage, which, None, 0, C.byref(n))
        out = np.zeros(max(n.value, 1), dtype=np.uint8)
        _check(lib.sc_wire_decoder_stage_small(self.handle, stage, which, out.ctypes.data_as(C.POINTER(C.c_uint8)),
                                               out.size, C.byref(n)), "sc_wire_decoder_stage_small")
        return out[: n.value].tobytes()

    def destroy(self) -> None:
        if self.handle:
            lib.sc_wire_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
