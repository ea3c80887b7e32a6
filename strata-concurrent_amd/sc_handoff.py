"""Python binding of libsc_handoff.so (include/sc_handoff.h) over ctypes, plus device-buffer helpers.

Device memory, streams and events come from the library itself (hipMalloc / hipStreamCreate through its C-ABI), so
a process that uses this module runs exactly one HIP runtime - the one the library links, as a C++ engine would.
Importing this module loads the built library and fails loudly when it is missing: there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("SC_HANDOFF_LIB", _HERE / "lib" / "libsc_handoff.so"))
if not LIB_PATH.exists():
    raise ImportError(f"libsc_handoff.so is not built ({LIB_PATH}); run __graft_entry__.build() first")
lib = C.CDLL(str(LIB_PATH))

SC_OK, SC_EINVAL, SC_EHIP, SC_ENOMEM, SC_ERANGE = 0, 1, 2, 3, 4
SC_ETIMEOUT = 7   # 5 and 6 are sc_arena.h's SC_EBUSY and SC_ESTALE
SC_FNV_FORCE_FAULT = 0xFFFFFFFF   # sc_fnv1a64_set_spin_limit: every look-back wait runs out (failure tests)
SC_DTYPE_F16, SC_DTYPE_F32 = 0, 1
SC_BLOB_K, SC_BLOB_V, SC_BLOB_GDN = 1, 2, 3


class Geometry(C.Structure):
    _fields_ = [(name, C.c_int64) for name in (
        "n_layers", "qsa_interval", "n_head_kv", "head_dim", "page_size", "ssm_state_size", "ssm_k_heads",
        "ssm_v_heads", "ssm_d_conv", "ssm_conv_channels", "idx_key_dim")]

    @property
    def n_qsa(self) -> int:
        return self.n_layers // self.qsa_interval

    @property
    def n_gdn(self) -> int:
        return self.n_layers - self.n_qsa

    @property
    def gdn_row_floats(self) -> int:
        s = self.ssm_state_size
        return s * self.ssm_v_heads * s + self.ssm_conv_channels * (self.ssm_d_conv - 1)

    def cells(self, tokens: int) -> int:
        ps = self.page_size
        return (tokens + ps - 1) // ps * ps


class PrefillView(C.Structure):
    _fields_ = [
        ("tokens", C.c_int64), ("pos0", C.c_int64), ("kv_dtype", C.c_int32), ("with_gdn", C.c_int32),
        ("k", C.POINTER(C.c_void_p)), ("v", C.POINTER(C.c_void_p)),
        ("rec", C.POINTER(C.c_void_p)), ("conv", C.POINTER(C.c_void_p)),
        ("conv_rows", C.c_int64), ("conv_ld", C.c_int64)]


class KvPools(C.Structure):
    """sc_kv_pools (strata::kernels::KvHostPools): a layer's host copy or staging pool; unused members NULL."""
    _fields_ = [("k_pool", C.c_void_p), ("v_pool", C.c_void_p), ("k_q", C.c_void_p), ("v_q", C.c_void_p),
                ("k_scale", C.c_void_p), ("v_scale", C.c_void_p), ("k_q4", C.c_void_p), ("v_q4", C.c_void_p)]


class DecodeSlot(C.Structure):
    _fields_ = [
        ("n_pages", C.c_int64), ("max_cells", C.c_int64),
        ("k_pool", C.POINTER(C.c_void_p)), ("v_pool", C.POINTER(C.c_void_p)),
        ("page_table", C.POINTER(C.c_void_p)), ("gdn_state", C.c_void_p),
        ("host", C.POINTER(KvPools)), ("stage", C.POINTER(KvPools))]


class KvRuns(C.Structure):
    _fields_ = [("src", C.c_void_p * 4), ("dst", C.c_void_p * 4), ("len", C.c_uint64 * 4), ("n", C.c_int32)]


class BatchDesc(C.Structure):
    _fields_ = [("n_slots", C.c_int32), ("lens", C.c_void_p), ("max_tokens", C.c_int64), ("staging", C.c_void_p),
                ("staging_bytes", C.c_uint64), ("chunk_tokens", C.c_int64),
                ("chunk_k", C.POINTER(C.c_void_p)), ("chunk_v", C.POINTER(C.c_void_p)),
                ("arena_k", C.POINTER(C.c_void_p)), ("arena_v", C.POINTER(C.c_void_p)), ("arena_pages", C.c_int64),
                ("tables", C.POINTER(C.c_void_p)), ("table_pages", C.c_int64), ("gdn", C.POINTER(C.c_void_p)),
                ("lens_out", C.c_void_p)]


SC_KV_F16, SC_KV_INT8, SC_KV_Q4, SC_KV_K8V4 = 0, 1, 2, 3


class QuantSlot(C.Structure):
    _fields_ = [("n_pages", C.c_int64), ("max_cells", C.c_int64), ("format", C.c_int32),
                ("k_codes", C.POINTER(C.c_void_p)), ("v_codes", C.POINTER(C.c_void_p)),
                ("k_scale", C.POINTER(C.c_void_p)), ("v_scale", C.POINTER(C.c_void_p)),
                ("page_table", C.POINTER(C.c_void_p)), ("gdn_state", C.c_void_p),
                ("host", C.POINTER(KvPools)), ("stage", C.POINTER(KvPools))]


class BlobMap(C.Structure):
    _fields_ = [("k_off", C.POINTER(C.c_uint64)), ("v_off", C.POINTER(C.c_uint64)), ("gdn_off", C.c_uint64),
                ("zero", C.POINTER(C.c_uint64)), ("n_zero", C.c_int64)]


SC_N_BUF = 5                     # K, V, K scales, V scales, indexer pooled rows (SC_BUF_* order)
ABSENT = 0xFFFFFFFFFFFFFFFF      # the offset of an empty blob in sc_image_layout_layers


class SlotLayers(C.Structure):
    _fields_ = [("format", C.c_int32), ("with_index", C.c_int32), ("max_cells", C.c_int64),
                ("pooled_capacity", C.c_int64), ("buf", C.POINTER(C.c_void_p) * SC_N_BUF), ("gdn_state", C.c_void_p)]


class LayersMap(C.Structure):
    _fields_ = [("off", C.POINTER(C.c_uint64)), ("zero", C.POINTER(C.c_uint64)), ("n_zero", C.c_int64)]


class ImageBlob(C.Structure):
    _fields_ = [("kind", C.c_int32), ("layer", C.c_int32), ("offset", C.c_uint64), ("bytes", C.c_uint64)]


_P = C.c_void_p
_I64, _U64 = C.c_int64, C.c_uint64
_GEO = C.POINTER(Geometry)
class Segments(C.Structure):
    """sc_segments: a payload held in segments (byte o at ptr[o // segment_bytes] + o % segment_bytes)."""
    _fields_ = [("n", C.c_int32), ("segment_bytes", C.c_uint64), ("ptr", C.POINTER(C.c_void_p))]


def segments_struct(ptrs, segment_bytes: int) -> tuple[Segments, object]:
    """A Segments struct over device pointers, plus the host array it points into (keep both alive)."""
    arr = (C.c_void_p * max(len(ptrs), 1))(*ptrs)
    return Segments(n=len(ptrs), segment_bytes=segment_bytes, ptr=C.cast(arr, C.POINTER(C.c_void_p))), arr


class IpcSegment(C.Structure):
    """sc_ipc_segment: one exported device allocation (a 64-byte memory handle and its size)."""
    _fields_ = [("handle", C.c_uint8 * 64), ("bytes", C.c_uint64)]


IPC_MAX_SEGMENT = 1 << 30
IPC_MAX_SEGMENTS = 64

_SIGS = {
    "sc_last_error": (C.c_char_p, []),
    "sc_version": (C.c_char_p, []),
    "sc_n_qsa_layers": (_I64, [_GEO]),
    "sc_n_gdn_layers": (_I64, [_GEO]),
    "sc_gdn_row_floats": (_I64, [_GEO]),
    "sc_kv_cells": (_I64, [_GEO, _I64]),
    "sc_payload_bytes": (_U64, [_GEO, _I64]),
    "sc_image_layout": (C.c_int, [_GEO, _I64, C.POINTER(ImageBlob), C.POINTER(_I64), C.POINTER(_U64)]),
    "sc_plan_carve": (C.c_int, [_GEO, C.POINTER(PrefillView), C.POINTER(DecodeSlot), C.POINTER(_P)]),
    "sc_plan_retarget": (C.c_int, [_P, C.POINTER(PrefillView), _P]),
    "sc_plan_gather": (C.c_int, [_GEO, C.POINTER(PrefillView), _P, _U64, C.POINTER(_P)]),
    "sc_plan_scatter": (C.c_int, [_GEO, _P, _U64, _I64, C.POINTER(DecodeSlot), C.POINTER(_P)]),
    "sc_plan_capture": (C.c_int, [_GEO, C.POINTER(DecodeSlot), _I64, _P, _U64, C.POINTER(_P)]),
    "sc_plan_copies": (C.c_int, [_P, C.c_int32, C.POINTER(_P)]),
    "sc_plan_launch": (C.c_int, [_P, _P]),
    "sc_plan_launch_gated": (C.c_int, [_P, _P, _P]),
    "sc_batch_staging_layout": (C.c_int, [_GEO, C.POINTER(_I64), C.c_int32, C.POINTER(_U64), C.POINTER(_U64)]),
    "sc_plan_resume_append": (C.c_int, [_GEO, C.POINTER(BatchDesc), C.POINTER(_P)]),
    "sc_plan_payload_bytes": (_U64, [_P]),
    "sc_plan_set_grid": (C.c_int, [_P, _I64]),
    "sc_set_order_min_pages": (_I64, [_I64]),
    "sc_plan_order_groups": (C.c_int, [_P]),
    "sc_plan_destroy": (C.c_int, [_P]),
    "sc_park_async": (C.c_int, [_GEO, C.POINTER(DecodeSlot), _I64, _P, _U64, _P, _P]),
    "sc_resume_async": (C.c_int, [_GEO, _P, _U64, _I64, C.POINTER(DecodeSlot), _P, _P]),
    "sc_kv_ring_restore": (C.c_int, [_P, _I64, _I64, _I64, _P]),
    "sc_kv_stage_from_host": (C.c_int, [_P, _I64, _P]),
    "sc_kv_ring_table": (C.c_int, [_P, _I64, _I64, _P]),
    "sc_kv_append_async": (C.c_int, [_P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, C.POINTER(KvPools),
                                     C.POINTER(KvPools)]),
    "sc_kv_append_q4_async": (C.c_int, [_P, _P, _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, C.POINTER(KvPools),
                                        C.POINTER(KvPools)]),
    "sc_kv_stream_reset": (C.c_int, [_P, _I64, _P, _P, _P, _I64, _P, _P]),
    "sc_kv_block_bytes": (_U64, [_I64, _I64, _I64, C.c_int32]),
    "sc_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "sc_get_device": (C.c_int, [C.POINTER(C.c_int)]),
    "sc_set_device": (C.c_int, [C.c_int]),
    "sc_device_alloc": (C.c_int, [C.POINTER(_P), _U64]),
    "sc_device_free": (C.c_int, [_P]),
    "sc_host_alloc": (C.c_int, [C.POINTER(_P), _U64]),
    "sc_host_free": (C.c_int, [_P]),
    "sc_host_range_mapped": (C.c_int, [_P, _U64, C.POINTER(C.c_int32)]),
    "sc_copy_async": (C.c_int, [_P, _P, _U64, _P]),
    "sc_fill_bytes_async": (C.c_int, [_P, C.c_uint8, _U64, _P]),
    "sc_stream_create": (C.c_int, [C.POINTER(_P)]),
    "sc_stream_destroy": (C.c_int, [_P]),
    "sc_stream_sync": (C.c_int, [_P]),
    "sc_device_sync": (C.c_int, []),
    "sc_event_create": (C.c_int, [C.POINTER(_P)]),
    "sc_event_destroy": (C.c_int, [_P]),
    "sc_event_record": (C.c_int, [_P, _P]),
    "sc_event_sync": (C.c_int, [_P]),
    "sc_event_elapsed_ms": (C.c_int, [_P, _P, C.POINTER(C.c_float)]),
    "sc_stream_wait_event": (C.c_int, [_P, _P]),
    "sc_probe_link": (C.c_int, [_U64, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "sc_fill_uniform_f16": (C.c_int, [_P, _U64, C.c_float, C.c_float, _U64, _U64, _P]),
    "sc_fill_uniform_f32": (C.c_int, [_P, _U64, C.c_float, C.c_float, _U64, _U64, _P]),
    "sc_fill_normal_f32": (C.c_int, [_P, _U64, _U64, _U64, _P]),
    "sc_decode_probe": (C.c_int, [_P, _U64, _P, _I64, _P]),
    "sc_delay_async": (C.c_int, [C.c_uint32, _P]),
    "sc_plan_carve_quant": (C.c_int, [_GEO, C.POINTER(PrefillView), C.POINTER(QuantSlot), C.POINTER(_P)]),
    "sc_plan_capture_map": (C.c_int, [_GEO, C.POINTER(DecodeSlot), _I64, _P, _U64, C.POINTER(BlobMap), C.POINTER(_P)]),
    "sc_plan_scatter_map": (C.c_int, [_GEO, _P, _U64, C.POINTER(BlobMap), _I64, C.POINTER(DecodeSlot), C.POINTER(_P)]),
    "sc_layer_blob_bytes": (C.c_int, [_GEO, C.c_int32, C.c_int32, _I64, C.POINTER(_U64)]),
    "sc_image_layout_layers": (C.c_int, [_GEO, C.c_int32, C.c_int32, _I64, C.POINTER(_U64), C.POINTER(_U64)]),
    "sc_plan_capture_layers": (C.c_int, [_GEO, C.POINTER(SlotLayers), _I64, _P, _U64, C.POINTER(LayersMap),
                                         C.POINTER(_P)]),
    "sc_plan_scatter_layers": (C.c_int, [_GEO, _P, _U64, C.POINTER(LayersMap), _I64, C.POINTER(SlotLayers),
                                         C.POINTER(_P)]),
    "sc_park_layers_async": (C.c_int, [_GEO, C.POINTER(SlotLayers), _I64, _P, _U64, _P, _P]),
    "sc_resume_layers_async": (C.c_int, [_GEO, _P, _U64, _I64, C.POINTER(SlotLayers), _P, _P]),
    "sc_fnv1a64_workspace_bytes": (_U64, [_U64]),
    "sc_fnv1a64_async": (C.c_int, [_P, _U64, _U64, _P, _P, _P, _U64, _P]),
    "sc_fnv1a64_chain_async": (C.c_int, [_P, _U64, _P, _P, _P, _U64, _P]),
    "sc_fnv1a64_check_async": (C.c_int, [_P, _U64, _U64, _U64, _P, _P, _P, _P, _U64, _P]),
    "sc_fnv1a64_device": (C.c_int, [_P, _U64, _U64, C.POINTER(_U64)]),
    "sc_fnv1a64_noalloc_async": (C.c_int, [_P, _U64, _U64, _P, _P, _P]),
    "sc_fnv1a64_set_spin_limit": (C.c_int, [C.c_uint32]),
    "sc_hash_map_create": (C.c_int, [C.POINTER(_P), C.c_int32, _P, _U64, C.POINTER(_P)]),
    "sc_hash_map_launch": (C.c_int, [_P, _U64, _P, _P, _P, _U64, _P]),
    "sc_hash_map_destroy": (C.c_int, [_P]),
    "sc_copy_device_async": (C.c_int, [_P, _P, _U64, _P]),
    "sc_ipc_export_create": (C.c_int, [_U64, _U64, C.POINTER(_P)]),
    "sc_ipc_export_count": (C.c_int32, [_P]),
    "sc_ipc_export_segments": (C.c_int, [_P, C.POINTER(IpcSegment), C.c_int32]),
    "sc_ipc_export_stage": (C.c_int, [_P, _P, _U64, _P]),
    "sc_ipc_export_destroy": (C.c_int, [_P]),
    "sc_ipc_import_open": (C.c_int, [C.POINTER(IpcSegment), C.c_int32, C.POINTER(_P)]),
    "sc_ipc_import_fetch": (C.c_int, [_P, _P, _U64, _P]),
    "sc_ipc_import_close": (C.c_int, [_P]),
    "sc_ipc_export_layout": (C.c_int, [_P, C.POINTER(_P), C.c_int32, C.POINTER(C.c_int32), C.POINTER(_U64)]),
    "sc_ipc_import_layout": (C.c_int, [_P, C.POINTER(_P), C.c_int32, C.POINTER(C.c_int32), C.POINTER(_U64)]),
    "sc_hash_map_create_segments": (C.c_int, [C.POINTER(_P), C.c_int32, _P, _U64, C.POINTER(Segments), C.POINTER(_P)]),
    "sc_hash_map_create_read": (C.c_int, [C.POINTER(Segments), _U64, C.POINTER(_P)]),
    "sc_hash_map_check_async": (C.c_int, [_P, _U64, _U64, _P, _P, _P, _P, _U64, _P]),
    "sc_fnv1a64_carry_bytes": (_U64, [_U64]),
    "sc_fnv1a64_carry_async": (C.c_int, [_P, _U64, _U64, _P, _P, _P, _P, _U64, _P]),
    "sc_fnv1a64_check_carried_async": (C.c_int, [_P, _U64, _U64, _U64, _P, _P, _P, _P, _P, _U64, _P]),
    "sc_hash_map_launch_carry": (C.c_int, [_P, _U64, _P, _P, _P, _P, _U64, _P]),
    "sc_hash_map_check_carried_async": (C.c_int, [_P, _U64, _U64, _P, _P, _P, _P, _P, _U64, _P]),
    "sc_plan_scatter_map_segments": (C.c_int, [_GEO, C.POINTER(Segments), _U64, C.POINTER(BlobMap), _I64,
                                               C.POINTER(DecodeSlot), C.POINTER(_P)]),
    "sc_plan_scatter_layers_segments": (C.c_int, [_GEO, C.POINTER(Segments), _U64, C.POINTER(LayersMap), _I64,
                                                  C.POINTER(SlotLayers), C.POINTER(_P)]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTS = tuple(_SIGS)


class ScError(RuntimeError):
    def __init__(self, code: int, where: str):
        self.code = code
        super().__init__(f"{where}: status {code}: {last_error()}")


def last_error() -> str:
    return lib.sc_last_error().decode()


def check(code: int, where: str) -> None:
    if code != SC_OK:
        raise ScError(code, where)


def geometry(**kw) -> Geometry:
    """A geometry with the configs' defaults (48 layers, QSA every 4th, K/V [2][256] f16, S=128, HV=32, C=8192)."""
    base = dict(n_layers=48, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=128,
                ssm_k_heads=16, ssm_v_heads=32, ssm_d_conv=4, ssm_conv_channels=8192, idx_key_dim=128)
    base.update(kw)
    return Geometry(**base)


def payload_bytes(geo: Geometry, tokens: int) -> int:
    return int(lib.sc_payload_bytes(C.byref(geo), tokens))


def image_layout(geo: Geometry, tokens: int) -> tuple[list[ImageBlob], int]:
    n = _I64(0)
    total = _U64(0)
    check(lib.sc_image_layout(C.byref(geo), tokens, None, C.byref(n), C.byref(total)), "sc_image_layout")
    blobs = (ImageBlob * max(n.value, 1))()
    check(lib.sc_image_layout(C.byref(geo), tokens, blobs, C.byref(n), C.byref(total)), "sc_image_layout")
    return list(blobs[: n.value]), int(total.value)


def _ptrs(values) -> C.Array:
    arr = (C.c_void_p * max(len(values), 1))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def _stream(stream) -> int | None:
    """A raw hipStream_t: None is the null stream; a Stream or any object with a `handle`."""
    if stream is None or isinstance(stream, int):
        return stream
    return stream.handle


def device_count() -> int:
    n = C.c_int(0)
    return n.value if lib.sc_device_count(C.byref(n)) == SC_OK else 0


def device_sync() -> None:
    check(lib.sc_device_sync(), "sc_device_sync")


class DeviceBuffer:
    """Device memory from the library (hipMalloc): a pointer, a dtype and a shape, nothing more."""

    def __init__(self, shape, dtype):
        import numpy as np
        self.shape = tuple(int(x) for x in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib.sc_device_alloc(C.byref(p), max(self.nbytes, 16)), "sc_device_alloc")
        self.ptr = p.value

    def data_ptr(self) -> int:
        return self.ptr

    def numel(self) -> int:
        return self.nbytes // self.dtype.itemsize

    def offset(self, index: int) -> int:
        """Address of flat element `index`."""
        return self.ptr + index * self.dtype.itemsize

    def fill(self, value: int, stream=None) -> None:
        fill_bytes(self.ptr, value, self.nbytes, stream)

    def numpy(self, count: int | None = None, start: int = 0):
        """Synchronously copy elements [start, start + count) (default: all) to a new host array."""
        import numpy as np
        n = self.numel() - start if count is None else count
        out = np.empty(max(n, 1), dtype=self.dtype)
        if n:
            check(lib.sc_copy_async(out.ctypes.data, self.offset(start), n * self.dtype.itemsize, None), "copy")
            device_sync()
        out = out[:n]
        return out.reshape(self.shape) if count is None and start == 0 else out

    def upload(self, array, start: int = 0) -> None:
        import numpy as np
        a = np.ascontiguousarray(array, dtype=self.dtype).reshape(-1)
        if a.size:
            check(lib.sc_copy_async(self.offset(start), a.ctypes.data, a.nbytes, None), "copy")
            device_sync()

    def free(self) -> None:
        if self.ptr:
            check(lib.sc_device_free(self.ptr), "sc_device_free")
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                lib.sc_device_free(self.ptr)
        except Exception:
            pass


def set_order_min_pages(pages: int) -> int:
    """Library-wide: tables of at least `pages` logical pages are visited in destination order by plans built from now
    on (<= 0: never).  Returns the previous value."""
    return int(lib.sc_set_order_min_pages(pages))


class Plan:
    """An owned sc_plan (a device-resident handoff table)."""

    def __init__(self, handle: int, keepalive=()):
        self.handle = handle
        self._keep = keepalive

    def launch(self, stream=None) -> None:
        check(lib.sc_plan_launch(self.handle, _stream(stream)), "sc_plan_launch")

    def retarget(self, prefill: "PrefillBuffers", pos0: int = 0, with_gdn: bool = True, stream=None) -> None:
        """Re-point a carve plan at another prefill sequence of the same slot (sc_plan_retarget)."""
        view, keep = prefill.view(pos0, with_gdn)
        check(lib.sc_plan_retarget(self.handle, C.byref(view), _stream(stream)), "sc_plan_retarget")
        self._target = prefill   # the device buffers the next launches read

    @property
    def payload_bytes(self) -> int:
        return int(lib.sc_plan_payload_bytes(self.handle))

    def set_grid(self, workgroups: int) -> None:
        check(lib.sc_plan_set_grid(self.handle, workgroups), "sc_plan_set_grid")

    @property
    def order_groups(self) -> int:
        """Page tables of the plan visited in destination order."""
        return int(lib.sc_plan_order_groups(self.handle))

    def destroy(self) -> None:
        if self.handle:
            check(lib.sc_plan_destroy(self.handle), "sc_plan_destroy")
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                lib.sc_plan_destroy(self.handle)
        except Exception:
            pass


# ---- device buffers of the two layouts ------------------------------------------------------------------------------


@dataclass
class PrefillBuffers:
    """One sequence in the prefill layout: per QSA layer K, V [T][H][D]; per GDN layer rec [HV][S][S] and the
    conv input rows [rows][C]."""
    geo: Geometry
    tokens: int
    k: list
    v: list
    rec: list
    conv: list
    conv_rows: int
    kv_dtype: int = SC_DTYPE_F16

    def view(self, pos0: int = 0, with_gdn: bool = True) -> tuple[PrefillView, tuple]:
        ks = _ptrs([t.data_ptr() for t in self.k])
        vs = _ptrs([t.data_ptr() for t in self.v])
        rs = _ptrs([t.data_ptr() for t in self.rec])
        cs = _ptrs([t.data_ptr() for t in self.conv])
        view = PrefillView(tokens=self.tokens, pos0=pos0, kv_dtype=self.kv_dtype, with_gdn=int(with_gdn),
                           k=C.cast(ks, C.POINTER(C.c_void_p)), v=C.cast(vs, C.POINTER(C.c_void_p)),
                           rec=C.cast(rs, C.POINTER(C.c_void_p)), conv=C.cast(cs, C.POINTER(C.c_void_p)),
                           conv_rows=self.conv_rows, conv_ld=self.geo.ssm_conv_channels)
        return view, (ks, vs, rs, cs)

    def host(self) -> dict:
        """The inputs read back to numpy (K/V as raw f16 bits, or f32)."""
        return {"k": [t.numpy() for t in self.k], "v": [t.numpy() for t in self.v],
                "rec": [t.numpy() for t in self.rec], "conv": [t.numpy() for t in self.conv],
                "tokens": self.tokens, "conv_rows": self.conv_rows, "kv_dtype": self.kv_dtype}


@dataclass
class Slot:
    """A decode slot: per QSA layer K/V pools [n_pages][H][ps][D] f16 bits, optional page tables, the GDN rows."""
    geo: Geometry
    n_pages: int
    max_cells: int
    k_pool: list
    v_pool: list
    gdn: object
    tables: list | None = None
    _keep: tuple = field(default=(), repr=False)
    host: list | None = None    # per QSA layer a KvPools (a streamed layer's host copy), or None
    stage: list | None = None   # per QSA layer a KvPools (the staging pool), or None

    def c_struct(self) -> DecodeSlot:
        ks = _ptrs([t.data_ptr() for t in self.k_pool])
        vs = _ptrs([t.data_ptr() for t in self.v_pool])
        ts = _ptrs([t.data_ptr() if t is not None else None for t in self.tables]) if self.tables else None
        hs, ss = _pools_array(self.host), _pools_array(self.stage)
        self._keep = (ks, vs, ts, hs, ss)
        return DecodeSlot(n_pages=self.n_pages, max_cells=self.max_cells,
                          k_pool=C.cast(ks, C.POINTER(C.c_void_p)), v_pool=C.cast(vs, C.POINTER(C.c_void_p)),
                          page_table=C.cast(ts, C.POINTER(C.c_void_p)) if ts is not None else None,
                          gdn_state=self.gdn.data_ptr() if self.gdn is not None else None,
                          host=C.cast(hs, C.POINTER(KvPools)) if hs is not None else None,
                          stage=C.cast(ss, C.POINTER(KvPools)) if ss is not None else None)

    def buffers(self) -> list:
        return [*self.k_pool, *self.v_pool, *([self.gdn] if self.gdn is not None else [])]

    def fill(self, value: int) -> None:
        for b in self.buffers():
            b.fill(value)

    def host_state(self) -> dict:
        out = {f"k{j}": t.numpy() for j, t in enumerate(self.k_pool)}
        out.update({f"v{j}": t.numpy() for j, t in enumerate(self.v_pool)})
        if self.gdn is not None:
            out["gdn"] = self.gdn.numpy()
        return out


def _pools_array(pools):
    """A ctypes array of KvPools (None entries are all-NULL pools), or None."""
    if not pools:
        return None
    return (KvPools * len(pools))(*[p if p is not None else KvPools() for p in pools])


def new_slot(geo: Geometry, max_cells: int, n_pages: int | None = None, tables=None, fill: int = 0) -> Slot:
    ps = geo.page_size
    n_pages = n_pages if n_pages is not None else (max_cells + ps - 1) // ps
    shape = (n_pages, geo.n_head_kv, ps, geo.head_dim)
    k = [DeviceBuffer(shape, "uint16") for _ in range(geo.n_qsa)]
    v = [DeviceBuffer(shape, "uint16") for _ in range(geo.n_qsa)]
    gdn = DeviceBuffer((geo.n_gdn, geo.gdn_row_floats), "float32") if geo.n_gdn else None
    slot = Slot(geo, n_pages, max_cells, k, v, gdn, tables)
    slot.fill(fill)
    return slot


def device_tables(tables) -> list | None:
    """Upload host page tables (one int32 array per QSA layer, or None for identity)."""
    if tables is None:
        return None
    out = []
    for t in tables:
        if t is None:
            out.append(None)
            continue
        b = DeviceBuffer(len(t), "int32")
        b.upload(t)
        out.append(b)
    return out


def fill_bytes(ptr: int, value: int, nbytes: int, stream=None) -> None:
    check(lib.sc_fill_bytes_async(ptr, value, nbytes, _stream(stream)), "sc_fill_bytes_async")


def plan_carve(geo: Geometry, prefill: PrefillBuffers, slot: Slot, pos0: int = 0, with_gdn: bool = True) -> Plan:
    view, keep = prefill.view(pos0, with_gdn)
    cs = slot.c_struct()
    h = C.c_void_p()
    check(lib.sc_plan_carve(C.byref(geo), C.byref(view), C.byref(cs), C.byref(h)), "sc_plan_carve")
    return Plan(h.value, (keep, slot._keep))


def plan_gather(geo: Geometry, prefill: PrefillBuffers, image_ptr: int, image_bytes: int) -> Plan:
    view, keep = prefill.view(0, True)
    h = C.c_void_p()
    check(lib.sc_plan_gather(C.byref(geo), C.byref(view), image_ptr, image_bytes, C.byref(h)), "sc_plan_gather")
    return Plan(h.value, keep)


def plan_scatter(geo: Geometry, image_ptr: int, image_bytes: int, tokens: int, slot: Slot) -> Plan:
    cs = slot.c_struct()
    h = C.c_void_p()
    check(lib.sc_plan_scatter(C.byref(geo), image_ptr, image_bytes, tokens, C.byref(cs), C.byref(h)),
          "sc_plan_scatter")
    return Plan(h.value, slot._keep)


def plan_capture(geo: Geometry, slot: Slot, tokens: int, image_ptr: int, image_bytes: int) -> Plan:
    cs = slot.c_struct()
    h = C.c_void_p()
    check(lib.sc_plan_capture(C.byref(geo), C.byref(cs), tokens, image_ptr, image_bytes, C.byref(h)),
          "sc_plan_capture")
    return Plan(h.value, slot._keep)


class CopyDesc(C.Structure):
    _fields_ = [("dst", C.c_void_p), ("src", C.c_void_p), ("bytes", C.c_uint64)]


def plan_copies(copies) -> Plan:
    """A plan of device-to-device copies (sc_plan_copies): `copies` is a list of (dst_ptr, src_ptr, nbytes)."""
    arr = (CopyDesc * max(len(copies), 1))(*[CopyDesc(d, s_, b) for d, s_, b in copies])
    h = C.c_void_p()
    check(lib.sc_plan_copies(C.cast(arr, C.c_void_p), len(copies), C.byref(h)), "sc_plan_copies")
    return Plan(h.value, (arr,))


def park_async(geo: Geometry, slot: Slot, tokens: int, host_ptr: int, host_bytes: int, stream=None,
               done=None) -> None:
    cs = slot.c_struct()
    check(lib.sc_park_async(C.byref(geo), C.byref(cs), tokens, host_ptr, host_bytes, _stream(stream), done),
          "sc_park_async")


def resume_async(geo: Geometry, host_ptr: int, host_bytes: int, tokens: int, slot: Slot, stream=None,
                 done=None) -> None:
    cs = slot.c_struct()
    check(lib.sc_resume_async(C.byref(geo), host_ptr, host_bytes, tokens, C.byref(cs), _stream(stream), done),
          "sc_resume_async")


class PinnedBuffer:
    """Pinned host memory from the library (hipHostMalloc), viewable as numpy."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib.sc_host_alloc(C.byref(p), nbytes), "sc_host_alloc")
        self.ptr, self.nbytes = p.value, nbytes

    def numpy(self):
        import numpy as np
        buf = (C.c_uint8 * self.nbytes).from_address(self.ptr)
        return np.frombuffer(buf, dtype=np.uint8)

    def free(self) -> None:
        if self.ptr:
            check(lib.sc_host_free(self.ptr), "sc_host_free")
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                lib.sc_host_free(self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(lib.sc_event_create(C.byref(p)), "sc_event_create")
        self.handle = p.value

    def record(self, stream=None) -> None:
        check(lib.sc_event_record(self.handle, _stream(stream)), "sc_event_record")

    def sync(self) -> None:
        check(lib.sc_event_sync(self.handle), "sc_event_sync")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib.sc_event_elapsed_ms(self.handle, end.handle, C.byref(ms)), "sc_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        try:
            lib.sc_event_destroy(self.handle)
        except Exception:
            pass


class Stream:
    """A non-blocking HIP stream at the default priority."""

    def __init__(self):
        p = C.c_void_p()
        check(lib.sc_stream_create(C.byref(p)), "sc_stream_create")
        self.handle = p.value
        self.cuda_stream = p.value

    def sync(self) -> None:
        check(lib.sc_stream_sync(self.handle), "sc_stream_sync")

    def wait(self, event: Event) -> None:
        check(lib.sc_stream_wait_event(self.handle, event.handle), "sc_stream_wait_event")

    def __del__(self):
        try:
            lib.sc_stream_destroy(self.handle)
        except Exception:
            pass


def delay_async(microseconds: int, stream=None) -> None:
    """Hold `stream` for `microseconds` with one sleeping wave (sc_delay_async): long work that always ends."""
    check(lib.sc_delay_async(microseconds, _stream(stream)), "sc_delay_async")


def probe_link(nbytes: int = 256 << 20, iters: int = 4) -> tuple[float, float]:
    h2d, d2h = C.c_double(), C.c_double()
    check(lib.sc_probe_link(nbytes, iters, C.byref(h2d), C.byref(d2h)), "sc_probe_link")
    return float(h2d.value), float(d2h.value)


# ---- batched ragged resume + append (many slots in one launch) ------------------------------------------------------

def staging_layout(geo: Geometry, lens) -> tuple[list[int], int]:
    n = len(lens)
    arr = (C.c_int64 * n)(*lens)
    offs = (C.c_uint64 * n)()
    total = C.c_uint64()
    check(lib.sc_batch_staging_layout(C.byref(geo), arr, n, offs, C.byref(total)), "sc_batch_staging_layout")
    return list(offs), int(total.value)


REFERENCE_FNV_SEED = 1469598103934665603   # the seed of every fnv1a64 call in the reference (conversation_wire.hpp:196)


def fnv1a64_device(ptr: int, nbytes: int, seed: int = REFERENCE_FNV_SEED) -> int:
    """FNV-1a 64 of `nbytes` device bytes at `ptr`, computed by the library's parallel hash (synchronous)."""
    out = _U64(0)
    check(lib.sc_fnv1a64_device(ptr, nbytes, seed, C.byref(out)), "sc_fnv1a64_device")
    return int(out.value)


class HashFault(RuntimeError):
    """A look-back wait of the device hash ran out (the launch's fault word is 1): the hash is not valid."""


FNV_FAULT_WAIT, FNV_FAULT_CARRY = 1, 2


def carry_bytes(nbytes: int) -> int:
    """Bytes of the carries of an `nbytes`-byte input (sc_fnv1a64_carry_bytes): one per 64 KiB boundary inside it."""
    return int(lib.sc_fnv1a64_carry_bytes(nbytes))


class HashPlan:
    """A reusable device workspace for sc_fnv1a64_async over inputs of up to `max_bytes` bytes, plus device words for
    the result and the launch's fault word."""

    def __init__(self, max_bytes: int):
        self.max_bytes = max_bytes
        self.ws_bytes = int(lib.sc_fnv1a64_workspace_bytes(max_bytes))
        self.ws = DeviceBuffer(self.ws_bytes, "uint8")
        self.out = DeviceBuffer(1, "uint64")
        self.fault = DeviceBuffer(1, "uint32")
        self.verdict = DeviceBuffer(1, "uint32")
        self.fault.fill(0)     # a launch that is given no fault word leaves this one clear
        self.verdict.fill(0)
        device_sync()          # before any launch on another stream writes them

    def launch(self, ptr: int, nbytes: int, seed: int = REFERENCE_FNV_SEED, stream=None) -> None:
        if nbytes > self.max_bytes:
            raise ValueError(f"hash input of {nbytes} bytes exceeds the plan's {self.max_bytes}")
        check(lib.sc_fnv1a64_async(ptr, nbytes, seed, self.out.ptr, self.fault.ptr, self.ws.ptr, self.ws_bytes,
                                   _stream(stream)),
              "sc_fnv1a64_async")

    def start(self, seed: int = REFERENCE_FNV_SEED) -> None:
        """Set the running hash of chain() to `seed` and clear the chain's fault word (synchronous uploads)."""
        self.out.upload([seed])
        self.fault.upload([0])

    def chain(self, ptr: int, nbytes: int, stream=None) -> None:
        """Continue the running hash over `nbytes` more device bytes at `ptr` (sc_fnv1a64_chain_async)."""
        if nbytes > self.max_bytes:
            raise ValueError(f"hash input of {nbytes} bytes exceeds the plan's {self.max_bytes}")
        check(lib.sc_fnv1a64_chain_async(ptr, nbytes, self.out.ptr, self.fault.ptr, self.ws.ptr, self.ws_bytes,
                                         _stream(stream)),
              "sc_fnv1a64_chain_async")

    def launch_carry(self, ptr: int, nbytes: int, carry_ptr: int, seed: int = REFERENCE_FNV_SEED, stream=None) -> None:
        """launch() that also writes the input's carries at `carry_ptr` (sc_fnv1a64_carry_async)."""
        if nbytes > self.max_bytes:
            raise ValueError(f"hash input of {nbytes} bytes exceeds the plan's {self.max_bytes}")
        check(lib.sc_fnv1a64_carry_async(ptr, nbytes, seed, self.out.ptr, self.fault.ptr, carry_ptr, self.ws.ptr,
                                         self.ws_bytes, _stream(stream)),
              "sc_fnv1a64_carry_async")

    def check_carried(self, ptr: int, nbytes: int, expected: int, carry_ptr: int, seed: int = REFERENCE_FNV_SEED,
                      stream=None) -> None:
        """The check of `expected` given the input's carries (sc_fnv1a64_check_carried_async): the hash in `out`, the
        verdict in `verdict`, the fault word (FNV_FAULT_CARRY when the input or the carries are not what was hashed)
        in `fault`."""
        if nbytes > self.max_bytes:
            raise ValueError(f"hash input of {nbytes} bytes exceeds the plan's {self.max_bytes}")
        check(lib.sc_fnv1a64_check_carried_async(ptr, nbytes, seed, expected, carry_ptr, self.out.ptr,
                                                 self.verdict.ptr, self.fault.ptr, self.ws.ptr, self.ws_bytes,
                                                 _stream(stream)),
              "sc_fnv1a64_check_carried_async")

    def fault_word(self) -> int:
        return int(self.fault.numpy()[0])

    def faulted(self) -> bool:
        return bool(self.fault.numpy()[0])

    def result(self) -> int:
        """The hash of the last launch (or chain); HashFault when a wait of it ran out."""
        if self.faulted():
            raise HashFault("a look-back wait of the device hash ran out; the hash is not valid")
        return int(self.out.numpy()[0])

    def free(self) -> None:
        self.ws.free()
        self.out.free()
        self.fault.free()
        self.verdict.free()


class HashMap:
    """Capture plans fused with the hash of the payload they write (sc_hash_map_*): launch() gathers and hashes in one
    read of the sources; the result and fault word land in `plan`'s words (a HashPlan sized for the payload)."""

    def __init__(self, plans, payload_ptr: int, nbytes: int):
        arr = (C.c_void_p * max(len(plans), 1))(*[p.handle for p in plans])
        h = C.c_void_p()
        check(lib.sc_hash_map_create(arr, len(plans), payload_ptr, nbytes, C.byref(h)), "sc_hash_map_create")
        self.handle, self.nbytes = h.value, nbytes

    def launch(self, hp: "HashPlan", seed: int = REFERENCE_FNV_SEED, stream=None) -> None:
        check(lib.sc_hash_map_launch(self.handle, seed, hp.out.ptr, hp.fault.ptr, hp.ws.ptr, hp.ws_bytes,
                                     _stream(stream)), "sc_hash_map_launch")

    @classmethod
    def segments(cls, plans, frame: int, nbytes: int, seg_ptrs, segment_bytes: int) -> "HashMap":
        """The map of `plans` (built for a contiguous payload at `frame`) writing into segments instead
        (sc_hash_map_create_segments)."""
        arr = (C.c_void_p * max(len(plans), 1))(*[p.handle for p in plans])
        segs, keep = segments_struct(seg_ptrs, segment_bytes)
        h = C.c_void_p()
        check(lib.sc_hash_map_create_segments(arr, len(plans), frame, nbytes, C.byref(segs), C.byref(h)),
              "sc_hash_map_create_segments")
        m = cls.__new__(cls)
        m.handle, m.nbytes = h.value, nbytes
        return m

    @classmethod
    def read(cls, seg_ptrs, segment_bytes: int, nbytes: int) -> "HashMap":
        """A map that only hashes a segmented payload where it lies (sc_hash_map_create_read)."""
        segs, keep = segments_struct(seg_ptrs, segment_bytes)
        h = C.c_void_p()
        check(lib.sc_hash_map_create_read(C.byref(segs), nbytes, C.byref(h)), "sc_hash_map_create_read")
        m = cls.__new__(cls)
        m.handle, m.nbytes = h.value, nbytes
        return m

    def check(self, hp: "HashPlan", expected: int, seed: int = REFERENCE_FNV_SEED, stream=None) -> None:
        """launch() that also leaves the verdict (1: equal and complete) in hp.verdict (sc_hash_map_check_async)."""
        check(lib.sc_hash_map_check_async(self.handle, seed, expected, hp.out.ptr, hp.verdict.ptr, hp.fault.ptr,
                                          hp.ws.ptr, hp.ws_bytes, _stream(stream)), "sc_hash_map_check_async")

    def launch_carry(self, hp: "HashPlan", carry_ptr: int, seed: int = REFERENCE_FNV_SEED, stream=None) -> None:
        """launch() that also writes the payload's carries at `carry_ptr` (sc_hash_map_launch_carry)."""
        check(lib.sc_hash_map_launch_carry(self.handle, seed, hp.out.ptr, hp.fault.ptr, carry_ptr, hp.ws.ptr,
                                           hp.ws_bytes, _stream(stream)), "sc_hash_map_launch_carry")

    def check_carried(self, hp: "HashPlan", expected: int, carry_ptr: int, seed: int = REFERENCE_FNV_SEED,
                      stream=None) -> None:
        """check() of a read map given the payload's carries (sc_hash_map_check_carried_async)."""
        check(lib.sc_hash_map_check_carried_async(self.handle, seed, expected, carry_ptr, hp.out.ptr, hp.verdict.ptr,
                                                  hp.fault.ptr, hp.ws.ptr, hp.ws_bytes, _stream(stream)),
              "sc_hash_map_check_carried_async")

    def destroy(self) -> None:
        if self.handle:
            check(lib.sc_hash_map_destroy(self.handle), "sc_hash_map_destroy")
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                lib.sc_hash_map_destroy(self.handle)
        except Exception:
            pass


@dataclass
class QuantPools:
    """Quantized decode pools of one slot: per QSA layer K and V codes (int8 [n_pages][H][ps][256] or q4_0
    [n_pages][H][ps][144] bytes) and int8 scales ([n_pages][H][ps][4] f16), plus the GDN rows."""
    geo: Geometry
    fmt: int
    n_pages: int
    max_cells: int
    k_codes: list
    v_codes: list
    k_scale: list
    v_scale: list
    gdn: object
    tables: list | None = None
    _keep: tuple = field(default=(), repr=False)
    host: list | None = None    # per QSA layer a KvPools (a streamed layer's host copy), or None
    stage: list | None = None   # per QSA layer a KvPools (the staging pool), or None

    def c_struct(self) -> QuantSlot:
        kc = _ptrs([t.ptr for t in self.k_codes])
        vc = _ptrs([t.ptr for t in self.v_codes])
        ks = _ptrs([t.ptr for t in self.k_scale]) if self.k_scale else None
        vs = _ptrs([t.ptr for t in self.v_scale]) if self.v_scale else None
        ts = _ptrs([t.data_ptr() if t is not None else None for t in self.tables]) if self.tables else None
        hs, ss = _pools_array(self.host), _pools_array(self.stage)
        self._keep = (kc, vc, ks, vs, ts, hs, ss)
        cast = lambda a: C.cast(a, C.POINTER(C.c_void_p)) if a is not None else None  # noqa: E731
        return QuantSlot(n_pages=self.n_pages, max_cells=self.max_cells, format=self.fmt, k_codes=cast(kc),
                         v_codes=cast(vc), k_scale=cast(ks), v_scale=cast(vs), page_table=cast(ts),
                         gdn_state=self.gdn.data_ptr() if self.gdn is not None else None,
                         host=C.cast(hs, C.POINTER(KvPools)) if hs is not None else None,
                         stage=C.cast(ss, C.POINTER(KvPools)) if ss is not None else None)

    def buffers(self) -> list:
        return [*self.k_codes, *self.v_codes, *self.k_scale, *self.v_scale, *([self.gdn] if self.gdn is not None else [])]


def new_quant_slot(geo: Geometry, fmt: int, max_cells: int, n_pages: int | None = None, tables=None,
                   fill: int = 0) -> QuantPools:
    ps, H = geo.page_size, geo.n_head_kv
    n_pages = n_pages if n_pages is not None else (max_cells + ps - 1) // ps
    rows = n_pages * H * ps
    k_int8, v_int8 = fmt != SC_KV_Q4, fmt == SC_KV_INT8
    k = [DeviceBuffer(rows * (256 if k_int8 else 144), "uint8") for _ in range(geo.n_qsa)]
    v = [DeviceBuffer(rows * (256 if v_int8 else 144), "uint8") for _ in range(geo.n_qsa)]
    ks = [DeviceBuffer(rows * 4, "uint16") for _ in range(geo.n_qsa)] if k_int8 else []
    vs = [DeviceBuffer(rows * 4, "uint16") for _ in range(geo.n_qsa)] if v_int8 else []
    gdn = DeviceBuffer((geo.n_gdn, geo.gdn_row_floats), "float32") if geo.n_gdn else None
    slot = QuantPools(geo, fmt, n_pages, max_cells, k, v, ks, vs, gdn, tables)
    for b in slot.buffers():
        b.fill(fill)
    return slot


def plan_carve_quant(geo: Geometry, prefill: PrefillBuffers, slot: QuantPools, pos0: int = 0,
                     with_gdn: bool = True) -> Plan:
    view, keep = prefill.view(pos0, with_gdn)
    cs = slot.c_struct()
    h = C.c_void_p()
    check(lib.sc_plan_carve_quant(C.byref(geo), C.byref(view), C.byref(cs), C.byref(h)), "sc_plan_carve_quant")
    return Plan(h.value, (keep, slot._keep))


# ---- slot images in every K/V format --------------------------------------------------------------------------------

def layer_blob_bytes(geo: Geometry, fmt: int, with_index: bool, tokens: int) -> list[int]:
    out = (_U64 * SC_N_BUF)()
    check(lib.sc_layer_blob_bytes(C.byref(geo), fmt, int(with_index), tokens, out), "sc_layer_blob_bytes")
    return [int(x) for x in out]


def image_layout_layers(geo: Geometry, fmt: int, with_index: bool, tokens: int) -> tuple[list[int | None], int]:
    """Offsets (five per QSA layer, then the GDN rows; None for an empty blob) and the total of the slot image."""
    offs = (_U64 * (geo.n_qsa * SC_N_BUF + 1))()
    total = _U64(0)
    check(lib.sc_image_layout_layers(C.byref(geo), fmt, int(with_index), tokens, offs, C.byref(total)),
          "sc_image_layout_layers")
    return [None if int(x) == ABSENT else int(x) for x in offs], int(total.value)


class LayerPools:
    """One slot's per-layer buffers in any format (identity layout), sized for `max_cells` cells, plus the GDN rows:
    the five SC_BUF_* buffers of each QSA layer (absent ones are None) and the indexer's pooled rows when with_index."""

    def __init__(self, geo: Geometry, fmt: int, max_cells: int, with_index: bool, buffers=None, gdn=None):
        self.geo, self.fmt, self.max_cells, self.with_index = geo, fmt, max_cells, with_index
        cap = layer_blob_bytes(geo, fmt, True, max_cells)       # a full pool, pooled rows for max_cells tokens
        self.pooled_capacity = (max_cells // 4 + 1) if with_index and max_cells > 0 else 0
        self.capacity = [cap[k] if (k != 4 or with_index) else 0 for k in range(SC_N_BUF)]
        if buffers is None:
            buffers = [[DeviceBuffer(n, "uint8") for _ in range(geo.n_qsa)] if n else None for n in self.capacity]
        self.bufs = buffers
        if gdn is None and geo.n_gdn:
            gdn = DeviceBuffer((geo.n_gdn, geo.gdn_row_floats), "float32")
        self.gdn = gdn
        self._keep = ()

    @classmethod
    def from_quant(cls, slot: "QuantPools", pooled=None) -> "LayerPools":
        """The pools of a quantizing carve's slot (identity tables), with optional indexer pooled-row buffers."""
        fmt = slot.fmt
        bufs = [list(slot.k_codes), list(slot.v_codes), list(slot.k_scale) or None, list(slot.v_scale) or None,
                list(pooled) if pooled else None]
        return cls(slot.geo, fmt, slot.max_cells, bool(pooled), buffers=bufs, gdn=slot.gdn)

    def c_struct(self) -> SlotLayers:
        arrs = [(_ptrs([b.ptr for b in bl]) if bl else None) for bl in self.bufs]
        self._keep = tuple(arrs)
        st = SlotLayers(format=self.fmt, with_index=int(self.with_index), max_cells=self.max_cells,
                        pooled_capacity=self.pooled_capacity,
                        gdn_state=self.gdn.ptr if self.gdn is not None else None)
        for k, a in enumerate(arrs):
            st.buf[k] = C.cast(a, C.POINTER(C.c_void_p)) if a is not None else None
        return st

    def buffers(self) -> list:
        out = [b for bl in self.bufs if bl for b in bl]
        return out + ([self.gdn] if self.gdn is not None else [])

    def randomize(self, seed: int) -> None:
        """Seeded pseudo-random contents in every buffer (device generator; each buffer its own stream)."""
        for i, b in enumerate(self.buffers()):
            check(lib.sc_fill_uniform_f16(b.ptr, b.nbytes // 2, -4.0, 4.0, seed, 7000 + i, None), "fill")

    def fill(self, value: int) -> None:
        for b in self.buffers():
            b.fill(value)

    def host(self) -> dict:
        import numpy as np
        out = {}
        for k, bl in enumerate(self.bufs):
            if bl:
                for j, b in enumerate(bl):
                    out[(k, j)] = b.numpy().view(np.uint8).reshape(-1)
        if self.gdn is not None:
            out["gdn"] = self.gdn.numpy().view(np.uint8).reshape(-1)
        return out

    def free(self) -> None:
        for b in self.buffers():
            b.free()


def _layers_map(offsets, zero) -> tuple:
    if offsets is None:
        return None, ()
    off = (_U64 * len(offsets))(*[ABSENT if x is None else x for x in offsets])
    z = (_U64 * max(len(zero or ()), 1))(*(zero or ()))
    m = LayersMap(off=C.cast(off, C.POINTER(_U64)), zero=C.cast(z, C.POINTER(_U64)), n_zero=len(zero or ()) // 2)
    return m, (off, z)


def plan_capture_layers(geo: Geometry, pools: LayerPools, tokens: int, ptr: int, nbytes: int, offsets=None,
                        zero=None) -> Plan:
    cs = pools.c_struct()
    m, keep = _layers_map(offsets, zero)
    h = C.c_void_p()
    check(lib.sc_plan_capture_layers(C.byref(geo), C.byref(cs), tokens, ptr, nbytes,
                                     C.byref(m) if m is not None else None, C.byref(h)), "sc_plan_capture_layers")
    return Plan(h.value, (pools._keep, keep))


def plan_scatter_layers(geo: Geometry, ptr: int, nbytes: int, tokens: int, pools: LayerPools, offsets=None) -> Plan:
    cs = pools.c_struct()
    m, keep = _layers_map(offsets, None)
    h = C.c_void_p()
    check(lib.sc_plan_scatter_layers(C.byref(geo), ptr, nbytes, C.byref(m) if m is not None else None, tokens,
                                     C.byref(cs), C.byref(h)), "sc_plan_scatter_layers")
    return Plan(h.value, (pools._keep, keep))


def park_layers_async(geo: Geometry, pools: LayerPools, tokens: int, host_ptr: int, host_bytes: int, stream=None,
                      done=None) -> None:
    cs = pools.c_struct()
    check(lib.sc_park_layers_async(C.byref(geo), C.byref(cs), tokens, host_ptr, host_bytes, _stream(stream), done),
          "sc_park_layers_async")


def resume_layers_async(geo: Geometry, host_ptr: int, host_bytes: int, tokens: int, pools: LayerPools, stream=None,
                        done=None) -> None:
    cs = pools.c_struct()
    check(lib.sc_resume_layers_async(C.byref(geo), host_ptr, host_bytes, tokens, C.byref(cs), _stream(stream), done),
          "sc_resume_layers_async")


def _layout(fn, handle) -> tuple[list[int], int]:
    arr = (C.c_void_p * IPC_MAX_SEGMENTS)()
    n, sb = C.c_int32(0), _U64(0)
    check(fn(handle, arr, IPC_MAX_SEGMENTS, C.byref(n), C.byref(sb)), "segment layout")
    return [int(arr[i]) for i in range(n.value)], int(sb.value)


class IpcExport:
    """The exporting side of a same-GPU hand-off: device segments allocated and exported once."""

    def __init__(self, capacity: int, segment_bytes: int = IPC_MAX_SEGMENT):
        h = C.c_void_p()
        check(lib.sc_ipc_export_create(capacity, segment_bytes, C.byref(h)), "sc_ipc_export_create")
        self.handle = h.value

    def segments(self) -> list:
        n = lib.sc_ipc_export_count(self.handle)
        arr = (IpcSegment * n)()
        check(lib.sc_ipc_export_segments(self.handle, arr, n), "sc_ipc_export_segments")
        return [(bytes(s.handle), int(s.bytes)) for s in arr]

    def stage(self, device_ptr: int, nbytes: int, stream=None) -> None:
        check(lib.sc_ipc_export_stage(self.handle, device_ptr, nbytes, _stream(stream)), "sc_ipc_export_stage")

    def layout(self) -> tuple[list[int], int]:
        """The segments' device addresses and the size of every one but the last (sc_ipc_export_layout)."""
        return _layout(lib.sc_ipc_export_layout, self.handle)

    def destroy(self) -> None:
        if self.handle:
            check(lib.sc_ipc_export_destroy(self.handle), "sc_ipc_export_destroy")
            self.handle = None


class IpcImport:
    """The importing side: another process's segments mapped into this one."""

    def __init__(self, segments):
        arr = (IpcSegment * len(segments))()
        for i, (handle, nbytes) in enumerate(segments):
            C.memmove(arr[i].handle, handle, 64)
            arr[i].bytes = nbytes
        h = C.c_void_p()
        check(lib.sc_ipc_import_open(arr, len(segments), C.byref(h)), "sc_ipc_import_open")
        self.handle = h.value

    def fetch(self, device_ptr: int, nbytes: int, stream=None) -> None:
        check(lib.sc_ipc_import_fetch(self.handle, device_ptr, nbytes, _stream(stream)), "sc_ipc_import_fetch")

    def layout(self) -> tuple[list[int], int]:
        """The imported segments' device addresses in this process and the segment size (sc_ipc_import_layout)."""
        return _layout(lib.sc_ipc_import_layout, self.handle)

    def close(self) -> None:
        if self.handle:
            check(lib.sc_ipc_import_close(self.handle), "sc_ipc_import_close")
            self.handle = None
