"""Python binding of libsc_handoff.so (include/sc_handoff.h) over ctypes, plus device-buffer helpers.

PyTorch provides device memory and streams here and nothing else: every byte of the handoff is moved by the
library's own HIP kernels and copies.  Importing this module loads the built library and fails loudly when it is
missing - there is no fallback.
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


class DecodeSlot(C.Structure):
    _fields_ = [
        ("n_pages", C.c_int64), ("max_cells", C.c_int64),
        ("k_pool", C.POINTER(C.c_void_p)), ("v_pool", C.POINTER(C.c_void_p)),
        ("page_table", C.POINTER(C.c_void_p)), ("gdn_state", C.c_void_p)]


class ImageBlob(C.Structure):
    _fields_ = [("kind", C.c_int32), ("layer", C.c_int32), ("offset", C.c_uint64), ("bytes", C.c_uint64)]


_P = C.c_void_p
_I64, _U64 = C.c_int64, C.c_uint64
_GEO = C.POINTER(Geometry)
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
    "sc_plan_gather": (C.c_int, [_GEO, C.POINTER(PrefillView), _P, _U64, C.POINTER(_P)]),
    "sc_plan_scatter": (C.c_int, [_GEO, _P, _U64, _I64, C.POINTER(DecodeSlot), C.POINTER(_P)]),
    "sc_plan_capture": (C.c_int, [_GEO, C.POINTER(DecodeSlot), _I64, _P, _U64, C.POINTER(_P)]),
    "sc_plan_launch": (C.c_int, [_P, _P]),
    "sc_plan_payload_bytes": (_U64, [_P]),
    "sc_plan_set_grid": (C.c_int, [_P, _I64]),
    "sc_plan_destroy": (C.c_int, [_P]),
    "sc_park_async": (C.c_int, [_GEO, C.POINTER(DecodeSlot), _I64, _P, _U64, _P, _P]),
    "sc_resume_async": (C.c_int, [_GEO, _P, _U64, _I64, C.POINTER(DecodeSlot), _P, _P]),
    "sc_device_alloc": (C.c_int, [C.POINTER(_P), _U64]),
    "sc_device_free": (C.c_int, [_P]),
    "sc_host_alloc": (C.c_int, [C.POINTER(_P), _U64]),
    "sc_host_free": (C.c_int, [_P]),
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
    """A raw hipStream_t from a torch stream, an int handle, or None (torch's current stream)."""
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class Plan:
    """An owned sc_plan (a device-resident handoff table)."""

    def __init__(self, handle: int, keepalive=()):
        self.handle = handle
        self._keep = keepalive

    def launch(self, stream=None) -> None:
        check(lib.sc_plan_launch(self.handle, _stream(stream)), "sc_plan_launch")

    @property
    def payload_bytes(self) -> int:
        return int(lib.sc_plan_payload_bytes(self.handle))

    def set_grid(self, workgroups: int) -> None:
        check(lib.sc_plan_set_grid(self.handle, workgroups), "sc_plan_set_grid")

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


# ---- device buffers (torch tensors as plain device memory) --------------------------------------------------------


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
        """The inputs read back to numpy (K/V as raw f16 bits)."""
        import numpy as np
        out = {}
        for name, ts in (("k", self.k), ("v", self.v)):
            out[name] = [_host_bits(t) for t in ts]
        out["rec"] = [t.cpu().numpy() for t in self.rec]
        out["conv"] = [t.cpu().numpy() for t in self.conv]
        out["tokens"] = self.tokens
        out["conv_rows"] = self.conv_rows
        out["kv_dtype"] = self.kv_dtype
        return out


def _host_bits(t):
    import torch
    if t.dtype == torch.float16:
        return t.view(torch.int16).cpu().numpy().view("uint16")
    return t.cpu().numpy()


@dataclass
class Slot:
    """A decode slot: per QSA layer K/V pools [n_pages][H][ps][D] f16, optional page tables, and the GDN rows."""
    geo: Geometry
    n_pages: int
    max_cells: int
    k_pool: list
    v_pool: list
    gdn: object
    tables: list | None = None
    _keep: tuple = field(default=(), repr=False)

    def c_struct(self) -> DecodeSlot:
        ks = _ptrs([t.data_ptr() for t in self.k_pool])
        vs = _ptrs([t.data_ptr() for t in self.v_pool])
        ts = _ptrs([t.data_ptr() if t is not None else None for t in self.tables]) if self.tables else None
        self._keep = (ks, vs, ts)
        return DecodeSlot(n_pages=self.n_pages, max_cells=self.max_cells,
                          k_pool=C.cast(ks, C.POINTER(C.c_void_p)), v_pool=C.cast(vs, C.POINTER(C.c_void_p)),
                          page_table=C.cast(ts, C.POINTER(C.c_void_p)) if ts is not None else None,
                          gdn_state=self.gdn.data_ptr() if self.gdn is not None else None)

    def host_state(self) -> dict:
        import numpy as np
        out = {}
        for j, t in enumerate(self.k_pool):
            out[f"k{j}"] = _host_bits(t)
        for j, t in enumerate(self.v_pool):
            out[f"v{j}"] = _host_bits(t)
        if self.gdn is not None:
            out["gdn"] = self.gdn.cpu().numpy()
        return out


def new_slot(geo: Geometry, max_cells: int, device="cuda:0", n_pages: int | None = None, tables=None,
             fill: int = 0) -> Slot:
    import torch
    ps = geo.page_size
    n_pages = n_pages if n_pages is not None else (max_cells + ps - 1) // ps
    shape = (n_pages, geo.n_head_kv, ps, geo.head_dim)
    k = [torch.empty(shape, dtype=torch.float16, device=device) for _ in range(geo.n_qsa)]
    v = [torch.empty(shape, dtype=torch.float16, device=device) for _ in range(geo.n_qsa)]
    gdn = torch.empty((geo.n_gdn, geo.gdn_row_floats), dtype=torch.float32, device=device) if geo.n_gdn else None
    for t in [*k, *v, *([gdn] if gdn is not None else [])]:
        fill_bytes(t.data_ptr(), fill, t.numel() * t.element_size())
    return Slot(geo, n_pages, max_cells, k, v, gdn, tables)


def fill_bytes(ptr: int, value: int, nbytes: int, stream=None) -> None:
    check(lib.sc_fill_bytes_async(ptr, value, nbytes, _stream(stream)), "sc_fill_bytes_async")


# Stream ids of the synthetic inputs (one counter stream per buffer).
def sid_k(j: int) -> int: return 1000 + 2 * j
def sid_v(j: int) -> int: return 1001 + 2 * j
def sid_rec(i: int) -> int: return 5000 + i
def sid_conv(i: int) -> int: return 9000 + i


def synthetic_prefill(geo: Geometry, tokens: int, seed: int, device="cuda:0", kv_dtype: int = SC_DTYPE_F16,
                      conv_rows: int | None = None) -> PrefillBuffers:
    """K/V ~ U[-4, 4] (f16, or f32 when kv_dtype is F32), recurrence and conv rows ~ N(0, 1) (Irwin-Hall 12),
    generated on the device by the library's counter-based generators."""
    import torch
    H, D = geo.n_head_kv, geo.head_dim
    S, HV, Cc = geo.ssm_state_size, geo.ssm_v_heads, geo.ssm_conv_channels
    conv_rows = min(tokens, geo.ssm_d_conv - 1) if conv_rows is None else conv_rows
    stream = _stream(None)
    ks, vs, recs, convs = [], [], [], []
    kv_t = torch.float16 if kv_dtype == SC_DTYPE_F16 else torch.float32
    for j in range(geo.n_qsa):
        for lst, sid in ((ks, sid_k(j)), (vs, sid_v(j))):
            t = torch.empty((max(tokens, 1), H, D), dtype=kv_t, device=device)
            n = tokens * H * D
            if kv_dtype == SC_DTYPE_F16:
                check(lib.sc_fill_uniform_f16(t.data_ptr(), n, -4.0, 4.0, seed, sid, stream), "fill")
            else:
                check(lib.sc_fill_uniform_f32(t.data_ptr(), n, -4.0, 4.0, seed, sid, stream), "fill")
            lst.append(t)
    for i in range(geo.n_gdn):
        r = torch.empty((HV, S, S), dtype=torch.float32, device=device)
        check(lib.sc_fill_normal_f32(r.data_ptr(), r.numel(), seed, sid_rec(i), stream), "fill")
        recs.append(r)
        c = torch.empty((max(conv_rows, 1), Cc), dtype=torch.float32, device=device)
        check(lib.sc_fill_normal_f32(c.data_ptr(), conv_rows * Cc, seed, sid_conv(i), stream), "fill")
        convs.append(c)
    return PrefillBuffers(geo, tokens, ks, vs, recs, convs, conv_rows, kv_dtype)


class SyntheticCase:
    """A seeded prefill sequence on the device plus the helpers smoke() and the tests use."""

    def __init__(self, geo: Geometry, tokens: int, seed: int, device="cuda:0", kv_dtype: int = SC_DTYPE_F16):
        self.geo, self.tokens, self.seed, self.device = geo, tokens, seed, device
        self.prefill = synthetic_prefill(geo, tokens, seed, device, kv_dtype)

    def new_slot(self, max_cells: int, **kw) -> Slot:
        return new_slot(self.geo, max_cells, self.device, **kw)

    def carve_into(self, slot: Slot, pos0: int = 0, stream=None) -> None:
        plan = plan_carve(self.geo, self.prefill, slot, pos0)
        plan.launch(stream)
        import torch
        torch.cuda.synchronize()
        plan.destroy()

    def host_inputs(self) -> dict:
        return self.prefill.host()


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


def probe_link(nbytes: int = 256 << 20, iters: int = 4) -> tuple[float, float]:
    h2d, d2h = C.c_double(), C.c_double()
    check(lib.sc_probe_link(nbytes, iters, C.byref(h2d), C.byref(d2h)), "sc_probe_link")
    return float(h2d.value), float(d2h.value)
