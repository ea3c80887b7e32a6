"""ctypes binding of the CPU oracle (oracle/sc_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or the timed CPU baseline.  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
if not _LIB_PATH.exists():
    raise ImportError(f"the oracle is not built ({_LIB_PATH}); run __graft_entry__.build() first")
lib = C.CDLL(str(_LIB_PATH))

REFERENCE_FNV_SEED = 1469598103934665603   # 0x14650fb0739d0383, every call site of the reference
TEXTBOOK_FNV_BASIS = 0xCBF29CE484222325


class Geometry(C.Structure):
    _fields_ = [(name, C.c_int64) for name in (
        "n_layers", "qsa_interval", "n_head_kv", "head_dim", "page_size", "ssm_state_size", "ssm_k_heads",
        "ssm_v_heads", "ssm_d_conv", "ssm_conv_channels", "idx_key_dim")]


class Blob(C.Structure):
    _fields_ = [("kind", C.c_int32), ("layer", C.c_int32), ("offset", C.c_uint64), ("bytes", C.c_uint64)]


_P = C.c_void_p
_I64, _U64 = C.c_int64, C.c_uint64
_G = C.POINTER(Geometry)
for _name, _res, _args in (
    ("sco_mix64", _U64, [_U64]),
    ("sco_synth_key", _U64, [_U64, _U64]),
    ("sco_f16_bits", C.c_uint16, [C.c_uint32]),
    ("sco_f16_from_f32", None, [_P, _P, _U64]),
    ("sco_fill_uniform_f32", None, [_P, _U64, C.c_float, C.c_float, _U64, _U64]),
    ("sco_fill_uniform_f16", None, [_P, _U64, C.c_float, C.c_float, _U64, _U64]),
    ("sco_fill_normal_f32", None, [_P, _U64, _U64, _U64]),
    ("sco_kv_append", None, [_P, C.c_int, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    ("sco_rec_carve", None, [_P, _I64, _I64, _P]),
    ("sco_conv_hist", None, [_P, _P, _I64, _I64, _I64, _I64, C.c_int]),
    ("sco_gdn_row_floats", _I64, [_G]),
    ("sco_cells", _I64, [_G, _I64]),
    ("sco_image_layout", _I64, [_G, _I64, C.POINTER(Blob), C.POINTER(_U64)]),
    ("sco_park", None, [_G, _I64, C.POINTER(_P), C.POINTER(_P), _P, _P]),
    ("sco_resume", None, [_G, _I64, _P, C.POINTER(_P), C.POINTER(_P), _P]),
    ("sco_fnv1a64", _U64, [_P, _U64, _U64]),
    ("sco_f32_of_f16", C.c_float, [C.c_uint16]),
    ("sco_q8_row", None, [_P, _I64, _P, _P]),
    ("sco_q4_row", None, [_P, _I64, _P]),
    ("sco_kv_append_quant", None, [_P, C.c_int, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P]),
    ("sco_handoff_carve", None, [_G, _I64, _I64, C.c_int, C.POINTER(_P), C.POINTER(_P), C.c_int, C.POINTER(_P),
                                 C.POINTER(_P), _I64, _I64, C.POINTER(_P), C.POINTER(_P), C.POINTER(_P), _I64, _P]),
    ("sco_cpu_handoff", _U64, [_P, _P, _U64, _P]),
    ("sco_memcpy_threads", C.c_int, [_P, _P, _U64, C.c_int]),
    ("sco_synth_kv_blob_hash", _U64, [_I64, _I64, _I64, _I64, _P, C.c_int32, C.c_uint8, _U64]),
    ("sco_synth_quant_blob_hash", _U64, [_I64, _I64, _I64, _I64, _U64, _U64, _I64, C.c_float, C.c_float, C.c_int32,
                                         C.c_int32, C.c_uint8, _U64]),
    ("sco_synth_gdn_hash", _U64, [_G, _U64, _U64, _U64, _I64, _U64]),
):
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def geometry_from(geo) -> Geometry:
    """Copy any object with the sc_geometry fields (e.g. the product binding's Geometry)."""
    return Geometry(*[getattr(geo, f) for f, _ in Geometry._fields_])


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _parr(arrays) -> C.Array:
    arr = (C.c_void_p * max(len(arrays), 1))()
    for i, a in enumerate(arrays):
        arr[i] = None if a is None else _ptr(a)
    return arr


# ---- generators --------------------------------------------------------------------------------------------------

def fill_uniform_f16(n: int, lo: float, hi: float, seed: int, sid: int) -> np.ndarray:
    out = np.empty(max(n, 1), dtype=np.uint16)
    lib.sco_fill_uniform_f16(_ptr(out), n, lo, hi, seed, sid)
    return out[:n]


def fill_uniform_f32(n: int, lo: float, hi: float, seed: int, sid: int) -> np.ndarray:
    out = np.empty(max(n, 1), dtype=np.float32)
    lib.sco_fill_uniform_f32(_ptr(out), n, lo, hi, seed, sid)
    return out[:n]


def fill_normal_f32(n: int, seed: int, sid: int) -> np.ndarray:
    out = np.empty(max(n, 1), dtype=np.float32)
    lib.sco_fill_normal_f32(_ptr(out), n, seed, sid)
    return out[:n]


def f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib.sco_f16_from_f32(_ptr(x), _ptr(out), x.size)
    return out


# ---- carve pieces ----------------------------------------------------------------------------------------------------

def kv_append(src: np.ndarray, T: int, pos0: int, table, n_pages: int, H: int, D: int, ps: int,
              pool: np.ndarray) -> None:
    src = np.ascontiguousarray(src)
    dtype = 0 if src.dtype == np.uint16 else 1
    tab = None if table is None else np.ascontiguousarray(table, dtype=np.int32)
    lib.sco_kv_append(_ptr(src), dtype, T, pos0, None if tab is None else _ptr(tab), n_pages, H, D, ps, _ptr(pool))


def rec_carve(src: np.ndarray, S: int, HV: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.empty(S * HV * S, dtype=np.float32)
    lib.sco_rec_carve(_ptr(src), S, HV, _ptr(out))
    return out


def conv_hist(hist: np.ndarray, qkv: np.ndarray, rows: int, ld: int, C_: int, nhist: int, fresh: bool) -> None:
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    lib.sco_conv_hist(_ptr(hist), _ptr(qkv) if qkv.size else None, rows, ld, C_, nhist, int(fresh))


def image_layout(geo, tokens: int) -> tuple[list[tuple[int, int, int, int]], int]:
    g = geometry_from(geo)
    blobs = (Blob * 4096)()
    total = _U64()
    n = lib.sco_image_layout(C.byref(g), tokens, blobs, C.byref(total))
    return [(b.kind, b.layer, b.offset, b.bytes) for b in blobs[:n]], int(total.value)


# ---- slot images in every K/V format ----------------------------------------------------------------------------------

KV_F16, KV_INT8, KV_Q4, KV_K8V4 = 0, 1, 2, 3
IDX_BLOCK = 4          # the indexer pools one key per 4 cells (include/strata/kernels/qsa.hpp:103,112)
BUF_NAMES = ("k", "v", "k_scale", "v_scale", "pooled")   # ConversationKv's buffers, in the wire pool order


def layer_blob_bytes(geo, fmt: int, with_index: bool, tokens: int) -> list[int]:
    """One QSA layer's five blob sizes (k, v, k_scale, v_scale, pooled) for `tokens` tokens, restating layout() of
    src/core/conversation_snapshot.cpp:27-66: cells = ceil(T/page_size)*page_size; per head f16 2D bytes, int8 D, q4_0
    (D/32)*18 (kv_q4_bytes_per_head, include/strata/kernels/kv_q4.hpp:33); int8 keys carry (D/64)*2 bytes of f16 scales
    per head; K8V4 (format 3) is int8 K with q4_0 V and no V scales; pooled rows T/4 + 1 of idx_key_dim f32 with the
    index."""
    g = geometry_from(geo)
    H, D, ps = g.n_head_kv, g.head_dim, g.page_size
    cells = (tokens + ps - 1) // ps * ps
    q4_head = D // 32 * 18
    per_head = {KV_F16: 2 * D, KV_INT8: D, KV_Q4: q4_head, KV_K8V4: D}[fmt]
    k = cells * H * per_head
    v = cells * H * (q4_head if fmt == KV_K8V4 else per_head)
    ks = cells * H * (D // 64) * 2 if fmt in (KV_INT8, KV_K8V4) else 0
    vs = ks if fmt == KV_INT8 else 0
    pooled = (tokens // IDX_BLOCK + 1) * g.idx_key_dim * 4 if with_index and tokens > 0 else 0
    return [k, v, ks, vs, pooled]


def image_layout_layers(geo, fmt: int, with_index: bool, tokens: int) -> tuple[list[int | None], int]:
    """The slot image in any format: for each QSA layer its nonempty blobs in BUF_NAMES order, then the GDN rows, each
    64-byte aligned (the pool order of src/core/conversation_wire.cpp:400-437).  Returns the offsets (layer-major,
    five per layer, None for an empty blob; the GDN rows last) and the total."""
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    n_gdn = g.n_layers - n_qsa
    sizes = layer_blob_bytes(geo, fmt, with_index, tokens)
    offs: list[int | None] = []
    at = 0
    for _ in range(n_qsa):
        for n in sizes:
            if n:
                at = (at + 63) // 64 * 64
                offs.append(at)
                at += n
            else:
                offs.append(None)
    if n_gdn:
        at = (at + 63) // 64 * 64
        offs.append(at)
        at += n_gdn * int(lib.sco_gdn_row_floats(C.byref(g))) * 4
    else:
        offs.append(None)
    return offs, (at + 63) // 64 * 64


def fnv1a64(data: bytes | np.ndarray, seed: int = REFERENCE_FNV_SEED) -> int:
    a = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else \
        np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    return int(lib.sco_fnv1a64(_ptr(a) if a.size else None, a.size, seed))


# ---- whole-blob hashes of synthetic sequences ------------------------------------------------------------------------

class KvSource(C.Structure):
    """Cells [t0, t0 + n) of a K/V blob hold tokens 0..n-1 of stream `sid` under `seed` (U[lo, hi] -> f16)."""
    _fields_ = [("seed", _U64), ("sid", _U64), ("t0", _I64), ("n", _I64), ("lo", C.c_float), ("hi", C.c_float)]


# Stream ids of the synthetic sequences the product binding generates (sc_handoff.synthetic_prefill): K of QSA layer j
# is stream 1000 + 2j, V 1001 + 2j, the recurrence of GDN layer i 5000 + i and its conv rows 9000 + i.
SID_K0, SID_V0, SID_REC0, SID_CONV0 = 1000, 1001, 5000, 9000


def kv_blob_hash(geo, cells: int, sources, tail: int = 0, seed: int = REFERENCE_FNV_SEED) -> int:
    """FNV-1a of an identity-layout K or V blob of `cells` cells; `sources` are (seed, sid, t0, n) tuples (U[-4, 4]),
    cells no source covers hold `tail` bytes (sco_synth_kv_blob_hash)."""
    arr = (KvSource * max(len(sources), 1))(*[KvSource(s, sid, t0, n, -4.0, 4.0) for s, sid, t0, n in sources])
    return int(lib.sco_synth_kv_blob_hash(geo.n_head_kv, geo.head_dim, geo.page_size, cells, C.addressof(arr),
                                          len(sources), tail, seed))


def gdn_blob_hash(geo, seed: int, conv_rows: int, fnv_seed: int = REFERENCE_FNV_SEED) -> int:
    """FNV-1a of the GDN blob of a sequence carved fresh (sco_synth_gdn_hash)."""
    g = geometry_from(geo)
    return int(lib.sco_synth_gdn_hash(C.byref(g), seed, SID_REC0, SID_CONV0, conv_rows, fnv_seed))


def synthetic_image_hashes(geo, tokens: int, seed: int, conv_rows: int | None = None, tail: int = 0,
                           chunk: tuple[int, int] | None = None, threads: int = 16) -> list[int]:
    """The FNV-1a of every blob of the image (sco_image_layout order: K, V per QSA layer, then the GDN rows) of a
    synthetic sequence of `tokens` tokens under `seed`, carved fresh into a slot whose untouched bytes are `tail`.
    `chunk` = (chunk_seed, chunk_tokens) appends a K/V-only chunk at cell `tokens` (the batched resume + append), so
    the blobs cover tokens + chunk_tokens tokens.  Blobs are hashed on `threads` threads."""
    from concurrent.futures import ThreadPoolExecutor
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    n_gdn = g.n_layers - n_qsa
    total = tokens + (chunk[1] if chunk else 0)
    cells = int(lib.sco_cells(C.byref(g), total))
    conv_rows = min(tokens, g.ssm_d_conv - 1) if conv_rows is None else conv_rows
    jobs = []
    for j in range(n_qsa):
        for sid in (SID_K0 + 2 * j, SID_V0 + 2 * j):
            src = [(seed, sid, 0, tokens)]
            if chunk:
                src.append((chunk[0], sid, tokens, chunk[1]))
            jobs.append(("kv", src))
    if n_gdn:
        jobs.append(("gdn", None))

    def run(job):
        kind, src = job
        return kv_blob_hash(g, cells, src, tail) if kind == "kv" else gdn_blob_hash(g, seed, conv_rows)

    with ThreadPoolExecutor(max_workers=threads) as pool:
        return list(pool.map(run, jobs))


def quant_blob_hash(geo, cells: int, seed: int, sid: int, tokens: int, fmt: int, part: int, tail: int = 0,
                    fnv_seed: int = REFERENCE_FNV_SEED) -> int:
    """The FNV-1a of one quantized pool blob (codes or int8 scales) of a synthetic f32 sequence, streamed from the
    generator through sco_q8_row / sco_q4_row (sco_synth_quant_blob_hash)."""
    return int(lib.sco_synth_quant_blob_hash(geo.n_head_kv, geo.head_dim, geo.page_size, cells, seed, sid, tokens,
                                             -4.0, 4.0, fmt, part, tail, fnv_seed))


QUANT_INT8, QUANT_Q4, QUANT_K8V4 = 1, 2, 3   # the slot formats (sc_handoff.h SC_KV_*)


def synthetic_quant_hashes(geo, tokens: int, seed: int, fmt: int, conv_rows: int | None = None, tail: int = 0,
                           threads: int = 16) -> list[int]:
    """The FNV-1a of every blob of a quantized slot a synthetic f32 sequence of `tokens` tokens under `seed` carves to
    (sc_plan_carve_quant): per QSA layer the K codes, the V codes, then the K and V scales where the format has them
    (int8: both; K8V4: int8 K with its scales, q4_0 V; q4_0: none), then the GDN rows; the first cells(tokens) cells of
    each identity pool, untouched cells holding `tail`.  Blobs are hashed on `threads` threads."""
    from concurrent.futures import ThreadPoolExecutor
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    n_gdn = g.n_layers - n_qsa
    cells = int(lib.sco_cells(C.byref(g), tokens))
    conv_rows = min(tokens, g.ssm_d_conv - 1) if conv_rows is None else conv_rows
    k_fmt = QUANT_Q4 if fmt == QUANT_Q4 else QUANT_INT8
    v_fmt = QUANT_INT8 if fmt == QUANT_INT8 else QUANT_Q4
    jobs = []
    for j in range(n_qsa):
        jobs.append((SID_K0 + 2 * j, k_fmt, 0))
        jobs.append((SID_V0 + 2 * j, v_fmt, 0))
        if k_fmt == QUANT_INT8:
            jobs.append((SID_K0 + 2 * j, k_fmt, 1))
        if v_fmt == QUANT_INT8:
            jobs.append((SID_V0 + 2 * j, v_fmt, 1))
    if n_gdn:
        jobs.append(None)

    def run(job):
        if job is None:
            return gdn_blob_hash(g, seed, conv_rows)
        sid, f, part = job
        return quant_blob_hash(g, cells, seed, sid, tokens, f, part, tail)

    with ThreadPoolExecutor(max_workers=threads) as pool:
        return list(pool.map(run, jobs))


# ---- whole handoff -------------------------------------------------------------------------------------------------

def expected_slot(geo, inputs: dict, slot_cells: int, pos0: int = 0, tables=None, n_pages: int | None = None,
                  initial: dict | None = None, with_gdn: bool = True) -> dict:
    """The decode slot after the fused carve of `inputs` (as PrefillBuffers.host() returns them), starting from
    `initial` (default: zeros) - the oracle of sc_plan_carve."""
    g = geometry_from(geo)
    n_pages = n_pages if n_pages is not None else (slot_cells + g.page_size - 1) // g.page_size
    out = new_state(geo, n_pages, initial)
    carve_into(geo, inputs, out, n_pages, pos0, tables, with_gdn)
    return out


def new_state(geo, n_pages: int, initial: dict | None = None) -> dict:
    """A host decode slot (Slot.host_state() keys): zeros, or a copy of `initial`."""
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    n_gdn = g.n_layers - n_qsa
    ps, H, D = g.page_size, g.n_head_kv, g.head_dim
    row = int(lib.sco_gdn_row_floats(C.byref(g)))
    out = {}
    for j in range(n_qsa):
        for name in ("k", "v"):
            key = f"{name}{j}"
            out[key] = (initial[key].copy() if initial else np.zeros((n_pages, H, ps, D), dtype=np.uint16))
            out[key] = np.ascontiguousarray(out[key].reshape(n_pages, H, ps, D))
    if n_gdn:
        out["gdn"] = initial["gdn"].copy() if initial else np.zeros((n_gdn, row), dtype=np.float32)
        out["gdn"] = np.ascontiguousarray(out["gdn"].reshape(n_gdn, row))
    return out


def carve_into(geo, inputs: dict, out: dict, n_pages: int, pos0: int = 0, tables=None, with_gdn: bool = True) -> None:
    """The fused carve of `inputs` into the host slot `out`, in place (sco_handoff_carve)."""
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    n_gdn = g.n_layers - n_qsa
    T = inputs["tokens"]
    ks = [np.ascontiguousarray(a) for a in inputs["k"]]
    vs = [np.ascontiguousarray(a) for a in inputs["v"]]
    recs = [np.ascontiguousarray(a, dtype=np.float32) for a in inputs["rec"]]
    convs = [np.ascontiguousarray(a, dtype=np.float32) for a in inputs["conv"]]
    dtype = 0 if (ks and ks[0].dtype == np.uint16) else 1
    tabs = None
    if tables is not None:
        tabs = [None if t is None else np.ascontiguousarray(t, dtype=np.int32) for t in tables]
    kp = _parr([out[f"k{j}"] for j in range(n_qsa)])
    vp = _parr([out[f"v{j}"] for j in range(n_qsa)])
    lib.sco_handoff_carve(C.byref(g), T, pos0, dtype, _parr(ks), _parr(vs), int(with_gdn), _parr(recs),
                          _parr(convs), inputs["conv_rows"], g.ssm_conv_channels, kp, vp,
                          _parr(tabs) if tabs is not None else None, n_pages,
                          _ptr(out["gdn"]) if n_gdn else None)


def park(geo, tokens: int, state: dict) -> np.ndarray:
    """The image sc_park_async writes for a slot (identity pools) in `state` (Slot.host_state() keys)."""
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    _, total = image_layout(geo, tokens)
    image = np.empty(max(total, 1), dtype=np.uint8)
    ks = [np.ascontiguousarray(state[f"k{j}"]) for j in range(n_qsa)]
    vs = [np.ascontiguousarray(state[f"v{j}"]) for j in range(n_qsa)]
    gdn = np.ascontiguousarray(state["gdn"]) if "gdn" in state else None
    lib.sco_park(C.byref(g), tokens, _parr(ks), _parr(vs), None if gdn is None else _ptr(gdn), _ptr(image))
    return image[:total]


def resume(geo, tokens: int, image: np.ndarray, state: dict) -> None:
    g = geometry_from(geo)
    n_qsa = g.n_layers // g.qsa_interval
    ks = [state[f"k{j}"] for j in range(n_qsa)]
    vs = [state[f"v{j}"] for j in range(n_qsa)]
    gdn = state.get("gdn")
    lib.sco_resume(C.byref(g), tokens, _ptr(np.ascontiguousarray(image)), _parr(ks), _parr(vs),
                   None if gdn is None else _ptr(gdn))


def cpu_handoff(src: np.ndarray, dst: np.ndarray, scratch: np.ndarray) -> int:
    return int(lib.sco_cpu_handoff(_ptr(src), _ptr(dst), src.size, _ptr(scratch)))


def memcpy_threads(src: np.ndarray, dst: np.ndarray, threads: int) -> None:
    """Not the reference's path: `threads` threads memcpy one share each (the host's plain copy ceiling)."""
    assert src.nbytes == dst.nbytes and lib.sco_memcpy_threads(_ptr(dst), _ptr(src), src.nbytes, threads) == 0


# ---- quantized K/V formats ---------------------------------------------------------------------------------------

def q8_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """int8 codes [rows][D] and f16 scale bits [rows][D/64] of f32 rows [rows][D] (sco_q8_row)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.reshape(-1, D)
    codes = np.zeros(rows.shape, dtype=np.int8)
    scales = np.zeros((rows.shape[0], D // 64), dtype=np.uint16)
    for r in range(rows.shape[0]):
        lib.sco_q8_row(_ptr(rows[r]), D, _ptr(codes[r]), _ptr(scales[r]))
    return codes, scales


def q4_rows(x: np.ndarray) -> np.ndarray:
    """q4_0 blocks [rows][D/32*18] of f32 rows [rows][D] (sco_q4_row)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.reshape(-1, D)
    out = np.zeros((rows.shape[0], D // 32 * 18), dtype=np.uint8)
    for r in range(rows.shape[0]):
        lib.sco_q4_row(_ptr(rows[r]), D, _ptr(out[r]))
    return out


def kv_append_quant(src: np.ndarray, fmt: int, T: int, pos0: int, table, n_pages: int, H: int, D: int, ps: int,
                    codes: np.ndarray, scales: np.ndarray | None) -> None:
    """In place: the quantizing carve of f32 [T][H][D] into a codes pool (and int8 scale pool) (sco_kv_append_quant)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    t = None if table is None else np.ascontiguousarray(table, dtype=np.int32)
    lib.sco_kv_append_quant(_ptr(src), fmt, T, pos0, _ptr(t) if t is not None else None, n_pages, H, D, ps,
                            _ptr(codes), _ptr(scales) if scales is not None else None)
