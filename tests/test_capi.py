"""The C-ABI library on the CPU: it loads, exports every entry point include/sc_handoff.h declares, and its host
logic (layout arithmetic, refusals before any HIP call) matches the oracle and the reference's error contract.
No test here makes a compute call: there is no GPU in this container."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "sc_handoff.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(sc):
    names = declared_symbols()
    assert len(names) >= 30
    for name in names:
        assert hasattr(sc.lib, name), name
    assert set(names) == set(sc.EXPORTS)


def test_version(sc):
    assert sc.lib.sc_version().decode().startswith("sc_handoff")


def test_layout_arithmetic_matches_oracle(sc, oracle):
    for kw in ({}, dict(n_layers=16), dict(ssm_v_heads=48, ssm_conv_channels=10240), dict(page_size=1)):
        geo = sc.geometry(**kw)
        for tokens in (0, 1, 3, 4, 5, 4096, 32768, 131071):
            blobs, total = sc.image_layout(geo, tokens)
            want, want_total = oracle.image_layout(geo, tokens)
            assert total == want_total
            assert [(b.kind, b.layer, b.offset, b.bytes) for b in blobs] == want
            assert sc.payload_bytes(geo, tokens) == sum(b[3] for b in want)
            assert sc.lib.sc_kv_cells(C.byref(geo), tokens) == oracle.lib.sco_cells(oracle.geometry_from(geo), tokens)
        assert sc.lib.sc_gdn_row_floats(C.byref(geo)) == geo.gdn_row_floats
        assert sc.lib.sc_n_qsa_layers(C.byref(geo)) == geo.n_layers // 4


def _fake_slot(sc, geo, max_cells, n_pages):
    # host addresses stand in for device pointers: every request below is refused before any HIP call
    fake = 1 << 40
    ks = (C.c_void_p * geo.n_qsa)(*[fake + 0x1000 * j for j in range(geo.n_qsa)])
    vs = (C.c_void_p * geo.n_qsa)(*[fake + 0x100000 + 0x1000 * j for j in range(geo.n_qsa)])
    slot = sc.DecodeSlot(n_pages=n_pages, max_cells=max_cells, k_pool=C.cast(ks, C.POINTER(C.c_void_p)),
                         v_pool=C.cast(vs, C.POINTER(C.c_void_p)), page_table=None, gdn_state=fake + 0x200000)
    return slot, (ks, vs)


def _fake_view(sc, geo, tokens, pos0=0):
    fake = 1 << 41
    arr = lambda n, base: (C.c_void_p * max(n, 1))(*[base + 0x1000 * i for i in range(n)])
    k, v, r, c = arr(geo.n_qsa, fake), arr(geo.n_qsa, fake + 1 << 30), arr(geo.n_gdn, fake + 2 << 30), \
        arr(geo.n_gdn, fake + 3 << 30)
    cast = lambda a: C.cast(a, C.POINTER(C.c_void_p))
    view = sc.PrefillView(tokens=tokens, pos0=pos0, kv_dtype=0, with_gdn=1, k=cast(k), v=cast(v), rec=cast(r),
                          conv=cast(c), conv_rows=3, conv_ld=geo.ssm_conv_channels)
    return view, (k, v, r, c)


@pytest.mark.parametrize("case", ["past_capacity", "pool_too_small", "bad_dtype", "missing_pool", "bad_geometry",
                                  "short_conv_ld", "misaligned"])
def test_carve_refusals_before_any_hip_call(sc, case):
    geo = sc.geometry(n_layers=8)
    slot, keep1 = _fake_slot(sc, geo, max_cells=64, n_pages=16)
    view, keep2 = _fake_view(sc, geo, tokens=60)
    if case == "past_capacity":
        view.pos0 = 8                      # 8 + 60 > 64 cells
    elif case == "pool_too_small":
        slot.n_pages = 8                   # identity pools hold 32 cells < max_cells
    elif case == "bad_dtype":
        view.kv_dtype = 7
    elif case == "missing_pool":
        keep1[0][1] = None
    elif case == "bad_geometry":
        geo.head_dim = 12                  # 24-byte rows
    elif case == "short_conv_ld":
        view.conv_ld = geo.ssm_conv_channels - 1
    elif case == "misaligned":
        keep2[0][0] = (1 << 41) + 8
    h = C.c_void_p()
    rc = sc.lib.sc_plan_carve(C.byref(geo), C.byref(view), C.byref(slot), C.byref(h))
    assert rc == sc.SC_EINVAL
    assert h.value is None
    msg = sc.last_error()
    assert msg.startswith("conversation snapshot:") or msg.startswith("sc_handoff:")


def test_image_refusals(sc):
    geo = sc.geometry(n_layers=8)
    slot, keep = _fake_slot(sc, geo, max_cells=64, n_pages=16)
    _, total = sc.image_layout(geo, 60)
    h = C.c_void_p()
    # an image smaller than the layout is refused, the reference's "invalid K/V payload size"
    assert sc.lib.sc_plan_scatter(C.byref(geo), 1 << 40, total - 64, 60, C.byref(slot), C.byref(h)) == sc.SC_EINVAL
    assert "invalid K/V payload size" in sc.last_error()
    # more tokens than the slot holds
    assert sc.lib.sc_plan_scatter(C.byref(geo), 1 << 40, 1 << 40, 65, C.byref(slot), C.byref(h)) == sc.SC_EINVAL
    assert sc.last_error() == "conversation snapshot: invalid K/V extent"
    # a paged slot's park is checked the same way before anything is enqueued: an image smaller than the layout, and
    # more tokens than the slot holds, are refused
    tab = (C.c_void_p * 2)(1 << 42, None)
    slot.page_table = C.cast(tab, C.POINTER(C.c_void_p))
    assert sc.lib.sc_park_async(C.byref(geo), C.byref(slot), 60, 1 << 40, total - 64, None, None) == sc.SC_EINVAL
    assert "invalid K/V payload size" in sc.last_error()
    assert sc.lib.sc_resume_async(C.byref(geo), 1 << 40, 1 << 40, 65, C.byref(slot), None, None) == sc.SC_EINVAL
    assert sc.last_error() == "conversation snapshot: invalid K/V extent"


def test_kv_append_range_refusals_before_any_hip_call(sc):
    """A per-layer append whose rows the tiles could not index (2^31 chunks or more) is refused on the host, before
    any launch: the pointers here are aligned stand-ins that are never dereferenced."""
    K, pools = 1 << 40, 1 << 41
    assert sc.lib.sc_kv_append_q4_async(pools, pools, None, 0, 1 << 30, K, K, 4, 256, 4, None, None,
                                        None) == sc.SC_ERANGE
    assert "2^31 chunks" in sc.last_error()
    assert sc.lib.sc_kv_append_async(K, K, 1 << 26, 0, None, 4, pools, pools, None, None, None, None, None, None,
                                     None) == sc.SC_ERANGE
    assert "2^31 chunks" in sc.last_error()


def test_noalloc_hash_refusals_before_any_hip_call(sc):
    """The hash without allocation refuses inputs past its static workspace, and missing pointers, on the host."""
    out = 1 << 40   # never dereferenced: the refusals come first
    fault = out + 8
    assert sc.lib.sc_fnv1a64_noalloc_async(1 << 40, (4 << 30) + 1, 0, out, fault, None) == sc.SC_ERANGE
    assert "at most 4 GiB" in sc.last_error()
    assert sc.lib.sc_fnv1a64_noalloc_async(None, 16, 0, out, fault, None) == sc.SC_EINVAL
    assert sc.lib.sc_fnv1a64_noalloc_async(1 << 40, 16, 0, None, fault, None) == sc.SC_EINVAL
    assert sc.lib.sc_fnv1a64_noalloc_async(1 << 40, 16, 0, out, None, None) == sc.SC_EINVAL
    assert "fault word" in sc.last_error()
    assert sc.lib.sc_fnv1a64_noalloc_async(1 << 40, 16, 0, out, fault + 1, None) == sc.SC_EINVAL
    assert "4-byte aligned" in sc.last_error()


def test_copy_plan_refusals_before_any_hip_call(sc):
    """A copy plan refuses copies that are not whole 16-byte chunks between 16-byte aligned addresses, and copies whose
    destinations overlap, on the host (host addresses stand in: nothing is allocated or dereferenced)."""
    base = 1 << 40
    out = C.c_void_p()
    for copies in ([(base + 8, base + 4096, 64)], [(base, base + 4096 + 4, 64)], [(base, base + 4096, 40)],
                   [(base, base + 4096, 64), (base + 32, base + 8192, 64)]):
        arr = (sc.CopyDesc * len(copies))(*[sc.CopyDesc(d, s_, b) for d, s_, b in copies])
        assert sc.lib.sc_plan_copies(C.cast(arr, C.c_void_p), len(copies), C.byref(out)) == sc.SC_EINVAL
    assert "same bytes" in sc.last_error()
    assert sc.lib.sc_plan_copies(None, 1, C.byref(out)) == sc.SC_EINVAL


def test_core_library_exports_the_wire_abi():
    """libsc_core.so exports every entry point include/sc_wire.h declares (the device payload path)."""
    import sc_wire
    text = (ROOT / "include" / "sc_wire.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = sorted(set(re.findall(r"\b(sc_wire_[a-z0-9_]+)\s*\(", text)))
    assert len(names) >= 10
    for name in names:
        assert hasattr(sc_wire.lib, name), name
    assert set(names) == set(sc_wire.EXPORTS)


def test_wire_refusals_before_any_hip_call(sc):
    """The device payload path refuses malformed requests on the host (no GPU needed)."""
    import sc_wire
    geo = sc.geometry(n_layers=8)
    h = C.c_void_p()
    assert sc_wire.lib.sc_wire_encoder_create(None, None, 0, None, 0, 0, C.byref(h)) == sc.SC_EINVAL
    assert "missing" in sc_wire.lib.sc_wire_last_error().decode()
    assert sc_wire.lib.sc_wire_decoder_open(None, 0, C.byref(geo), None, None, 0, 0, 0, 0, 0, C.byref(h)) == sc.SC_EINVAL


def test_core_library_exports_the_arena_abi():
    """libsc_core.so exports every entry point include/sc_arena.h declares (the hand-off arena and its movers)."""
    import sc_arena
    text = (ROOT / "include" / "sc_arena.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = sorted(set(re.findall(r"\b(sc_(?:arena|mover)_[a-z0-9_]+)\s*\(", text)))
    assert len(names) >= 19
    for name in names:
        assert hasattr(sc_arena.lib, name), name
    assert set(names) == set(sc_arena.EXPORTS)


def test_ipc_refusals_before_any_hip_call(sc):
    """Same-GPU hand-off segments over 1 GiB, of odd sizes or too many are refused on the host (no handle opened)."""
    h = C.c_void_p()
    assert sc.lib.sc_ipc_export_create(1 << 20, (1 << 30) + 4096, C.byref(h)) == sc.SC_ERANGE
    assert sc.lib.sc_ipc_export_create(1 << 20, 1000, C.byref(h)) == sc.SC_ERANGE
    assert sc.lib.sc_ipc_export_create(65 << 20, 1 << 20, C.byref(h)) == sc.SC_ERANGE   # 65 segments
    assert sc.lib.sc_ipc_export_create(0, 1 << 20, C.byref(h)) == sc.SC_ERANGE
    seg = (sc.IpcSegment * 2)()
    seg[0].bytes, seg[1].bytes = 1 << 20, (1 << 30) + 1
    assert sc.lib.sc_ipc_import_open(seg, 2, C.byref(h)) == sc.SC_ERANGE
    assert "SC_IPC_MAX_SEGMENT" in sc.last_error()
    assert sc.lib.sc_ipc_import_open(seg, 65, C.byref(h)) == sc.SC_ERANGE


def test_kv_block_bytes_per_format(sc):
    """sc_kv_block_bytes (kv_block_bytes, src/kernels/cuda/kv_stream.cu:192-197): one block (page) of K and V.  At the
    real model's shapes (2 KV heads of 256, 4 cells per page, include/strata/kernels/qsa.hpp:96-117) the reference's own
    per-cell figures fix it: f16 2 048 B, int8 1 056 B (the --kv help text, src/program/generate.cpp:532-537), and
    K8V4's 816 B (same text) is half an int8 cell plus half a q4_0 cell, which fixes q4_0 at 576 B.  Other shapes follow
    the per-format row sizes: f16 2 * head_dim, int8 head_dim + one f16 scale per 64, q4_0 18 B per 32 values."""
    f16, int8, q4 = (int(sc.lib.sc_kv_block_bytes(2, 256, 4, fmt)) for fmt in (0, 1, 2))
    assert (f16, int8) == (4 * 2048, 4 * 1056)
    assert (int8 + q4) // 2 == 4 * 816 and q4 == 4 * 576
    for heads, dim, ps in ((1, 64, 1), (4, 128, 8), (2, 512, 16), (3, 256, 2)):
        rows = heads * ps
        assert sc.lib.sc_kv_block_bytes(heads, dim, ps, 0) == rows * dim * 2 * 2
        assert sc.lib.sc_kv_block_bytes(heads, dim, ps, 1) == rows * (dim + dim // 64 * 2) * 2
        assert sc.lib.sc_kv_block_bytes(heads, dim, ps, 2) == rows * (dim // 32 * 18) * 2
