"""The handoff path over geometries other than the configs' one, against the oracle, byte for byte.

The reference's geometry is a runtime value (include/strata/core/layout.hpp:27-59: its real model has HV = 48 value
heads and C = 10240 conv channels, the configs HV = 32 and C = 8192), and so are the pool's page size and head shape.
Every kernel derives its row, page and chunk arithmetic from the geometry, so each shape here runs the fused carve
(through identity, reversed and holed page tables, from a mid-page pos0), the two-pass gather -> scatter and a
park -> resume round trip, and every byte of the slot must equal the oracle's.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

BASE = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
            ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
GEOMETRIES = {
    "ps1_d64_h1": dict(BASE, page_size=1, head_dim=64, n_head_kv=1, ssm_state_size=16, ssm_v_heads=4,
                       ssm_conv_channels=72),
    "ps8_d128_h4": dict(BASE, page_size=8, head_dim=128, n_head_kv=4),
    "ps16_real_gdn": dict(BASE, page_size=16, ssm_state_size=128, ssm_v_heads=48, ssm_conv_channels=10240),
    "dconv3": dict(BASE, ssm_d_conv=3, ssm_conv_channels=1024),
    "dconv5_qsa3": dict(BASE, n_layers=12, qsa_interval=3, ssm_d_conv=5, ssm_conv_channels=260),
}


def _tables(sc, kind, n_qsa, n_pages):
    if kind == "identity":
        return None, None
    t = np.arange(n_pages, dtype=np.int32)
    if kind == "reversed":
        t = t[::-1].copy()
    else:
        t[1::3] = -1
    return sc.device_tables([t] * n_qsa), [t] * n_qsa


def _compare(want, got):
    for name in want:
        w, g = want[name].reshape(-1).view(np.uint8), got[name].reshape(-1).view(np.uint8)
        if not np.array_equal(w, g):
            bad = np.flatnonzero(w != g)
            raise AssertionError(f"{name}: {bad.size} bytes differ, first at byte {bad[0]}")


@pytest.mark.parametrize("name", sorted(GEOMETRIES))
@pytest.mark.parametrize("table,pos0", [("identity", 0), ("reversed", 0), ("holes", 5)])
def test_fused_carve(sc, oracle, cuda, name, table, pos0):
    print(f"case geometry {name} {table} pos0={pos0}", flush=True)
    geo = sc.geometry(**GEOMETRIES[name])
    tokens = 67
    ps = GEOMETRIES[name]["page_size"]
    max_cells = (pos0 + tokens + ps - 1) // ps * ps + 2 * ps
    n_pages = max_cells // ps
    case = synth.SyntheticCase(geo, tokens=tokens, seed=len(name) * 101 + pos0)
    dev_tabs, host_tabs = _tables(sc, table, geo.n_qsa, n_pages)
    slot = case.new_slot(max_cells=max_cells, tables=dev_tabs, fill=0xA5)
    sc.device_sync()
    initial = slot.host_state()
    case.carve_into(slot, pos0=pos0)
    want = oracle.expected_slot(geo, case.host_inputs(), slot_cells=max_cells, pos0=pos0, tables=host_tabs,
                                n_pages=n_pages, initial=initial)
    _compare(want, slot.host_state())


@pytest.mark.parametrize("name", sorted(GEOMETRIES))
def test_gather_scatter_and_park_resume(sc, oracle, cuda, name):
    print(f"case geometry {name} two-pass + park/resume", flush=True)
    geo = sc.geometry(**GEOMETRIES[name])
    tokens = 45
    case = synth.SyntheticCase(geo, tokens=tokens, seed=len(name))
    _, total = sc.image_layout(geo, tokens)
    image = sc.DeviceBuffer(max(total, 16), "uint8")
    image.fill(0xEE)
    sc.plan_gather(geo, case.prefill, image.data_ptr(), total).launch()
    sc.device_sync()
    cells = geo.cells(tokens)
    expected = oracle.expected_slot(geo, case.host_inputs(), slot_cells=cells)
    assert np.array_equal(image.numpy(total), oracle.park(geo, tokens, expected))
    # scatter the image into a reversed-table slot; it must equal the fused carve into the same slot
    ps = GEOMETRIES[name]["page_size"]
    max_cells = cells + 2 * ps
    n_pages = max_cells // ps
    dev_tabs, host_tabs = _tables(sc, "reversed", geo.n_qsa, n_pages)
    slot = case.new_slot(max_cells=max_cells, tables=dev_tabs)
    sc.plan_scatter(geo, image.data_ptr(), total, tokens, slot).launch()
    sc.device_sync()
    want = oracle.expected_slot(geo, case.host_inputs(), slot_cells=max_cells, tables=host_tabs, n_pages=n_pages)
    _compare(want, slot.host_state())
    # park an identity slot carved from the same inputs to pinned memory (one copy per blob) and resume it into a
    # fresh identity slot
    parked = case.new_slot(max_cells=max_cells)
    case.carve_into(parked)
    sc.device_sync()
    host = sc.PinnedBuffer(total)
    host.numpy()[:] = 0x77
    side, done = sc.Stream(), sc.Event()
    sc.park_async(geo, parked, tokens, host.ptr, total, stream=side, done=done.handle)
    done.sync()
    assert np.array_equal(host.numpy()[:total], image.numpy(total))
    fresh = case.new_slot(max_cells=max_cells, fill=0x5A)
    sc.device_sync()
    sc.resume_async(geo, host.ptr, total, tokens, fresh, stream=side, done=done.handle)
    done.sync()
    ident = oracle.expected_slot(geo, case.host_inputs(), slot_cells=max_cells)
    got = fresh.host_state()
    extent = cells // ps
    for key in ident:
        if key == "gdn":
            assert np.array_equal(got[key].view(np.uint8), ident[key].view(np.uint8))
        else:
            assert np.array_equal(got[key][:extent], ident[key][:extent]), key
            assert np.all(got[key][extent:].view(np.uint8) == 0x5A), key
    # park the paged slot itself (its pages gathered through the tables straight into pinned memory) and resume the
    # image into a fresh paged slot (scattered through the tables straight from pinned memory)
    host.numpy()[:] = 0x33
    sc.park_async(geo, slot, tokens, host.ptr, total, stream=side, done=done.handle)
    done.sync()
    assert np.array_equal(host.numpy()[:total], image.numpy(total)), "paged park"
    fresh_paged = case.new_slot(max_cells=max_cells, tables=dev_tabs, fill=0)
    sc.device_sync()
    sc.resume_async(geo, host.ptr, total, tokens, fresh_paged, stream=side, done=done.handle)
    done.sync()
    _compare(want, fresh_paged.host_state())
    host.free()


def test_paged_park_resume_beyond_one_launch(sc, cuda):
    """40 QSA layers: the paged park and resume take two launches of 32 and 8 layers; the parked image equals the
    capture of the slot and the resumed slot reads back as the same image."""
    geo = sc.geometry(n_layers=40, qsa_interval=1, n_head_kv=1, head_dim=64, page_size=8, ssm_state_size=16,
                      ssm_k_heads=2, ssm_v_heads=2, ssm_d_conv=4, ssm_conv_channels=64, idx_key_dim=64)
    assert geo.n_qsa == 40
    tokens, max_cells = 75, 96
    n_pages = max_cells // geo.page_size + 4
    rng = np.random.default_rng(40)
    tabs = sc.device_tables([rng.permutation(n_pages)[: max_cells // geo.page_size].astype(np.int32)
                             for _ in range(geo.n_qsa)])
    case = synth.SyntheticCase(geo, tokens, seed=404)
    slot = case.new_slot(max_cells=max_cells, n_pages=n_pages, tables=tabs)
    case.carve_into(slot)
    _, total = sc.image_layout(geo, tokens)
    image = sc.DeviceBuffer(total, "uint8")
    image.fill(0)
    sc.plan_capture(geo, slot, tokens, image.ptr, total).launch()
    sc.device_sync()
    host = sc.PinnedBuffer(total)
    host.numpy()[:] = 0
    side, done = sc.Stream(), sc.Event()
    sc.park_async(geo, slot, tokens, host.ptr, total, stream=side, done=done.handle)
    done.sync()
    assert np.array_equal(host.numpy()[:total], image.numpy(total)), "paged park"
    back = case.new_slot(max_cells=max_cells, n_pages=n_pages, tables=tabs, fill=0)
    sc.device_sync()
    sc.resume_async(geo, host.ptr, total, tokens, back, stream=side, done=done.handle)
    done.sync()
    again = sc.DeviceBuffer(total, "uint8")
    again.fill(0xAA)
    sc.plan_capture(geo, back, tokens, again.ptr, total).launch()
    sc.device_sync()
    assert np.array_equal(again.numpy(total), image.numpy(total)), "paged resume"
    host.free()


def test_paged_park_refuses_an_image_the_device_cannot_reach(sc, cuda):
    """A paged slot's pages are moved by a kernel that reads or writes the host image itself, so the image must be
    pinned memory mapped for the device: a pageable buffer is refused before anything is enqueued.  The park and the
    resume are only attempted after sc_host_range_mapped has reported the buffer unmapped, the same check they make."""
    import ctypes as C
    geo = sc.geometry(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
                      ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=512)
    tokens, max_cells = 61, 96
    n_pages = max_cells // geo.page_size + 3
    rng = np.random.default_rng(61)
    tabs = sc.device_tables([rng.permutation(n_pages)[: max_cells // geo.page_size].astype(np.int32)
                             for _ in range(geo.n_qsa)])
    case = synth.SyntheticCase(geo, tokens, seed=611)
    slot = case.new_slot(max_cells=max_cells, n_pages=n_pages, tables=tabs, fill=0x5A)
    sc.device_sync()
    _, total = sc.image_layout(geo, tokens)
    pageable = np.full(total, 0x33, dtype=np.uint8)
    mapped = C.c_int32(-1)
    assert sc.lib.sc_host_range_mapped(pageable.ctypes.data, total, C.byref(mapped)) == sc.SC_OK
    if mapped.value != 0:
        pytest.fail("a pageable buffer reads as mapped for the device; the refusal below cannot be tested safely")
    cs = slot.c_struct()
    assert sc.lib.sc_park_async(C.byref(geo), C.byref(cs), tokens, pageable.ctypes.data, total, None, None) == \
        sc.SC_EINVAL
    assert "pinned memory mapped for the device" in sc.last_error()
    assert sc.lib.sc_resume_async(C.byref(geo), pageable.ctypes.data, total, tokens, C.byref(cs), None, None) == \
        sc.SC_EINVAL
    sc.device_sync()
    assert np.all(pageable == 0x33)
    for name, pool in slot.host_state().items():
        if name != "gdn":
            assert np.all(pool.view(np.uint8) == 0x5A), name   # nothing was written
    pinned = sc.PinnedBuffer(total)
    assert sc.lib.sc_host_range_mapped(pinned.ptr, total, C.byref(mapped)) == sc.SC_OK
    assert mapped.value == 1
    pinned.free()
