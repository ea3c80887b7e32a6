"""Parity of the HIP handoff path with the CPU oracle, through the C-ABI (libsc_handoff.so).

Bar: bit-exact for every byte (the path is integer / byte movement, plus an RNE f32->f16 rounding that is exact by
definition).  Small and toy-config cases compare every byte with the oracle; the full-depth 32K and 128K configs are
checked through properties that hold at any size: the fused carve equals the two-pass gather -> scatter, a park ->
resume round trip is the identity, sampled rows sit where the reference's closed forms put them, and the whole
conv history matches the oracle.
"""
import ctypes as C

import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
TOY = dict(n_layers=16)   # config 1: 4 QSA + 12 GDN layers at the configs' per-layer geometry


def _sync():
    import sc_handoff
    sc_handoff.device_sync()


def _device_u8(nbytes):
    import sc_handoff
    return sc_handoff.DeviceBuffer(max(nbytes, 16), "uint8")


def _tables(kind, n_qsa, n_pages):
    import sc_handoff
    if kind == "identity":
        return None, None
    if kind == "reversed":
        t = np.arange(n_pages)[::-1].astype(np.int32)
    elif kind == "holes":
        t = np.arange(n_pages).astype(np.int32)
        t[1::3] = -1
    elif kind == "shuffled":
        t = np.random.default_rng(n_pages).permutation(n_pages).astype(np.int32)
    else:
        raise ValueError(kind)
    return sc_handoff.device_tables([t] * n_qsa), [t] * n_qsa


def _compare(want, got):
    assert set(want) <= set(got)
    for name in want:
        w, g = want[name].reshape(-1), got[name].reshape(-1)
        if not np.array_equal(w.view(np.uint8), g.view(np.uint8)):
            bad = np.nonzero(w.view(np.uint8) != g.view(np.uint8))[0]
            raise AssertionError(f"{name}: {bad.size} bytes differ, first at byte {bad[0]}")


# ---- generators --------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 1000, 4097, 1 << 20])
def test_device_generators_match_oracle(sc, oracle, cuda, n):
    a = sc.DeviceBuffer(n, "uint16")
    sc.check(sc.lib.sc_fill_uniform_f16(a.ptr, n, -4.0, 4.0, 0x5EED, 17, None), "fill")
    b = sc.DeviceBuffer(n, "float32")
    sc.check(sc.lib.sc_fill_normal_f32(b.ptr, n, 0x5EED, 18, None), "fill")
    c = sc.DeviceBuffer(n, "float32")
    sc.check(sc.lib.sc_fill_uniform_f32(c.ptr, n, -4.0, 4.0, 99, 3, None), "fill")
    _sync()
    assert np.array_equal(a.numpy(), oracle.fill_uniform_f16(n, -4.0, 4.0, 0x5EED, 17))
    assert np.array_equal(b.numpy().view(np.uint32), oracle.fill_normal_f32(n, 0x5EED, 18).view(np.uint32))
    assert np.array_equal(c.numpy().view(np.uint32), oracle.fill_uniform_f32(n, -4.0, 4.0, 99, 3).view(np.uint32))


# ---- the fused carve -> scatter, every byte against the oracle -----------------------------------------------------

def test_toy_config_fused_carve_bit_exact(sc, oracle, cuda):
    """Config 1: 16 layers (4 QSA, 12 GDN), 4096 tokens, K/V U[-4,4] f16, state N(0,1), one decode slot."""
    geo = sc.geometry(**TOY)
    case = synth.SyntheticCase(geo, tokens=4096, seed=0x5EED)
    slot = case.new_slot(max_cells=4096)
    case.carve_into(slot)
    want = oracle.expected_slot(geo, case.host_inputs(), slot_cells=4096)
    _compare(want, slot.host_state())
    assert sc.payload_bytes(geo, 4096) == 59_899_904


@pytest.mark.parametrize("tokens,pos0,max_cells,table,dtype", [
    (77, 0, 128, "identity", "f16"),     # partial last page
    (77, 3, 128, "identity", "f16"),     # an append starting mid-page, older conv history kept
    (96, 0, 96, "reversed", "f16"),      # the reference's reversed-table fixture (qsa_parity.cpp:458)
    (61, 6, 80, "holes", "f16"),         # non-resident pages are skipped
    (100, 0, 104, "shuffled", "f16"),
    (53, 0, 64, "identity", "f32"),      # f32 K/V rounded to f16 (kv_append's arithmetic)
    (2, 0, 8, "identity", "f16"),        # a chunk shorter than the conv history, fresh sequence
    (1, 5, 8, "identity", "f16"),        # ... and appended: older history rows survive
    (0, 0, 8, "identity", "f16"),        # no tokens: only the running state moves
])
def test_fused_carve_cases(sc, oracle, cuda, tokens, pos0, max_cells, table, dtype):
    geo = sc.geometry(**SMALL)
    kv_dtype = sc.SC_DTYPE_F16 if dtype == "f16" else sc.SC_DTYPE_F32
    case = synth.SyntheticCase(geo, tokens=tokens, seed=tokens * 31 + pos0, kv_dtype=kv_dtype)
    n_pages = max_cells // geo.page_size
    dev_tabs, host_tabs = _tables(table, geo.n_qsa, n_pages)
    slot = case.new_slot(max_cells=max_cells, tables=dev_tabs, fill=0xA5)
    _sync()
    initial = slot.host_state()
    case.carve_into(slot, pos0=pos0)
    want = oracle.expected_slot(geo, case.host_inputs(), slot_cells=max_cells, pos0=pos0, tables=host_tabs,
                                n_pages=n_pages, initial=initial)
    _compare(want, slot.host_state())


def test_kv_only_chunk_leaves_running_state(sc, oracle, cuda):
    geo = sc.geometry(**SMALL)
    case = synth.SyntheticCase(geo, tokens=40, seed=5)
    slot = case.new_slot(max_cells=64, fill=0x3C)
    _sync()
    initial = slot.host_state()
    plan = sc.plan_carve(geo, case.prefill, slot, pos0=9, with_gdn=False)
    plan.launch()
    _sync()
    want = oracle.expected_slot(geo, case.host_inputs(), slot_cells=64, pos0=9, initial=initial, with_gdn=False)
    got = slot.host_state()
    _compare(want, got)
    assert np.array_equal(got["gdn"].view(np.uint32), initial["gdn"].view(np.uint32))


# ---- two-pass: gather into the transfer buffer, scatter into the slot ---------------------------------------------

@pytest.mark.parametrize("tokens,table", [(77, "identity"), (96, "reversed"), (4096, "identity")])
def test_gather_then_scatter(sc, oracle, cuda, tokens, table):
    geo = sc.geometry(**(SMALL if tokens < 1000 else TOY))
    case = synth.SyntheticCase(geo, tokens=tokens, seed=tokens)
    _, total = sc.image_layout(geo, tokens)
    image = _device_u8(total)
    image.fill(0xEE)
    gather = sc.plan_gather(geo, case.prefill, image.data_ptr(), total)
    gather.launch()
    _sync()
    # the image is the park image of the fused carve into a zeroed identity slot
    cells = geo.cells(tokens)
    expected = oracle.expected_slot(geo, case.host_inputs(), slot_cells=cells)
    want_image = oracle.park(geo, tokens, expected)
    got_image = image.numpy(total)
    assert np.array_equal(got_image, want_image)
    # scatter into a decode slot (possibly paged) == the fused carve into the same kind of slot
    max_cells = cells + 8
    n_pages = max_cells // geo.page_size
    dev_tabs, host_tabs = _tables(table, geo.n_qsa, n_pages)
    slot = case.new_slot(max_cells=max_cells, tables=dev_tabs)
    fused = case.new_slot(max_cells=max_cells, tables=dev_tabs)
    scatter = sc.plan_scatter(geo, image.data_ptr(), total, tokens, slot)
    scatter.launch()
    case.carve_into(fused)
    _sync()
    _compare(fused.host_state(), slot.host_state())
    want = oracle.expected_slot(geo, case.host_inputs(), slot_cells=max_cells, tables=host_tabs, n_pages=n_pages)
    _compare(want, slot.host_state())


@pytest.mark.parametrize("table", ["identity", "reversed", "shuffled"])
def test_capture_reads_through_the_page_table(sc, oracle, cuda, table):
    geo = sc.geometry(**SMALL)
    tokens, max_cells = 90, 96
    case = synth.SyntheticCase(geo, tokens=tokens, seed=77)
    n_pages = max_cells // geo.page_size
    dev_tabs, host_tabs = _tables(table, geo.n_qsa, n_pages)
    slot = case.new_slot(max_cells=max_cells, tables=dev_tabs)
    case.carve_into(slot)
    _, total = sc.image_layout(geo, tokens)
    image = _device_u8(total)
    image.fill(0x11)
    plan = sc.plan_capture(geo, slot, tokens, image.data_ptr(), total)
    plan.launch()
    _sync()
    # un-page on the host: logical page p lives at physical page table[p]
    state = slot.host_state()
    cells = geo.cells(tokens)
    logical = {}
    for key, pool in state.items():
        if key == "gdn":
            logical[key] = pool
            continue
        order = np.arange(cells // geo.page_size) if host_tabs is None else host_tabs[0][: cells // geo.page_size]
        logical[key] = np.ascontiguousarray(pool[order])
    assert np.array_equal(image.numpy(total), oracle.park(geo, tokens, logical))


# ---- park / resume: pinned host RAM on a side stream ---------------------------------------------------------------

def test_park_resume_round_trip(sc, oracle, cuda):
    geo = sc.geometry(**TOY)
    tokens = 4093
    case = synth.SyntheticCase(geo, tokens=tokens, seed=4093)
    slot = case.new_slot(max_cells=4096)
    case.carve_into(slot)
    _, total = sc.image_layout(geo, tokens)
    host = sc.PinnedBuffer(total)
    host.numpy()[:] = 0x77
    side = sc.Stream()
    done = sc.Event()
    sc.park_async(geo, slot, tokens, host.ptr, total, stream=side, done=done.handle)
    done.sync()
    state = slot.host_state()
    assert np.array_equal(host.numpy(), oracle.park(geo, tokens, state))
    fresh = case.new_slot(max_cells=4096, fill=0x5A)
    _sync()   # the fill ran on the null stream; the non-blocking side stream does not wait for it
    sc.resume_async(geo, host.ptr, total, tokens, fresh, stream=side, done=done.handle)
    done.sync()
    got = fresh.host_state()
    extent = geo.cells(tokens) // geo.page_size
    for key in state:
        if key == "gdn":
            assert np.array_equal(got[key].view(np.uint32), state[key].view(np.uint32))
        else:
            assert np.array_equal(got[key][:extent], state[key][:extent])
            assert np.all(got[key][extent:].view(np.uint8) == 0x5A)   # nothing past the parked extent is touched
    host.free()


def test_refusal_writes_nothing(sc, cuda):
    """Invalid requests are refused before the first write (conversation_snapshot.hpp:104-105)."""
    geo = sc.geometry(**SMALL)
    case = synth.SyntheticCase(geo, tokens=60, seed=1)
    slot = case.new_slot(max_cells=64, fill=0xA5)
    _sync()
    before = slot.host_state()
    with pytest.raises(sc.ScError) as err:
        sc.plan_carve(geo, case.prefill, slot, pos0=8)   # 68 cells into a 64-cell slot
    assert err.value.code == sc.SC_EINVAL
    assert "invalid K/V extent" in str(err.value)
    _, total = sc.image_layout(geo, 60)
    host = sc.PinnedBuffer(total)
    with pytest.raises(sc.ScError):
        sc.resume_async(geo, host.ptr, total - 64, 60, slot)
    _sync()
    after = slot.host_state()
    for key in before:
        assert np.array_equal(before[key].view(np.uint8), after[key].view(np.uint8))
    host.free()


# ---- full-depth configs: size-independent properties ----------------------------------------------------------------

def _sampled_rows_check(sc, oracle, geo, case, slot, n_samples=4096, seed=0):
    """Sampled K/V rows and recurrence rows sit where the reference's closed forms put them (kv_append's row for
    cell t of head h: page t // ps, in-page t % ps; the recurrence's (i, h) row of (S, HV, S)); the whole conv
    history of every GDN layer matches the oracle."""
    rng = np.random.default_rng(seed)
    T, H, ps, S, HV = case.tokens, geo.n_head_kv, geo.page_size, geo.ssm_state_size, geo.ssm_v_heads
    for j in rng.choice(geo.n_qsa, size=3, replace=False):
        t = rng.integers(0, T, size=n_samples)
        h = rng.integers(0, H, size=n_samples)
        for src, pool in ((case.prefill.k[j], slot.k_pool[j]), (case.prefill.v[j], slot.v_pool[j])):
            src_h, pool_h = src.numpy(), pool.numpy()
            assert np.array_equal(src_h[t, h], pool_h[t // ps, h, t % ps])
    for g in rng.choice(geo.n_gdn, size=4, replace=False):
        i = rng.integers(0, S, size=n_samples)
        hv = rng.integers(0, HV, size=n_samples)
        rec = slot.gdn.numpy(S * HV * S, int(g) * geo.gdn_row_floats).reshape(S, HV, S)
        src = case.prefill.rec[g].numpy()
        assert np.array_equal(src[hv, i].view(np.uint32), rec[i, hv].view(np.uint32))
    Cc, nh = geo.ssm_conv_channels, geo.ssm_d_conv - 1
    gdn = slot.gdn.numpy()
    for g in range(geo.n_gdn):
        hist = np.zeros((Cc, nh), dtype=np.float32)
        oracle.conv_hist(hist, case.prefill.conv[g].numpy(), case.prefill.conv_rows, Cc, Cc, nh, True)
        assert np.array_equal(gdn[g, S * HV * S:].view(np.uint32), hist.reshape(-1).view(np.uint32))


def _equal_buffers(a_list, b_list):
    for a, b in zip(a_list, b_list):
        assert a.nbytes == b.nbytes
        assert np.array_equal(a.numpy().view(np.uint8), b.numpy().view(np.uint8))


@pytest.mark.parametrize("tokens", [32768, 131072])
def test_full_depth_properties(sc, oracle, cuda, tokens):
    """Configs 2 and 3: 48 layers (12 QSA, 36 GDN) at 32K and 128K tokens."""
    geo = sc.geometry()
    case = synth.SyntheticCase(geo, tokens=tokens, seed=0x5EED + tokens)
    fused = case.new_slot(max_cells=tokens)
    case.carve_into(fused)
    _sampled_rows_check(sc, oracle, geo, case, fused, seed=tokens)
    # two-pass through a transfer buffer gives the same slot
    _, total = sc.image_layout(geo, tokens)
    assert total == sc.payload_bytes(geo, tokens)
    image = _device_u8(total)
    gather = sc.plan_gather(geo, case.prefill, image.ptr, total)
    gather.launch()
    two_pass = case.new_slot(max_cells=tokens, fill=0x33)
    scatter = sc.plan_scatter(geo, image.ptr, total, tokens, two_pass)
    scatter.launch()
    _sync()
    _equal_buffers(fused.buffers(), two_pass.buffers())
    # park -> resume round trip through pinned host memory on a side stream
    host = sc.PinnedBuffer(total)
    side = sc.Stream()
    done = sc.Event()
    sc.park_async(geo, fused, tokens, host.ptr, total, stream=side, done=done.handle)
    done.sync()
    assert np.array_equal(host.numpy(), image.numpy(total))   # the parked image is the gathered transfer buffer
    two_pass.fill(0)
    _sync()
    sc.resume_async(geo, host.ptr, total, tokens, two_pass, stream=side, done=done.handle)
    done.sync()
    _equal_buffers(fused.buffers(), two_pass.buffers())
    host.free()
