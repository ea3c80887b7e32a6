"""Destination-ordered page tiles (sc_set_order_min_pages, MoveRow::order): a plan whose rows write through a page
table visits the logical pages in the order of their physical pages, the order rebuilt on the device before every
launch.  The bytes written must not change: every case here compares the pools with the CPU oracle's placement
(sco_kv_append, pinned in tests/test_oracle.py) or with the same move in source order, byte for byte, including
tables with holes (-1: a page that is not resident, skipped as the reference's kv_append skips it,
src/prefill/kernels.cu:577), entries past the pool, pools larger than the pages written, a table changed between
two launches of one plan, and the scatter of a parked image into a paged slot.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

GEO = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32, ssm_k_heads=4,
           ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
SENTINEL = 0xEE


@pytest.fixture
def ordered(sc):
    """Every table gets the destination order, however few pages it covers."""
    prev = sc.set_order_min_pages(1)
    yield
    sc.set_order_min_pages(prev)


def _table(rng, logical, n_pages, kind):
    if kind == "permuted":
        return rng.permutation(n_pages)[:logical].astype(np.int32)
    if kind == "holes":
        t = rng.permutation(n_pages)[:logical].astype(np.int32)
        t[1::3] = -1
        return t
    if kind == "past_pool":   # entries at or past the pool's end are skipped like holes
        t = rng.permutation(n_pages)[:logical].astype(np.int32)
        t[::5] = n_pages + np.arange(len(t[::5]), dtype=np.int32)
        return t
    raise ValueError(kind)


def _expected_pools(oracle, geo, inputs, T, pos0, tables, n_pages):
    H, D, ps = geo.n_head_kv, geo.head_dim, geo.page_size
    out = {}
    for j in range(geo.n_qsa):
        for kv in ("k", "v"):
            pool = np.full(n_pages * H * ps * D, SENTINEL | SENTINEL << 8, dtype=np.uint16)
            oracle.kv_append(inputs[kv][j], T, pos0, tables[j], n_pages, H, D, ps, pool)
            out[f"{kv}{j}"] = pool
    return out


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("kind", ["permuted", "holes", "past_pool"])
@pytest.mark.parametrize("T,pos0,spare", [(77, 0, 0), (61, 6, 5), (40, 3, 40)])
def test_ordered_carve_equals_oracle(sc, oracle, cuda, ordered, dtype, kind, T, pos0, spare):
    print(f"case ordered carve {dtype} {kind} T={T} pos0={pos0} spare={spare}", flush=True)
    geo = sc.geometry(**GEO)
    ps = geo.page_size
    logical = (pos0 + T + ps - 1) // ps + 1
    n_pages = logical + spare   # spare: physical pages the table never names
    rng = np.random.default_rng(T * 7 + spare)
    tables = [_table(rng, logical, n_pages, kind) for _ in range(geo.n_qsa)]
    case = synth.SyntheticCase(geo, tokens=T, seed=900 + T,
                            kv_dtype=sc.SC_DTYPE_F16 if dtype == "f16" else sc.SC_DTYPE_F32)
    slot = sc.new_slot(geo, logical * ps, n_pages=n_pages, tables=sc.device_tables(tables), fill=SENTINEL)
    sc.device_sync()
    plan = sc.plan_carve(geo, case.prefill, slot, pos0=pos0, with_gdn=False)
    assert plan.order_groups == geo.n_qsa
    plan.launch()
    sc.device_sync()
    want = _expected_pools(oracle, geo, case.host_inputs(), T, pos0, tables, n_pages)
    got = slot.host_state()
    for name, w in want.items():
        assert np.array_equal(got[name].reshape(-1), w), f"{name} differs"
    plan.destroy()


def test_table_changed_between_launches(sc, oracle, cuda, ordered):
    """The order is rebuilt on every launch: a new table between two launches of one plan is followed."""
    geo = sc.geometry(**GEO)
    T, ps = 93, geo.page_size
    logical = (T + ps - 1) // ps
    n_pages = logical + 7
    rng = np.random.default_rng(11)
    case = synth.SyntheticCase(geo, tokens=T, seed=77)
    first = [_table(rng, logical, n_pages, "permuted") for _ in range(geo.n_qsa)]
    second = [_table(rng, logical, n_pages, "holes") for _ in range(geo.n_qsa)]
    dev = sc.device_tables(first)
    slot = sc.new_slot(geo, logical * ps, n_pages=n_pages, tables=dev, fill=SENTINEL)
    plan = sc.plan_carve(geo, case.prefill, slot, with_gdn=False)
    assert plan.order_groups == geo.n_qsa
    for tables in (first, second):
        for j, t in enumerate(tables):
            dev[j].upload(t)
        for b in slot.buffers():
            b.fill(SENTINEL)
        sc.device_sync()
        plan.launch()
        sc.device_sync()
        want = _expected_pools(oracle, geo, case.host_inputs(), T, 0, tables, n_pages)
        got = slot.host_state()
        for name, w in want.items():
            assert np.array_equal(got[name].reshape(-1), w), f"{name} differs"
    plan.destroy()


def test_ordered_scatter_of_an_image(sc, cuda, ordered):
    """A parked image scattered into a paged slot in destination order reads back as the same image."""
    geo = sc.geometry(**GEO)
    T, ps = 101, geo.page_size
    case = synth.SyntheticCase(geo, tokens=T, seed=5)
    flat = case.new_slot(max_cells=128)
    case.carve_into(flat)
    _, total = sc.image_layout(geo, T)
    image = sc.DeviceBuffer(total, "uint8")
    sc.plan_capture(geo, flat, T, image.ptr, total).launch()
    n_pages = 40
    rng = np.random.default_rng(3)
    tables = sc.device_tables([rng.permutation(n_pages).astype(np.int32) for _ in range(geo.n_qsa)])
    paged = sc.new_slot(geo, 128, n_pages=n_pages, tables=tables, fill=SENTINEL)
    scatter = sc.plan_scatter(geo, image.ptr, total, T, paged)
    assert scatter.order_groups == geo.n_qsa
    scatter.launch()
    back = sc.DeviceBuffer(total, "uint8")
    back.fill(0x5A)
    sc.plan_capture(geo, paged, T, back.ptr, total).launch()
    sc.device_sync()
    assert np.array_equal(image.numpy(), back.numpy())


def test_default_threshold_orders_large_tables_only(sc, oracle, cuda):
    """With the library default, a table covering >= 2048 pages is ordered and one covering fewer is not; both place
    every byte as the oracle does."""
    geo = sc.geometry(**GEO)
    ps = geo.page_size
    for T, ordered_groups in ((8192, geo.n_qsa), (1024, 0)):
        print(f"case default threshold T={T}", flush=True)
        logical = T // ps
        rng = np.random.default_rng(T)
        tables = [rng.permutation(logical).astype(np.int32) for _ in range(geo.n_qsa)]
        case = synth.SyntheticCase(geo, tokens=T, seed=31 + T)
        slot = sc.new_slot(geo, T, n_pages=logical, tables=sc.device_tables(tables), fill=SENTINEL)
        sc.device_sync()
        plan = sc.plan_carve(geo, case.prefill, slot, with_gdn=False)
        assert plan.order_groups == ordered_groups
        plan.launch()
        sc.device_sync()
        want = _expected_pools(oracle, geo, case.host_inputs(), T, 0, tables, logical)
        got = slot.host_state()
        for name, w in want.items():
            assert np.array_equal(got[name].reshape(-1), w), f"T={T}: {name} differs"
        plan.destroy()


@pytest.mark.parametrize("fmt", ["int8", "q4"])
@pytest.mark.parametrize("kind", ["permuted", "holes"])
@pytest.mark.parametrize("T,pos0,spare", [(77, 0, 0), (61, 6, 9)])
def test_quantizing_carve_keeps_source_order(sc, oracle, cuda, ordered, fmt, kind, T, pos0, spare):
    """Quantizing rows keep the source order even where every table would be ordered; their pools still equal the
    oracle's."""
    print(f"case quant carve {fmt} {kind} T={T} pos0={pos0} spare={spare}", flush=True)
    geo = sc.geometry(**GEO)
    H, D, ps = geo.n_head_kv, geo.head_dim, geo.page_size
    logical = (pos0 + T + ps - 1) // ps + 1
    n_pages = logical + spare
    rng = np.random.default_rng(T * 3 + spare)
    tables = [_table(rng, logical, n_pages, kind) for _ in range(geo.n_qsa)]
    case = synth.SyntheticCase(geo, tokens=T, seed=600 + T, kv_dtype=sc.SC_DTYPE_F32)
    code = sc.SC_KV_INT8 if fmt == "int8" else sc.SC_KV_Q4
    slot = sc.new_quant_slot(geo, code, logical * ps, n_pages=n_pages, tables=sc.device_tables(tables),
                             fill=SENTINEL)
    sc.device_sync()
    plan = sc.plan_carve_quant(geo, case.prefill, slot, pos0=pos0, with_gdn=False)
    assert plan.order_groups == 0   # quantizing rows keep the source order
    plan.launch()
    sc.device_sync()
    inputs = case.host_inputs()
    row = 256 if fmt == "int8" else 144
    for j in range(geo.n_qsa):
        for kv in ("k", "v"):
            codes = np.full(n_pages * H * ps * row, SENTINEL, dtype=np.uint8)
            scales = np.full(n_pages * H * ps * 4, SENTINEL | SENTINEL << 8, dtype=np.uint16) if fmt == "int8" else None
            oracle.kv_append_quant(inputs[kv][j], 1 if fmt == "int8" else 2, T, pos0, tables[j], n_pages, H, D, ps,
                                   codes, scales)
            got = (slot.k_codes if kv == "k" else slot.v_codes)[j].numpy().view(np.uint8).reshape(-1)
            assert np.array_equal(got, codes), f"{kv}{j} codes differ"
            if scales is not None:
                got_s = (slot.k_scale if kv == "k" else slot.v_scale)[j].numpy().view(np.uint8).reshape(-1)
                assert np.array_equal(got_s, scales.view(np.uint8)), f"{kv}{j} scales differ"
    plan.destroy()
