"""Streamed layers in the one-launch carves: sc_plan_carve / sc_plan_carve_quant with a host copy and a staging pool.

The reference's prefill writer puts every appended cell into the paged pool when its page is resident (a negative table
entry skips it), into the layer's authoritative host copy and into the prompt path's staging pool, both in the identity
layout (src/prefill/kernels.cu:574-577,587-600; src/kernels/cuda/kv_q4.cu:124-128).  The one-launch carve does all
three for every QSA layer in one launch; here the host copy is pinned host memory the kernel writes directly, the
staging pool device memory, and every byte of all three (written or not) must equal the oracle's placement
(sco_kv_append / sco_kv_append_quant, pinned in tests/test_oracle.py and tests/test_oracle_quant.py).
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

GEO = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32, ssm_k_heads=4,
           ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)
SENTINEL = 0xEE
ROW = {"f16": 512, "int8": 256, "q4": 144}


def _buf(sc, nbytes, host):
    if host:
        b = sc.PinnedBuffer(nbytes)
        b.numpy()[:] = SENTINEL
    else:
        b = sc.DeviceBuffer(nbytes, "uint8")
        b.fill(SENTINEL)
    return b


def _read(sc, b):
    if isinstance(b, sc.PinnedBuffer):
        return b.numpy().copy()
    return b.numpy()


def _extra(sc, geo, fmt, pages, host):
    """Per QSA layer the K/V pools (+ int8 scales) of `pages` identity pages, and their KvPools records."""
    rows = pages * geo.n_head_kv * geo.page_size
    bufs, pools = [], []
    for _ in range(geo.n_qsa):
        b = {"k": _buf(sc, rows * ROW[fmt], host), "v": _buf(sc, rows * ROW[fmt], host)}
        kp = sc.KvPools()
        if fmt == "f16":
            kp.k_pool, kp.v_pool = b["k"].ptr, b["v"].ptr
        elif fmt == "int8":
            b["ks"], b["vs"] = _buf(sc, rows * 8, host), _buf(sc, rows * 8, host)
            kp.k_q, kp.v_q, kp.k_scale, kp.v_scale = b["k"].ptr, b["v"].ptr, b["ks"].ptr, b["vs"].ptr
        else:
            kp.k_q4, kp.v_q4 = b["k"].ptr, b["v"].ptr
        bufs.append(b)
        pools.append(kp)
    return bufs, pools


def _want(oracle, geo, fmt, x, T, pos0, table, pages):
    """The oracle's pool bytes (codes) and int8 scale bytes after the carve, from sentinel bytes."""
    H, D, ps = geo.n_head_kv, geo.head_dim, geo.page_size
    rows = pages * H * ps
    if fmt == "f16":
        pool = np.full(rows * D, SENTINEL | SENTINEL << 8, dtype=np.uint16)
        oracle.kv_append(x, T, pos0, table, pages, H, D, ps, pool)
        return pool.view(np.uint8), None
    codes = np.full(rows * ROW[fmt], SENTINEL, dtype=np.uint8)
    scales = np.full(rows * 4, SENTINEL | SENTINEL << 8, dtype=np.uint16) if fmt == "int8" else None
    oracle.kv_append_quant(x, 1 if fmt == "int8" else 2, T, pos0, table, pages, H, D, ps, codes, scales)
    return codes, None if scales is None else scales.view(np.uint8)


@pytest.mark.parametrize("fmt,dtype", [("f16", "f16"), ("f16", "f32"), ("int8", "f32"), ("q4", "f32")])
@pytest.mark.parametrize("table_kind", ["identity", "holes"])
@pytest.mark.parametrize("T,pos0", [(37, 0), (29, 6)])
def test_carve_writes_pool_host_copy_and_staging(sc, oracle, cuda, fmt, dtype, table_kind, T, pos0):
    print(f"case streamed carve {fmt} from {dtype} {table_kind} T={T} pos0={pos0}", flush=True)
    geo = sc.geometry(**GEO)
    logical = (pos0 + T + geo.page_size - 1) // geo.page_size + 2
    max_cells = logical * geo.page_size
    n_pages = logical if table_kind == "identity" else logical + 3
    table = None
    if table_kind == "holes":   # a streamed layer: some pages are not resident in VRAM
        table = np.random.default_rng(T).permutation(n_pages)[:logical].astype(np.int32)
        table[1::3] = -1
    kv_dtype = sc.SC_DTYPE_F16 if dtype == "f16" else sc.SC_DTYPE_F32
    case = synth.SyntheticCase(geo, tokens=T, seed=700 + T, kv_dtype=kv_dtype)
    tabs = None if table is None else sc.device_tables([table] * geo.n_qsa)
    host_bufs, host_pools = _extra(sc, geo, fmt, logical, host=True)
    stage_bufs, stage_pools = _extra(sc, geo, fmt, logical, host=False)
    if fmt == "f16":
        slot = sc.new_slot(geo, max_cells, n_pages=n_pages, tables=tabs, fill=SENTINEL)
        slot.host, slot.stage = host_pools, stage_pools
        sc.device_sync()
        plan = sc.plan_carve(geo, case.prefill, slot, pos0=pos0, with_gdn=False)
        pool_bufs = [{"k": slot.k_pool[j], "v": slot.v_pool[j]} for j in range(geo.n_qsa)]
    else:
        code = sc.SC_KV_INT8 if fmt == "int8" else sc.SC_KV_Q4
        slot = sc.new_quant_slot(geo, code, max_cells, n_pages=n_pages, tables=tabs, fill=SENTINEL)
        slot.host, slot.stage = host_pools, stage_pools
        sc.device_sync()
        plan = sc.plan_carve_quant(geo, case.prefill, slot, pos0=pos0, with_gdn=False)
        pool_bufs = [{"k": slot.k_codes[j], "v": slot.v_codes[j],
                      **({"ks": slot.k_scale[j], "vs": slot.v_scale[j]} if fmt == "int8" else {})}
                     for j in range(geo.n_qsa)]
    plan.launch()
    sc.device_sync()
    inputs = case.host_inputs()
    for j in range(geo.n_qsa):
        for kv in ("k", "v"):
            x = inputs[kv][j]
            for name, bufs, tab, pages in (("pool", pool_bufs, table, n_pages), ("host copy", host_bufs, None, logical),
                                           ("staging pool", stage_bufs, None, logical)):
                codes, scales = _want(oracle, geo, fmt, x, T, pos0, tab, pages)
                got = _read(sc, bufs[j][kv]).view(np.uint8).reshape(-1)
                assert np.array_equal(got, codes), f"{name} {kv}{j} differs"
                if scales is not None:
                    got = _read(sc, bufs[j][kv + "s"]).view(np.uint8).reshape(-1)
                    assert np.array_equal(got, scales), f"{name} {kv}{j} scales differ"
    plan.destroy()


def test_k8v4_slot_refuses_host_copies(sc, cuda):
    """K8V4 is resident only (the reference's hybrid rule): a host copy is refused before anything is written."""
    geo = sc.geometry(**GEO)
    case = synth.SyntheticCase(geo, tokens=8, seed=3, kv_dtype=sc.SC_DTYPE_F32)
    slot = sc.new_quant_slot(geo, sc.SC_KV_K8V4, 16, fill=SENTINEL)
    _, pools = _extra(sc, geo, "int8", 4, host=False)
    slot.host = pools
    with pytest.raises(sc.ScError) as err:
        sc.plan_carve_quant(geo, case.prefill, slot, with_gdn=False)
    assert err.value.code == sc.SC_EINVAL and "hybrid K8V4" in str(err.value)


def test_host_copy_must_be_mapped_pinned_memory(sc, cuda):
    """The kernels write a host copy straight into host memory, so its pools must be pinned memory mapped for the
    device: pageable buffers (and device memory) are refused when the plan is built, and by the per-layer append before
    its launch (attempted only after sc_host_range_mapped has reported the buffer unmapped, the same check it makes)."""
    import ctypes as C
    geo = sc.geometry(**GEO)
    T, logical = 12, 5
    case = synth.SyntheticCase(geo, tokens=T, seed=5, kv_dtype=sc.SC_DTYPE_F32)
    rows = logical * geo.n_head_kv * geo.page_size
    pageable = [np.zeros(rows * ROW["f16"], np.uint8) for _ in range(2 * geo.n_qsa)]
    pools = []
    for j in range(geo.n_qsa):
        kp = sc.KvPools()
        kp.k_pool, kp.v_pool = pageable[2 * j].ctypes.data, pageable[2 * j + 1].ctypes.data
        pools.append(kp)
    mapped = C.c_int32(-1)
    assert sc.lib.sc_host_range_mapped(pageable[0].ctypes.data, pageable[0].nbytes, C.byref(mapped)) == sc.SC_OK
    assert mapped.value == 0
    slot = sc.new_slot(geo, logical * geo.page_size, fill=SENTINEL)
    slot.host = pools
    with pytest.raises(sc.ScError) as err:
        sc.plan_carve(geo, case.prefill, slot, with_gdn=False)
    assert err.value.code == sc.SC_EINVAL and "pinned memory mapped for the device" in str(err.value)
    # device memory is not a host copy either
    dev_bufs, dev_pools = _extra(sc, geo, "f16", logical, host=False)
    slot.host = dev_pools
    with pytest.raises(sc.ScError):
        sc.plan_carve(geo, case.prefill, slot, with_gdn=False)
    # the per-layer append, f16 pools with a pageable host copy
    kp = pools[0]
    rc = sc.lib.sc_kv_append_async(case.prefill.k[0].data_ptr(), case.prefill.v[0].data_ptr(), T, 0, None,
                                   geo.page_size, slot.k_pool[0].data_ptr(), slot.v_pool[0].data_ptr(), None, None,
                                   None, None, None, C.byref(kp), None)
    assert rc == sc.SC_EINVAL and "pinned memory mapped for the device" in sc.last_error()
    sc.device_sync()
    assert all(np.all(b == 0) for b in pageable)
    assert np.all(slot.host_state()["k0"].view(np.uint8) == SENTINEL)   # nothing was launched
