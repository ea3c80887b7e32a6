"""Slot images in every K/V format on the device: capture, scatter, park and resume (sc_*_layers) byte for byte.

The expected image is built on the host from the pools' own bytes placed at the oracle's offsets (image_layout_layers,
pinned in tests/test_layers_layout.py against the reference codec's pool order), with every gap zero.  Scatters and
resumes must restore exactly the blob prefixes and leave every byte past them as it was.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)


def _expected_image(oracle, geo, pools, fmt, index, tokens):
    offs, total = oracle.image_layout_layers(geo, fmt, index, tokens)
    sizes = oracle.layer_blob_bytes(geo, fmt, index, tokens)
    host = pools.host()
    want = np.zeros(total, np.uint8)
    for j in range(geo.n_qsa):
        for b in range(5):
            if sizes[b]:
                o = offs[j * 5 + b]
                want[o:o + sizes[b]] = host[(b, j)][:sizes[b]]
    if geo.n_gdn:
        g = host["gdn"]
        want[offs[-1]:offs[-1] + g.size] = g
    return want, sizes, host


def _check_restored(geo, dst, src_host, sizes, fill):
    got = dst.host()
    for j in range(geo.n_qsa):
        for b in range(5):
            if (b, j) not in got:
                continue
            g, s, n = got[(b, j)], src_host[(b, j)], sizes[b]
            assert np.array_equal(g[:n], s[:n]), f"buffer {b} of layer {j}: restored bytes differ"
            assert (g[n:] == fill).all(), f"buffer {b} of layer {j}: bytes past the image were written"
    if geo.n_gdn:
        assert np.array_equal(got["gdn"], src_host["gdn"])


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("index", [False, True])
@pytest.mark.parametrize("tokens", [1, 77, 4096])
def test_capture_scatter_round_trip(sc, oracle, cuda, fmt, index, tokens):
    geo = sc.geometry(**SMALL)
    max_cells = (tokens + 3) // 4 * 4 + 8
    pools = sc.LayerPools(geo, fmt, max_cells, index)
    pools.randomize(0x5EED + tokens + 10 * fmt)
    want, sizes, host = _expected_image(oracle, geo, pools, fmt, index, tokens)
    image = sc.DeviceBuffer(want.size, "uint8")
    image.fill(0xEE)                       # the capture must clear every gap
    plan = sc.plan_capture_layers(geo, pools, tokens, image.ptr, want.size)
    plan.launch()
    sc.device_sync()
    got = image.numpy()
    if not np.array_equal(got, want):
        bad = np.flatnonzero(got != want)
        raise AssertionError(f"captured image differs at {bad.size} bytes, first {bad[0]}")
    gdn_bytes = host["gdn"].size if geo.n_gdn else 0
    assert plan.payload_bytes == geo.n_qsa * sum(sizes) + gdn_bytes
    dst = sc.LayerPools(geo, fmt, max_cells, index)
    dst.fill(0xA5)
    back = sc.plan_scatter_layers(geo, image.ptr, want.size, tokens, dst)
    back.launch()
    sc.device_sync()
    _check_restored(geo, dst, host, sizes, 0xA5)
    for p in (plan, back):
        p.destroy()
    for b in pools.buffers() + dst.buffers() + [image]:
        b.free()


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("index", [False, True])
def test_park_resume_round_trip(sc, oracle, cuda, fmt, index):
    geo = sc.geometry(**SMALL)
    tokens = 301
    max_cells = 320
    pools = sc.LayerPools(geo, fmt, max_cells, index)
    pools.randomize(0xBEEF + fmt)
    want, sizes, host = _expected_image(oracle, geo, pools, fmt, index, tokens)
    pinned = sc.PinnedBuffer(want.size)
    pinned.numpy()[:] = 0xEE
    st = sc.Stream()
    done = sc.Event()
    sc.park_layers_async(geo, pools, tokens, pinned.ptr, want.size, stream=st, done=done.handle)
    done.sync()
    assert np.array_equal(pinned.numpy(), want)
    dst = sc.LayerPools(geo, fmt, max_cells, index)
    dst.fill(0x3C)
    sc.resume_layers_async(geo, pinned.ptr, want.size, tokens, dst, stream=st)
    st.sync()
    _check_restored(geo, dst, host, sizes, 0x3C)
    pinned.free()
    for b in pools.buffers() + dst.buffers():
        b.free()


def test_quantized_carve_parks_and_resumes(sc, oracle, cuda):
    """The quantizing carve's pools (int8 K and V with scales) plus indexer rows, parked and resumed into fresh pools:
    codes, scales, rows and the GDN state come back bit for bit, and the image equals the host-built one."""
    geo = sc.geometry(**SMALL)
    T = 501
    case = synth.SyntheticCase(geo, T, seed=0x5EED, kv_dtype=sc.SC_DTYPE_F32)
    cap = (T + 3) // 4 * 4 + 16
    slot = sc.new_quant_slot(geo, sc.SC_KV_INT8, cap)
    sc.plan_carve_quant(geo, case.prefill, slot).launch()
    pooled = [sc.DeviceBuffer((cap // 4 + 1) * geo.idx_key_dim * 4, "uint8") for _ in range(geo.n_qsa)]
    for i, b in enumerate(pooled):
        sc.check(sc.lib.sc_fill_uniform_f16(b.ptr, b.nbytes // 2, -1.0, 1.0, 77, i, None), "fill")
    sc.device_sync()
    pools = sc.LayerPools.from_quant(slot, pooled)
    want, sizes, host = _expected_image(oracle, geo, pools, sc.SC_KV_INT8, True, T)
    pinned = sc.PinnedBuffer(want.size)
    sc.park_layers_async(geo, pools, T, pinned.ptr, want.size)
    sc.device_sync()
    assert np.array_equal(pinned.numpy(), want)
    fresh = sc.new_quant_slot(geo, sc.SC_KV_INT8, cap, fill=0x11)
    fresh_pooled = [sc.DeviceBuffer(b.nbytes, "uint8") for b in pooled]
    for b in fresh_pooled:
        b.fill(0x11)
    dst = sc.LayerPools.from_quant(fresh, fresh_pooled)
    sc.resume_layers_async(geo, pinned.ptr, want.size, T, dst)
    sc.device_sync()
    _check_restored(geo, dst, host, sizes, 0x11)


def test_full_depth_int8_with_index(sc, oracle, cuda):
    """Config-2 geometry at 32K, int8 with the index: capture -> scatter into fresh pools equals the source."""
    geo = sc.geometry()
    T = 32768
    pools = sc.LayerPools(geo, sc.SC_KV_INT8, T, True)
    pools.randomize(9)
    offs, total = sc.image_layout_layers(geo, sc.SC_KV_INT8, True, T)
    image = sc.DeviceBuffer(total, "uint8")
    cap = sc.plan_capture_layers(geo, pools, T, image.ptr, total)
    dst = sc.LayerPools(geo, sc.SC_KV_INT8, T, True)
    dst.fill(0)
    back = sc.plan_scatter_layers(geo, image.ptr, total, T, dst)
    cap.launch()
    back.launch()
    sc.device_sync()
    a, b = pools.host(), dst.host()
    for key in a:
        assert np.array_equal(a[key], b[key]), key
    # and the image carries each blob where the layout says (sampled: layer 5's scales, the GDN rows)
    sizes = sc.layer_blob_bytes(geo, sc.SC_KV_INT8, True, T)
    o = offs[5 * 5 + 2]
    assert np.array_equal(image.numpy(sizes[2], start=o), a[(2, 5)][:sizes[2]])
    assert np.array_equal(image.numpy(a["gdn"].size, start=offs[-1]), a["gdn"])
