"""The quantizing carve (sc_plan_carve_quant: int8, q4_0, K8V4) against the oracle, byte for byte.

The oracle's rules (sco_q8_row, sco_q4_row) are pinned in tests/test_oracle_quant.py by independent numpy forms of the
reference's int8 kv_append and kv_append_q4 quantizers.  Here every code byte, every scale and every untouched byte of
the device pools must equal the oracle's, for every table shape the f16 carve is tested with, a start in the middle of
a page, and rows built to hit the edge cases (zero groups, tied magnitudes, exact .5 quotients, tiny and huge scales,
NaN and infinite values, signed zeros).
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)


def _edge_rows(src: np.ndarray) -> np.ndarray:
    """Overwrite a few (token, head) rows of [T][H][256] f32 with edge-case groups."""
    x = src.copy()
    T = x.shape[0]
    if T > 0:
        x[0, 0] = 0.0
    if T > 1:
        x[1, 0, :64] = np.linspace(-127, 127, 64, dtype=np.float32)
        x[1, 1, :32] = 2.0
        x[1, 1, 5], x[1, 1, 9] = -5.0, 5.0
    if T > 2:
        x[2, 0] = x[2, 0] * np.float32(1e-4)
        x[2, 1] = x[2, 1] * np.float32(5e3)
    if T > 3:
        x[3, 0, :64] = np.float32(127) * np.arange(64, dtype=np.float32) / np.float32(64) + np.float32(0.5)
    if T > 6:
        x[4, 0, :64] = np.nan                       # a group / blocks of NaNs
        x[4, 1, 0], x[4, 1, 37] = np.nan, np.nan    # NaN first in a group, NaN inside a block
        # a negative quiet NaN, a signalling NaN and the largest-payload negative NaN: never a block's maximum
        x[4, 1, 40:43] = np.array([0xFFC00001, 0x7F800001, 0xFFFFFFFF], np.uint32).view(np.float32)
        x[5, 0, 2], x[5, 0, 9] = np.inf, -np.inf    # infinite scale; inf / inf
        x[5, 1, :32] = -np.float32(0)
        x[5, 1, 3] = np.float32(0)                  # -0 first among zeros
        x[6, 0, 1] = np.float32(1e7)                # max / 127 beyond f16: infinite scale
    if T > 7:
        # q4_0 blocks with values where a fused and a separately rounded x * id + 8.5 give different codes
        from quant_cases import boundary_blocks
        x[7] = boundary_blocks(2 * 8).reshape(2, 256)
    return x


def _tables(sc, kind, n_qsa, n_pages):
    if kind == "identity":
        return None, None
    if kind == "reversed":
        t = np.arange(n_pages)[::-1].astype(np.int32)
    elif kind == "holes":
        t = np.arange(n_pages).astype(np.int32)
        t[1::3] = -1
    else:
        t = np.random.default_rng(n_pages).permutation(n_pages).astype(np.int32)
    return sc.device_tables([t] * n_qsa), [t] * n_qsa


@pytest.mark.parametrize("fmt", ["int8", "q4", "k8v4"])
@pytest.mark.parametrize("tokens,pos0,table", [(77, 0, "identity"), (77, 5, "reversed"), (61, 2, "holes"),
                                               (4096, 0, "shuffled"), (1, 3, "identity")])
def test_quant_carve_matches_oracle(sc, oracle, cuda, fmt, tokens, pos0, table):
    geo = sc.geometry(**SMALL)
    code = {"int8": sc.SC_KV_INT8, "q4": sc.SC_KV_Q4, "k8v4": sc.SC_KV_K8V4}[fmt]
    case = synth.SyntheticCase(geo, tokens, seed=0x5EED + tokens, kv_dtype=sc.SC_DTYPE_F32)
    # plant the edge rows in every layer's K and V
    for buf in case.prefill.k + case.prefill.v:
        host = buf.numpy()
        buf.upload(_edge_rows(host.reshape(-1, geo.n_head_kv, 256)[:tokens]).reshape(-1))
    max_cells = ((pos0 + tokens + 3) // 4 + 2) * 4
    n_pages = max_cells // 4
    tdev, thost = _tables(sc, table, geo.n_qsa, n_pages)
    slot = sc.new_quant_slot(geo, code, max_cells, n_pages=n_pages, tables=tdev, fill=0xA5)
    plan = sc.plan_carve_quant(geo, case.prefill, slot, pos0=pos0)
    plan.launch()
    sc.device_sync()
    inputs = case.host_inputs()
    k_int8, v_int8 = code != sc.SC_KV_Q4, code == sc.SC_KV_INT8
    H = geo.n_head_kv
    for j in range(geo.n_qsa):
        for name, srcs, codes, scales, is8 in (("k", inputs["k"], slot.k_codes, slot.k_scale, k_int8),
                                               ("v", inputs["v"], slot.v_codes, slot.v_scale, v_int8)):
            row_bytes = 256 if is8 else 144
            want_codes = np.full((n_pages, H, 4, row_bytes), 0xA5, np.uint8)
            want_scales = np.full((n_pages, H, 4, 4), 0xA5A5, np.uint16) if is8 else None
            oracle.kv_append_quant(srcs[j].reshape(-1)[: tokens * H * 256], 1 if is8 else 2, tokens, pos0,
                                   thost[j] if thost else None, n_pages, H, 256, 4, want_codes, want_scales)
            got = codes[j].numpy().reshape(want_codes.shape)
            if not np.array_equal(got, want_codes):
                bad = np.argwhere(got != want_codes)
                raise AssertionError(f"{fmt} {name}{j} codes: {len(bad)} bytes differ, first at {bad[0].tolist()}")
            if is8:
                assert np.array_equal((scales[j] if name == "k" else scales[j]).numpy().reshape(want_scales.shape),
                                      want_scales), f"{fmt} {name}{j} scales"
    # the running state is carved exactly as the f16 carve carves it
    # (older conv history rows of a short continuing chunk come from the slot's previous contents: the 0xA5 fill)
    initial = {f"{n}{j}": np.zeros((n_pages, H, 4, 256), np.uint16) for j in range(geo.n_qsa) for n in "kv"}
    initial["gdn"] = np.full((geo.n_gdn, geo.gdn_row_floats), 0xA5A5A5A5, np.uint32).view(np.float32)
    want = oracle.expected_slot(geo, inputs, slot_cells=max_cells, pos0=pos0, initial=initial)
    assert np.array_equal(slot.gdn.numpy().view(np.uint32), want["gdn"].view(np.uint32))


def test_quant_carve_refusals(sc, cuda):
    geo = sc.geometry(**SMALL)
    case16 = synth.SyntheticCase(geo, 8, seed=1)                       # f16 rows: refused, the carve reads f32
    slot = sc.new_quant_slot(geo, sc.SC_KV_INT8, 16)
    with pytest.raises(sc.ScError):
        sc.plan_carve_quant(geo, case16.prefill, slot)
    case = synth.SyntheticCase(geo, 8, seed=1, kv_dtype=sc.SC_DTYPE_F32)
    small = sc.new_quant_slot(geo, sc.SC_KV_INT8, 4)                 # 8 tokens do not fit 4 cells
    with pytest.raises(sc.ScError):
        sc.plan_carve_quant(geo, case.prefill, small)
    other = sc.geometry(**dict(SMALL, head_dim=128))                 # head_dim 256 only
    with pytest.raises(sc.ScError):
        sc.plan_carve_quant(other, synth.SyntheticCase(other, 8, seed=1, kv_dtype=sc.SC_DTYPE_F32).prefill,
                            sc.new_quant_slot(other, sc.SC_KV_INT8, 16))


def test_quant_carve_full_depth_int8(sc, oracle, cuda):
    """Config 2 geometry (48 layers) at 32K tokens, int8: sampled rows of every layer against the oracle, and the
    scales' decoded magnitudes bound every code's reconstruction error by half a step."""
    geo = sc.geometry()
    T = 32768
    case = synth.SyntheticCase(geo, T, seed=0x5EED, kv_dtype=sc.SC_DTYPE_F32)
    slot = sc.new_quant_slot(geo, sc.SC_KV_INT8, T)
    plan = sc.plan_carve_quant(geo, case.prefill, slot)
    plan.launch()
    sc.device_sync()
    rng = np.random.default_rng(3)
    H = geo.n_head_kv
    for j in range(geo.n_qsa):
        codes = slot.k_codes[j].numpy().reshape(-1, 256).view(np.int8)
        scales = slot.k_scale[j].numpy().reshape(-1, 4)
        for t in rng.integers(0, T, size=16):
            for h in range(H):
                x = case.prefill.k[j].numpy(256, start=(int(t) * H + h) * 256)
                c, s = oracle.q8_rows(x[None])
                row = (int(t) // 4 * H + h) * 4 + int(t) % 4
                assert np.array_equal(codes[row], c[0]) and np.array_equal(scales[row], s[0])
                sf = np.repeat(s[0].view(np.float16).astype(np.float32), 64)
                err = np.abs(x - codes[row].astype(np.float32) * sf)
                assert np.all(err <= sf * np.float32(0.5) * np.float32(1 + 1e-6))
