"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

Each test checks the oracle against something that shares no code with it and that a plausible mistake (a
dropped term, a wrong index, a transposed operand) would fail: the reference's own golden vectors, numpy
formulations of the layouts, the reference's rival-layout test, published totals and textbook hash vectors.
"""
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- f32 -> f16 (kv_append's rounding, src/prefill/kernels.cu:575) ------------------------------------------------

def test_f16_matches_reference_golden_vectors(oracle):
    pairs = json.loads((GOLDEN / "f16_oracle_vectors.json").read_text())["pairs_f32_f16"]
    assert len(pairs) == 395
    for f32_bits, f16_bits in pairs:
        assert oracle.lib.sco_f16_bits(f32_bits) == f16_bits, hex(f32_bits)


def test_f16_matches_numpy_on_random_and_edge_bits(oracle):
    rng = np.random.default_rng(12345)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    edges = []
    for e in range(96, 145):   # every exponent around the f16 range, with tie / near-tie mantissas
        for m in (0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x3000, 0x7FF000, 0x7FEFFF, 0x7FFFFF):
            edges.append((e << 23) | m)
            edges.append((1 << 31) | (e << 23) | m)
    bits = np.concatenate([bits, np.array(edges, dtype=np.uint32)])
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    with np.errstate(over="ignore"):
        want = x[finite].astype(np.float16).view(np.uint16)
    got = oracle.f16_bits(x[finite])
    assert np.array_equal(got, want)
    # non-finite: infinities stay infinities, NaNs stay NaNs (quiet, sign kept)
    nf = oracle.f16_bits(x[~finite])
    assert np.all((nf & 0x7C00) == 0x7C00)
    assert np.array_equal((nf & 0x3FF) != 0, np.isnan(x[~finite]))


# ---- synthetic generators ------------------------------------------------------------------------------------------

def test_splitmix64_published_sequence(oracle):
    # SplitMix64 from state 0 (Steele, Lea, Flood 2014; Vigna's splitmix64.c): the first outputs
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    golden = 0x9E3779B97F4A7C15
    got = [oracle.lib.sco_mix64((golden * (i + 1)) & (2**64 - 1)) for i in range(4)]
    assert got == want


def test_uniform_and_normal_moments(oracle):
    u = oracle.fill_uniform_f16(1 << 20, -4.0, 4.0, 0x5EED, 7).view(np.float16).astype(np.float64)
    assert u.min() >= -4.0 and u.max() <= 4.0
    assert abs(u.mean()) < 0.02 and abs(u.var() - 64 / 12) < 0.05
    z = oracle.fill_normal_f32(1 << 20, 0x5EED, 8).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1.0) < 0.01 and np.abs(z).max() <= 6.0
    # f16 uniform is the f32 uniform rounded to f16, and different streams differ
    uf = oracle.fill_uniform_f32(4096, -4.0, 4.0, 0x5EED, 7)
    assert np.array_equal(oracle.fill_uniform_f16(4096, -4.0, 4.0, 0x5EED, 7), uf.astype(np.float16).view(np.uint16))
    assert not np.array_equal(oracle.fill_normal_f32(64, 1, 2), oracle.fill_normal_f32(64, 1, 3))


# ---- the K/V carve (kv_append, src/prefill/kernels.cu:560-601) --------------------------------------------------------

def _numpy_paged(src, T, H, D, ps, table, n_pages, pos0=0):
    """[T][H][D] -> pool [n_pages][H][ps][D] by array operations (no index formula shared with the oracle)."""
    pool = np.zeros((n_pages, H, ps, D), dtype=src.dtype)
    cells = np.arange(T) + pos0
    logical = cells // ps
    phys = logical if table is None else np.asarray(table)[logical]
    ok = (phys >= 0) & (phys < n_pages)
    for h in range(H):
        pool[phys[ok], h, (cells % ps)[ok], :] = src[:T][ok, h, :]
    return pool


@pytest.mark.parametrize("ps,table_kind,pos0,T", [(4, "identity", 0, 96), (4, "reversed", 0, 96),
                                                  (1, "reversed", 0, 40), (4, "identity", 3, 57),
                                                  (4, "holes", 6, 70), (8, "reversed", 5, 90)])
def test_kv_append_matches_numpy_layout(oracle, ps, table_kind, pos0, T):
    H, D = 2, 64
    rng = np.random.default_rng(ps * 1000 + T)
    n_pages = (pos0 + T + ps - 1) // ps
    src = rng.integers(0, 2**16, size=(T, H, D), dtype=np.uint16)
    if table_kind == "identity":
        table = None
    elif table_kind == "reversed":     # qsa_parity.cpp:458: the table REVERSED
        table = np.arange(n_pages)[::-1].astype(np.int32)
    else:                              # non-resident pages (-1) are skipped, as kernels.cu:577 skips them
        table = np.arange(n_pages).astype(np.int32)
        table[1::3] = -1
    pool = np.zeros((n_pages, H, ps, D), dtype=np.uint16)
    oracle.kv_append(src, T, pos0, table, n_pages, H, D, ps, pool)
    assert np.array_equal(pool, _numpy_paged(src, T, H, D, ps, table, n_pages, pos0))


def test_kv_append_rival_layouts_differ(oracle):
    """src/kernels/qsa_parity.cpp:489-515 restated: the declared [page][kv_head][page_size][head_dim] layout must be
    observable - the linear (table ignored) and cell-major-in-page rivals must both disagree with it."""
    H, D, ps, T = 2, 32, 4, 64
    n_pages = T // ps
    rng = np.random.default_rng(7)
    src = rng.integers(1, 2**16, size=(T, H, D), dtype=np.uint16)
    table = np.arange(n_pages)[::-1].astype(np.int32)
    pool = np.zeros((n_pages, H, ps, D), dtype=np.uint16)
    oracle.kv_append(src, T, 0, table, n_pages, H, D, ps, pool)
    rows = pool.reshape(-1, D)
    mism_lin = mism_cell = 0
    for cell in range(T):
        for h in range(H):
            declared = (table[cell // ps] * H + h) * ps + cell % ps
            assert np.array_equal(rows[declared], src[cell, h])
            linear = (cell * H + h) * ps + cell % ps
            cell_major = (table[cell // ps] * ps + cell % ps) * H + h
            mism_lin += linear >= len(rows) or not np.array_equal(rows[linear], src[cell, h])
            mism_cell += cell_major >= len(rows) or not np.array_equal(rows[cell_major], src[cell, h])
    assert mism_lin / (T * H) > 0.5 and mism_cell / (T * H) > 0.5


def test_kv_append_f32_rounds_like_numpy(oracle):
    H, D, ps, T = 2, 64, 4, 20
    rng = np.random.default_rng(3)
    src = (rng.standard_normal((T, H, D)) * 3).astype(np.float32)
    src[0, 0, :4] = [65504.0, 65520.0, 1e-8, -2.0**-24 * 1.5]   # f16 max, overflow tie, underflow, subnormal tie
    pool = np.zeros((T // ps, H, ps, D), dtype=np.uint16)
    oracle.kv_append(src, T, 0, None, T // ps, H, D, ps, pool)
    with np.errstate(over="ignore"):
        want = _numpy_paged(src.astype(np.float16).view(np.uint16), T, H, D, ps, None, T // ps)
    assert np.array_equal(pool, want)


# ---- GDN state (gdn.cu:75 layout; gdn_conv_hist_kernel, kernels.cu:219-228) ----------------------------------------

def test_rec_carve_is_the_sh_v_s_layout(oracle):
    S, HV = 16, 6
    rng = np.random.default_rng(11)
    src = rng.standard_normal((HV, S, S)).astype(np.float32)
    got = oracle.rec_carve(src, S, HV).reshape(S, HV, S)
    assert np.array_equal(got, src.transpose(1, 0, 2))
    # the decode kernel's index: element (i, h, j) at i*HV*S + h*S + j (gdn.cu:75 `col[i*stride]`, stride HV*S)
    flat = got.reshape(-1)
    for (i, h, j) in [(0, 0, 0), (3, 5, 7), (S - 1, HV - 1, S - 1), (7, 2, 0)]:
        assert flat[i * HV * S + h * S + j] == src[h, i, j]
    assert not np.array_equal(got, src.reshape(S, HV, S))   # a missing transpose is visible


@pytest.mark.parametrize("rows", [3, 9, 2, 1, 0])
@pytest.mark.parametrize("fresh", [False, True])
def test_conv_hist(oracle, rows, fresh):
    Cc, nh, ld = 40, 3, 48
    rng = np.random.default_rng(rows)
    qkv = rng.standard_normal((max(rows, 1), ld)).astype(np.float32)
    old = rng.standard_normal((Cc, nh)).astype(np.float32)
    hist = old.copy()
    oracle.conv_hist(hist, qkv, rows, ld, Cc, nh, fresh)
    prev = np.zeros_like(old) if fresh else old
    # the history is a shift register of the last nh inputs per channel: previous history, then this chunk's rows
    stream = np.concatenate([prev, qkv[:rows, :Cc].T], axis=1)
    assert np.array_equal(hist, stream[:, -nh:])
    if rows >= nh:
        assert np.array_equal(hist, qkv[rows - nh:rows, :Cc].T)


# ---- image layout and payload accounting ---------------------------------------------------------------------------

CONFIG_GEO = dict(n_layers=48, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=128,
                  ssm_k_heads=16, ssm_v_heads=32, ssm_d_conv=4, ssm_conv_channels=8192, idx_key_dim=128)


def _geo(oracle, **kw):
    return oracle.Geometry(**{**CONFIG_GEO, **kw})


@pytest.mark.parametrize("layers,tokens,payload", [
    (16, 4096, 59_899_904),        # config 1: the toy handoff of 16 layers at 4096 tokens
    (48, 32768, 884_342_784),      # config 2
    (48, 131072, 3_300_261_888),   # config 3
    (48, 8192, 280_363_008),       # config 4, 8K slot
    (48, 98304, 2_494_955_520),    # config 4, 96K slot
])
def test_payload_totals_match_published(oracle, layers, tokens, payload):
    blobs, total = oracle.image_layout(_geo(oracle, n_layers=layers), tokens)
    assert total == payload
    assert sum(b[3] for b in blobs) == payload


def test_image_layout_closed_forms(oracle):
    g = _geo(oracle)
    for tokens in (1, 2, 3, 4, 5, 4097, 32768):
        blobs, total = oracle.image_layout(g, tokens)
        cells = -(-tokens // 4) * 4
        assert oracle.lib.sco_cells(g, tokens) == cells
        kv = [b for b in blobs if b[0] in (1, 2)]
        assert len(kv) == 24 and all(b[3] == cells * 2 * 256 * 2 for b in kv)
        assert [b[0] for b in kv] == [1, 2] * 12 and [b[1] for b in kv] == [j for j in range(12) for _ in (0, 1)]
        gdn = [b for b in blobs if b[0] == 3]
        assert len(gdn) == 1 and gdn[0][3] == 36 * (128 * 32 * 128 + 8192 * 3) * 4 == 36 * 2_195_456
        assert all(b[2] % 64 == 0 for b in blobs)
        assert all(blobs[i][2] >= blobs[i - 1][2] + blobs[i - 1][3] for i in range(1, len(blobs)))
        assert total % 64 == 0 and total >= blobs[-1][2] + blobs[-1][3]


def test_park_resume_round_trip_aba(oracle):
    """conversation_snapshot_test.cpp:136-159 restated on the oracle: save A, save B, restore A => A's bytes."""
    g = _geo(oracle, n_layers=8, ssm_state_size=8, ssm_v_heads=4, ssm_conv_channels=64)
    tokens, n_pages = 37, 12
    rng = np.random.default_rng(5)

    def state():
        s = {f"{n}{j}": rng.integers(0, 2**16, size=(n_pages, 2, 4, 256), dtype=np.uint16)
             for j in range(2) for n in ("k", "v")}
        s["gdn"] = rng.standard_normal((6, 8 * 4 * 8 + 64 * 3)).astype(np.float32)
        return s

    a, b = state(), state()
    img_a, img_b = oracle.park(g, tokens, a), oracle.park(g, tokens, b)
    assert not np.array_equal(img_a, img_b)
    oracle.resume(g, tokens, img_a, b)
    cells = 40
    for j in range(2):
        for n in ("k", "v"):
            flat_a = a[f"{n}{j}"].reshape(-1)
            flat_b = b[f"{n}{j}"].reshape(-1)
            extent = cells * 2 * 256
            assert np.array_equal(flat_b[:extent], flat_a[:extent])
    assert np.array_equal(a["gdn"], b["gdn"])
    assert np.array_equal(oracle.park(g, tokens, b), img_a)


# ---- FNV-1a 64 (src/core/pinned.cu:594-601) --------------------------------------------------------------------------

def test_fnv1a64_textbook_vectors(oracle):
    basis = oracle.TEXTBOOK_FNV_BASIS
    assert oracle.fnv1a64(b"", basis) == 0xCBF29CE484222325
    assert oracle.fnv1a64(b"a", basis) == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64(b"foobar", basis) == 0x85944171F73967E8


def test_fnv1a64_reference_seed(oracle):
    assert oracle.REFERENCE_FNV_SEED == 0x14650FB0739D0383
    assert oracle.fnv1a64(b"") == 0x14650FB0739D0383
    # chaining: hashing in pieces equals hashing at once (how the codec streams it)
    data = bytes(range(256)) * 9
    h = oracle.REFERENCE_FNV_SEED
    for i in range(0, len(data), 100):
        h = oracle.fnv1a64(data[i:i + 100], h)
    assert h == oracle.fnv1a64(data)


def test_cpu_handoff_pipeline_round_trip(oracle):
    src = np.random.default_rng(9).integers(0, 256, size=3 << 20, dtype=np.uint8)
    dst = np.zeros_like(src)
    scratch = np.empty(3 * src.size, dtype=np.uint8)
    h = oracle.cpu_handoff(src, dst, scratch)
    assert h == oracle.fnv1a64(src) and np.array_equal(src, dst)


def test_memcpy_threads_copies_every_byte(oracle):
    """The CPU baseline's labelled N-core copy ceiling copies the buffer exactly, for share boundaries that fall
    inside the buffer, past its end, and for one thread."""
    data = np.random.default_rng(5).integers(0, 256, 1_000_003, dtype=np.uint8)
    for threads in (1, 3, 8, 64):
        out = np.zeros_like(data)
        oracle.memcpy_threads(data, out, threads)
        assert np.array_equal(out, data), threads


# ---- whole-blob hashes of synthetic sequences (the full-size parity checker) -----------------------------------------

def _synthetic_inputs(oracle, g, tokens, seed, conv_rows, dtype=0):
    """What the product's synthetic_prefill generates, from the oracle's generators (host arrays)."""
    H, D, S, HV, Cc = g.n_head_kv, g.head_dim, g.ssm_state_size, g.ssm_v_heads, g.ssm_conv_channels
    n_qsa = g.n_layers // g.qsa_interval
    n_gdn = g.n_layers - n_qsa
    fill = oracle.fill_uniform_f16 if dtype == 0 else oracle.fill_uniform_f32
    k = [fill(tokens * H * D, -4.0, 4.0, seed, oracle.SID_K0 + 2 * j).reshape(tokens, H, D) for j in range(n_qsa)]
    v = [fill(tokens * H * D, -4.0, 4.0, seed, oracle.SID_V0 + 2 * j).reshape(tokens, H, D) for j in range(n_qsa)]
    rec = [oracle.fill_normal_f32(HV * S * S, seed, oracle.SID_REC0 + i).reshape(HV, S, S) for i in range(n_gdn)]
    conv = [oracle.fill_normal_f32(max(conv_rows, 1) * Cc, seed, oracle.SID_CONV0 + i).reshape(-1, Cc)
            for i in range(n_gdn)]
    return {"k": k, "v": v, "rec": rec, "conv": conv, "tokens": tokens, "conv_rows": conv_rows}


def _blob_hashes(oracle, geo, tokens, image):
    blobs, _ = oracle.image_layout(geo, tokens)
    return [oracle.fnv1a64(image[off:off + n]) for _, _, off, n in blobs]


SMALL_GEO = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=64, page_size=4, ssm_state_size=16,
                 ssm_k_heads=2, ssm_v_heads=4, ssm_d_conv=4, ssm_conv_channels=96, idx_key_dim=32)


@pytest.mark.parametrize("tokens,conv_rows,dtype,tail", [(37, 3, 0, 0), (40, 3, 1, 0), (2, 2, 0, 0x5A),
                                                         (13, 0, 0, 0x11)])
def test_synthetic_image_hashes_equal_fill_carve_park(oracle, tokens, conv_rows, dtype, tail):
    """sco_synth_*_hash == FNV-1a of each blob of sco_park(sco_handoff_carve(sco_fill_*)): the streaming checker of
    the full-size configs computes exactly the bytes the pinned oracle chain produces (f16 and f32 sources, a page
    tail of untouched bytes, short conv histories)."""
    g = oracle.Geometry(*SMALL_GEO.values())
    inputs = _synthetic_inputs(oracle, g, tokens, seed=77, conv_rows=conv_rows, dtype=dtype)
    n_pages = (tokens + g.page_size - 1) // g.page_size
    initial = oracle.new_state(g, n_pages)
    for key in initial:
        initial[key].view(np.uint8)[:] = tail
    state = oracle.expected_slot(g, inputs, slot_cells=n_pages * g.page_size, initial=initial)
    want = _blob_hashes(oracle, g, tokens, oracle.park(g, tokens, state))
    got = oracle.synthetic_image_hashes(g, tokens, 77, conv_rows=conv_rows, tail=tail, threads=3)
    assert got == want


def test_synthetic_image_hashes_with_appended_chunk(oracle):
    """Two sources per K/V blob (a parked prefix of L tokens, then a chunk appended at cell L mid-page): the form the
    batched resume + append is checked with."""
    g = oracle.Geometry(*SMALL_GEO.values())
    L, chunk = 21, 10
    first = _synthetic_inputs(oracle, g, L, seed=5, conv_rows=3)
    second = _synthetic_inputs(oracle, g, chunk, seed=905, conv_rows=0)
    n_pages = (L + chunk + g.page_size - 1) // g.page_size
    state = oracle.expected_slot(g, first, slot_cells=n_pages * g.page_size)
    oracle.carve_into(g, second, state, n_pages, pos0=L, with_gdn=False)
    want = _blob_hashes(oracle, g, L + chunk, oracle.park(g, L + chunk, state))
    got = oracle.synthetic_image_hashes(g, L, 5, chunk=(905, chunk), threads=2)
    assert got == want
    # a plausible mistake fails: the chunk placed one cell early, or the recurrence left head-major
    assert oracle.synthetic_image_hashes(g, L - 1, 5, chunk=(905, chunk), threads=2)[0] != want[0]
    bad = dict(state)
    rec_len = g.ssm_state_size * g.ssm_v_heads * g.ssm_state_size
    bad["gdn"] = state["gdn"].copy()
    bad["gdn"][0, :rec_len] = first["rec"][0].reshape(-1)
    assert _blob_hashes(oracle, g, L + chunk, oracle.park(g, L + chunk, bad))[-1] != want[-1]


@pytest.mark.parametrize("fmt", [1, 2, 3])
@pytest.mark.parametrize("tokens,tail", [(37, 0x5A), (40, 0)])
def test_synthetic_quant_hashes_equal_fill_quantize(oracle, fmt, tokens, tail):
    """sco_synth_quant_blob_hash == FNV-1a of each pool blob of sco_kv_append_quant(sco_fill_uniform_f32): the
    streaming checker of the full-size quantizing carves computes exactly the bytes of the pinned quantizers (int8
    codes and scales, q4_0 blocks, K8V4's int8 K with q4_0 V), over pools whose untouched tail cells hold `tail`."""
    g = oracle.Geometry(*SMALL_GEO.values())
    H, D, ps = g.n_head_kv, g.head_dim, g.page_size
    n_qsa = g.n_layers // g.qsa_interval
    inputs = _synthetic_inputs(oracle, g, tokens, seed=31, conv_rows=3, dtype=1)
    n_pages = (tokens + ps - 1) // ps
    rows = n_pages * H * ps
    want = []
    for j in range(n_qsa):
        k_fmt = 2 if fmt == 2 else 1
        v_fmt = 1 if fmt == 1 else 2
        scale_blobs = []
        for x, f in ((inputs["k"][j], k_fmt), (inputs["v"][j], v_fmt)):
            row_bytes = D if f == 1 else D // 32 * 18
            codes = np.full(rows * row_bytes, tail, dtype=np.uint8)
            scales = np.full(rows * (D // 64), tail | tail << 8, dtype=np.uint16) if f == 1 else None
            oracle.kv_append_quant(x, f, tokens, 0, None, n_pages, H, D, ps, codes, scales)
            want.append(oracle.fnv1a64(codes))
            if scales is not None:
                scale_blobs.append(oracle.fnv1a64(scales.view(np.uint8)))
        want += scale_blobs
    state = oracle.expected_slot(g, inputs, slot_cells=n_pages * ps)
    want.append(oracle.fnv1a64(state["gdn"].view(np.uint8)))
    got = oracle.synthetic_quant_hashes(g, tokens, 31, fmt, tail=tail, threads=3)
    assert got == want
    # a plausible mistake fails: the V rows quantized from the K stream
    if fmt == 1:
        bad = oracle.quant_blob_hash(g, n_pages * ps, 31, oracle.SID_K0, tokens, 1, 0, tail)
        assert bad != want[1]
