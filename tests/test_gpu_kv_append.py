"""The per-layer prefill writers with the reference's arguments (sc_kv_append_async, sc_kv_append_q4_async; the
reference's kv_append, src/prefill/kernels.cu:558-625, and kv_append_q4, src/kernels/cuda/kv_q4.cu:110-135,205-215)
against the oracle, byte for byte.

Each call writes K and V of T cells from pos0 into the paged pool through the page table (a negative entry skips its
cells), into the host copy (pinned memory the kernel writes directly) and into the staging pool, both identity layout.
The oracle's placement (sco_kv_append, sco_kv_append_quant) and quantizers (sco_q8_row, sco_q4_row) are pinned by
tests/test_oracle.py and tests/test_oracle_quant.py; here every pool byte, written or not, must equal the oracle's.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, D, PS = 2, 256, 4
ROW = {"f16": D * 2, "int8": D, "q4": D // 32 * 18}
SENTINEL = 0xEE


def _source(T: int, seed: int) -> np.ndarray:
    x = (np.random.default_rng(seed).standard_normal((T, H, D)) * 3).astype(np.float32)
    if T > 3:
        x[0, 0] = 0.0
        x[1, 1, :32] = 2.0
        x[1, 1, 5], x[1, 1, 9] = -5.0, 5.0          # tied magnitudes in a q4_0 block
        x[2, 0, :64] = np.nan                          # a group of NaNs
        x[2, 1, 7] = np.inf
        x[3, 0] *= np.float32(1e-5)
        x[3, 1, :3] = np.float32(70000.0)             # beyond f16: rounds to inf in the f16 pool
    return x


def _pools(sc, fmt: str, n_pages: int, host: bool):
    """K and V codes (+ int8 scales) of n_pages pages, sentinel-filled: device buffers, or pinned host memory."""
    def buf(nbytes):
        if host:
            b = sc.PinnedBuffer(nbytes)
            b.numpy()[:] = SENTINEL
        else:
            b = sc.DeviceBuffer(nbytes, "uint8")
            b.fill(SENTINEL)
        return b
    rows = n_pages * H * PS
    out = {"k": buf(rows * ROW[fmt]), "v": buf(rows * ROW[fmt])}
    if fmt == "int8":
        out["ks"], out["vs"] = buf(rows * 8), buf(rows * 8)
    return out


def _read(sc, b) -> np.ndarray:
    if isinstance(b, sc.PinnedBuffer):
        return b.numpy().copy()
    sc.device_sync()
    return b.numpy()


def _expected(oracle, fmt: str, x: np.ndarray, T: int, pos0: int, table, n_pages: int):
    """The oracle's pool (codes, scales) after the append, starting from sentinel bytes."""
    rows = n_pages * H * PS
    if fmt == "f16":
        pool = np.full(rows * D, SENTINEL | SENTINEL << 8, dtype=np.uint16)
        oracle.kv_append(x, T, pos0, table, n_pages, H, D, PS, pool)
        return pool.view(np.uint8), None
    codes = np.full(rows * ROW[fmt], SENTINEL, dtype=np.uint8)
    scales = np.full(rows * 4, SENTINEL | SENTINEL << 8, dtype=np.uint16) if fmt == "int8" else None
    oracle.kv_append_quant(x, 1 if fmt == "int8" else 2, T, pos0, table, n_pages, H, D, PS, codes, scales)
    return codes, None if scales is None else scales.view(np.uint8)


def _kv_pools(sc, fmt: str, p) -> "sc.KvPools":
    kp = sc.KvPools()
    if fmt == "f16":
        kp.k_pool, kp.v_pool = p["k"].ptr, p["v"].ptr
    elif fmt == "int8":
        kp.k_q, kp.v_q, kp.k_scale, kp.v_scale = p["k"].ptr, p["v"].ptr, p["ks"].ptr, p["vs"].ptr
    else:
        kp.k_q4, kp.v_q4 = p["k"].ptr, p["v"].ptr
    return kp


def _append(sc, fmt, K, V, T, pos0, table_ptr, pool, host=None, stage=None, stream=None):
    h = C.byref(host) if host is not None else None
    s = C.byref(stage) if stage is not None else None
    if fmt == "q4":
        return sc.lib.sc_kv_append_q4_async(pool["k"].ptr, pool["v"].ptr, table_ptr, pos0, T, K, V, H, D, PS, stream,
                                            h, s)
    if fmt == "f16":
        return sc.lib.sc_kv_append_async(K, V, T, pos0, table_ptr, PS, pool["k"].ptr, pool["v"].ptr, None, None, None,
                                         None, stream, h, s)
    return sc.lib.sc_kv_append_async(K, V, T, pos0, table_ptr, PS, None, None, pool["k"].ptr, pool["v"].ptr,
                                     pool["ks"].ptr, pool["vs"].ptr, stream, h, s)


TABLES = ["identity", "reversed", "holes"]


def _table(kind: str, n_logical: int, n_pages: int):
    if kind == "identity":
        return None
    t = np.arange(n_logical, dtype=np.int32)[::-1] % n_pages if kind == "reversed" else \
        np.random.default_rng(n_logical).permutation(n_pages)[:n_logical].astype(np.int32)
    if kind == "holes":
        t[1::3] = -1                                   # pages that are not resident
    return np.ascontiguousarray(t, dtype=np.int32)


@pytest.mark.parametrize("fmt", ["f16", "int8", "q4"])
@pytest.mark.parametrize("table_kind", TABLES)
@pytest.mark.parametrize("T,pos0", [(37, 0), (29, 6), (1, 13)])
def test_append_matches_oracle(sc, oracle, cuda, fmt, table_kind, T, pos0):
    print(f"case kv_append {fmt} {table_kind} T={T} pos0={pos0}", flush=True)
    n_logical = (pos0 + T + PS - 1) // PS
    n_pages = n_logical + 3
    x_k, x_v = _source(T, 1000 + T), _source(T, 2000 + T)
    K, V = sc.DeviceBuffer(x_k.size, "float32"), sc.DeviceBuffer(x_v.size, "float32")
    K.upload(x_k)
    V.upload(x_v)
    table = _table(table_kind, n_logical, n_pages)
    tab = None
    if table is not None:
        tab = sc.DeviceBuffer(table.size, "int32")
        tab.upload(table)
    pool = _pools(sc, fmt, n_pages, host=False)
    host = _pools(sc, fmt, n_logical, host=True)       # the host copy: identity, every cell
    stage = _pools(sc, fmt, n_logical, host=False)     # the staging pool: identity, every cell
    stream = sc.Stream()
    rc = _append(sc, fmt, K.ptr, V.ptr, T, pos0, tab.ptr if tab is not None else None, pool,
                 _kv_pools(sc, fmt, host), _kv_pools(sc, fmt, stage), stream.handle)
    assert rc == 0, sc.last_error()
    stream.sync()
    for name, dest, pages, tbl in (("pool", pool, n_pages, table), ("host", host, n_logical, None),
                                   ("stage", stage, n_logical, None)):
        for kv, x in (("k", x_k), ("v", x_v)):
            want_codes, want_scales = _expected(oracle, fmt, x, T, pos0, tbl, pages)
            got = _read(sc, dest[kv])
            assert np.array_equal(got, want_codes), (name, kv, np.flatnonzero(got != want_codes)[:8])
            if want_scales is not None:
                got_s = _read(sc, dest[kv + "s"])
                assert np.array_equal(got_s, want_scales), (name, kv, "scales")


def test_k8v4_aliased_calls(sc, oracle, cuda):
    """The reference's K8V4 prompt path appends K alone (K == V, k_q == v_q) and V alone into the q4_0 pool
    (src/prefill/prefill.cpp:1325-1331): the aliased rows write the same bytes, and the pools equal the oracle's."""
    T, pos0 = 23, 2
    n_pages = (pos0 + T + PS - 1) // PS + 1
    x_k, x_v = _source(T, 7), _source(T, 8)
    K, V = sc.DeviceBuffer(x_k.size, "float32"), sc.DeviceBuffer(x_v.size, "float32")
    K.upload(x_k)
    V.upload(x_v)
    kq = _pools(sc, "int8", n_pages, host=False)
    vq4 = _pools(sc, "q4", n_pages, host=False)
    assert sc.lib.sc_kv_append_async(K.ptr, K.ptr, T, pos0, None, PS, None, None, kq["k"].ptr, kq["k"].ptr,
                                     kq["ks"].ptr, kq["ks"].ptr, None, None, None) == 0, sc.last_error()
    assert sc.lib.sc_kv_append_q4_async(vq4["v"].ptr, vq4["v"].ptr, None, pos0, T, V.ptr, V.ptr, H, D, PS, None,
                                        None, None) == 0, sc.last_error()
    want_k, want_ks = _expected(oracle, "int8", x_k, T, pos0, None, n_pages)
    want_v, _ = _expected(oracle, "q4", x_v, T, pos0, None, n_pages)
    assert np.array_equal(_read(sc, kq["k"]), want_k) and np.array_equal(_read(sc, kq["ks"]), want_ks)
    assert np.array_equal(_read(sc, vq4["v"]), want_v)
    assert (_read(sc, kq["v"]) == SENTINEL).all() and (_read(sc, vq4["k"]) == SENTINEL).all()


def test_q4_pool_aligned_to_two_bytes(sc, oracle, cuda):
    """q4_0 pools need only 2-byte alignment (the reference's block is 18 bytes): a pool that starts 2 bytes past a
    16-byte boundary takes the 2-byte store path and must hold the same bytes as the oracle's."""
    T, pos0 = 19, 1
    n_pages = (pos0 + T + PS - 1) // PS + 1
    x_k, x_v = _source(T, 31), _source(T, 32)
    K, V = sc.DeviceBuffer(x_k.size, "float32"), sc.DeviceBuffer(x_v.size, "float32")
    K.upload(x_k)
    V.upload(x_v)
    rows = n_pages * H * PS
    kb, vb = sc.DeviceBuffer(rows * ROW["q4"] + 16, "uint8"), sc.DeviceBuffer(rows * ROW["q4"] + 16, "uint8")
    kb.fill(SENTINEL)
    vb.fill(SENTINEL)
    assert sc.lib.sc_kv_append_q4_async(kb.ptr + 2, vb.ptr + 2, None, pos0, T, K.ptr, V.ptr, H, D, PS, None, None,
                                        None) == 0, sc.last_error()
    for buf, x in ((kb, x_k), (vb, x_v)):
        want, _ = _expected(oracle, "q4", x, T, pos0, None, n_pages)
        got = _read(sc, buf)
        assert np.array_equal(got[2:2 + want.size], want)
        assert (got[:2] == SENTINEL).all() and (got[2 + want.size:] == SENTINEL).all()


def test_refusals_write_nothing(sc, cuda):
    T = 8
    K = sc.DeviceBuffer(T * H * D + 16, "float32")
    pool = _pools(sc, "f16", 4, host=False)
    q8 = _pools(sc, "int8", 4, host=False)
    q4 = _pools(sc, "q4", 4, host=False)
    cases = [
        lambda: sc.lib.sc_kv_append_async(K.ptr + 4, K.ptr, T, 0, None, PS, pool["k"].ptr, pool["v"].ptr, None, None,
                                          None, None, None, None, None),                 # misaligned K
        lambda: sc.lib.sc_kv_append_async(K.ptr, K.ptr, T, 0, None, PS, pool["k"].ptr, None, None, None, None, None,
                                          None, None, None),                               # f16 K pool without V
        lambda: sc.lib.sc_kv_append_async(K.ptr, K.ptr, T, 0, None, PS, None, None, q8["k"].ptr, q8["v"].ptr, None,
                                          None, None, None, None),                         # int8 without scales
        lambda: sc.lib.sc_kv_append_async(K.ptr, K.ptr, T, -1, None, PS, pool["k"].ptr, pool["v"].ptr, None, None,
                                          None, None, None, None, None),                   # negative pos0
        lambda: sc.lib.sc_kv_append_async(K.ptr, K.ptr, T, 0, None, 0, pool["k"].ptr, pool["v"].ptr, None, None,
                                          None, None, None, None, None),                   # page size 0
        lambda: sc.lib.sc_kv_append_q4_async(q4["k"].ptr, q4["v"].ptr, None, 0, T, K.ptr, K.ptr, H, 128, PS, None,
                                             None, None),                                  # head_dim 128
        lambda: sc.lib.sc_kv_append_async(None, K.ptr, T, 0, None, PS, pool["k"].ptr, pool["v"].ptr, None, None,
                                          None, None, None, None, None),                   # no K
    ]
    for i, call in enumerate(cases):
        assert call() == sc.SC_EINVAL, (i, sc.last_error())
        assert "kv_append" in sc.last_error(), i
    # T <= 0 launches nothing and succeeds, as the reference returns early
    assert sc.lib.sc_kv_append_async(None, None, 0, 0, None, PS, None, None, None, None, None, None, None, None,
                                     None) == 0
    assert sc.lib.sc_kv_append_q4_async(None, None, None, 0, -3, None, None, H, 64, PS, None, None, None) == 0
    for p in (pool, q8, q4):
        for b in p.values():
            assert (_read(sc, b) == SENTINEL).all()
