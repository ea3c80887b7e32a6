"""The prompt path of a streamed layer (src/prefill/prefill.cpp:1313-1340): before each chunk, the layer's cells
[0, p0) come back from its pinned host copy into the staging pool with kv_stage_from_host (sc_kv_stage_from_host;
the reference's kv_stream.cu:244-252: the first ceil(p0 / page_size) blocks of each run, one copy per run), then the
chunk is appended into the paged pool, the host copy and the staging pool (sc_kv_append_async /
sc_kv_append_q4_async).  After two chunks, with the staging pool reused (overwritten) in between as another layer
would, the staging pool and the host copy must equal the oracle's: the first chunk's appends, its first blocks
restored, the second chunk's appends on top, every other byte untouched.  f16, int8 (codes and scales) and q4_0."""
import numpy as np
import pytest

from test_gpu_kv_append import H, D, PS, ROW, SENTINEL, _append, _expected, _kv_pools, _pools, _read, _source

pytestmark = pytest.mark.gpu

REUSED = 0x77   # what another layer left in the staging pool


def _runs(sc, fmt, dst, src):
    """sc_kv_runs of the format (the reference's runs_of, kv_stream.cu:33-55): K and V codes, then the int8 scales;
    `len` is one block's bytes of that array."""
    rows = H * PS
    r = sc.KvRuns()
    names = ("k", "v", "ks", "vs") if fmt == "int8" else ("k", "v")
    for i, name in enumerate(names):
        r.src[i], r.dst[i] = src[name].ptr, dst[name].ptr
        r.len[i] = rows * (ROW[fmt] if name in ("k", "v") else (D // 64) * 2)
    r.n = len(names)
    return r


def _stage_blocks(arr: np.ndarray, host: np.ndarray, n_blocks: int, block: int) -> np.ndarray:
    """kv_stage_from_host's effect on one run: its first n_blocks blocks are the host copy's."""
    out = arr.copy()
    out[: n_blocks * block] = host[: n_blocks * block]
    return out


@pytest.mark.parametrize("fmt", ["f16", "int8", "q4"])
@pytest.mark.parametrize("T1,T2", [(37, 21), (40, 9), (1, 50)])
def test_streamed_layer_prompt_path(sc, oracle, cuda, fmt, T1, T2):
    print(f"case kv_stage_from_host {fmt} T1={T1} T2={T2}", flush=True)
    total = T1 + T2
    n_logical = (total + PS - 1) // PS
    n_pages = n_logical + 2
    table = np.random.default_rng(total).permutation(n_pages)[:n_logical].astype(np.int32)
    tab = sc.DeviceBuffer(table.size, "int32")
    tab.upload(table)
    xs = {c: (_source(T, 100 * c + T), _source(T, 100 * c + 50 + T)) for c, T in ((1, T1), (2, T2))}
    pool = _pools(sc, fmt, n_pages, host=False)       # the VRAM pool, through the page table
    host = _pools(sc, fmt, n_logical, host=True)      # the pinned host copy: identity, every cell
    stage = _pools(sc, fmt, n_logical, host=False)    # the staging pool: identity, every cell
    stream = sc.Stream()
    bufs = []
    for chunk, (T, p0) in ((1, (T1, 0)), (2, (T2, T1))):
        if chunk == 2:
            for b in stage.values():   # another layer used the staging pool in between
                b.fill(REUSED)
            sc.device_sync()
            runs = _runs(sc, fmt, stage, host)
            assert sc.lib.sc_kv_stage_from_host(sc.C.byref(runs), (p0 + PS - 1) // PS, stream.handle) == 0, \
                sc.last_error()
        K, V = sc.DeviceBuffer(xs[chunk][0].size, "float32"), sc.DeviceBuffer(xs[chunk][1].size, "float32")
        K.upload(xs[chunk][0])
        V.upload(xs[chunk][1])
        bufs += [K, V]
        assert _append(sc, fmt, K.ptr, V.ptr, T, p0, tab.ptr, pool, _kv_pools(sc, fmt, host), _kv_pools(sc, fmt, stage),
                       stream.handle) == 0, sc.last_error()
        stream.sync()
    n_staged = (T1 + PS - 1) // PS
    for kv, i in (("k", 0), ("v", 1)):
        # the host copy: both chunks appended onto its sentinel bytes
        c1, s1 = _expected(oracle, fmt, xs[1][i], T1, 0, None, n_logical)
        want_host = c1.copy()
        want_host_s = None if s1 is None else s1.copy()
        if fmt == "f16":
            pool16 = want_host.view(np.uint16).copy()
            oracle.kv_append(xs[2][i], T2, T1, None, n_logical, H, D, PS, pool16)
            want_host = pool16.view(np.uint8)
        else:
            scales = None if s1 is None else s1.view(np.uint16).copy()
            codes = want_host.copy()
            oracle.kv_append_quant(xs[2][i], 1 if fmt == "int8" else 2, T2, T1, None, n_logical, H, D, PS, codes,
                                   scales)
            want_host, want_host_s = codes, None if scales is None else scales.view(np.uint8)
        assert np.array_equal(_read(sc, host[kv]), want_host), (fmt, kv, "host copy")
        # the staging pool: the reused bytes, its first blocks from the host copy after chunk 1, then chunk 2
        block = H * PS * ROW[fmt]
        staged = _stage_blocks(np.full(c1.size, REUSED, np.uint8), c1, n_staged, block)
        if fmt == "f16":
            p16 = staged.view(np.uint16).copy()
            oracle.kv_append(xs[2][i], T2, T1, None, n_logical, H, D, PS, p16)
            want_stage, want_stage_s = p16.view(np.uint8), None
        else:
            sblock = H * PS * (D // 64) * 2
            sc_in = None if s1 is None else _stage_blocks(np.full(s1.size, REUSED, np.uint8), s1, n_staged, sblock)
            scales = None if sc_in is None else sc_in.view(np.uint16).copy()
            codes = staged.copy()
            oracle.kv_append_quant(xs[2][i], 1 if fmt == "int8" else 2, T2, T1, None, n_logical, H, D, PS, codes,
                                   scales)
            want_stage, want_stage_s = codes, None if scales is None else scales.view(np.uint8)
        got = _read(sc, stage[kv])
        assert np.array_equal(got, want_stage), (fmt, kv, "staging pool", np.flatnonzero(got != want_stage)[:8])
        if want_host_s is not None:
            assert np.array_equal(_read(sc, host[kv + "s"]), want_host_s), (fmt, kv, "host scales")
            assert np.array_equal(_read(sc, stage[kv + "s"]), want_stage_s), (fmt, kv, "staging scales")
    for b in bufs + [tab]:
        b.free()


def test_stage_from_host_refusals_and_empty(sc, cuda):
    """No blocks copies nothing; a malformed run list is refused before any copy."""
    a = sc.DeviceBuffer(4096, "uint8")
    b = sc.DeviceBuffer(4096, "uint8")
    a.fill(1)
    b.fill(2)
    r = sc.KvRuns()
    r.src[0], r.dst[0], r.len[0], r.n = a.ptr, b.ptr, 1024, 1
    assert sc.lib.sc_kv_stage_from_host(sc.C.byref(r), 0, None) == 0
    sc.device_sync()
    assert (b.numpy() == 2).all()
    bad = sc.KvRuns()
    bad.n = 5
    assert sc.lib.sc_kv_stage_from_host(sc.C.byref(bad), 1, None) == sc.SC_EINVAL
    bad.n, bad.src[0], bad.dst[0], bad.len[0] = 1, a.ptr, None, 1024
    assert sc.lib.sc_kv_stage_from_host(sc.C.byref(bad), 1, None) == sc.SC_EINVAL
    sc.device_sync()
    assert (b.numpy() == 2).all()
    a.free()
    b.free()
