"""The hash that allocates nothing (sc_fnv1a64_noalloc_async, a static per-GPU workspace) against the same hash with a
caller workspace (sc_fnv1a64_async), through the C-ABI: two calls in a row on one stream, the second with a smaller,
ragged, misaligned input, each bit-identical to the workspace form; the small one also to the oracle's byte loop."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_noalloc_hash_equals_workspace_hash(sc, oracle, cuda):
    big, small = (1 << 30) + 4096, 3 * (1 << 20) + 5
    buf = sc.DeviceBuffer(big + 64, "uint8")
    sc.check(sc.lib.sc_fill_uniform_f16(buf.ptr, (big + 64) // 2, -4.0, 4.0, 7, 1, None), "fill")
    hp = sc.HashPlan(big)
    out = sc.DeviceBuffer(1, "uint64")
    stream = sc.Stream()
    got = []
    for n, at in ((big, 0), (small, 3)):
        print(f"no-allocation hash of {n} bytes at offset {at}", flush=True)
        hp.launch(buf.ptr + at, n, stream=stream)
        stream.sync()
        want = hp.result()
        out.fill(0)
        sc.device_sync()
        sc.check(sc.lib.sc_fnv1a64_noalloc_async(buf.ptr + at, n, sc.REFERENCE_FNV_SEED, out.ptr, stream.handle),
                 "sc_fnv1a64_noalloc_async")
        stream.sync()
        got.append(int(out.numpy()[0]))
        assert got[-1] == want, (n, hex(got[-1]), hex(want))
    assert got[1] == oracle.fnv1a64(buf.numpy(small, start=3).tobytes())
    hp.free()
