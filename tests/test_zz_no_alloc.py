"""The hash that allocates nothing (sc_fnv1a64_noalloc_async, a static per-GPU workspace) against the same hash with a
caller workspace (sc_fnv1a64_async), through the C-ABI: two calls in a row on one stream, the second with a smaller,
ragged, misaligned input, each bit-identical to the workspace form and to the oracle's byte loop, each with a clear
fault word."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_noalloc_hash_equals_workspace_hash(sc, oracle, cuda):
    big, small = (1 << 30) + 4096, 3 * (1 << 20) + 5
    buf = sc.DeviceBuffer(big + 64, "uint8")
    sc.check(sc.lib.sc_fill_uniform_f16(buf.ptr, (big + 64) // 2, -4.0, 4.0, 7, 1, None), "fill")
    # the fill ran on the null stream and the hashes below run on a non-blocking stream, which does not wait for it
    sc.device_sync()
    host = sc.PinnedBuffer(big + 64)
    sc.check(sc.lib.sc_copy_async(host.ptr, buf.ptr, big + 64, None), "copy")
    sc.device_sync()
    hp = sc.HashPlan(big)
    words = sc.DeviceBuffer(2, "uint64")   # [hash, fault word]
    stream = sc.Stream()
    try:
        for n, at in ((big, 0), (small, 3)):
            print(f"no-allocation hash of {n} bytes at offset {at}", flush=True)
            hp.launch(buf.ptr + at, n, stream=stream)
            stream.sync()
            want = hp.result()
            words.fill(0xEE)
            sc.device_sync()
            sc.check(sc.lib.sc_fnv1a64_noalloc_async(buf.ptr + at, n, sc.REFERENCE_FNV_SEED, words.ptr, words.ptr + 8,
                                                     stream.handle),
                     "sc_fnv1a64_noalloc_async")
            stream.sync()
            got = words.numpy()
            assert int(got[1]) & 0xFFFFFFFF == 0, (n, "fault word")
            assert int(got[0]) == want, (n, hex(int(got[0])), hex(want))
            assert want == oracle.fnv1a64(host.numpy()[at:at + n], sc.REFERENCE_FNV_SEED), n
    finally:
        hp.free()
        host.free()
        buf.free()
        words.free()
