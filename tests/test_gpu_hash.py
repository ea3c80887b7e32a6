"""The device FNV-1a 64 (sc_fnv1a64_*) against the oracle's byte loop, bit for bit.

The oracle (sco_fnv1a64) restates the reference's fnv1a64 (src/core/pinned.cu:594-601) and is pinned by the published
FNV-1a 64 test vectors in tests/test_oracle.py.  Here the parallel device hash must equal it on every size class the
segmenting can get wrong (empty, shorter than a segment, exact multiples of the 256-byte segment, of a workgroup's
64 KiB and of a scan block, ragged tails), from misaligned starts (the byte path), from any seed, and at the size of a
full 128K hand-off payload.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

SEEDS = [1469598103934665603, 0xCBF29CE484222325, 0, 0xFFFFFFFFFFFFFFFF, 0x0123456789ABCDEF]


def _upload(sc, data: np.ndarray, pad: int = 0):
    buf = sc.DeviceBuffer(max(data.size + pad, 16), "uint8")
    if data.size:
        buf.upload(data, start=pad)
    return buf


# sizes include one workgroup's 64 KiB and the look-back's window of 64 workgroups (4 MiB) with neighbours, so a
# workgroup's window reaches before the input's start, holds only maps, or starts exactly on a workgroup boundary
@pytest.mark.parametrize("n", [0, 1, 2, 15, 16, 17, 255, 256, 257, 1000, 4095, 4096, 65535, 65536, 65537,
                               3 * 65536 + 100, 1 << 20, (1 << 20) + 255, 64 << 16, (64 << 16) + 1, (65 << 16) + 300,
                               (129 << 16) - 7, 12_345_679, (257 << 16) + 3])
def test_device_hash_equals_byte_loop(sc, oracle, cuda, n):
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, size=n, dtype=np.uint8)
    buf = _upload(sc, data)
    for seed in SEEDS[: 2 if n > 100000 else len(SEEDS)]:
        assert sc.fnv1a64_device(buf.ptr, n, seed) == oracle.fnv1a64(data.tobytes(), seed), (n, hex(seed))
    buf.free()


def test_published_vectors_on_device(sc, cuda):
    basis = 0xCBF29CE484222325   # the textbook offset basis (the published vectors use it)
    for text, want in [(b"", basis), (b"a", 0xAF63DC4C8601EC8C), (b"foobar", 0x85944171F73967E8)]:
        arr = np.frombuffer(text, dtype=np.uint8)
        buf = _upload(sc, arr)
        assert sc.fnv1a64_device(buf.ptr, arr.size, basis) == want, text
        buf.free()


@pytest.mark.parametrize("offset", [1, 3, 8, 15])
def test_misaligned_start(sc, oracle, cuda, offset):
    n = 70_001
    data = np.random.default_rng(offset).integers(0, 256, size=n, dtype=np.uint8)
    buf = _upload(sc, data, pad=offset)
    assert sc.fnv1a64_device(buf.ptr + offset, n) == oracle.fnv1a64(data.tobytes())
    buf.free()


def test_low_entropy_inputs(sc, oracle, cuda):
    """All-zero, all-0xFF and a repeating ramp: inputs whose low-byte state walks short cycles."""
    n = 300_000
    for data in (np.zeros(n, np.uint8), np.full(n, 0xFF, np.uint8), (np.arange(n) % 251).astype(np.uint8)):
        buf = _upload(sc, data)
        assert sc.fnv1a64_device(buf.ptr, n) == oracle.fnv1a64(data.tobytes())
        buf.free()


def test_async_plan_on_a_stream_and_reuse(sc, oracle, cuda):
    """One workspace hashes inputs of different sizes back to back on a non-blocking stream."""
    plan = sc.HashPlan(1 << 22)
    stream = sc.Stream()
    for n in (1 << 22, 123_457, 0, 4096):
        data = np.random.default_rng(n + 7).integers(0, 256, size=n, dtype=np.uint8)
        buf = _upload(sc, data)
        plan.launch(buf.ptr, n, stream=stream)
        stream.sync()
        assert plan.result() == oracle.fnv1a64(data.tobytes()), n
        buf.free()
    plan.free()


@pytest.mark.parametrize("seed", [1469598103934665603, 0xFFFFFFFFFFFFFFFF])
def test_chained_pieces_equal_the_one_shot_hash(sc, oracle, cuda, seed):
    """sc_fnv1a64_chain_async over consecutive pieces (empty ones, ragged and misaligned boundaries, pieces shorter
    than a segment and spanning several workgroups) ends at the one-shot hash of the whole buffer, and the running
    hash after each piece is the byte loop's hash of the prefix so far."""
    rng = np.random.default_rng(seed & 0xFFFF)
    n = 5_000_011
    data = rng.integers(0, 256, size=n, dtype=np.uint8)
    buf = _upload(sc, data)
    cuts = [0, 0, 1, 17, 256, 4096 + 3, 65_536 * 3 + 5, 65_536 * 3 + 5, 1_000_000, 3_333_333, n - 1, n]
    plan = sc.HashPlan(n)
    stream = sc.Stream()
    plan.start(seed)
    for a, b in zip(cuts, cuts[1:]):
        plan.chain(buf.ptr + a, b - a, stream=stream)
        stream.sync()
        assert plan.result() == oracle.fnv1a64(data[:b].tobytes(), seed), (a, b)
    assert plan.result() == sc.fnv1a64_device(buf.ptr, n, seed)
    # queued back to back without waiting in between, the result is the same
    plan.start(seed)
    for a, b in zip(cuts, cuts[1:]):
        plan.chain(buf.ptr + a, b - a, stream=stream)
    stream.sync()
    assert plan.result() == oracle.fnv1a64(data.tobytes(), seed)
    plan.free()
    buf.free()


def test_workspace_refusals(sc, cuda):
    buf = sc.DeviceBuffer(1 << 16, "uint8")
    out = sc.DeviceBuffer(1, "uint64")
    small = int(sc.lib.sc_fnv1a64_workspace_bytes(1 << 16)) - 256
    ws = sc.DeviceBuffer(max(small, 16), "uint8")
    fault = out.ptr + 16   # inside the workspace buffer's allocation is not needed: refusals come first
    rc = sc.lib.sc_fnv1a64_async(buf.ptr, 1 << 16, 0, out.ptr, fault, ws.ptr, small, None)
    assert rc == sc.SC_EINVAL and "workspace" in sc.last_error()
    rc = sc.lib.sc_fnv1a64_chain_async(buf.ptr, 1 << 16, out.ptr, fault, ws.ptr, small, None)
    assert rc == sc.SC_EINVAL and "workspace" in sc.last_error()
    rc = sc.lib.sc_fnv1a64_chain_async(buf.ptr, 16, out.ptr + 4, fault, ws.ptr, small, None)
    assert rc == sc.SC_EINVAL and "aligned" in sc.last_error()
    rc = sc.lib.sc_fnv1a64_async(buf.ptr, 16, 0, out.ptr, None, ws.ptr, small, None)
    assert rc == sc.SC_EINVAL and "fault word" in sc.last_error()
    rc = sc.lib.sc_fnv1a64_chain_async(buf.ptr, 16, out.ptr, fault + 2, ws.ptr, small, None)
    assert rc == sc.SC_EINVAL and "fault word" in sc.last_error()
    for b in (buf, out, ws):
        b.free()


def test_full_payload_size(sc, oracle, cuda):
    """A buffer of the 128K hand-off payload's size (3 300 261 888 bytes), against the byte loop."""
    n = 3_300_261_888
    buf = sc.DeviceBuffer(n, "uint8")
    sc.lib.sc_fill_uniform_f16(buf.ptr, n // 2, -4.0, 4.0, 0x5EED, 77, None)
    sc.device_sync()
    host = sc.PinnedBuffer(n)
    sc.check(sc.lib.sc_copy_async(host.ptr, buf.ptr, n, None), "copy")
    sc.device_sync()
    want = oracle.fnv1a64(host.numpy())
    assert sc.fnv1a64_device(buf.ptr, n) == want
    host.free()
    buf.free()


def test_a_look_back_wait_that_runs_out_fails_the_verdict(sc, oracle, cuda):
    """The hash kernel's waits on earlier workgroups are bounded.  With the bound forced down to one read, waits run
    out (thousands of workgroups start together, and most cannot find their start state on their first reads): the
    launch still ends, and the verdict is 0 even though the expected hash is the true one.  With the default bound
    the same check passes."""
    n = 256 << 20
    buf = sc.DeviceBuffer(n, "uint8")
    sc.lib.sc_fill_uniform_f16(buf.ptr, n // 2, -4.0, 4.0, 0x5EED, 91, None)
    sc.device_sync()
    host = sc.PinnedBuffer(n)
    sc.check(sc.lib.sc_copy_async(host.ptr, buf.ptr, n, None), "copy")
    sc.device_sync()
    want = oracle.fnv1a64(host.numpy(), sc.REFERENCE_FNV_SEED)
    hp = sc.HashPlan(n)
    verdict = sc.DeviceBuffer(1, "uint32")
    try:
        for limit, passes in ((1, False), (0, True)):
            sc.check(sc.lib.sc_fnv1a64_set_spin_limit(limit), "spin limit")
            verdict.fill(0xAB)
            sc.check(sc.lib.sc_fnv1a64_check_async(buf.ptr, n, sc.REFERENCE_FNV_SEED, want, hp.out.ptr, verdict.ptr,
                                                   hp.fault.ptr, hp.ws.ptr, hp.ws_bytes, None), "check")
            sc.device_sync()
            print(f"case spin limit {limit}: verdict {int(verdict.numpy()[0])}", flush=True)
            assert int(verdict.numpy()[0]) == (1 if passes else 0)
            assert hp.faulted() == (not passes)
            if passes:
                assert hp.result() == want
    finally:
        sc.check(sc.lib.sc_fnv1a64_set_spin_limit(0), "spin limit")
        for b in (buf, host, verdict):
            b.free()
        hp.free()


def test_gated_scatter_writes_all_or_nothing(sc, oracle, cuda):
    """sc_fnv1a64_check_async leaves a verdict on the device and sc_plan_launch_gated scatters only when it is 1: a
    wrong expected hash leaves the slot untouched, the right one mounts it, with no host round trip in between."""
    geo = sc.geometry(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
                      ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520)
    tokens = 53
    case = synth.SyntheticCase(geo, tokens=tokens, seed=99)
    _, total = sc.image_layout(geo, tokens)
    image = sc.DeviceBuffer(total, "uint8")
    gather = sc.plan_gather(geo, case.prefill, image.ptr, total)
    gather.launch()
    sc.device_sync()
    want = oracle.fnv1a64(image.numpy(total))
    slot = case.new_slot(max_cells=64, fill=0x5C)
    scatter = sc.plan_scatter(geo, image.ptr, total, tokens, slot)
    hp = sc.HashPlan(total)
    verdict = sc.DeviceBuffer(1, "uint32")
    for expected, mounted in ((want ^ 1, False), (want, True)):
        verdict.fill(0xAB)
        sc.device_sync()
        sc.check(sc.lib.sc_fnv1a64_check_async(image.ptr, total, sc.REFERENCE_FNV_SEED, expected, hp.out.ptr,
                                               verdict.ptr, None, hp.ws.ptr, hp.ws_bytes, None), "check")
        sc.check(sc.lib.sc_plan_launch_gated(scatter.handle, verdict.ptr, None), "gated launch")
        sc.device_sync()
        assert hp.result() == want
        assert int(verdict.numpy()[0]) == int(mounted)
        state = slot.host_state()
        if mounted:
            assert np.array_equal(oracle.park(geo, tokens, state), image.numpy(total))
        else:
            assert all(np.all(v.view(np.uint8) == 0x5C) for v in state.values())
    hp.free()


def test_every_hash_form_reports_a_wait_that_ran_out(sc, oracle, cuda):
    """With every look-back wait forced to run out (SC_FNV_FORCE_FAULT; the launches still end), the one-shot form
    sets its fault word to 1, a chain's fault word stays 1 through a later piece that finishes cleanly, the form without
    allocation sets its fault word, and the synchronous form returns SC_ETIMEOUT instead of a hash.  With the default
    bound every fault word is 0 and every hash equals the byte loop's."""
    n = 16 << 20
    buf = sc.DeviceBuffer(n, "uint8")
    sc.check(sc.lib.sc_fill_uniform_f16(buf.ptr, n // 2, -4.0, 4.0, 0x5EED, 93, None), "fill")
    sc.device_sync()
    want = oracle.fnv1a64(buf.numpy(), sc.REFERENCE_FNV_SEED)
    hp = sc.HashPlan(n)
    words = sc.DeviceBuffer(4, "uint64")   # the form without allocation: [hash, fault]
    try:
        for limit in (sc.SC_FNV_FORCE_FAULT, 0):
            forced = limit != 0
            print(f"case spin limit {limit:#x}", flush=True)
            sc.check(sc.lib.sc_fnv1a64_set_spin_limit(limit), "spin limit")
            hp.fault.fill(0xAB)
            hp.launch(buf.ptr, n)
            sc.device_sync()
            assert int(hp.fault.numpy()[0]) == int(forced)
            if forced:
                with pytest.raises(sc.HashFault):
                    hp.result()
            else:
                assert hp.result() == want
            # a chain: the faulting piece first, then a small clean one (a single workgroup never waits)
            hp.start()
            hp.chain(buf.ptr, n - 1000)
            hp.chain(buf.ptr + n - 1000, 1000)
            sc.device_sync()
            assert int(hp.fault.numpy()[0]) == int(forced)
            if not forced:
                assert hp.result() == want
            words.fill(0xCD)
            sc.check(sc.lib.sc_fnv1a64_noalloc_async(buf.ptr, n, sc.REFERENCE_FNV_SEED, words.ptr, words.ptr + 8,
                                                     None), "noalloc")
            sc.device_sync()
            got = words.numpy()
            assert int(got[1]) & 0xFFFFFFFF == int(forced)
            if not forced:
                assert int(got[0]) == want
            # one workgroup's worth of input never waits, so it never faults
            hp.launch(buf.ptr, 65536)
            sc.device_sync()
            assert hp.result() == oracle.fnv1a64(buf.numpy(65536), sc.REFERENCE_FNV_SEED)
            out = sc._U64(0)
            rc = sc.lib.sc_fnv1a64_device(buf.ptr, n, sc.REFERENCE_FNV_SEED, sc.C.byref(out))
            if forced:
                assert rc == sc.SC_ETIMEOUT and "ran out" in sc.last_error()
            else:
                assert rc == sc.SC_OK and int(out.value) == want
    finally:
        sc.check(sc.lib.sc_fnv1a64_set_spin_limit(0), "spin limit")
        for b in (buf, words):
            b.free()
        hp.free()
