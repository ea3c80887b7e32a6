"""The hash's carries (sc_fnv1a64_carry_async, sc_fnv1a64_check_carried_async and their map forms) against the
oracle's byte loop.

A producer's hash writes the low byte of the running hash after every whole 64 KiB of its input (the carries); a check
given them starts every 64 KiB workgroup from the carry before it instead of looking back, and verifies that it ends
with the carry after it.  Here: the carries equal the low bytes the byte loop reaches at every 64 KiB boundary (chained
sco_fnv1a64 over the 64 KiB pieces); the check with them gives the byte loop's hash and a 1 verdict; a carry with one
bit flipped (first, middle, last) gives a 0 verdict with SC_FNV_FAULT_CARRY; a payload byte flipped, with the original
carries, gives a 0 verdict; the fused capture + hash writes the same carries as the plain hash of its payload; and a
payload held in segments is checked where it lies with the same result.
"""
import numpy as np
import pytest

import sc_synthetic as synth

pytestmark = pytest.mark.gpu

GROUP = 64 << 10


def oracle_carries(oracle, data, seed):
    out, h = [], seed
    for k in range((len(data) - 1) // GROUP if len(data) else 0):
        h = oracle.fnv1a64(data[k * GROUP:(k + 1) * GROUP], h)
        out.append(h & 0xFF)
    return np.array(out, dtype=np.uint8)


@pytest.mark.parametrize("n,offset", [(1, 0), (255, 0), (GROUP, 0), (GROUP + 1, 0), (3 * GROUP + 77, 0),
                                      (5 * (1 << 20) + 3, 3), (64 * (1 << 20) + 200, 0), (64 * (1 << 20), 5)])
def test_carries_and_the_check_given_them(sc, oracle, cuda, n, offset):
    print(f"case carries n={n} offset={offset}", flush=True)
    seed = sc.REFERENCE_FNV_SEED if n % 2 else 0x0123456789ABCDEF
    data = np.random.default_rng(n + offset).integers(0, 256, size=n, dtype=np.uint8)
    buf = sc.DeviceBuffer(n + offset + 16, "uint8")
    buf.upload(np.concatenate([np.zeros(offset, np.uint8), data, np.zeros(16, np.uint8)]))
    nc = sc.carry_bytes(n)
    assert nc == (n - 1) // GROUP
    carry = sc.DeviceBuffer(max(nc, 1) + 16, "uint8")
    hp = sc.HashPlan(n)
    try:
        want = oracle.fnv1a64(data, seed)
        want_carry = oracle_carries(oracle, data, seed)
        carry.fill(0xEE)
        hp.fault.fill(0xAB)
        hp.launch_carry(buf.ptr + offset, n, carry.ptr, seed=seed)
        sc.device_sync()
        assert hp.fault_word() == 0 and hp.result() == want
        got = carry.numpy(max(nc, 1) + 16)
        assert np.array_equal(got[:nc], want_carry), np.flatnonzero(got[:nc] != want_carry)[:8]
        assert (got[nc:] == 0xEE).all()   # nothing past the carries is written
        # the check given them
        hp.fault.fill(0xAB)
        hp.verdict.fill(0)
        hp.check_carried(buf.ptr + offset, n, want, carry.ptr, seed=seed)
        sc.device_sync()
        assert int(hp.verdict.numpy()[0]) == 1 and hp.fault_word() == 0 and int(hp.out.numpy()[0]) == want
        # one carry bit flipped: refused, and the fault says why
        for k in sorted({0, nc // 2, nc - 1}) if nc else []:
            bad = want_carry.copy()
            bad[k] ^= 1 << (k % 8)
            carry.upload(bad)
            hp.fault.fill(0)
            hp.verdict.fill(1)
            hp.check_carried(buf.ptr + offset, n, want, carry.ptr, seed=seed)
            sc.device_sync()
            assert int(hp.verdict.numpy()[0]) == 0, k
            assert hp.fault_word() & sc.FNV_FAULT_CARRY, k
        # one payload byte flipped with the carries of the original: refused
        carry.upload(want_carry if nc else np.zeros(1, np.uint8))
        for at in sorted({0, n // 2, n - 1}):
            flipped = data.copy()
            flipped[at] ^= 0x5A
            buf.upload(np.concatenate([np.zeros(offset, np.uint8), flipped]))
            hp.verdict.fill(1)
            hp.check_carried(buf.ptr + offset, n, want, carry.ptr, seed=seed)
            sc.device_sync()
            assert int(hp.verdict.numpy()[0]) == 0, at
    finally:
        hp.free()
        carry.free()
        buf.free()


SMALL = dict(n_layers=8, qsa_interval=4, n_head_kv=2, head_dim=256, page_size=4, ssm_state_size=32,
             ssm_k_heads=4, ssm_v_heads=8, ssm_d_conv=4, ssm_conv_channels=520, idx_key_dim=128)


@pytest.mark.parametrize("tokens", [300, 77])
def test_fused_capture_writes_the_carries_of_its_payload(sc, oracle, cuda, tokens):
    geo = sc.geometry(**SMALL)
    print(f"case fused carries {tokens} tokens", flush=True)
    case = synth.SyntheticCase(geo, tokens, seed=0xCA77 + tokens)
    slot = case.new_slot(max_cells=tokens + 8)
    case.carve_into(slot)
    _, total = sc.image_layout(geo, tokens)
    head = 4096 + 48   # a head the plans do not write, then the blobs
    nbytes = head + total + 16 * 5   # and a tail under one lane segment past the last 64 KiB boundary
    payload = sc.DeviceBuffer(nbytes, "uint8")
    payload.fill(0x3C)
    plan = sc.plan_capture(geo, slot, tokens, payload.ptr + head, total)
    nc = sc.carry_bytes(nbytes)
    assert nc >= 2
    carry, carry_plain = sc.DeviceBuffer(nc, "uint8"), sc.DeviceBuffer(nc, "uint8")
    hp = sc.HashPlan(nbytes)
    hmap = sc.HashMap([plan], payload.ptr, nbytes)
    try:
        hmap.launch_carry(hp, carry.ptr)
        sc.device_sync()
        h_fused = hp.result()
        data = payload.numpy(nbytes).copy()
        assert h_fused == oracle.fnv1a64(data)
        assert np.array_equal(carry.numpy(nc), oracle_carries(oracle, data, sc.REFERENCE_FNV_SEED))
        hp.launch_carry(payload.ptr, nbytes, carry_plain.ptr)
        sc.device_sync()
        assert hp.result() == h_fused and np.array_equal(carry_plain.numpy(nc), carry.numpy(nc))
        # the payload held in segments, checked where it lies with the fused kernel's carries
        seg = 2 * GROUP
        n_seg = (nbytes + seg - 1) // seg
        segs = [sc.DeviceBuffer(seg, "uint8") for _ in range(n_seg)]
        for i, s in enumerate(segs):
            part = data[i * seg:(i + 1) * seg]
            s.upload(part)
        rmap = sc.HashMap.read([s.ptr for s in segs], seg, nbytes)
        hp.verdict.fill(0)
        hp.fault.fill(0xAB)
        rmap.check_carried(hp, h_fused, carry.ptr)
        sc.device_sync()
        assert int(hp.verdict.numpy()[0]) == 1 and hp.fault_word() == 0 and int(hp.out.numpy()[0]) == h_fused
        bad = carry.numpy(nc).copy()
        bad[-1] ^= 0x80
        carry_plain.upload(bad)
        hp.verdict.fill(1)
        rmap.check_carried(hp, h_fused, carry_plain.ptr)
        sc.device_sync()
        assert int(hp.verdict.numpy()[0]) == 0 and hp.fault_word() & sc.FNV_FAULT_CARRY
        rmap.destroy()
        for s in segs:
            s.free()
    finally:
        hmap.destroy()
        hp.free()
        carry.free()
        carry_plain.free()
        payload.free()
