"""The arithmetic the device FNV-1a's levels rest on (strata-concurrent_amd/csrc/sc_hash.hip), checked on the CPU
against brute force: the low byte of the FNV-1a state is the machine l' = ((l ^ b) * 179) mod 256, and a level's
map of a run of bytes says where the level's bits go given the true lower bits.

The kernel computes a k-bit level's map from 2^(k-2) machine runs plus the byte parities of the run (the top two
bits' terms follow from the term of the bit below and the parity of that bit), runs each 256-byte lane segment as two
128-byte halves side by side, takes the lane's map as the second half's after the first's, and gets the bits at the
midpoint by applying the first half's map to the start bits.  Each of these steps is restated here the way the kernel
does it and compared with running the machine from every start value, so a wrong parity bit, a swapped composition
order or a wrong midpoint fails.  The device kernel itself is compared with the byte loop in tests/test_gpu_hash.py.
"""
import numpy as np
import pytest

PRIME_LOW = 179   # 1099511628211 mod 256


def run(l, data):
    for b in data:
        l = ((l ^ int(b)) * PRIME_LOW) & 0xFF
    return l


def brute_map(low, j, k, data):
    """The level's map (t, v0, v1[, w00, w01, w10, w11]) read off the machine run from every start of the level."""
    ends = {st: (run(low | (st << j), data) >> j) & ((1 << k) - 1) for st in range(1 << k)}
    t = ends[0] & 1
    v = [((ends[a] >> 1) & 1) for a in (0, 1)]
    for a in (0, 1):   # the term of bit j + 1 does not depend on the start value of bit j + 1
        assert all(((ends[a | (c << 1)] >> 1) & 1) ^ c == v[a] for c in (0, 1))
    bits = [t] + v
    if k == 3:
        bits += [((ends[a | (c << 1)] >> 2) & 1) for a in (0, 1) for c in (0, 1)]
    return sum(bit << i for i, bit in enumerate(bits))


def shortcut_map(low, j, k, data):
    """The kernel's form (map3_of / map2_of): 2^(k-2) machines, the rest from the byte parities."""
    par = 0
    for b in data:
        par ^= int(b)
    odd = len(data) & 1
    if k == 2:
        e = run(low, data)
        t, v0 = (e >> j) & 1, (e >> (j + 1)) & 1
        return t | (v0 << 1) | ((v0 ^ t ^ ((par >> j) & 1) ^ odd) << 2)
    e0, e1 = run(low, data), run(low | (1 << j), data)
    t = (e0 >> j) & 1
    v0, v1 = (e0 >> (j + 1)) & 1, (e1 >> (j + 1)) & 1
    w00, w10 = (e0 >> (j + 2)) & 1, (e1 >> (j + 2)) & 1
    q = ((par >> (j + 1)) & 1) ^ odd
    return t | (v0 << 1) | (v1 << 2) | (w00 << 3) | ((w00 ^ v0 ^ q) << 4) | (w10 << 5) | ((w10 ^ v1 ^ q) << 6)


def map_v(m, a):
    return (m >> (1 + a)) & 1


def map_w(m, a, c):
    return (m >> (3 + 2 * a + c)) & 1


def compose(k, g, f):
    """g after f, as compose<k> in the kernel."""
    tf = f & 1
    r = tf ^ (g & 1)
    for a in (0, 1):
        r |= (map_v(f, a) ^ map_v(g, a ^ tf)) << (1 + a)
    if k == 3:
        for a in (0, 1):
            for c in (0, 1):
                r |= (map_w(f, a, c) ^ map_w(g, a ^ tf, c ^ map_v(f, a))) << (3 + 2 * a + c)
    return r


def apply(k, m, st):
    a, c = st & 1, (st >> 1) & 1
    r = (a ^ (m & 1)) | ((c ^ map_v(m, a)) << 1)
    if k == 3:
        r |= (((st >> 2) & 1) ^ map_w(m, a, c)) << 2
    return r


LEVELS = ((0, 3), (3, 3), (6, 2))


def runs(rng, count):
    for i in range(count):
        n = int(rng.integers(0, 300))
        data = rng.integers(0, 256, n)
        if i % 3 == 0:
            data &= int(rng.integers(0, 256))   # low-entropy runs: some bits constant
        yield data


@pytest.mark.parametrize("j,k", LEVELS + ((0, 2), (2, 3), (4, 2), (5, 3)))
def test_level_map_from_fewer_machines_equals_every_start(j, k):
    rng = np.random.default_rng(100 + 8 * j + k)
    for data in runs(rng, 400):
        low = int(rng.integers(0, 256)) & ((1 << j) - 1)
        assert shortcut_map(low, j, k, data) == brute_map(low, j, k, data), (j, k, len(data))


def test_the_parity_term_matters():
    # a shortcut without the parity (or without the length's parity) is wrong on some runs: the check above has teeth
    rng = np.random.default_rng(7)
    wrong = 0
    for data in runs(rng, 200):
        e0 = run(0, data)
        t, v0 = e0 & 1, (e0 >> 1) & 1
        if (t | (v0 << 1) | ((v0 ^ t) << 2)) != brute_map(0, 0, 2, data):
            wrong += 1
    assert wrong > 20


def test_halves_compose_to_the_segment_and_give_the_midpoint():
    """A 256-byte segment as two 128-byte halves, level by level, as the kernel's level1/2/3_maps and the kernel body:
    the lane's map is the second half's after the first's, and the first half's map applied to the true start bits
    gives the bits at the midpoint, where the next level's second-half machines start."""
    rng = np.random.default_rng(31)
    for trial in range(600):
        seg = rng.integers(0, 256, 256)
        if trial % 4 == 0:
            seg &= int(rng.integers(0, 256))
        a_half, b_half = seg[:128], seg[128:]
        true0 = int(rng.integers(0, 256))
        true_mid = run(true0, a_half)
        true_end = run(true_mid, b_half)
        low_a = low_b = 0
        for j, k in LEVELS:
            ma, mb = shortcut_map(low_a, j, k, a_half), shortcut_map(low_b, j, k, b_half)
            lane = compose(k, mb, ma)
            st = (true0 >> j) & ((1 << k) - 1)
            assert apply(k, lane, st) == (true_end >> j) & ((1 << k) - 1)
            mid = apply(k, ma, st)
            assert mid == (true_mid >> j) & ((1 << k) - 1)
            low_a |= st << j
            low_b |= mid << j
        assert (low_a, low_b) == (true0, true_mid)


def test_workgroup_maps_compose_in_order():
    # maps of consecutive runs compose associatively and in run order (the look-back's scan relies on both)
    rng = np.random.default_rng(5)
    for _ in range(200):
        parts = [rng.integers(0, 256, int(rng.integers(1, 40))) for _ in range(3)]
        j, k = LEVELS[int(rng.integers(0, 3))]
        low = int(rng.integers(0, 256)) & ((1 << j) - 1)
        # the lower bits at each part's start follow the machine from `low`
        lows, l = [], low
        for p in parts:
            lows.append(l & ((1 << j) - 1))
            l = run(l, p)
        m = [brute_map(lows[i], j, k, parts[i]) for i in range(3)]
        whole = brute_map(low, j, k, np.concatenate(parts))
        assert compose(k, m[2], compose(k, m[1], m[0])) == whole
        assert compose(k, compose(k, m[2], m[1]), m[0]) == whole
