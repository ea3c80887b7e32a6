"""Pins the oracle's quantized K/V formats (sco_q8_row, sco_q4_row, sco_kv_append_quant) with independent numpy
restatements of the reference's rules and with hand-computed groups.

int8 (src/prefill/kernels.cu:578-600; kv_q8.cu:29-64; host form kv_q8_parity.cpp:78-92): per 64 values the scale is
f16(max|x| / 127) rounded to nearest even, codes rint(x / f32(scale)) clamped to +-127 (0 when the scale is 0).
q4_0 (kv_q4.cu:72-89; host form kv_q4_parity.cpp:64-87): per 32 values d = (value of largest |x|, ties to the larger)
/ -8, codes trunc(x * (1/d) + 8.5) rounded once (the device writer's fused multiply-add), clamped to [0, 15], packed
j | j+16 << 4 after the f16 scale.  numpy float32 arithmetic is IEEE single precision with no contraction; the fused
q4 sum is formed exactly in float64 (the product of two binary32 values is exact there) with an error-free TwoSum
deciding the rare ties.  So these vectorised forms are the same definitions computed a different way: a wrong group
size, a dropped clamp, a rounding mode, a separately rounded product or a nibble order fails them.
"""
import numpy as np
import pytest

F32 = np.float32


def q8_numpy(x):
    g = x.reshape(-1, 64).astype(F32)
    a = np.abs(g)
    amax = np.max(np.where(np.isnan(a), F32(0), a), axis=1)      # NaNs do not count toward the maximum
    with np.errstate(over="ignore"):
        scale = (amax / F32(127)).astype(np.float16)
    scale = np.where(np.isnan(g).all(axis=1), np.uint16(0x7E00).view(np.float16), scale)   # only NaNs: an f16 NaN
    sf = scale.astype(F32)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(g / np.where(sf > 0, sf, F32(1)))
    ok = (sf > 0) & ~np.isnan(g) & ~np.isnan(q)                   # a NaN quotient (inf / inf) codes 0
    q = np.where(ok, np.clip(np.where(ok, q, 0), -127, 127), 0).astype(np.int8)
    return q.reshape(x.shape), scale.view(np.uint16).reshape(x.shape[:-1] + (x.shape[-1] // 64,))


def fma_f32(a, b, c):
    """RN_binary32(a * b + c) for binary32 arrays, rounded once: a * b is exact in float64, the float64 sum's error is
    recovered exactly (Knuth's TwoSum), and where the float64 sum sits exactly halfway between two binary32 values the
    error decides the side (elsewhere the float64 sum rounds to the same binary32 value as the exact one)."""
    with np.errstate(invalid="ignore", over="ignore"):
        p = a.astype(np.float64) * b.astype(np.float64)
        c64 = np.float64(c)
        s = p + c64
        bb = s - p
        err = (p - (s - bb)) + (c64 - bb)
        f = s.astype(F32)
        back = f.astype(np.float64)
        other = np.where(back < s, np.nextafter(f, F32(np.inf)), np.nextafter(f, F32(-np.inf))).astype(np.float64)
        tie = np.isfinite(s) & (back != s) & (s - back == other - s)
        up, down = np.maximum(back, other), np.minimum(back, other)
        fixed = np.where(err > 0, up, down).astype(F32)
        return np.where(tie & (err != 0), fixed, f).astype(F32)


def q4_numpy(x):
    g = x.reshape(-1, 32).astype(F32)
    a = np.abs(g)
    a = np.where(np.isnan(a), F32(-1), a)                         # a NaN is never the maximum
    amax = a.max(axis=1, keepdims=True)
    with np.errstate(invalid="ignore"):
        mval = np.where(a == amax, g, -np.inf).max(axis=1)
    first = g[np.arange(g.shape[0]), np.argmax(a == amax, axis=1)]
    mval = np.where(mval == 0, first, mval)                       # +0 and -0 tie: the first in index order
    mval = np.where(amax[:, 0] < 0, F32(0), mval).astype(F32)     # a block of NaNs: +0
    d = (mval / F32(-8)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        idv = np.where(d != 0, F32(1) / np.where(d != 0, d, F32(1)), F32(0)).astype(F32)
        s = fma_f32(g, idv[:, None], F32(8.5))
    q = np.where(np.isnan(s), 0, np.clip(np.trunc(np.where(np.isnan(s), 0, s)), 0, 15)).astype(np.uint8)
    packed = (q[:, :16] | (q[:, 16:] << 4)).astype(np.uint8)
    with np.errstate(over="ignore"):
        dh = d.astype(np.float16).view(np.uint16)
    out = np.zeros((g.shape[0], 18), np.uint8)
    out[:, 0] = dh & 0xFF
    out[:, 1] = dh >> 8
    out[:, 2:] = packed
    return out.reshape(x.shape[:-1] + (x.shape[-1] // 32 * 18,))


def _groups(rng, n, D):
    x = rng.standard_normal((n, D)).astype(F32) * F32(3)
    x[0] = 0                                       # an all-zero row: scale 0, codes 0 / d 0, codes 8
    n64 = min(D, 64)
    x[1, :n64] = np.linspace(-127, 127, n64, dtype=F32)     # exact integer quotients
    x[2, :32] = F32(2.0)
    x[2, 5] = F32(-5.0)
    x[2, 9] = F32(5.0)                             # tied magnitudes: the positive value is the q4 maximum
    x[3] = rng.standard_normal(D).astype(F32) * F32(1e-3)   # tiny values: f16 scales near the subnormal range
    x[4] = rng.standard_normal(D).astype(F32) * F32(2e4)    # large values: scales near the f16 top
    x[5, :n64] = F32(127) * np.arange(n64, dtype=F32) / F32(64) + F32(0.5)   # quotients near .5
    x[6, 0] = np.nan                               # NaN first in its group: never the maximum, codes 0
    x[7, 5] = np.nan
    x[7, 9] = F32(50)                              # ... and NaN before the group's maximum
    x[7, n64 - 3:n64] = np.array([0xFFC00001, 0x7F800001, 0xFFFFFFFF], np.uint32).view(F32)   # negative, signalling
    x[8, :n64] = np.nan                            # a group of NaNs: scale NaN / d -0, codes 0 / 0
    x[9, 2], x[9, 7] = F32(np.inf), -F32(np.inf)   # infinities: an infinite scale; inf / inf codes 0
    x[10, :32] = -F32(0)
    x[10, 3] = F32(0)                              # -0 first among zeros: d = -0 / -8 = +0
    x[11, 1] = F32(1e7)                            # max / 127 beyond the f16 range: an infinite scale
    x[12, :32] = 0                                 # a q4_0 block with a subnormal d: 1/d overflows to -inf, so
    x[12, 0], x[12, 1] = F32(2.0 ** -146), -F32(2.0 ** -147)   # x * id + 8.5 is -inf (code 0) and +inf (code 15)
    return x


def test_f32_of_f16_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(F32)
    got = np.array([oracle.lib.sco_f32_of_f16(int(b)) for b in bits], dtype=F32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


@pytest.mark.parametrize("D", [64, 256, 512])
def test_q8_matches_numpy(oracle, D):
    x = _groups(np.random.default_rng(D), 200, D)
    codes, scales = oracle.q8_rows(x)
    wc, ws = q8_numpy(x)
    assert np.array_equal(codes, wc)
    assert np.array_equal(scales, ws)


def test_q8_hand_computed(oracle):
    x = np.zeros(64, F32)
    x[0], x[1], x[2], x[3] = F32(127), F32(-63.5), F32(0.49999997), F32(-127)
    codes, scales = oracle.q8_rows(x[None])
    assert scales[0, 0] == 0x3C00                  # 127 / 127 = 1.0
    assert list(codes[0, :4]) == [127, -64, 0, -127]   # -63.5 rounds half to even: -64
    y = np.zeros(64, F32)
    y[0] = F32(1e-9)                              # 1e-9 / 127 is below half the smallest f16 subnormal: scale 0
    codes, scales = oracle.q8_rows(y[None])
    assert scales[0, 0] == 0 and not codes.any()


@pytest.mark.parametrize("D", [32, 256])
def test_q4_matches_numpy(oracle, D):
    x = _groups(np.random.default_rng(D + 1), 200, D)
    assert np.array_equal(oracle.q4_rows(x), q4_numpy(x))


def test_q4_hand_computed(oracle):
    x = np.zeros(32, F32)
    x[0], x[16], x[3], x[19] = F32(-8), F32(4), F32(1), F32(-8)   # tie at |8|: both -8, so d = -8 / -8 = 1
    blk = oracle.q4_rows(x[None])[0]
    assert int(blk[0]) | (int(blk[1]) << 8) == 0x3C00       # d = 1.0
    # codes: trunc(x / 1 + 8.5): -8 -> 0, 4 -> 12, 1 -> 9, 0 -> 8
    assert blk[2 + 0] == (0 | (12 << 4))
    assert blk[2 + 3] == (9 | (0 << 4))
    assert blk[2 + 1] == (8 | (8 << 4))
    z = np.zeros(32, F32)
    zb = oracle.q4_rows(z[None])[0]
    # all +0: the maximum is +0, d = +0 / -8 = -0 (f16 0x8000), id 0, every code trunc(8.5) = 8
    assert zb[0] == 0 and zb[1] == 0x80 and all(b == 0x88 for b in zb[2:])
    t = np.zeros(32, F32)
    t[0], t[1] = F32(-3), F32(3)                   # tied magnitudes: the larger value (+3) is the maximum
    tb = oracle.q4_rows(t[None])[0]
    d = F32(3) / F32(-8)
    assert int(tb[0]) | (int(tb[1]) << 8) == int(np.array([d], F32).astype(np.float16).view(np.uint16)[0])


def test_q4_codes_round_once_like_the_device_writer(oracle):
    """Blocks with values on code boundaries, where trunc(RN(x * id + 8.5)) and trunc(RN(RN(x * id) + 8.5)) differ
    (found with exact rational arithmetic): the oracle follows the fused form, code for code, and the numpy form agrees
    with it; the separately rounded form would fail."""
    from quant_cases import boundary_blocks, fused_code, separate_code
    blocks = boundary_blocks(8)
    got = oracle.q4_rows(blocks)
    assert np.array_equal(got, q4_numpy(blocks))
    differing = 0
    for row, blk in zip(blocks, got):
        d = F32(row[0] / F32(-8))
        idv = F32(F32(1) / d)
        codes = [(blk[2 + (t % 16)] >> (4 * (t // 16))) & 15 for t in range(32)]
        assert codes == [fused_code(x, idv) for x in row]
        differing += sum(fused_code(x, idv) != separate_code(x, idv) for x in row)
    assert differing >= 8


def test_q4_overflowing_reciprocal_hand_computed(oracle):
    """d = 2^-146 / -8 = -2^-149 is the smallest subnormal, 1/d overflows to -inf: a positive value codes 0, a negative
    one 15 (a saturating conversion of +inf), a zero 0 (0 * inf is NaN)."""
    x = np.zeros(32, F32)
    x[0], x[1] = F32(2.0 ** -146), -F32(2.0 ** -147)
    blk = oracle.q4_rows(x[None])[0]
    assert int(blk[0]) | (int(blk[1]) << 8) == 0x8000               # d = -2^-149 rounds to -0 in f16
    assert blk[2] == 0 and blk[3] == 15 and not blk[4:].any()


def test_nan_and_infinity_hand_computed(oracle):
    nan8 = np.full(64, np.nan, F32)
    codes, scales = oracle.q8_rows(nan8[None])
    assert scales[0, 0] == 0x7E00 and not codes.any()             # only NaNs: the device writers' NaN maximum
    y = np.zeros(64, F32)
    y[0], y[1], y[2] = F32(np.inf), F32(1), F32(-np.inf)
    codes, scales = oracle.q8_rows(y[None])
    assert scales[0, 0] == 0x7C00 and not codes.any()             # scale inf: x / inf is 0, inf / inf codes 0
    blk = oracle.q4_rows(np.full(32, np.nan, F32)[None])[0]
    assert blk[0] == 0 and blk[1] == 0x80 and not blk[2:].any()   # d = +0 / -8 = -0; NaN codes 0
    z = np.zeros(32, F32)
    z[0], z[1], z[2] = np.nan, F32(-4), F32(2)                    # the NaN is passed over: d = -4 / -8 = 0.5
    blk = oracle.q4_rows(z[None])[0]
    assert int(blk[0]) | (int(blk[1]) << 8) == 0x3800
    assert blk[2] == 0 | (8 << 4) and blk[3] == 0 | (8 << 4) and blk[4] == 12 | (8 << 4)


@pytest.mark.parametrize("fmt", [1, 2])
def test_quant_placement(oracle, fmt):
    """The quantizing carve places row (t, h) where kv_append places it, and skips non-resident pages."""
    T, H, D, ps, n_pages, pos0 = 11, 2, 256, 4, 8, 3
    rng = np.random.default_rng(fmt)
    src = rng.standard_normal((T, H, D)).astype(F32)
    table = np.array([5, -1, 0, 7, 2, 1, 3, 4], np.int32)
    row_bytes = D if fmt == 1 else D // 32 * 18
    codes = np.full((n_pages, H, ps, row_bytes), 0xEE, np.uint8)
    scales = np.full((n_pages, H, ps, D // 64), 0xEEEE, np.uint16)
    oracle.kv_append_quant(src, fmt, T, pos0, table, n_pages, H, D, ps, codes, scales if fmt == 1 else None)
    for t in range(T):
        pos = pos0 + t
        page = table[pos // ps]
        for h in range(H):
            if page < 0:
                continue
            got = codes[page, h, pos % ps]
            if fmt == 1:
                c, s = q8_numpy(src[t, h])
                assert np.array_equal(got.view(np.int8), c) and np.array_equal(scales[page, h, pos % ps], s)
            else:
                assert np.array_equal(got, q4_numpy(src[t, h]))
    # the page behind the -1 entry (cells 4..7) is never written
    untouched = [p for p in range(n_pages) if p not in set(table[table >= 0][: (pos0 + T + ps - 1) // ps].tolist())]
    for p in untouched:
        assert (codes[p] == 0xEE).all()
