// sc_hash.hip - FNV-1a 64 of a device buffer, bit-identical to the byte loop, computed in parallel.
//
// The engine's one content hash is FNV-1a 64: for every byte, h = (h ^ b) * p mod 2^64 with the prime
// p = 1099511628211 (the reference's fnv1a64, src/core/pinned.cu:594-601).  As written it is one long serial chain,
// about 1 GB/s on a CPU core, and the reference runs it twice over a multi-GB hand-off payload.  Two facts make the
// exact same value computable in parallel:
//
//   1. The low byte of the state is a finite-state machine of its own.  Multiplication mod 2^64 keeps the low 8 bits
//      a function of the low 8 bits, and xor with a byte touches only the low 8 bits, so
//          l' = ((l ^ b) * 179) mod 256          (179 = p mod 256).
//      Moreover bit j of l' depends only on bits 0..j of l and b (multiplication by an odd constant and xor are both
//      "triangular"), and it is bit j of l xor a term that involves only the lower bits:
//          l'_j = l_j ^ t_j,   t_j = b_j ^ bit_j(((l ^ b) mod 2^j) * 179).
//      So once bits 0..j-1 of the state are known at every position, bit j at every position is an exclusive xor
//      prefix of the t_j terms: a scan.  Eight levels of scans recover the low byte at every position.
//   2. With the low byte known, the rest is linear.  Writing h ^ b = h + d with d = (l ^ b) - l (a small signed
//      number), h_N = h_0 p^N + sum_n d_n p^(N-n) mod 2^64: independent per-segment Horner sums, folded with powers
//      of p in any order.
//
// The buffer is split into lane segments of kFnvLaneBytes bytes, and the low byte is resolved in three passes over
// the data: bits 0-2, 3-5 and 6-7.  A pass for bits j .. j + k - 1 runs every segment's machine from its known start
// bits 0..j-1 once per combination of the unknown start bits j .. j + k - 2, with the pass's top bit started at 0:
// the end value of a bit in a machine started from the true lower bits is the segment's xor term for that bit (the
// term of a bit depends only on the lower start bits).  Two machines share one 24-bit multiply (bytes 0 and 2 of a
// register); the first pass needs only bits 0..2, which follow l' = (l ^ b) * 3 mod 8, so its four machines share
// one register a byte each.  Per pass: the data pass ballots the terms, each workgroup leaves its map of the k-bit
// state (a byte), one workgroup scans the maps, and the next pass derives each lane's start bits from its
// workgroup's state and the ballots by xor-prefix arithmetic.  The last data pass runs the full machine from the now
// complete start byte, forms each segment's Horner sum, scales it by p^(bytes after the segment) and reduces; a final
// workgroup adds h_0 p^N.  Four reads of the input in all.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "sc_handoff.h"
#include "sc_internal.hpp"

namespace sc {
namespace {

constexpr uint64_t kFnvPrime = 1099511628211ull;
constexpr uint32_t kPrimeLow = 179u;   // kFnvPrime mod 256
constexpr int kScanThreads = 1024;

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;
using gu32x4 = __attribute__((address_space(1))) u32x4;

__device__ __forceinline__ uint64_t pow_prime(uint64_t e) {
    uint64_t r = 1, b = kFnvPrime;
    while (e) {
        if (e & 1) r *= b;
        b *= b;
        e >>= 1;
    }
    return r;
}

// The 16 dwords of one full, 16-byte aligned lane segment.
__device__ __forceinline__ void load_segment(const uint8_t* p, uint32_t (&w)[kFnvLaneBytes / 4]) {
#pragma unroll
    for (int k = 0; k < kFnvLaneBytes / 16; ++k) {
        const u32x4 v = *(const gu32x4*) (p + 16 * k);
        w[4 * k + 0] = v.x;
        w[4 * k + 1] = v.y;
        w[4 * k + 2] = v.z;
        w[4 * k + 3] = v.w;
    }
}

// Two low-byte machines side by side, in bytes 0 and 2 of `x`: xor the byte into both, drop the products' high
// bytes, one 24-bit multiply (byte 0's product stays below bit 16).  `bb` holds the byte in bytes 0 and 2.  (A packed
// 16-bit multiply, v_pk_mul_lo_u16, needs no mask but measured slower here: 843 against 777 us for bits 3-5 of 3.3 GB.)
__device__ __forceinline__ uint32_t step_pair(uint32_t x, uint32_t bb) {
    return __umul24((x ^ bb) & 0x00FF00FFu, kPrimeLow);
}
// Packed 16-bit subtraction of the two halves of a word (v_pk_sub_i16).
typedef short v2i16 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_sub(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2i16, a) - __builtin_bit_cast(v2i16, b));
}
// Byte k of w, in bytes 0 and 2 (v_perm_b32: selector 0x0c gives a zero byte).
template <int k>
__device__ __forceinline__ uint32_t spread(uint32_t w) {
    return __builtin_amdgcn_perm(0u, w, uint32_t(k | 0x0c00 | (k << 16) | 0x0c000000));
}

__device__ __forceinline__ uint32_t run_pair(const uint8_t* p, uint64_t n, bool full, uint32_t x) {
    if (full) {
        uint32_t w[kFnvLaneBytes / 4];
        load_segment(p, w);
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 4; ++k) {
            x = step_pair(x, spread<0>(w[k]));
            x = step_pair(x, spread<1>(w[k]));
            x = step_pair(x, spread<2>(w[k]));
            x = step_pair(x, spread<3>(w[k]));
        }
        return x;
    }
    for (uint64_t i = 0; i < n; ++i) x = step_pair(x, uint32_t(p[i]) * 0x10001u);
    return x;
}

// p^k mod 2^64 for k = 1..K as four signed 16-bit digits, digit[K - k] for the byte k places before a block's end:
// p^k = sum_j digit[j] 2^(16 j) mod 2^64 with every digit in [-2^15, 2^15) (balanced base 2^16; the carry out of the
// top digit is a multiple of 2^64 and drops).  The digits of bytes c and c + 1 of a block pair up as one 32-bit word,
// the operand layout of the packed 16-bit dot product.
template <int K>
struct PowDigits {
    uint32_t pair[K / 2][4];   // [c / 2][j]: digit of byte c in the low half, of byte c + 1 in the high half
};
template <int K>
constexpr PowDigits<K> pow_digits() {
    int32_t digit[K][4] = {};
    uint64_t pk = 1;
    for (int k = 1; k <= K; ++k) {
        pk *= kFnvPrime;
        uint64_t v = pk;
        for (int j = 0; j < 4; ++j) {
            const int32_t d = int32_t(int16_t(uint16_t(v & 0xFFFFu)));
            digit[K - k][j] = d;
            v = (v - uint64_t(int64_t(d))) >> 16;
        }
    }
    PowDigits<K> t{};
    for (int c = 0; c < K; c += 2)
        for (int j = 0; j < 4; ++j)
            t.pair[c / 2][j] = (uint32_t(digit[c][j]) & 0xFFFFu) | (uint32_t(digit[c + 1][j]) << 16);
    return t;
}
template <int K>
constexpr uint64_t prime_pow() {
    uint64_t r = 1;
    for (int k = 0; k < K; ++k) r *= kFnvPrime;
    return r;
}
constexpr PowDigits<16> kPowDigits = pow_digits<16>();
constexpr uint64_t kPrime16 = prime_pow<16>();

// The Horner sum of 16 bytes given the true low byte `l` before them: sum over c of d_c p^(16-c), d_c = (l ^ b) - l.
// Per digit j, S_j = sum_c d_c digit[c][j]: |d| <= 255 and |digit| <= 2^15, so |S_j| < 16 * 255 * 2^15 < 2^28 and the
// sums are exact in 32-bit integers.  Two bytes' d values share one word as signed 16-bit halves, so each S_j takes
// one packed dot product (v_dot2_i32_i16) per byte pair: 2 operations per byte for the four digits.
__device__ __forceinline__ int32_t dot2(uint32_t a, uint32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b), acc, false);
}
// sum_j S_j 2^(16 j) mod 2^64.
__device__ __forceinline__ uint64_t digit_sum(int32_t s0, int32_t s1, int32_t s2, int32_t s3) {
    return uint64_t(int64_t(s0)) + (uint64_t(int64_t(s1)) << 16) + (uint64_t(int64_t(s2)) << 32) +
           (uint64_t(int64_t(s3)) << 48);
}
__device__ __forceinline__ uint64_t block_sum(const u32x4 v, uint32_t& l) {
    const uint32_t dw[4] = {v.x, v.y, v.z, v.w};
    int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    // `m` carries the low byte's product unmasked: only its low 8 bits are ever read
    uint32_t m = l;
#pragma unroll
    for (int c = 0; c < 16; c += 2) {
        const uint32_t x0 = (m ^ (dw[c >> 2] >> (8 * (c & 3)))) & 0xFFu;
        const uint32_t d0 = x0 - (m & 0xFFu);
        m = __umul24(x0, kPrimeLow);
        const uint32_t x1 = (m ^ (dw[(c + 1) >> 2] >> (8 * ((c + 1) & 3)))) & 0xFFu;
        const uint32_t d1 = x1 - (m & 0xFFu);
        m = __umul24(x1, kPrimeLow);
        const uint32_t dp = __builtin_amdgcn_perm(d1, d0, 0x05040100u);   // low halves: d0 | d1 << 16
        s0 = dot2(dp, kPowDigits.pair[c / 2][0], s0);
        s1 = dot2(dp, kPowDigits.pair[c / 2][1], s1);
        s2 = dot2(dp, kPowDigits.pair[c / 2][2], s2);
        s3 = dot2(dp, kPowDigits.pair[c / 2][3], s3);
    }
    l = m & 0xFFu;
    return digit_sum(s0, s1, s2, s3);
}

// Byte k of `a` in byte 0 and byte k of `b` in byte 2, zeros elsewhere (v_perm_b32: selector 0x0c gives a zero byte).
__device__ __forceinline__ uint32_t pair_byte(uint32_t a, uint32_t b, int k) {
    return __builtin_amdgcn_perm(b, a, uint32_t(k) | 0x0c00u | (uint32_t(4 + k) << 16) | 0x0c000000u);
}

// The Horner sums of 128 bytes of two segments at once, as one sum: the true low bytes of their states sit in the
// low bytes of the halves of `m` (segment A low, B high, each half's high byte 0), and B starts kPairGap bytes after
// A.  Per step one permute lines up a byte of each, one xor, one packed subtract gives both d values (A's in the low
// half), one 24-bit multiply and a mask the next low bytes (the masked byte A's product stays below bit 16, as in
// step_pair).  Byte c of B is weighted by p^(128 - c) and byte c of A by p^(kPairGap + 128 - c), so each digit sum
// takes one packed dot product per step against a word holding both digits, and the block sum is A's and B's scaled
// to B's block end; the 64-bit sums are formed once per 128 bytes (|S_j| < 128 * 2 * 255 * 2^15 < 2^31 stays exact).
// About 4 VALU operations per byte of each segment, against 7.5 for one segment at a time.
constexpr int kPairBytes = 128;
constexpr uint64_t kPairGap = uint64_t(kThreads) * kFnvLaneBytes;   // a lane's two segments, a workgroup apart
constexpr uint64_t prime_pow_of(uint64_t e) {
    uint64_t r = 1, b = kFnvPrime;
    for (; e; e >>= 1, b *= b)
        if (e & 1) r *= b;
    return r;
}
struct PairDigits {
    uint32_t w[kPairBytes][4];   // [c][j]: digit j of p^(kPairGap + 128 - c) in the low half, of p^(128 - c) above
};
constexpr PairDigits pair_digits() {
    PairDigits t{};
    for (int c = 0; c < kPairBytes; ++c) {
        uint64_t va = prime_pow_of(kPairGap + kPairBytes - c), vb = prime_pow_of(kPairBytes - c);
        for (int j = 0; j < 4; ++j) {
            const int32_t da = int32_t(int16_t(uint16_t(va & 0xFFFFu))), db = int32_t(int16_t(uint16_t(vb & 0xFFFFu)));
            t.w[c][j] = (uint32_t(da) & 0xFFFFu) | (uint32_t(db) << 16);
            va = (va - uint64_t(int64_t(da))) >> 16;
            vb = (vb - uint64_t(int64_t(db))) >> 16;
        }
    }
    return t;
}
constexpr PairDigits kPairDigits = pair_digits();
constexpr uint64_t kPrimePair = prime_pow<kPairBytes>();
// p^(256 (63 - l)) for lane l: a lane's sum, relative to the end of its segment B, times this is relative to the end of
// the wave's last segment B.
struct LanePow {
    uint64_t v[64];
};
constexpr LanePow lane_pow() {
    LanePow t{};
    for (int l = 0; l < 64; ++l) t.v[l] = prime_pow_of(uint64_t(kFnvLaneBytes) * uint64_t(63 - l));
    return t;
}
__constant__ LanePow kLanePow = lane_pow();
__device__ __forceinline__ uint64_t run_sum2(const u32x4 (&va)[kPairBytes / 16], const u32x4 (&vb)[kPairBytes / 16],
                                             uint32_t& m) {
    int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
    for (int c = 0; c < kPairBytes; ++c) {
        const int w = c >> 2;   // the dword of byte c
        const uint32_t x = m ^ pair_byte(va[w >> 2][w & 3], vb[w >> 2][w & 3], c & 3);
        const uint32_t d = pk_sub(x, m);
        m = __umul24(x, kPrimeLow) & 0x00FF00FFu;
        s0 = dot2(d, kPairDigits.w[c][0], s0);
        s1 = dot2(d, kPairDigits.w[c][1], s1);
        s2 = dot2(d, kPairDigits.w[c][2], s2);
        s3 = dot2(d, kPairDigits.w[c][3], s3);
    }
    return digit_sum(s0, s1, s2, s3);
}

// One step of the full hash given the true low byte `l` of the state: accumulate d = (l ^ b) - l, then multiply.
__device__ __forceinline__ void step_full(uint32_t b, uint32_t& l, uint64_t& acc) {
    const uint32_t x = (l ^ b) & 0xFFu;
    acc = (acc + uint64_t(int64_t(int32_t(x) - int32_t(l)))) * kFnvPrime;
    l = __umul24(x, kPrimeLow) & 0xFFu;
}

// Exclusive xor prefix of a 64-bit word: bit i of the result is the xor of bits 0..i-1.
__device__ __forceinline__ uint64_t xor_prefix_excl(uint64_t x) {
    x ^= x << 1;
    x ^= x << 2;
    x ^= x << 4;
    x ^= x << 8;
    x ^= x << 16;
    x ^= x << 32;
    return x << 1;
}

// The ballots of one pass, per wave: the terms of the lowest unresolved bit j (T), of bit j + 1 for either start
// value a of bit j (U_a), and, in a three-bit pass, of bit j + 2 for each start pair (a, c) of bits j, j + 1 (W_ac).
// A bit's term over a run is the xor of per-byte contributions that depend only on the lower bits of the state, so
// each is the end value of that bit in a machine started from the right lower bits with the bit itself 0.
constexpr int kMaxPassWords = 7;   // T, U0, U1, W00, W01, W10, W11
struct PassWords {
    uint64_t* w[kMaxPassWords];
};
template <int kBits>
constexpr int pass_words() { return kBits == 3 ? 7 : 3; }

// The lanes' true start bits of one wave, as masks, from `st` (bit j in bit 0, j + 1 in bit 1, j + 2 in bit 2) at
// the wave's first segment; `st` advances past the wave.  Each lane's term for a bit is chosen by its own true lower
// bits, and the bit at a lane is the wave's incoming bit xor the terms of the lanes before it.
template <int kBits>
__device__ __forceinline__ void wave_masks(const uint64_t (&wd)[kMaxPassWords], uint32_t& st, uint64_t (&m)[3]) {
    const uint32_t a = st & 1u, c = (st >> 1) & 1u;
    const uint64_t sj = xor_prefix_excl(wd[0]) ^ (a ? ~0ull : 0ull);
    const uint64_t v = (sj & wd[2]) | (~sj & wd[1]);
    const uint64_t sc = xor_prefix_excl(v) ^ (c ? ~0ull : 0ull);
    m[0] = sj;
    m[1] = sc;
    uint32_t next = (a ^ (uint32_t(__popcll(wd[0])) & 1u)) | ((c ^ (uint32_t(__popcll(v)) & 1u)) << 1);
    if constexpr (kBits == 3) {
        const uint32_t e = (st >> 2) & 1u;
        const uint64_t x = (~sj & ~sc & wd[3]) | (~sj & sc & wd[4]) | (sj & ~sc & wd[5]) | (sj & sc & wd[6]);
        m[2] = xor_prefix_excl(x) ^ (e ? ~0ull : 0ull);
        next |= (e ^ (uint32_t(__popcll(x)) & 1u)) << 2;
    }
    st = next;
}

// This lane's true start bits j .. j + kBits - 1 (bit 0 of the result upward) in the pass's workgroup `group`, from
// that workgroup's start state and the ballots of its waves.
template <int kBits>
__device__ __forceinline__ uint32_t lane_bits(uint64_t group, uint32_t gstate, const PassWords& w) {
    // the wave index is read as wave-uniform, so the masks below are scalar work
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t base = group * 4;
    uint32_t st = gstate;
    uint64_t m[3] = {0, 0, 0};
    // every word this lane may need is loaded before the first step, so the loads overlap
    uint64_t wd[kThreads / 64][kMaxPassWords] = {};
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k)
#pragma unroll
        for (int i = 0; i < pass_words<kBits>(); ++i)
            if (k <= wave) wd[k][i] = w.w[i][base + k];
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k)
        if (k <= wave) wave_masks<kBits>(wd[k], st, m);
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < kBits; ++i) bits |= (uint32_t(m[i] >> lane) & 1u) << i;
    return bits;
}

// The first pass only needs bits 0..2 of the state, which follow l' = ((l ^ b) * 3) mod 8 (179 = 3 mod 8): four
// such machines share one register, one per byte (a 3-bit state times 3 stays below 2^8, so nothing carries across
// bytes; the product's bits above 2 are masked by the next step).  Machine (a, c) - start bits 0, 1 = a, c - sits in
// byte a + 2c.
template <int k>
__device__ __forceinline__ uint32_t spread4(uint32_t w) {
    return __builtin_amdgcn_perm(0u, w, uint32_t(k | (k << 8) | (k << 16) | (k << 24)));
}
__device__ __forceinline__ uint32_t step_low3(uint32_t x, uint32_t b4) {
    const uint32_t y = (x ^ b4) & 0x07070707u;
    return y + (y << 1);
}
__device__ __forceinline__ uint32_t run_low3(const uint8_t* p, uint64_t n, bool full) {
    uint32_t x = 0x03020100u;
    if (full) {
        uint32_t w[kFnvLaneBytes / 4];
        load_segment(p, w);
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 4; ++k) {
            x = step_low3(x, spread4<0>(w[k]));
            x = step_low3(x, spread4<1>(w[k]));
            x = step_low3(x, spread4<2>(w[k]));
            x = step_low3(x, spread4<3>(w[k]));
        }
    } else {
        for (uint64_t i = 0; i < n; ++i) x = step_low3(x, uint32_t(p[i]) * 0x01010101u);
    }
    return x & 0x07070707u;
}

// Four low-byte machines in two registers (bytes 0 and 2 of each), one spread byte for both.
__device__ __forceinline__ void run_quad(const uint8_t* p, uint64_t n, bool full, uint32_t& xa, uint32_t& xb) {
    if (full) {
        uint32_t w[kFnvLaneBytes / 4];
        load_segment(p, w);
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 4; ++k) {
            uint32_t bb = spread<0>(w[k]);
            xa = step_pair(xa, bb);
            xb = step_pair(xb, bb);
            bb = spread<1>(w[k]);
            xa = step_pair(xa, bb);
            xb = step_pair(xb, bb);
            bb = spread<2>(w[k]);
            xa = step_pair(xa, bb);
            xb = step_pair(xb, bb);
            bb = spread<3>(w[k]);
            xa = step_pair(xa, bb);
            xb = step_pair(xb, bb);
        }
        return;
    }
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t bb = uint32_t(p[i]) * 0x10001u;
        xa = step_pair(xa, bb);
        xb = step_pair(xb, bb);
    }
}

__device__ __forceinline__ uint32_t map_v(uint32_t m, uint32_t a) { return (m >> (1u + a)) & 1u; }
__device__ __forceinline__ uint32_t map_w(uint32_t m, uint32_t a, uint32_t c) { return (m >> (3u + 2u * a + c)) & 1u; }
template <int kBits>
__device__ __forceinline__ uint32_t compose(uint32_t g, uint32_t f) {
    const uint32_t tf = f & 1u;
    uint32_t r = tf ^ (g & 1u);
#pragma unroll
    for (uint32_t a = 0; a < 2; ++a) r |= (map_v(f, a) ^ map_v(g, a ^ tf)) << (1u + a);
    if constexpr (kBits == 3) {
#pragma unroll
        for (uint32_t a = 0; a < 2; ++a)
#pragma unroll
            for (uint32_t c = 0; c < 2; ++c)
                r |= (map_w(f, a, c) ^ map_w(g, a ^ tf, c ^ map_v(f, a))) << (3u + 2u * a + c);
    }
    return r;
}
template <int kBits>
__device__ __forceinline__ uint32_t apply(uint32_t m, uint32_t st) {
    const uint32_t a = st & 1u, c = (st >> 1) & 1u;
    uint32_t r = (a ^ (m & 1u)) | ((c ^ map_v(m, a)) << 1);
    if constexpr (kBits == 3) r |= (((st >> 2) & 1u) ^ map_w(m, a, c)) << 2;
    return r;
}

// Data pass for bits j .. j + kBits - 1.  First completes each segment's start bits from the previous pass (which
// resolved kPrevBits bits; the bits below it are in start[]), then runs the machines - two (start bit j = 0, 1) for
// a two-bit pass, four (start bits j, j + 1 = 00, 10, 01, 11) for a three-bit one - ballots the terms, and leaves
// the workgroup's summary: its map of the state at its first segment (bit 0 t, bits 1-2 v_a, bits 3-6 w_ac).
template <int kBits, int kPrevBits>
__global__ void __launch_bounds__(kThreads) fnv_pass_kernel(const uint8_t* data, uint64_t n, int j, bool aligned,
                                                             uint8_t* start, PassWords prev, const uint8_t* gstate_prev,
                                                             PassWords out, uint8_t* summary) {
    const uint64_t seg = uint64_t(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t begin = seg * kFnvLaneBytes;
    const bool live = begin < n;
    uint32_t s = 0;
    if constexpr (kPrevBits > 0) {
        const uint32_t bits = lane_bits<kPrevBits>(blockIdx.x, gstate_prev[blockIdx.x], prev);
        const int lo = j - kPrevBits;
        s = (lo > 0 && live ? uint32_t(start[seg]) : 0u) | (bits << lo);
        if (live) start[seg] = uint8_t(s);
    }
    uint32_t ea = 0, eb = 0;
    if constexpr (kBits == 3 && kPrevBits == 0) {
        // bits 0..2 (j = 0): the four machines of run_low3 end in bytes a + 2c; regroup them into the layout the
        // ballots below read (ea: machines (0, 0) in byte 0 and (1, 0) in byte 2; eb: (0, 1) and (1, 1))
        if (live) {
            const uint64_t len = n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
            const uint32_t x = run_low3(data + begin, len, aligned && len == kFnvLaneBytes);
            ea = (x & 0xFFu) | (((x >> 8) & 0xFFu) << 16);
            eb = ((x >> 16) & 0xFFu) | ((x >> 24) << 16);
        }
    } else if (live) {
        const uint64_t len = n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
        const bool full = aligned && len == kFnvLaneBytes;
        ea = s | ((s | (1u << j)) << 16);
        if constexpr (kBits == 2) {
            ea = run_pair(data + begin, len, full, ea);
        } else {
            const uint32_t sc = s | (1u << (j + 1));
            eb = sc | ((sc | (1u << j)) << 16);
            run_quad(data + begin, len, full, ea, eb);
        }
    }
    uint64_t bw[kMaxPassWords] = {};
    bw[0] = __ballot((ea >> j) & 1u);
    bw[1] = __ballot((ea >> (j + 1)) & 1u);
    bw[2] = __ballot((ea >> (16 + j + 1)) & 1u);
    if constexpr (kBits == 3) {
        bw[3] = __ballot((ea >> (j + 2)) & 1u);        // start (a, c) = (0, 0)
        bw[4] = __ballot((eb >> (j + 2)) & 1u);        // (0, 1)
        bw[5] = __ballot((ea >> (16 + j + 2)) & 1u);   // (1, 0)
        bw[6] = __ballot((eb >> (16 + j + 2)) & 1u);   // (1, 1)
    }
    // this wave's map of the state at its first segment, from its ballots (wave-uniform, so scalar work); the
    // workgroup's map is the four waves' maps composed in order
    uint32_t wmap = 0;
#pragma unroll
    for (uint32_t in = 0; in < (1u << (kBits - 1)); ++in) {   // start (a, c) = (in & 1, in >> 1), e = 0
        const uint32_t a = in & 1u, c = (in >> 1) & 1u;
        uint32_t st = in;
        uint64_t m[3];
        wave_masks<kBits>(bw, st, m);
        if (in == 0) wmap |= st & 1u;                                  // t
        if (c == 0) wmap |= ((st >> 1) & 1u) << (1 + a);               // v_a: the end bit j + 1 from c = 0
        if constexpr (kBits == 3) wmap |= ((st >> 2) & 1u) << (3 + 2 * a + c);   // w_ac: end bit j + 2 from e = 0
    }
    __shared__ uint32_t s_map[kThreads / 64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if ((threadIdx.x & 63) == 0) {
        const uint64_t at = uint64_t(blockIdx.x) * 4 + wave;
#pragma unroll
        for (int i = 0; i < pass_words<kBits>(); ++i) out.w[i][at] = bw[i];
        s_map[wave] = wmap;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t sum = s_map[0];
        for (int k = 1; k < kThreads / 64; ++k) sum = compose<kBits>(s_map[k], sum);
        summary[blockIdx.x] = uint8_t(sum);
    }
}

// The state the hash starts from: the launch's seed, or the running hash at `seed_dev` when the input continues an
// earlier one (read by every kernel that needs it, so one stream can chain pieces without a host round trip).
__device__ __forceinline__ uint64_t start_state(uint64_t seed, const uint64_t* seed_dev) {
    return seed_dev ? *seed_dev : seed;
}

// The workgroups' start states for one pass, in one workgroup.  Workgroup g maps the state (a, c, e) = (bit j,
// j + 1, j + 2) at its first segment to (a ^ t, c ^ v_a, e ^ w_ac) at the next workgroup's, and its summary byte is
// that map (bit 0 t, bits 1-2 v_0 v_1, bits 3-6 w_00 w_01 w_10 w_11; a two-bit pass has no e and no w).  Maps compose
// as (g after f): t = t_f ^ t_g, v_a = v_a(f) ^ v_(a ^ t_f)(g), w_ac = w_ac(f) ^ w_(a ^ t_f, c ^ v_a(f))(g).
// Each thread composes its run of summaries (read 16 bytes at a time), the runs are scanned across threads in LDS,
// and each thread then walks its run again from its start state, writing the states 16 at a time.
constexpr uint64_t kScanVec = 16;   // summary bytes per vector load / state bytes per vector store

template <int kBits>
__global__ void __launch_bounds__(kScanThreads) fnv_scan_kernel(const uint8_t* summary, uint64_t groups, int j,
                                                                 uint64_t seed, const uint64_t* seed_dev,
                                                                 uint8_t* gstate) {
    constexpr uint32_t kMask = kBits == 3 ? 0x7Fu : 0x7u;
    const uint32_t init = uint32_t(start_state(seed, seed_dev) >> j) & ((1u << kBits) - 1u);
    // runs of whole 16-byte vectors: the summaries and states live in 256-byte aligned buffers padded to 256 bytes,
    // so a vector that starts before `groups` stays inside its buffer
    const uint64_t per = ((groups + kScanThreads - 1) / kScanThreads + kScanVec - 1) / kScanVec * kScanVec;
    const uint64_t b = uint64_t(threadIdx.x) * per;
    const uint64_t e = b + per < groups ? b + per : groups;
    uint32_t f = 0;
    for (uint64_t c = b; c < e; c += kScanVec) {
        const u32x4 w = *(const gu32x4*) (summary + c);
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < int(kScanVec); ++k)
            if (c + uint64_t(k) < e) f = compose<kBits>((words[k >> 2] >> (8 * (k & 3))) & kMask, f);
    }
    // inclusive scan of the run maps (Hillis-Steele), then the exclusive prefix of this thread's run
    __shared__ uint32_t s_map[kScanThreads];
    s_map[threadIdx.x] = f;
    __syncthreads();
    for (int o = 1; o < kScanThreads; o <<= 1) {
        const uint32_t earlier = threadIdx.x >= uint32_t(o) ? s_map[threadIdx.x - o] : 0u;
        __syncthreads();
        s_map[threadIdx.x] = compose<kBits>(s_map[threadIdx.x], earlier);
        __syncthreads();
    }
    uint32_t st = apply<kBits>(threadIdx.x ? s_map[threadIdx.x - 1] : 0u, init);
    for (uint64_t c = b; c < e; c += kScanVec) {
        const u32x4 w = *(const gu32x4*) (summary + c);
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
        uint32_t out[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < int(kScanVec); ++k) {
            out[k >> 2] |= st << (8 * (k & 3));
            st = apply<kBits>((words[k >> 2] >> (8 * (k & 3))) & kMask, st);
        }
        if (c + kScanVec <= e) {
            *(gu32x4*) (gstate + c) = u32x4{out[0], out[1], out[2], out[3]};
        } else {
            for (uint64_t k = 0; c + k < e; ++k) gstate[c + k] = uint8_t(out[k >> 2] >> (8 * (k & 3)));
        }
    }
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(uint32_t(v), m), hi = __shfl_xor(uint32_t(v >> 32), m);
    return (uint64_t(hi) << 32) | lo;
}

// One segment's Horner sum, scaled by p^(bytes after it), from the true low byte `l` at its start.
__device__ __forceinline__ uint64_t segment_sum(const uint8_t* data, uint64_t n, uint64_t begin, bool aligned,
                                                uint32_t l) {
    const uint64_t len = n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
    const uint8_t* p = data + begin;
    uint64_t acc = 0;
    if (aligned && len == kFnvLaneBytes) {
        u32x4 v[kFnvLaneBytes / 16];
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 16; ++k) v[k] = *(const gu32x4*) (p + 16 * k);
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 16; ++k) acc = acc * kPrime16 + block_sum(v[k], l);
    } else {
        for (uint64_t i = 0; i < len; ++i) step_full(p[i], l, acc);
    }
    return acc * pow_prime(n - begin - len);
}

// Each lane takes two segments, its own in the pass's workgroups 2g and 2g + 1, and runs their machines side by side
// (run_sum2).  A lane's segment is read in two halves of 128 bytes, each half of both segments loaded before it is
// summed (lanes are 256 bytes apart, so each half is one 128-byte line per segment, read by eight loads issued
// together).  The last, partial segments and unaligned data take the one-segment path.
__global__ void __launch_bounds__(kThreads) fnv_final_kernel(const uint8_t* data, uint64_t n, uint64_t groups,
                                                              bool aligned, const uint8_t* start, PassWords prev,
                                                              const uint8_t* gstate_prev, uint64_t* partial) {
    const uint64_t ga = uint64_t(blockIdx.x) * 2, gb = ga + 1;
    const uint64_t sa = ga * kThreads + threadIdx.x, sb = gb * kThreads + threadIdx.x;
    const uint64_t ba = sa * kFnvLaneBytes, bb = sb * kFnvLaneBytes;
    const uint32_t bits_a = lane_bits<2>(ga, gstate_prev[ga], prev);
    const uint32_t bits_b = gb < groups ? lane_bits<2>(gb, gstate_prev[gb], prev) : 0u;
    // p^(n - r), r the end of the wave's last segment B: wave-uniform, one power per wave rather than one per lane.  p
    // has order dividing 2^62 modulo 2^64, so the exponent is taken modulo 2^62 (r passes n in the buffer's last wave)
    const uint64_t wave_end =
        (gb * kThreads + uint64_t(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * 64 + 64) * kFnvLaneBytes;
    const uint64_t wave_pow = pow_prime((n - wave_end) & ((uint64_t(1) << 62) - 1));
    uint64_t acc = 0;
    if (aligned && bb + kFnvLaneBytes <= n) {   // both segments whole
        uint32_t m = (uint32_t(start[sa]) | (bits_a << 6)) | ((uint32_t(start[sb]) | (bits_b << 6)) << 16);
        uint64_t acc2 = 0;
#pragma unroll 1
        for (int h = 0; h < kFnvLaneBytes; h += kPairBytes) {
            u32x4 va[kPairBytes / 16], vb[kPairBytes / 16];
#pragma unroll
            for (int k = 0; k < kPairBytes / 16; ++k) {
                va[k] = *(const gu32x4*) (data + ba + h + 16 * k);
                vb[k] = *(const gu32x4*) (data + bb + h + 16 * k);
            }
            acc2 = acc2 * kPrimePair + run_sum2(va, vb, m);
        }
        acc = acc2 * kLanePow.v[threadIdx.x & 63] * wave_pow;   // both segments, scaled to the input's end
    } else {
        if (ba < n) acc += segment_sum(data, n, ba, aligned, uint32_t(start[sa]) | (bits_a << 6));
        if (bb < n) acc += segment_sum(data, n, bb, aligned, uint32_t(start[sb]) | (bits_b << 6));
    }
    for (int m = 32; m > 0; m >>= 1) acc += shfl_xor64(acc, m);
    __shared__ uint64_t s_sum[kThreads / 64];
    if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
}

// h = seed * p^n + sum of the partial sums (mod 2^64; the order of the additions does not matter).  With `verdict`,
// also 1 there when h equals `expected`, else 0: a later kernel on the stream can act on the check without a host
// round trip.
__global__ void __launch_bounds__(kScanThreads) fnv_reduce_kernel(const uint64_t* partial, uint64_t groups, uint64_t seed,
                                                                   const uint64_t* seed_dev, uint64_t n, uint64_t* out,
                                                                   uint64_t expected, uint32_t* verdict) {
    uint64_t acc = 0;
    for (uint64_t i = threadIdx.x; i < groups; i += kScanThreads) acc += partial[i];
    for (int m = 32; m > 0; m >>= 1) acc += shfl_xor64(acc, m);
    __shared__ uint64_t s_sum[kScanThreads / 64];
    if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t h = start_state(seed, seed_dev) * pow_prime(n);
        for (int w = 0; w < kScanThreads / 64; ++w) h += s_sum[w];
        out[0] = h;
        if (verdict) verdict[0] = h == expected ? 1u : 0u;
    }
}

}  // namespace

// Workspace: [start bytes: one per segment][ballot words T, U0, U1, W00..W11: two sets (this pass, the previous)]
// [summaries][workgroup start states: two sets][partial sums].
FnvWorkspace fnv_workspace(uint64_t n) {
    FnvWorkspace w{};
    w.segments = (n + kFnvLaneBytes - 1) / kFnvLaneBytes;
    w.groups = (w.segments + kThreads - 1) / kThreads;
    auto up = [](uint64_t x) { return (x + 255) / 256 * 256; };
    w.off_start = 0;
    w.off_word0 = up(w.segments);
    w.off_word1 = w.off_word0 + kMaxPassWords * up(w.groups * 4 * 8);
    w.off_parity = w.off_word1 + kMaxPassWords * up(w.groups * 4 * 8);   // summaries
    w.off_prefix = w.off_parity + up(w.groups);               // start states, two sets
    w.off_partial = w.off_prefix + 2 * up(w.groups);
    w.bytes = w.off_partial + up(w.groups * 8 > 8 ? w.groups * 8 : 8);
    return w;
}

hipError_t launch_fnv1a64(const void* data, uint64_t n, uint64_t seed, const uint64_t* seed_dev, uint64_t* out,
                          void* workspace, hipStream_t stream, uint64_t expected, uint32_t* verdict) {
    const FnvWorkspace w = fnv_workspace(n);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const uint8_t* src = static_cast<const uint8_t*>(data);
    const bool aligned = (reinterpret_cast<uintptr_t>(data) & 15u) == 0;
    const uint64_t word_bytes = (w.off_word1 - w.off_word0) / kMaxPassWords;
    auto words = [&](uint64_t off) {
        PassWords p{};
        for (int k = 0; k < kMaxPassWords; ++k) p.w[k] = reinterpret_cast<uint64_t*>(ws + off + k * word_bytes);
        return p;
    };
    const PassWords set[2] = {words(w.off_word0), words(w.off_word1)};
    uint8_t* start = ws + w.off_start;
    uint8_t* summary = ws + w.off_parity;
    const uint64_t half = (w.off_partial - w.off_prefix) / 2;
    uint8_t* gstate[2] = {ws + w.off_prefix, ws + w.off_prefix + half};
    uint64_t* partial = reinterpret_cast<uint64_t*>(ws + w.off_partial);
    const uint64_t final_groups = (w.groups + 1) / 2;   // the final pass takes two of the passes' workgroups each
    if (w.groups > 0) {
        // bits 0-2, then 3-5 (four machines per lane), then 6-7 (two): three reads of the data before the final one;
        // each pass reads the previous pass's ballots and workgroup states
        const dim3 grid(unsigned(w.groups)), block(kThreads), one(1), scan(kScanThreads);
        hipLaunchKernelGGL((fnv_pass_kernel<3, 0>), grid, block, 0, stream, src, n, 0, aligned, start, set[1],
                           gstate[1], set[0], summary);
        hipLaunchKernelGGL(fnv_scan_kernel<3>, one, scan, 0, stream, summary, w.groups, 0, seed, seed_dev, gstate[0]);
        hipLaunchKernelGGL((fnv_pass_kernel<3, 3>), grid, block, 0, stream, src, n, 3, aligned, start, set[0],
                           gstate[0], set[1], summary);
        hipLaunchKernelGGL(fnv_scan_kernel<3>, one, scan, 0, stream, summary, w.groups, 3, seed, seed_dev, gstate[1]);
        hipLaunchKernelGGL((fnv_pass_kernel<2, 3>), grid, block, 0, stream, src, n, 6, aligned, start, set[1],
                           gstate[1], set[0], summary);
        hipLaunchKernelGGL(fnv_scan_kernel<2>, one, scan, 0, stream, summary, w.groups, 6, seed, seed_dev, gstate[0]);
        hipLaunchKernelGGL(fnv_final_kernel, dim3(unsigned(final_groups)), block, 0, stream, src, n, w.groups, aligned,
                           start, set[0], gstate[0], partial);
    }
    // the reduce reads the start state before it writes `out`, so `out` may be `seed_dev` itself
    hipLaunchKernelGGL(fnv_reduce_kernel, dim3(1), dim3(kScanThreads), 0, stream, partial, final_groups, seed, seed_dev,
                       n, out, expected, verdict);
    return hipGetLastError();
}

}  // namespace sc

// ---- the hash that allocates nothing ----------------------------------------------------------------------------------
// For callers that cannot allocate (code under HIP graph capture, tight serving loops): the workspace is `scratch`, one
// array per GPU that the library holds until the process ends, sized for inputs of up to SC_FNV_NOALLOC_MAX_BYTES
// (fnv_workspace(4 GiB) is 44.7 MiB).  Its kernels write every workspace word they later read, so nothing in it is
// cleared between calls; a call after another on the same stream is ordered after it, and calls that overlap on one
// GPU (on different streams) race on the one array.
namespace {

constexpr uint64_t kScratchBytes = 48ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};   // the device address of `scratch` on each GPU, looked up once per GPU

// The current device's copy of `scratch`.  In host code the array's name is only a stand-in for the device symbol, so
// kernels get the address the runtime reports for it, looked up with the device current.
hipError_t scratch_of_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" int sc_fnv1a64_noalloc_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, void* stream) {
    if (!out || (bytes && !data)) return sc::record_error(SC_EINVAL, "sc_handoff: missing hash input or output");
    if (bytes > SC_FNV_NOALLOC_MAX_BYTES || sc::fnv_workspace(bytes).bytes > kScratchBytes)
        return sc::record_error(SC_ERANGE, "sc_handoff: the hash without allocation takes at most 4 GiB "
                                           "(SC_FNV_NOALLOC_MAX_BYTES); use sc_fnv1a64_async with a workspace");
    void* ws = nullptr;
    hipError_t e = scratch_of_current_device(&ws);
    if (e != hipSuccess)
        return sc::record_error(SC_EHIP, std::string("sc_handoff hash scratch: ") + hipGetErrorString(e));
    e = sc::launch_fnv1a64(data, bytes, seed, nullptr, out, ws, static_cast<hipStream_t>(stream), 0, nullptr);
    if (e != hipSuccess) return sc::record_error(SC_EHIP, std::string("sc_handoff hash launch: ") + hipGetErrorString(e));
    return sc::record_ok();
}
