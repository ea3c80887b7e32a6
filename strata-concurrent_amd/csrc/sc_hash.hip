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
// The buffer is split into lane segments of kFnvLaneBytes bytes, a workgroup's 256 lanes covering 64 KiB, and the
// low byte is resolved in three levels: bits 0-2, 3-5 and 6-7.  A level's map of a run of bytes takes the level's bits
// at the run's start to their values at its end, given the true lower bits.  The term of a bit depends only on the
// lower start bits, so the end value of a bit in a machine started from the true lower bits, with the bit itself 0,
// is the run's term for that bit.  The top two bits of a level need no machines of their own: flipping start bit i
// (the bits below it fixed) flips bit i at every position, which changes the term of bit i + 1 by the xor over the run
// of 1 ^ y_i, y_i being bit i of ((l ^ b) mod 2^i) * 179; and y_i = l_i ^ l'_i ^ b_i, so that xor is
//     (length mod 2) ^ (term of bit i) ^ (parity of bit i over the run's bytes).
// A level for bits j .. j + k - 1 therefore runs 2^(k-2) machines (one per value of the unknown start bits
// j .. j + k - 3): two for a three-bit level (start bit j = 0, 1) and one for a two-bit level.  Each lane runs its
// segment as two halves of 128 bytes side by side: both halves' machines share the multiplies (two 8-bit machines per
// 24-bit multiply, bytes 0 and 2; the first level needs only bits 0..2, which follow l' = (l ^ b) * 3 mod 8, so four
// machines share one register a byte each), each half's map comes from its machines and its byte parities, and the
// lane's map is the second half's after the first's.  Per level: the lanes ballot their maps, each workgroup forms
// its map of the k-bit state from them, finds its start state by a look-back over the workgroups before it, each
// lane derives its start bits from the workgroup's state and the ballots by xor-prefix arithmetic, and its first
// half's map gives the bits at its midpoint.  After the third level every lane runs the full machine of both halves
// from their now complete start bytes and forms its segment's Horner sum, scaled by p^(bytes after the segment); the
// workgroups' sums are added, and a last kernel adds h_0 p^N.  All of it is one kernel that reads the input once (the
// one-pass hash, below).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "sc_handoff.h"
#include "sc_internal.hpp"

namespace sc {
namespace {

constexpr uint64_t kFnvPrime = 1099511628211ull;
constexpr uint32_t kPrimeLow = 179u;   // kFnvPrime mod 256

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

// The Horner sum of a run of bytes is sum over c of d_c p^(len - c), d_c = (l ^ b) - l.  Each power of p is written
// as four signed 16-bit digits (balanced base 2^16: p^k = sum_j digit_j 2^(16 j) mod 2^64, every digit in
// [-2^15, 2^15); the carry out of the top digit is a multiple of 2^64 and drops), so per digit j the sum
// S_j = sum_c d_c digit_j is exact in 32 bits (|d| <= 255), and two d values packed as signed 16-bit halves take one
// packed dot product (v_dot2_i32_i16) per digit.
__device__ __forceinline__ int32_t dot2(uint32_t a, uint32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b), acc, false);
}
// sum_j S_j 2^(16 j) mod 2^64.
__device__ __forceinline__ uint64_t digit_sum(int32_t s0, int32_t s1, int32_t s2, int32_t s3) {
    return uint64_t(int64_t(s0)) + (uint64_t(int64_t(s1)) << 16) + (uint64_t(int64_t(s2)) << 32) +
           (uint64_t(int64_t(s3)) << 48);
}

// Byte k of `a` in byte 0 and byte k of `b` in byte 2, zeros elsewhere (v_perm_b32: selector 0x0c gives a zero byte).
__device__ __forceinline__ uint32_t pair_byte(uint32_t a, uint32_t b, int k) {
    return __builtin_amdgcn_perm(b, a, uint32_t(k) | 0x0c00u | (uint32_t(4 + k) << 16) | 0x0c000000u);
}

// A lane's segment is summed as two halves of 128 bytes, their machines side by side in one register: the true low
// bytes of their states sit in the low bytes of the halves of `m` (half A low, half B high, each half's high byte 0).
// Per step one permute lines up a byte of each, one xor, one packed subtract gives both d values (A's in the low
// half), one 24-bit multiply and a mask the next low bytes (the masked byte A's product stays below bit 16, as in
// step_pair).  Byte c of B is weighted by p^(128 - c) and byte c of A by p^(256 - c), so each digit sum takes one
// packed dot product per step against a word holding both digits, and the one sum is the segment's Horner sum
// relative to its end (|S_j| < 128 * 2 * 255 * 2^15 < 2^31 stays exact).  About 4 VALU operations per byte, against
// 7.5 for one byte at a time.
constexpr int kPairBytes = 128, kHalfWords = kPairBytes / 4;
constexpr uint64_t prime_pow_of(uint64_t e) {
    uint64_t r = 1, b = kFnvPrime;
    for (; e; e >>= 1, b *= b)
        if (e & 1) r *= b;
    return r;
}
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
struct HalfDigits {
    uint32_t w[kPairBytes][4];   // [c][j]: digit j of p^(256 - c) in the low half, of p^(128 - c) above
};
constexpr HalfDigits half_digits() {
    HalfDigits t{};
    for (int c = 0; c < kPairBytes; ++c) {
        uint64_t va = prime_pow_of(2 * kPairBytes - c), vb = prime_pow_of(kPairBytes - c);
        for (int j = 0; j < 4; ++j) {
            const int32_t da = int32_t(int16_t(uint16_t(va & 0xFFFFu))), db = int32_t(int16_t(uint16_t(vb & 0xFFFFu)));
            t.w[c][j] = (uint32_t(da) & 0xFFFFu) | (uint32_t(db) << 16);
            va = (va - uint64_t(int64_t(da))) >> 16;
            vb = (vb - uint64_t(int64_t(db))) >> 16;
        }
    }
    return t;
}
constexpr HalfDigits kHalfDigits = half_digits();
// `m`: the true low byte at the segment's start in the low half, at its midpoint in the high half.
__device__ __forceinline__ uint64_t halves_sum(const uint32_t (&w)[kFnvLaneBytes / 4], uint32_t m) {
    int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
    for (int c = 0; c < kPairBytes; ++c) {
        const uint32_t x = m ^ pair_byte(w[c >> 2], w[kHalfWords + (c >> 2)], c & 3);
        const uint32_t d = pk_sub(x, m);
        m = __umul24(x, kPrimeLow) & 0x00FF00FFu;
        s0 = dot2(d, kHalfDigits.w[c][0], s0);
        s1 = dot2(d, kHalfDigits.w[c][1], s1);
        s2 = dot2(d, kHalfDigits.w[c][2], s2);
        s3 = dot2(d, kHalfDigits.w[c][3], s3);
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

// The ballots of one level, per wave: the bits of the lanes' maps of the level (below) - the term of the lowest
// unresolved bit j (T), of bit j + 1 for either start value a of bit j (U_a), and, in a three-bit level, of bit j + 2
// for each start pair (a, c) of bits j, j + 1 (W_ac).
constexpr int kMaxLevelWords = 7;   // T, U0, U1, W00, W01, W10, W11
template <int kBits>
constexpr int level_words() { return kBits == 3 ? 7 : 3; }

// The lanes' true start bits of one wave, as masks, from `st` (bit j in bit 0, j + 1 in bit 1, j + 2 in bit 2) at
// the wave's first segment; `st` advances past the wave.  Each lane's term for a bit is chosen by its own true lower
// bits, and the bit at a lane is the wave's incoming bit xor the terms of the lanes before it.
template <int kBits>
__device__ __forceinline__ void wave_masks(const uint64_t (&wd)[kMaxLevelWords], uint32_t& st, uint64_t (&m)[3]) {
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

// The first level only needs bits 0..2 of the state, which follow l' = ((l ^ b) * 3) mod 8 (179 = 3 mod 8): four
// such machines share one register, one per byte (a 3-bit state times 3 stays below 2^8, so nothing carries across
// bytes; the product's bits above 2 are masked by the next step).
__device__ __forceinline__ uint32_t step_low3(uint32_t x, uint32_t b4) {
    const uint32_t y = (x ^ b4) & 0x07070707u;
    return y + (y << 1);
}

// A run's map of a level from its machines' end states.  Three-bit level for bits j..j+2: e0 and e1 ended the machines
// started from the true lower bits with bit j = 0 and 1 (bits j + 1, j + 2 = 0); two-bit level for bits j, j + 1: e
// ended the one machine started with both 0.  The bits the machines do not give follow from the term of the bit below,
// the parity of that bit over the run's bytes (bit i of `par`, the xor of the bytes) and the run's length (`odd`).
template <int j>
__device__ __forceinline__ uint32_t map3_of(uint32_t e0, uint32_t e1, uint32_t par, uint32_t odd) {
    const uint32_t t = (e0 >> j) & 1u, v0 = (e0 >> (j + 1)) & 1u, v1 = (e1 >> (j + 1)) & 1u;
    const uint32_t w00 = (e0 >> (j + 2)) & 1u, w10 = (e1 >> (j + 2)) & 1u, q = ((par >> (j + 1)) & 1u) ^ odd;
    return t | (v0 << 1) | (v1 << 2) | (w00 << 3) | ((w00 ^ v0 ^ q) << 4) | (w10 << 5) | ((w10 ^ v1 ^ q) << 6);
}
template <int j>
__device__ __forceinline__ uint32_t map2_of(uint32_t e, uint32_t par, uint32_t odd) {
    const uint32_t t = (e >> j) & 1u, v0 = (e >> (j + 1)) & 1u;
    return t | (v0 << 1) | ((v0 ^ t ^ ((par >> j) & 1u) ^ odd) << 2);
}

// The same maps of a partial or unaligned segment (whole segments run from registers, below), a byte at a time from
// memory; `low` holds the true bits below j at the segment's start.
template <int j>
__device__ __forceinline__ uint32_t map3_bytes(const uint8_t* p, uint64_t n, uint32_t low) {
    uint32_t x = low | ((low | (1u << j)) << 16), par = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t b = p[i];
        par ^= b;
        x = step_pair(x, b * 0x10001u);
    }
    return map3_of<j>(x & 0xFFFFu, x >> 16, par, uint32_t(n & 1u));
}
template <int j>
__device__ __forceinline__ uint32_t map2_bytes(const uint8_t* p, uint64_t n, uint32_t low) {
    uint32_t x = low, par = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t b = p[i];
        par ^= b;
        x = step_pair(x, b * 0x10001u);
    }
    return map2_of<j>(x, par, uint32_t(n & 1u));
}

// A workgroup's map of a level's state: (a, c, e) = (bit j, j + 1, j + 2) at its first segment goes to
// (a ^ t, c ^ v_a, e ^ w_ac) at the next workgroup's first segment; the map is a byte (bit 0 t, bits 1-2 v_0 v_1,
// bits 3-6 w_00 w_01 w_10 w_11; a two-bit level has no e and no w), 0 being the identity.  Maps compose as
// (g after f): t = t_f ^ t_g, v_a = v_a(f) ^ v_(a ^ t_f)(g), w_ac = w_ac(f) ^ w_(a ^ t_f, c ^ v_a(f))(g).
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

// The state the hash starts from: the launch's seed, or the running hash at `seed_dev` when the input continues an
// earlier one (read by every kernel that needs it, so one stream can chain pieces without a host round trip).
__device__ __forceinline__ uint64_t start_state(uint64_t seed, const uint64_t* seed_dev) {
    return seed_dev ? *seed_dev : seed;
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(uint32_t(v), m), hi = __shfl_xor(uint32_t(v >> 32), m);
    return (uint64_t(hi) << 32) | lo;
}

// One partial or unaligned segment's Horner sum, scaled by p^(bytes after it), from the true low byte `l` at its
// start, a byte at a time.
__device__ __forceinline__ uint64_t segment_sum(const uint8_t* p, uint64_t n, uint64_t begin, uint32_t l) {
    const uint64_t len = n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
    uint64_t acc = 0;
    for (uint64_t i = 0; i < len; ++i) step_full(p[i], l, acc);
    return acc * pow_prime(n - begin - len);
}

// h = seed * p^n + the sum of the workgroups' sums (mod 2^64; the order of the additions does not matter), `acc` being
// that sum, or null for an empty input.  `fault` is the launch's fault word (null for an empty input, which has no
// waits): a wait that ran out (kFaultWait) or carries that do not match the input (kFaultCarry) make h unusable, and the
// launch says so at `fault_out` - the fault word, 0 for none, or, for a chained piece (`sticky`), or'ed into what the
// earlier pieces left there, so a chain reports a fault of any of its pieces.  With `verdict`, also 1 there when h
// equals `expected` and the launch has no fault, else 0: a later kernel on the stream can act on the check without a
// host round trip.
__global__ void fnv_finish_kernel(const uint64_t* acc, uint64_t seed, const uint64_t* seed_dev, uint64_t n, uint64_t* out,
                                  uint32_t* fault_out, bool sticky, uint64_t expected, uint32_t* verdict,
                                  const uint32_t* fault, const uint8_t* tail, uint32_t tail_len) {
    uint64_t h = start_state(seed, seed_dev) * pow_prime(n) + (acc ? acc[0] : 0u);
    // the mapped hash leaves the payload's last partial lane segment (under 256 bytes, whole 16-byte chunks at a 16-byte
    // aligned address) to this thread: its chunks are loaded at once, then hashed a byte at a time from registers
    // (a loop of byte loads took 14 us, each load waiting on the one before)
    if (tail_len) {
        u32x4 c[kFnvLaneBytes / 16];
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 16; ++k)
            c[k] = uint32_t(k) * 16u < tail_len ? *(const gu32x4*) (tail + 16 * k) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 16; ++k) {
            if (uint32_t(k) * 16u >= tail_len) break;
            const uint32_t word[4] = {c[k].x, c[k].y, c[k].z, c[k].w};
#pragma unroll
            for (int b = 0; b < 16; ++b)
                if (uint32_t(k) * 16u + uint32_t(b) < tail_len) h = (h ^ ((word[b / 4] >> (8 * (b % 4))) & 0xFFu)) * kFnvPrime;
        }
    }
    const uint32_t bad = fault ? fault[0] : 0u;   // kFaultWait and / or kFaultCarry
    out[0] = h;
    if (fault_out) fault_out[0] = sticky ? (fault_out[0] | bad) : bad;
    if (verdict) verdict[0] = h == expected && !bad ? 1u : 0u;
}

// ---- the one-pass hash ---------------------------------------------------------------------------------------------
// One kernel reads the input once: each lane keeps its 256-byte segment in registers through the three levels of the
// low byte and the Horner sums.  A level's workgroup start state comes from a decoupled look-back rather than a scan
// kernel: workgroups take their index from a ticket counter in the order they start, publish their map of the level's
// state as soon as they have it and their end state once they know their start, and a workgroup finds its start by
// reading the words of the 64 workgroups before it at once and composing maps back to the nearest end state.  A
// workgroup waits only on lower tickets, held by workgroups that are running or done, so every wait ends; each wait is
// also bounded (kSpinLimit reads), after which the launch records a fault that fails the verdict and the workgroup
// publishes an end state anyway, so no other workgroup waits on it.
// The lane within its wave, from the exec-independent lane count (two VALU operations): used where keeping threadIdx.x
// live across the kernel would spill it and reload it from scratch, a memory round trip each time.
__device__ __forceinline__ int lane_id() { return int(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u))); }
constexpr uint32_t kHasMap = 1u << 8, kHasState = 1u << 9;   // a status word: 0, kHasMap | map, kHasState | state
// Sleeps of 64 x 64 cycles before a look-back's first read of its window (the mapped kernel's last level writes its
// gathered payload instead): 3.3 GB hashed in 1.77 ms with two, 1.79 ms with none
constexpr int kFirstSleeps = 2, kFirstSleepsMapped = 0;
constexpr uint32_t kSpinLimit = 1u << 16;   // reads of one window, about 0.2 s (sc_fnv1a64_set_spin_limit)
// A bound the host sets only to test failure handling: every look-back of a workgroup after the first runs out at
// once, so any input of more than one workgroup (64 KiB) ends with the fault set, deterministically.
constexpr uint32_t kForceFault = 0xFFFFFFFFu;

// The launch's fault word: 0, or the or of kFaultWait (a look-back wait ran out) and kFaultCarry (a workgroup of a check
// given carries did not end with the carry after it: the input or its carries are not what was hashed).
constexpr uint32_t kFaultWait = SC_FNV_FAULT_WAIT, kFaultCarry = SC_FNV_FAULT_CARRY;
__device__ __forceinline__ void flag_fault(uint32_t* fault, uint32_t v) {
    __hip_atomic_fetch_or(fault, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish(uint32_t* word, uint32_t v) {
    __hip_atomic_store(word, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t peek(uint32_t* word) {
    return __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup g's start state at one level, run by one whole wave (the result is wave-uniform); publishes g's map
// before the look-back and its end state after.  `init` is the state before workgroup 0.  Lane l reads the word of
// workgroup top - l.  The maps of lanes 0..l compose in one inclusive scan across the wave (six shuffle steps), so
// resolving a window costs the same wherever its nearest end state lies.
template <int kBits>
__device__ __forceinline__ uint32_t look_back(uint32_t* status, uint64_t g, uint32_t map, uint32_t init, uint32_t* fault,
                                              uint32_t spin_limit, int first_sleeps) {
    const int lane = lane_id();
    if (g == 0) {
        if (lane == 0) publish(status, kHasState | apply<kBits>(map, init));
        return init;
    }
    if (spin_limit == kForceFault) {   // the failure-handling tests' forced fault (never set otherwise)
        if (lane == 0) {
            flag_fault(fault, kFaultWait);
            publish(status + g, kHasState | apply<kBits>(map, 0u));
        }
        return 0u;
    }
    // the caller has published g's map.  The workgroups just before g publish theirs a few microseconds after g on
    // average (their work varies with what shares their SIMDs), so a read right away would mostly find the window
    // incomplete and cost a round trip and a sleep anyway
    for (int i = 0; i < first_sleeps; ++i) __builtin_amdgcn_s_sleep(64);
    uint32_t acc = 0;                  // the maps of the workgroups from above the window up to g, composed
    int64_t top = int64_t(g) - 1;      // the window is workgroups top, top - 1, ...; before workgroup 0 stands `init`
    uint32_t spins = 0;
    for (;;) {
        const int64_t h = top - lane;
        const uint32_t word = h >= 0 ? peek(status + h) : (kHasState | init);
        const uint64_t have_state = __ballot((word & kHasState) != 0u);
        const uint64_t ready = __ballot((word & (kHasMap | kHasState)) != 0u);
        const int first = have_state ? __builtin_ctzll(have_state) : 64;   // the lane of the nearest end state
        const uint64_t need = first == 64 ? ~0ull : (1ull << first) - 1ull;
        if ((ready & need) != need) {   // a workgroup between g and that end state has not published its map yet
            if (++spins > spin_limit) {   // never in a correct launch; successors still get an end state
                if (lane == 0) {
                    flag_fault(fault, kFaultWait);
                    publish(status + g, kHasState | apply<kBits>(map, 0u));
                }
                return 0u;
            }
            // a long sleep (64 x 64 cycles, about 1.7 us) leaves the SIMD's issue slots to the other waves' level work:
            // sleeps of 16 or 32 between reads measured slower (1.77-1.78 against 1.76 ms for 3.3 GB; the fused
            // capture 2.42-2.47 against 2.37 ms), and so did 1 in the earlier form of the levels
            __builtin_amdgcn_s_sleep(64);
            continue;
        }
        // x_l = map_0 o map_1 o ... o map_l (map_l applied first); the lanes from `first` on are not used
        uint32_t x = word & 0xFFu;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t lower = uint32_t(__shfl_up(int(x), d));
            if (lane >= d) x = compose<kBits>(lower, x);
        }
        if (first < 64) {
            uint32_t st = uint32_t(__builtin_amdgcn_readlane(int(word), first)) & 0xFFu;
            if (first > 0) st = apply<kBits>(uint32_t(__builtin_amdgcn_readlane(int(x), first - 1)), st);
            st = apply<kBits>(acc, st);
            if (lane == 0) publish(status + g, kHasState | apply<kBits>(map, st));
            return st;
        }
        acc = compose<kBits>(acc, uint32_t(__builtin_amdgcn_readlane(int(x), 63)));   // all maps: read the window before
        top -= 64;
        spins = 0;
    }
}

struct LevelLds {
    uint64_t bw[kFnvThreads / 64][kMaxLevelWords];
    uint32_t map[kFnvThreads / 64];
    uint32_t state;
};

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    return uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v))))) |
           (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v >> 32))))) << 32);
}

// One level (bits j .. j + kBits - 1) once every lane has its map of the level (`lane_map`, the identity 0 for a lane
// past the input): ballots the maps, forms and publishes the workgroup's map, runs `during` in every wave (work that
// does not need the level's result, done while the look-back waits), looks back for the workgroup's start state after
// `first_sleeps` sleeps of 64 x 64 cycles, and returns this lane's start bits of the level (bit 0 upward).
template <int kBits, typename During>
__device__ __forceinline__ uint32_t resolve_level(int wave, uint32_t lane_map, uint64_t g, uint32_t* status, uint32_t init,
                                                  uint32_t* fault, uint32_t spin_limit, LevelLds& L, int first_sleeps,
                                                  During during, int j, const uint8_t* carry_in, uint64_t carry_count,
                                                  uint32_t& end_bits) {
    uint64_t bw[kMaxLevelWords] = {};
#pragma unroll
    for (int i = 0; i < level_words<kBits>(); ++i) bw[i] = __ballot((lane_map >> i) & 1u);
    uint32_t wmap = 0;
#pragma unroll
    for (uint32_t in = 0; in < (1u << (kBits - 1)); ++in) {
        const uint32_t a = in & 1u, c = (in >> 1) & 1u;
        uint32_t st = in;
        uint64_t m[3];
        wave_masks<kBits>(bw, st, m);
        if (in == 0) wmap |= st & 1u;
        if (c == 0) wmap |= ((st >> 1) & 1u) << (1 + a);
        if constexpr (kBits == 3) wmap |= ((st >> 2) & 1u) << (3 + 2 * a + c);
    }
    const int lane = lane_id();
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < level_words<kBits>(); ++i) L.bw[wave][i] = bw[i];
        L.map[wave] = wmap;
    }
    __syncthreads();
    uint32_t sum = L.map[0];
    if (wave == 0) {
        for (int k = 1; k < kFnvThreads / 64; ++k) sum = compose<kBits>(L.map[k], sum);
        sum = __builtin_amdgcn_readfirstlane(sum);
        if (lane == 0 && g > 0 && !carry_in) publish(status + g, kHasMap | sum);
    }
    during();
    if (wave == 0) {
        constexpr uint32_t kMask = (1u << kBits) - 1u;
        uint32_t st;
        if (carry_in) {   // the start is the carry before the workgroup, checked by the one after it
            st = g == 0 ? init : (uint32_t(carry_in[g - 1]) >> j) & kMask;
            if (g < carry_count && apply<kBits>(sum, st) != ((uint32_t(carry_in[g]) >> j) & kMask) && lane == 0)
                flag_fault(fault, kFaultCarry);
        } else {
            st = look_back<kBits>(status, g, sum, init, fault, spin_limit, first_sleeps);
        }
        if (lane == 0) L.state = st;
        end_bits |= apply<kBits>(sum, st) << j;
    }
    __syncthreads();
    uint32_t st = __builtin_amdgcn_readfirstlane(L.state);
    uint64_t m[3] = {0, 0, 0};
#pragma unroll
    for (int k = 0; k < kFnvThreads / 64; ++k) {
        if (k > wave) break;
        uint64_t wd[kMaxLevelWords] = {};
#pragma unroll
        for (int i = 0; i < level_words<kBits>(); ++i) wd[i] = uniform64(L.bw[k][i]);
        wave_masks<kBits>(wd, st, m);
    }
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < kBits; ++i) bits |= (uint32_t(m[i] >> lane) & 1u) << i;
    __syncthreads();   // the next level rewrites L
    return bits;
}

// The levels of a whole segment held in registers, run as its two halves of kPairBytes bytes side by side (half A the
// first, half B the second): each returns half A's map of the level in its low 16 bits and half B's above.  `par` holds
// the xor of half A's bytes in byte 0 and of half B's in byte 2, `low` the true bits below the level at half A's start
// in byte 0 and at half B's in byte 2.
__device__ __forceinline__ uint32_t half_parities(const uint32_t (&w)[kFnvLaneBytes / 4]) {
    uint32_t a = 0, b = 0;
#pragma unroll
    for (int k = 0; k < kHalfWords; ++k) {
        a ^= w[k];
        b ^= w[kHalfWords + k];
    }
    a ^= a >> 16;
    a ^= a >> 8;
    b ^= b >> 16;
    b ^= b >> 8;
    return (a & 0xFFu) | ((b & 0xFFu) << 16);
}
// Byte k of `a` in bytes 0 and 1, byte k of `b` in bytes 2 and 3.
__device__ __forceinline__ uint32_t pair_byte2(uint32_t a, uint32_t b, int k) {
    return __builtin_amdgcn_perm(b, a, uint32_t(k) | (uint32_t(k) << 8) | (uint32_t(4 + k) << 16) | (uint32_t(4 + k) << 24));
}
// Bits 0-2: four 3-bit machines, half A's started from bit 0 = 0 and 1 in bytes 0 and 1, half B's in bytes 2 and 3.
__device__ __forceinline__ uint32_t level1_maps(const uint32_t (&w)[kFnvLaneBytes / 4], uint32_t par) {
    uint32_t x = 0x01000100u;
#pragma unroll
    for (int k = 0; k < kHalfWords; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) x = step_low3(x, pair_byte2(w[k], w[kHalfWords + k], i));
    return map3_of<0>(x & 0xFFu, (x >> 8) & 0xFFu, par, 0u) |
           (map3_of<0>((x >> 16) & 0xFFu, x >> 24, par >> 16, 0u) << 16);
}
// Bits 3-5: half A's machines in byte 0 of r0 (start bit 3 = 0) and r1 (= 1), half B's in their byte 2.
__device__ __forceinline__ uint32_t level2_maps(const uint32_t (&w)[kFnvLaneBytes / 4], uint32_t low, uint32_t par) {
    uint32_t r0 = low, r1 = low | 0x00080008u;
#pragma unroll
    for (int k = 0; k < kHalfWords; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t bb = pair_byte(w[k], w[kHalfWords + k], i);
            r0 = step_pair(r0, bb);
            r1 = step_pair(r1, bb);
        }
    return map3_of<3>(r0 & 0xFFu, r1 & 0xFFu, par, 0u) |
           (map3_of<3>((r0 >> 16) & 0xFFu, (r1 >> 16) & 0xFFu, par >> 16, 0u) << 16);
}
// Bits 6-7: one machine per half, half A's in byte 0, half B's in byte 2.
__device__ __forceinline__ uint32_t level3_maps(const uint32_t (&w)[kFnvLaneBytes / 4], uint32_t low, uint32_t par) {
    uint32_t r = low;
#pragma unroll
    for (int k = 0; k < kHalfWords; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) r = step_pair(r, pair_byte(w[k], w[kHalfWords + k], i));
    return map2_of<6>(r & 0xFFu, par, 0u) | (map2_of<6>((r >> 16) & 0xFFu, par >> 16, 0u) << 16);
}

// ---- the gather fused with the hash -------------------------------------------------------------------------------
// A lane of the mapped hash gathers its segment of the payload from the extents' sources into its registers, stores it
// into the payload and hashes it from the registers, so a capture's payload is written and hashed in one read of the
// slot.  Most segments lie inside one extent and one contiguous source (a 256-byte segment of a 4 KiB page); the
// others, at extent and page boundaries, take their chunks one at a time.
__device__ __forceinline__ void put16(uint8_t* p, u32x4 v) { *(gu32x4*) p = v; }

// A run of the payload from payload offset `o`: bytes [o, end) come from one contiguous source `src` (a copy extent, a
// page of a pages extent, the payload itself for a self extent or an unplaced page) or are zeros (src null); `store`
// says whether the gather writes them (self bytes stay as the payload holds them).
struct Run {
    const uint8_t* src;
    uint64_t end;
    bool store;
};
__device__ __forceinline__ Run run_at(const HashExtent& x, uint64_t o, uint8_t* dst_o) {
    Run r{dst_o, x.end, false};
    if (x.kind == kExtCopy) {
        r.src = x.src + (o - x.off);
        r.store = true;
    } else if (x.kind == kExtZero) {
        r.src = nullptr;
        r.store = true;
    } else if (x.kind == kExtPages) {
        const uint32_t q = uint32_t((o - x.off) >> 4), page = q / x.page_chunks, ch = q - page * x.page_chunks;
        const uint64_t page_end = x.off + (uint64_t(page) + 1u) * x.page_chunks * 16u;
        r.end = page_end < x.end ? page_end : x.end;
        const int64_t phys = x.table ? int64_t(x.table[page]) : int64_t(page);
        if (phys >= 0 && phys < x.ld) {
            r.src = x.src + (uint64_t(phys) * x.page_chunks + ch) * 16u;
            r.store = true;
        }
    }
    return r;
}

__device__ u32x4 g_hash_zero_chunk;   // read for zero runs, so every chunk takes the same load

// A lane's 256-byte segment from run a (its first ka chunks) and run b (the rest): 16 loads issued at once, a zero run's
// from one zero chunk.
__device__ __forceinline__ void load_runs(const Run& a, const Run& b, uint32_t ka, uint32_t (&w)[kFnvLaneBytes / 4]) {
    const uint8_t* za = a.src ? a.src : reinterpret_cast<const uint8_t*>(&g_hash_zero_chunk);
    const uint8_t* zb = b.src ? b.src : reinterpret_cast<const uint8_t*>(&g_hash_zero_chunk);
    const uint64_t sa = a.src ? 16u : 0u, sb = b.src ? 16u : 0u;
#pragma unroll
    for (int k = 0; k < kFnvLaneBytes / 16; ++k) {
        const bool in_a = uint32_t(k) < ka;
        const uint8_t* q = in_a ? za + sa * uint64_t(k) : zb + sb * uint64_t(k - int(ka));
        const u32x4 v = *(const gu32x4*) q;
        w[4 * k] = v.x;
        w[4 * k + 1] = v.y;
        w[4 * k + 2] = v.z;
        w[4 * k + 3] = v.w;
    }
}

// A lane's whole segment inside extent X, where X holds the lane's whole wave and is wave-uniform (its fields stay in
// scalar registers and no lane reads the extent table): a copy or the payload's own bytes in one run from one base, as
// the plain hash loads, zeros without a load, pages in one run or two (across one page boundary).  False for a segment
// over three pages or more (pages under 256 bytes), which the caller gathers chunk by chunk.
__device__ __forceinline__ bool gather_in_extent(const HashExtent& X, uint8_t* base, uint64_t begin,
                                                 uint32_t (&w)[kFnvLaneBytes / 4]) {
    if (X.kind == kExtCopy) {
        load_segment(X.src + (begin - X.off), w);
        return true;
    }
    if (X.kind == kExtSelf) {
        load_segment(base + begin, w);
        return true;
    }
    if (X.kind == kExtZero) {
#pragma unroll
        for (int i = 0; i < kFnvLaneBytes / 4; ++i) w[i] = 0u;
        return true;
    }
    const uint64_t seg_end = begin + kFnvLaneBytes;
    const Run a = run_at(X, begin, base + begin);
    Run b = a;
    uint32_t ka = kFnvLaneBytes / 16;
    if (a.end < seg_end) {
        ka = uint32_t((a.end - begin) >> 4);
        b = run_at(X, a.end, base + a.end);
        if (b.end < seg_end) return false;
    }
    load_runs(a, b, ka, w);
    return true;
}

// The lane's segment [begin, begin + len) gathered into w, walking the extent table from the workgroup's first extent
// (a wave over an extent boundary, a workgroup over three extents or more, the payload's last wave).  A segment in one
// run or two issues its 16 loads at once from one or two bases; a segment over three runs or more, and the payload's
// last partial segment, goes chunk by chunk into the payload, which the lane then reads back (its own stores, after a
// fence).  The payload is written by store_wave below (the last partial segment only here).
__device__ __forceinline__ void gather_segment(const HashMapArgs& m, uint8_t* base, uint32_t e_group, uint64_t begin,
                                               uint64_t len, uint32_t (&w)[kFnvLaneBytes / 4]) {
    uint32_t e = e_group;
    while (m.ext[e].end <= begin) ++e;
    HashExtent x = m.ext[e];
    uint8_t* dst = base + begin;   // `base` + o addresses payload byte o of this workgroup's segment
    const uint64_t seg_end = begin + len;
    const Run a = run_at(x, begin, dst);
    if (len == kFnvLaneBytes) {
        Run b = a;
        uint32_t ka = kFnvLaneBytes / 16;   // chunks from run a
        bool two = a.end >= seg_end;
        if (!two) {
            ka = uint32_t((a.end - begin) >> 4);
            if (a.end >= x.end) x = m.ext[++e];
            b = run_at(x, a.end, dst + 16u * ka);
            two = b.end >= seg_end;
        }
        if (two) {
            load_runs(a, b, ka, w);
            return;
        }
        // three runs or more: walk from the workgroup's first extent again (the look-ahead above may have moved past
        // the extent holding `begin`)
        e = e_group;
        while (m.ext[e].end <= begin) ++e;
        x = m.ext[e];
    }
#pragma unroll 1
    for (uint64_t o = begin; o < seg_end;) {
        while (x.end <= o) x = m.ext[++e];
        const Run r = run_at(x, o, base + o);
        const uint64_t o0 = o, end = r.end < seg_end ? r.end : seg_end;
        for (; o < end; o += 16)
            if (r.store && m.store) put16(base + o, r.src ? *(const gu32x4*) (r.src + (o - o0)) : u32x4{0u, 0u, 0u, 0u});
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");   // the lane's stores complete before its reads
    if (len == kFnvLaneBytes) load_segment(dst, w);
}

// The wave's 16 KiB of gathered payload into the payload with coalesced stores: each lane holds 256 contiguous bytes,
// so stores straight from the registers would put 64 lines under every store instruction (measured: the fused kernel
// 3.3-3.7 ms with them against 2.3 ms without any store, and 8.2 ms with non-temporal ones).  Four passes of 4 KiB: a
// quarter of the lanes write their segments into the wave's LDS rows (17 chunks apart, so the 16 writers of a
// 16-byte column fall in different banks), then every lane reads back 16 bytes per 1 KiB and stores it, 1 KiB
// contiguous per instruction, non-temporal.  Bytes at or past `limit` (the part hashed in the kernel) are not written
// here.
constexpr int kXposeRow = kFnvLaneBytes / 16 + 1;   // chunks per LDS row: a lane's 16 and one of padding
__device__ __forceinline__ void store_wave(u32x4 (&lds)[16 * kXposeRow], const uint32_t (&w)[kFnvLaneBytes / 4],
                                           uint8_t* dst, uint64_t wave_begin, uint64_t limit, int lane) {
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        if ((lane >> 4) == pass) {
            const int row = (lane & 15) * kXposeRow;
#pragma unroll
            for (int k = 0; k < kFnvLaneBytes / 16; ++k)
                lds[row + k] = u32x4{w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int c = r * 64 + lane;   // chunk of this pass's 4 KiB: lane c / 16's chunk c % 16
            const u32x4 v = lds[(c >> 4) * kXposeRow + (c & 15)];
            const uint64_t o = wave_begin + uint64_t(pass) * 4096u + uint64_t(c) * 16u;
            // non-temporal: the fused 128K capture 2.75 against 2.79-2.81 ms with regular stores
            if (o < limit) __builtin_nontemporal_store(v, (gu32x4*) (dst + o));
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// status: three arrays of `stride` words (one per level); ctl: [0] the ticket counter, [1] the fault word, [2..3] the
// sum of the workgroups' sums (each workgroup adds its own with one 64-bit atomic).  kMapped: the payload is gathered
// through `map` (stored, and hashed up to `n`, its whole lane segments) instead of read from `data`.  Not kMapped,
// with `map.seg` set: the payload is read where its segments hold it (`data` unused).
// Five waves per SIMD (the mapped instance would take 110 VGPRs and four; held to 96 it spills 5 words and runs the
// fused 128K capture in 2.78-2.85 ms against 2.82 at four waves).  Every value the gather keeps live past its look-ahead
// costs spills here: an extra extent index held across it spilled 35 words and took the capture to 3.03 ms.
template <bool kMapped>
__global__ void __launch_bounds__(kFnvThreads) __attribute__((amdgpu_waves_per_eu(5, 8))) fnv_onepass_kernel(const uint8_t* data, uint64_t n, bool aligned,
                                                                uint64_t seed, const uint64_t* seed_dev,
                                                                uint32_t* status, uint64_t stride, uint32_t* ctl,
                                                                uint32_t spin_limit, HashMapArgs map,
                                                                FnvCarries carries, uint64_t carry_count) {
    __shared__ LevelLds L;
    __shared__ uint32_t s_ticket;
    __shared__ uint64_t s_sum[kFnvThreads / 64];
    __shared__ u32x4 s_xpose[kMapped ? kFnvThreads / 64 : 1][16 * kXposeRow];
    if (threadIdx.x == 0) s_ticket = atomicAdd(ctl, 1u);
    __syncthreads();
    const uint64_t g = uint32_t(__builtin_amdgcn_readfirstlane(int(s_ticket)));
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t begin = (g * kFnvThreads + threadIdx.x) * kFnvLaneBytes;
    const bool live = begin < n;
    const uint64_t len = !live ? 0 : n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
    // the mapped instance hashes whole lane segments only (its launch passes n rounded down to them, the closing kernel
    // takes the rest), so every live lane is whole there and the byte-at-a-time forms below drop out of it
    const bool full = kMapped ? live : aligned && len == kFnvLaneBytes;
    const uint8_t* p = data + begin;
    if (!kMapped && map.seg) {
        // a payload read where its segments hold it: this workgroup's 64 KiB lie in segment k
        const uint64_t k = g * uint64_t(kFnvGroupBytes) / map.seg_bytes;
        p = map.seg[k] + (begin - k * map.seg_bytes);
    }
    uint32_t* fault = ctl + 1;
    uint32_t w[kFnvLaneBytes / 4] = {};
    uint8_t* base = nullptr;   // mapped: `base` + o addresses payload byte o in the segment holding this workgroup's bytes
    if constexpr (kMapped) {
        // the workgroup's part of the map in one round trip: its 14 words read together through the constant address
        // space (scalar loads; the map does not change during the launch) and held from here, rather than each field
        // loaded in the branch that first needs it, one round trip after another
        typedef const __attribute__((address_space(4))) uint64_t ConstWord;
        const ConstWord* q = (const ConstWord*) (map.grp + g);
        uint64_t h[14];
#pragma unroll
        for (int i = 0; i < 14; ++i) h[i] = q[i];
        asm volatile("" ::"s"(h[0]), "s"(h[1]), "s"(h[2]), "s"(h[3]), "s"(h[4]), "s"(h[5]), "s"(h[6]), "s"(h[7]),
                     "s"(h[8]), "s"(h[9]), "s"(h[10]), "s"(h[11]), "s"(h[12]), "s"(h[13]));
        HashGroup hg;
        static_assert(offsetof(HashGroup, pad) == 14 * 8, "the words read are the group's fields");
        __builtin_memcpy(&hg, h, sizeof(h));
        base = hg.base;
        if (begin < map.n_total) {
            const uint64_t wave_lo = (g * kFnvThreads + uint64_t(wave) * 64) * kFnvLaneBytes;
            const uint64_t wave_hi = wave_lo + 64u * kFnvLaneBytes;
            bool done = false;
            if (hg.two && wave_hi <= map.n_total) {   // every lane of the wave whole, inside one of the two extents
                if (wave_hi <= hg.x[0].end)
                    done = gather_in_extent(hg.x[0], base, begin, w);
                else if (wave_lo >= hg.x[0].end)
                    done = gather_in_extent(hg.x[1], base, begin, w);
            }
            if (!done) {
                const uint64_t left = map.n_total - begin;
                gather_segment(map, base, hg.first, begin, left < kFnvLaneBytes ? left : kFnvLaneBytes, w);
            }
        }
    } else if (full) {
        load_segment(p, w);
    }
    const uint64_t h0 = start_state(seed, seed_dev);

    // the three levels: every lane's map of the level (a whole segment from its two halves in registers, a partial or
    // unaligned one a byte at a time), then the workgroup's look-back.  `s` gathers the true start bits at the lane's
    // segment, `sb` at its midpoint (its first half's map applied to the level's start bits)
    const uint32_t par = full ? half_parities(w) : 0u;
    uint32_t halves = 0, lane_map = 0;
    if (full) {
        halves = level1_maps(w, par);
        lane_map = compose<3>(halves >> 16, halves & 0xFFFFu);
    } else if (live) {
        lane_map = map3_bytes<0>(p, len, 0u);
    }
    // the gathered payload is written while the last look-back waits: 2.05 ms for the 128K capture + hash, against
    // 2.22 ms while the first waits, 2.15 ms while the second waits and 2.18 ms after the last (stores issued earlier
    // meet the next workgroups' gathers)
    const auto store_gathered = [&] {
        if constexpr (kMapped)
            if (map.store)
                store_wave(s_xpose[wave], w, base, (g * kFnvThreads + uint64_t(wave) * 64) * kFnvLaneBytes, n, lane);
    };
    uint32_t end_bits = 0;   // wave 0: the workgroup's end state, level by level (its carry)
    uint32_t s = resolve_level<3>(wave, lane_map, g, status, uint32_t(h0) & 7u, fault, spin_limit, L,
                                  kFirstSleeps, [] {}, 0, carries.in, carry_count, end_bits);
    uint32_t sb = apply<3>(halves & 0xFFFFu, s);

    lane_map = 0;
    if (full) {
        halves = level2_maps(w, s | (sb << 16), par);
        lane_map = compose<3>(halves >> 16, halves & 0xFFFFu);
    } else if (live) {
        lane_map = map3_bytes<3>(p, len, s);
    }
    uint32_t st = resolve_level<3>(wave, lane_map, g, status + stride, uint32_t(h0 >> 3) & 7u, fault, spin_limit, L,
                                   kFirstSleeps, [] {}, 3, carries.in, carry_count, end_bits);
    s |= st << 3;
    sb |= apply<3>(halves & 0xFFFFu, st) << 3;

    lane_map = 0;
    if (full) {
        halves = level3_maps(w, s | (sb << 16), par);
        lane_map = compose<2>(halves >> 16, halves & 0xFFFFu);
    } else if (live) {
        lane_map = map2_bytes<6>(p, len, s);
    }
    st = resolve_level<2>(wave, lane_map, g, status + 2 * stride, uint32_t(h0 >> 6) & 3u, fault, spin_limit, L,
                          kMapped ? kFirstSleepsMapped : kFirstSleeps, store_gathered, 6, carries.in, carry_count,
                          end_bits);
    if (carries.out && threadIdx.x == 0 && g < carry_count) carries.out[g] = uint8_t(end_bits);
    s |= st << 6;
    sb |= apply<2>(halves & 0xFFFFu, st) << 6;

    // the Horner sums, from the true low bytes at the segment's start and midpoint
    uint64_t acc = 0;
    if (full) {
        // p^(n - r), r the end of the wave's last segment: wave-uniform.  p has order dividing 2^62 modulo 2^64, so
        // the exponent is taken modulo 2^62 (r passes n in the buffer's last wave)
        const uint64_t wave_end = ((g * kFnvThreads) + uint64_t(wave) * 64 + 64) * kFnvLaneBytes;
        const uint64_t wave_pow = pow_prime((n - wave_end) & ((uint64_t(1) << 62) - 1));
        acc = halves_sum(w, s | (sb << 16)) * kLanePow.v[lane] * wave_pow;
    } else if (live) {
        acc = segment_sum(p, n, begin, s);
    }
    for (int m = 32; m > 0; m >>= 1) acc += shfl_xor64(acc, m);
    if (lane == 0) s_sum[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t sum = 0;
#pragma unroll
        for (int k = 0; k < kFnvThreads / 64; ++k) sum += s_sum[k];
        atomicAdd(reinterpret_cast<unsigned long long*>(ctl + 2), (unsigned long long) sum);
    }
}

// Clears the status words, the ticket and fault words and the sum before a launch (a kernel rather than a memset, so a
// graph may hold it).
__global__ void __launch_bounds__(kThreads) fnv_onepass_init_kernel(uint32_t* status, uint64_t words, uint32_t* ctl) {
    const uint64_t stride = uint64_t(gridDim.x) * kThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < words; i += stride) status[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < 4) ctl[threadIdx.x] = 0u;
}
}  // namespace

// The bound on each look-back wait, in window reads; tests lower it to force a wait to run out.
std::atomic<uint32_t> g_spin_limit{kSpinLimit};

// Workspace: [ticket, fault and sum words][status words: three levels of `stride` words].
FnvWorkspace fnv_workspace(uint64_t n) {
    FnvWorkspace w{};
    w.segments = (n + kFnvLaneBytes - 1) / kFnvLaneBytes;
    w.groups = (w.segments + kFnvThreads - 1) / kFnvThreads;
    auto up = [](uint64_t x) { return (x + 255) / 256 * 256; };
    w.off_ctl = 0;
    w.off_status = 256;
    w.stride = up(w.groups * 4) / 4;
    w.bytes = w.off_status + 3 * w.stride * 4;
    return w;
}

hipError_t launch_fnv1a64(const void* data, uint64_t n, uint64_t seed, const uint64_t* seed_dev, uint64_t* out,
                          uint32_t* fault_out, void* workspace, hipStream_t stream, uint64_t expected, uint32_t* verdict,
                          const FnvCarries& carries) {
    const FnvWorkspace w = fnv_workspace(n);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const uint8_t* src = static_cast<const uint8_t*>(data);
    const bool aligned = (reinterpret_cast<uintptr_t>(data) & 15u) == 0;
    uint32_t* ctl = reinterpret_cast<uint32_t*>(ws + w.off_ctl);
    uint32_t* status = reinterpret_cast<uint32_t*>(ws + w.off_status);
    if (w.groups > 0) {
        const uint64_t words = 3 * w.stride;
        const uint64_t init_blocks = (words + kThreads - 1) / kThreads < 1024 ? (words + kThreads - 1) / kThreads : 1024;
        hipLaunchKernelGGL(fnv_onepass_init_kernel, dim3(unsigned(init_blocks)), dim3(kThreads), 0, stream, status, words,
                           ctl);
        hipLaunchKernelGGL(fnv_onepass_kernel<false>, dim3(unsigned(w.groups)), dim3(kFnvThreads), 0, stream, src, n, aligned,
                           seed, seed_dev, status, w.stride, ctl, g_spin_limit.load(), HashMapArgs{}, carries,
                           fnv_carry_count(n));
    }
    // the finish reads the start state before it writes `out`, so `out` may be `seed_dev` itself
    const bool any = w.groups > 0;
    hipLaunchKernelGGL(fnv_finish_kernel, dim3(1), dim3(1), 0, stream, any ? reinterpret_cast<const uint64_t*>(ctl + 2) : nullptr,
                       seed, seed_dev, n, out, fault_out, seed_dev != nullptr, expected, verdict, any ? ctl + 1 : nullptr,
                       nullptr, 0u);
    return hipGetLastError();
}

// Each hash workgroup's part of a map (HashGroup), one thread per workgroup: the extent holding the workgroup's first
// byte (extents tile [0, bytes) in order, so the first whose end lies past it), that extent and the next, whether the
// workgroup's bytes lie in those two, and where its segment puts payload byte 0.  Built on the device so that a map's
// creation uploads its extents only (the parts are 128 bytes per 64 KiB: 6.4 MB for a 3.3 GB payload).
__global__ void hash_groups_kernel(const HashExtent* ext, uint32_t n_ext, uint64_t bytes, uint8_t* const* segs,
                                   uint32_t n_segs, uint64_t seg_bytes, HashGroup* grp, uint64_t groups) {
    const uint64_t g = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const uint64_t o = g * uint64_t(kFnvGroupBytes), o_end = o + kFnvGroupBytes < bytes ? o + kFnvGroupBytes : bytes;
    uint32_t lo = 0, hi = n_ext - 1;   // the first extent whose end lies past o (the last one at most)
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (ext[mid].end > o) hi = mid;
        else lo = mid + 1;
    }
    HashGroup h{};
    const uint64_t k = o / seg_bytes;
    h.base = reinterpret_cast<uint8_t*>(reinterpret_cast<uintptr_t>(segs[k < n_segs ? k : n_segs - 1]) - k * seg_bytes);
    h.first = lo;
    h.x[0] = ext[lo];
    if (lo + 1 < n_ext) h.x[1] = ext[lo + 1];
    h.two = ext[lo].end >= o_end || (lo + 1 < n_ext && ext[lo + 1].end >= o_end) ? 1u : 0u;
    grp[g] = h;
}

hipError_t launch_hash_groups(const HashExtent* ext, uint32_t n_ext, uint64_t bytes, uint8_t* const* segs,
                              uint32_t n_segs, uint64_t seg_bytes, HashGroup* grp, uint64_t groups, hipStream_t stream) {
    if (!groups) return hipSuccess;
    if (!n_ext || !n_segs || !seg_bytes) return hipErrorInvalidValue;
    hipLaunchKernelGGL(hash_groups_kernel, dim3(unsigned((groups + 255) / 256)), dim3(256), 0, stream, ext, n_ext, bytes,
                       segs, n_segs, seg_bytes, grp, groups);
    return hipGetLastError();
}

// The gather fused with the hash: the payload's `map.n_total` bytes gathered into its segments and hashed, the whole
// lane segments in the one-pass kernel and the last partial one (under 256 bytes, at `tail`) by the closing kernel,
// which runs after every byte is in place.  With `verdict`, the closing kernel also leaves the check of the hash
// against `expected` there, as sc_fnv1a64_check_async does.  The carries are those of the whole payload (`n_total`
// bytes): a carry at a boundary inside the last partial lane segment cannot occur (boundaries are 64 KiB apart).
hipError_t launch_fnv1a64_mapped(const HashMapArgs& map, const uint8_t* tail, uint64_t seed, uint64_t* out,
                                 uint32_t* fault_out, void* workspace, hipStream_t stream, uint64_t expected,
                                 uint32_t* verdict, const FnvCarries& carries) {
    const uint64_t n_total = map.n_total, n_full = n_total & ~uint64_t(kFnvLaneBytes - 1);
    if (n_total % 16) return hipErrorInvalidValue;   // maps hold whole 16-byte chunks (the closing kernel loads them)
    const FnvWorkspace w = fnv_workspace(n_total);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint32_t* ctl = reinterpret_cast<uint32_t*>(ws + w.off_ctl);
    uint32_t* status = reinterpret_cast<uint32_t*>(ws + w.off_status);
    if (!map.store) {
        // a map that only reads: the plain kernel hashes the payload where its segments hold it, the last partial
        // lane segment included (no gather, so nothing waits for bytes to be placed)
        if (w.groups > 0) {
            const uint64_t words = 3 * w.stride;
            const uint64_t init_blocks = (words + kThreads - 1) / kThreads < 1024 ? (words + kThreads - 1) / kThreads : 1024;
            hipLaunchKernelGGL(fnv_onepass_init_kernel, dim3(unsigned(init_blocks)), dim3(kThreads), 0, stream, status,
                               words, ctl);
            hipLaunchKernelGGL(fnv_onepass_kernel<false>, dim3(unsigned(w.groups)), dim3(kFnvThreads), 0, stream, nullptr,
                               n_total, true, seed, nullptr, status, w.stride, ctl, g_spin_limit.load(), map, carries,
                               fnv_carry_count(n_total));
        }
        const bool any = w.groups > 0;
        hipLaunchKernelGGL(fnv_finish_kernel, dim3(1), dim3(1), 0, stream,
                           any ? reinterpret_cast<const uint64_t*>(ctl + 2) : nullptr, seed, nullptr, n_total, out,
                           fault_out, false, expected, verdict, any ? ctl + 1 : nullptr, nullptr, 0u);
        return hipGetLastError();
    }
    if (w.groups > 0) {
        const uint64_t words = 3 * w.stride;
        const uint64_t init_blocks = (words + kThreads - 1) / kThreads < 1024 ? (words + kThreads - 1) / kThreads : 1024;
        hipLaunchKernelGGL(fnv_onepass_init_kernel, dim3(unsigned(init_blocks)), dim3(kThreads), 0, stream, status, words,
                           ctl);
        hipLaunchKernelGGL(fnv_onepass_kernel<true>, dim3(unsigned(w.groups)), dim3(kFnvThreads), 0, stream, nullptr, n_full,
                           true, seed, nullptr, status, w.stride, ctl, g_spin_limit.load(), map, carries,
                           fnv_carry_count(n_total));
    }
    const bool any = w.groups > 0;
    hipLaunchKernelGGL(fnv_finish_kernel, dim3(1), dim3(1), 0, stream, any ? reinterpret_cast<const uint64_t*>(ctl + 2) : nullptr,
                       seed, nullptr, n_full, out, fault_out, false, expected, verdict, any ? ctl + 1 : nullptr,
                       tail, uint32_t(n_total - n_full));
    return hipGetLastError();
}

}  // namespace sc

// ---- the hash that allocates nothing ----------------------------------------------------------------------------------
// For callers that cannot allocate (code under HIP graph capture, tight serving loops): the workspace is `scratch`, one
// array per GPU that the library holds until the process ends, sized for inputs of up to SC_FNV_NOALLOC_MAX_BYTES
// (fnv_workspace(4 GiB) is 0.75 MiB).  Every call clears all of it that it uses (the ticket, the fault word, the sum
// and the look-back's status words) with a kernel of its own before the hash kernel; a call after another on the same
// stream is ordered after it, and calls that overlap on one GPU (on different streams) race on the one array.
namespace {

constexpr uint64_t kScratchBytes = 2ull << 20;
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

extern "C" int sc_fnv1a64_noalloc_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, uint32_t* fault,
                                        void* stream) {
    if (!out || !fault || (bytes && !data))
        return sc::record_error(SC_EINVAL, "sc_handoff: missing hash input, output or fault word");
    if (reinterpret_cast<uintptr_t>(fault) & 3u)
        return sc::record_error(SC_EINVAL, "sc_handoff: the hash fault word must be 4-byte aligned");
    if (bytes > SC_FNV_NOALLOC_MAX_BYTES || sc::fnv_workspace(bytes).bytes > kScratchBytes)
        return sc::record_error(SC_ERANGE, "sc_handoff: the hash without allocation takes at most 4 GiB "
                                           "(SC_FNV_NOALLOC_MAX_BYTES); use sc_fnv1a64_async with a workspace");
    void* ws = nullptr;
    hipError_t e = scratch_of_current_device(&ws);
    if (e != hipSuccess)
        return sc::record_error(SC_EHIP, std::string("sc_handoff hash scratch: ") + hipGetErrorString(e));
    e = sc::launch_fnv1a64(data, bytes, seed, nullptr, out, fault, ws, static_cast<hipStream_t>(stream), 0, nullptr,
                           sc::FnvCarries{});
    if (e != hipSuccess) return sc::record_error(SC_EHIP, std::string("sc_handoff hash launch: ") + hipGetErrorString(e));
    return sc::record_ok();
}

extern "C" int sc_fnv1a64_set_spin_limit(uint32_t reads) {
    static_assert(sc::kForceFault == SC_FNV_FORCE_FAULT, "the forced-fault bound is the header's");
    sc::g_spin_limit.store(reads ? reads : sc::kSpinLimit);
    return sc::record_ok();
}
