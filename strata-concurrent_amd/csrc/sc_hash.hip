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
// The buffer is split into lane segments of kFnvLaneBytes bytes.  Level j (one launch each) runs every segment's
// (j+1)-bit machine serially from its known start bits with bit j set to 0 - the end value of bit j is then the
// segment's xor of t_j - and ballots those bits; a single-workgroup scan turns the per-workgroup parities into
// exclusive prefixes, and the next level derives bit j of each segment's start from them.  The last launch runs the
// full machine from the now complete start byte, forms each segment's Horner sum, scales it by p^(bytes after the
// segment) and reduces; a final workgroup adds h_0 p^N.  Every kernel reads each input byte once; ten launches in all.
#include <hip/hip_runtime.h>

#include <cstdint>

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

// The low-bit machine over a segment from state `l`.  Only the low 8 bits of the result are meaningful: the 24-bit
// multiply reads the low 24 bits of its operands and its low 8 result bits depend only on their low 8 bits, so the
// other bytes of a dword may ride along unmasked.
__device__ __forceinline__ uint32_t run_low(const uint8_t* p, uint64_t n, bool full, uint32_t l) {
    if (full) {
        uint32_t w[kFnvLaneBytes / 4];
        load_segment(p, w);
#pragma unroll
        for (int k = 0; k < kFnvLaneBytes / 4; ++k) {
            l = __umul24(l ^ w[k], kPrimeLow);
            l = __umul24(l ^ (w[k] >> 8), kPrimeLow);
            l = __umul24(l ^ (w[k] >> 16), kPrimeLow);
            l = __umul24(l ^ (w[k] >> 24), kPrimeLow);
        }
        return l;
    }
    for (uint64_t i = 0; i < n; ++i) l = __umul24(l ^ uint32_t(p[i]), kPrimeLow);
    return l;
}

// One step of the full hash given the true low byte `l` of the state: accumulate d = (l ^ b) - l, then multiply.
__device__ __forceinline__ void step_full(uint32_t b, uint32_t& l, uint64_t& acc) {
    const uint32_t x = (l ^ b) & 0xFFu;
    acc = (acc + uint64_t(int64_t(int32_t(x) - int32_t(l)))) * kFnvPrime;
    l = __umul24(x, kPrimeLow) & 0xFFu;
}

// Bit `bit` of the start state of this lane's segment, from the previous level's ballots and scan: the seed's bit,
// xor the parity of every earlier workgroup (scan), of the earlier waves of this workgroup, and of the earlier lanes
// of this wave.
__device__ __forceinline__ uint32_t start_bit(uint64_t seed, int bit, const uint64_t* word, const uint8_t* prefix) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t v = uint32_t(seed >> bit) & 1u;
    v ^= prefix[blockIdx.x];
    for (int w = 0; w < wave; ++w) v ^= uint32_t(__popcll(word[uint64_t(blockIdx.x) * 4 + w])) & 1u;
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    v ^= uint32_t(__popcll(word[uint64_t(blockIdx.x) * 4 + wave] & below)) & 1u;
    return v;
}

__global__ void __launch_bounds__(kThreads) fnv_level_kernel(const uint8_t* data, uint64_t n, int level, uint64_t seed,
                                                              bool aligned, uint8_t* start, const uint64_t* word_prev,
                                                              const uint8_t* prefix, uint64_t* word, uint8_t* parity) {
    const uint64_t seg = uint64_t(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t begin = seg * kFnvLaneBytes;
    const bool live = begin < n;
    uint32_t s = 0;
    if (level > 0) {
        const uint32_t bit = start_bit(seed, level - 1, word_prev, prefix);
        s = (level > 1 && live ? uint32_t(start[seg]) : 0u) | (bit << (level - 1));
        if (live) start[seg] = uint8_t(s);
    }
    uint32_t t = 0;
    if (live) {
        const uint64_t len = n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
        t = (run_low(data + begin, len, aligned && len == kFnvLaneBytes, s) >> level) & 1u;
    }
    const uint64_t ballot = __ballot(t);
    __shared__ uint64_t s_word[kThreads / 64];
    if ((threadIdx.x & 63) == 0) {
        word[uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)] = ballot;
        s_word[threadIdx.x >> 6] = ballot;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        parity[blockIdx.x] = uint8_t(__popcll(s_word[0] ^ s_word[1] ^ s_word[2] ^ s_word[3]) & 1);
}

// Exclusive xor prefix of the per-workgroup parities, in one workgroup: each thread folds a contiguous run, a ballot
// scan joins the runs.
__global__ void __launch_bounds__(kScanThreads) fnv_scan_kernel(const uint8_t* parity, uint64_t groups, uint8_t* prefix) {
    const uint64_t per = (groups + kScanThreads - 1) / kScanThreads;
    const uint64_t b = uint64_t(threadIdx.x) * per;
    const uint64_t e = b + per < groups ? b + per : groups;
    uint32_t p = 0;
    for (uint64_t i = b; i < e; ++i) p ^= parity[i];
    const uint64_t ballot = __ballot(p & 1u);
    __shared__ uint64_t s_word[kScanThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) s_word[wave] = ballot;
    __syncthreads();
    uint32_t pre = 0;
    for (int w = 0; w < wave; ++w) pre ^= uint32_t(__popcll(s_word[w])) & 1u;
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    pre ^= uint32_t(__popcll(ballot & below)) & 1u;
    for (uint64_t i = b; i < e; ++i) {
        prefix[i] = uint8_t(pre);
        pre ^= parity[i];
    }
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(uint32_t(v), m), hi = __shfl_xor(uint32_t(v >> 32), m);
    return (uint64_t(hi) << 32) | lo;
}

__global__ void __launch_bounds__(kThreads) fnv_final_kernel(const uint8_t* data, uint64_t n, uint64_t seed, bool aligned,
                                                              const uint8_t* start, const uint64_t* word_prev,
                                                              const uint8_t* prefix, uint64_t* partial) {
    const uint64_t seg = uint64_t(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t begin = seg * kFnvLaneBytes;
    const uint32_t bit7 = start_bit(seed, 7, word_prev, prefix);
    uint64_t acc = 0;
    if (begin < n) {
        uint32_t l = uint32_t(start[seg]) | (bit7 << 7);
        const uint64_t len = n - begin < kFnvLaneBytes ? n - begin : kFnvLaneBytes;
        const uint8_t* p = data + begin;
        if (aligned && len == kFnvLaneBytes) {
            // 16 bytes per iteration: the Horner step is ~20 instructions, so a fully unrolled segment would not fit
            // the instruction cache; the next chunk's load is issued before this chunk's steps.
            u32x4 next = *(const gu32x4*) p;
            for (int k = 0; k < kFnvLaneBytes / 16; ++k) {
                const u32x4 v = next;
                if (k + 1 < kFnvLaneBytes / 16) next = *(const gu32x4*) (p + 16 * (k + 1));
                const uint32_t dw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    step_full(dw[c] & 0xFFu, l, acc);
                    step_full((dw[c] >> 8) & 0xFFu, l, acc);
                    step_full((dw[c] >> 16) & 0xFFu, l, acc);
                    step_full(dw[c] >> 24, l, acc);
                }
            }
        } else {
            for (uint64_t i = 0; i < len; ++i) step_full(p[i], l, acc);
        }
        acc *= pow_prime(n - begin - len);
    }
    for (int m = 32; m > 0; m >>= 1) acc += shfl_xor64(acc, m);
    __shared__ uint64_t s_sum[kThreads / 64];
    if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
}

// h = seed * p^n + sum of the partial sums (mod 2^64; the order of the additions does not matter).
__global__ void __launch_bounds__(kScanThreads) fnv_reduce_kernel(const uint64_t* partial, uint64_t groups, uint64_t seed,
                                                                   uint64_t n, uint64_t* out) {
    uint64_t acc = 0;
    for (uint64_t i = threadIdx.x; i < groups; i += kScanThreads) acc += partial[i];
    for (int m = 32; m > 0; m >>= 1) acc += shfl_xor64(acc, m);
    __shared__ uint64_t s_sum[kScanThreads / 64];
    if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t h = seed * pow_prime(n);
        for (int w = 0; w < kScanThreads / 64; ++w) h += s_sum[w];
        out[0] = h;
    }
}

}  // namespace

// Workspace: [start bytes: one per segment][ballot words, two sets][parities][prefixes][partial sums].
FnvWorkspace fnv_workspace(uint64_t n) {
    FnvWorkspace w{};
    w.segments = (n + kFnvLaneBytes - 1) / kFnvLaneBytes;
    w.groups = (w.segments + kThreads - 1) / kThreads;
    auto up = [](uint64_t x) { return (x + 255) / 256 * 256; };
    w.off_start = 0;
    w.off_word0 = up(w.segments);
    w.off_word1 = w.off_word0 + up(w.groups * 4 * 8);
    w.off_parity = w.off_word1 + up(w.groups * 4 * 8);
    w.off_prefix = w.off_parity + up(w.groups);
    w.off_partial = w.off_prefix + up(w.groups);
    w.bytes = w.off_partial + up(w.groups * 8 > 8 ? w.groups * 8 : 8);
    return w;
}

hipError_t launch_fnv1a64(const void* data, uint64_t n, uint64_t seed, uint64_t* out, void* workspace,
                          hipStream_t stream) {
    const FnvWorkspace w = fnv_workspace(n);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const uint8_t* src = static_cast<const uint8_t*>(data);
    const bool aligned = (reinterpret_cast<uintptr_t>(data) & 15u) == 0;
    uint8_t* start = ws + w.off_start;
    uint64_t* words[2] = {reinterpret_cast<uint64_t*>(ws + w.off_word0), reinterpret_cast<uint64_t*>(ws + w.off_word1)};
    uint8_t* parity = ws + w.off_parity;
    uint8_t* prefix = ws + w.off_prefix;
    uint64_t* partial = reinterpret_cast<uint64_t*>(ws + w.off_partial);
    if (w.groups > 0) {
        for (int level = 0; level < 8; ++level) {
            hipLaunchKernelGGL(fnv_level_kernel, dim3(unsigned(w.groups)), dim3(kThreads), 0, stream, src, n, level,
                               seed, aligned, start, words[(level + 1) & 1], prefix, words[level & 1], parity);
            hipLaunchKernelGGL(fnv_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, parity, w.groups, prefix);
        }
        hipLaunchKernelGGL(fnv_final_kernel, dim3(unsigned(w.groups)), dim3(kThreads), 0, stream, src, n, seed, aligned,
                           start, words[1], prefix, partial);
    }
    hipLaunchKernelGGL(fnv_reduce_kernel, dim3(1), dim3(kScanThreads), 0, stream, partial, w.groups, seed, n, out);
    return hipGetLastError();
}

}  // namespace sc
