// sc_kernels.hip - the CDNA4 (gfx950) kernels of the prefill->decode cache handoff.
//
// All of it is data movement, so every kernel here is bounded by HBM bandwidth, not by the matrix cores:
//   * sc_move_kernel  - walks a handoff table (sc_internal.hpp) in 8 KiB tiles.  Every K/V, recurrence, page
//                       and copy row moves whole 16-byte chunks: 64 lanes x 16 B = 1 KiB per wave instruction,
//                       and a 512-byte pool row is one contiguous run on both sides, so both the loads and the
//                       stores are fully coalesced without LDS.  The conv history is the one real transpose
//                       ([rows][C] -> [C][3], 4-byte granules) and goes through LDS.
//   * fill / generator kernels for synthetic inputs, and the decode probe used to measure overlap.
//
// The K/V address map is the reference's kv_append (src/prefill/kernels.cu:567-573): prefill token t of kv head
// h goes to cell pos0 + t, i.e. pool row (table[cell / ps] * H + h) * ps + cell % ps; a negative table entry is
// a page that is not resident and is skipped, as kv_append skips it (kernels.cu:577).  The recurrence map is
// the (S, HV, S) layout of src/kernels/cuda/gdn.cu:75 (element (i, h, j) at i*HV*S + h*S + j), taken from a
// head-major [HV][S][S] prefill image.  The history map is gdn_conv_hist_kernel (kernels.cu:219-228).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sc_arith.hpp"
#include "sc_convert.hpp"
#include "sc_internal.hpp"

namespace sc {
namespace {

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    const uint32_t hi = __umulhi(n, f.m);
    return uint32_t((uint64_t(hi) + uint64_t(n)) >> f.s);
}

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

// Every buffer the handoff touches is global memory: say so, so the 16-byte accesses are global_load/store_dwordx4
// rather than flat ones that also arbitrate for LDS.  Loads and stores are non-temporal: a handoff reads each source
// byte once and writes each destination byte once, and nothing reads them back soon.  Streaming the stores past the
// caches measured faster (5.83 vs 5.57 TB/s on the 128K handoff) than write-allocating them; streaming the loads as
// well, 1% faster on the 128K carve (four alternating rounds), 4-6% on an image scattered into pages and 4% on a
// plain tile copy.
using gu32x4 = __attribute__((address_space(1))) u32x4;
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) { return __builtin_nontemporal_load((const gu32x4*) (p)); }
// A regular load, for the quantizing rows: with non-temporal loads the int8 carve through a shuffled table took
// 1.628 ms against 1.548 and the per-layer int8 appends 1.509 against 1.396 ms (the f16 rows gained).
__device__ __forceinline__ u32x4 ld16_cached(const uint8_t* p) { return *(const gu32x4*) (p); }
__device__ __forceinline__ void st16(uint8_t* p, u32x4 v) { __builtin_nontemporal_store(v, (gu32x4*) (p)); }

// Thirty-two zero bytes in global memory, which no kernel writes.  A lane with nothing to read (past its row, in a
// row's zero-filled tail, on a page the table does not place) loads from here instead of skipping its load, so every
// lane of a tile issues the same loads in the same order.  The compiler can then count them, and each store waits for
// its own load only.  With loads skipped on some lanes it waited for every earlier memory operation before each
// store, and this part counts stores and loads in one counter: every store waited for the previous store's
// acknowledgement.
__device__ u32x4 g_zero_chunks[2];
__device__ __forceinline__ const uint8_t* zero_chunks() { return reinterpret_cast<const uint8_t*>(g_zero_chunks); }

// The tile a workgroup starts on.  Workgroups are dispatched to the part's eight XCDs in turn (workgroup b to XCD
// b mod 8), each XCD with its own L2; numbering the tiles so that each XCD takes one contiguous eighth of them, in
// order, measured faster than tile b on workgroup b for the identity carve: 128K 1.066-1.075 against 1.088-1.118 ms.
// The host chooses it per plan (sc_plan::xcd).  Any numbering is correct (this one is a permutation of 0 .. n - 1);
// only the speed depends on the dispatch order.
__device__ __forceinline__ uint64_t xcd_tile(uint32_t b, uint32_t n) {
    const uint32_t q = n / 8, r = n % 8, x = b % 8;
    return uint64_t(x) * q + (x < r ? x : r) + b / 8;
}

// Page tables are read through global loads.  Every tile issues all of its loads, table entries included, before
// its first store: a table load placed after a store (which might alias the table) waits for it, and the
// per-chunk load -> store chains that result measured 10-14% slower on the 128K handoff through a page table.
// Whether the row has a table is a template argument, so the entry's load is never skipped (see g_zero_chunks).
using gi32 = __attribute__((address_space(1))) const int32_t;
template <bool kTable>
__device__ __forceinline__ int32_t table_entry(const MoveRow& r, uint32_t page) {
    if constexpr (kTable) return *(gi32*) (r.table + page);
    return int32_t(page);
}
// The same entry for a wave-uniform page, read with a scalar load (through the constant address space: no kernel
// writes a table).  A vector load would share the wave's in-order load counter, so taking its value into a scalar
// register would first wait for every row load issued before it.
using ci32 = __attribute__((address_space(4))) const int32_t;
__device__ __forceinline__ int32_t table_entry_uniform(const MoveRow& r, uint32_t page) {
    return r.table ? *((ci32*) r.table + page) : int32_t(page);
}

// The (cell, head) address of K/V source row `src_row` (token-major [T][H]): the logical page, and the row's
// place inside a physical page.
struct KvCell {
    uint32_t page, h, in_page;
};
__device__ __forceinline__ KvCell kv_cell(const MoveRow& r, const MoveGeo& g, uint32_t src_row) {
    const uint32_t t = fdiv(src_row, g.heads);
    const uint32_t cell = uint32_t(r.pos0 + int64_t(t));
    const uint32_t page = fdiv(cell, g.page_size);
    return {page, src_row - t * g.heads.d, cell - page * g.page_size.d};
}
// Pool row of a K/V row in physical page `phys`; -1 when the page is not resident or out of the pool.
__device__ __forceinline__ int64_t pool_row(const MoveRow& r, const MoveGeo& g, int32_t phys, const KvCell& c) {
    if (phys < 0 || int64_t(phys) >= r.ld) return -1;
    return (int64_t(phys) * g.heads.d + c.h) * g.page_size.d + c.in_page;
}

// Destination order (MoveRow::order): virtual chunk vq of a row is in-page chunk vq % page_chunks of the order's
// entry vq / page_chunks, a logical page (-1 past the pages the table places).  Its source rows are that page's cells
// in token-major order, so the page's chunks are one contiguous run of the row's source: the source chunk is
// (lp * ps - pos0) * H * row_chunks plus the in-page index.  Returns ~0u (>= every row's chunk count) for a -1 entry
// and for cells outside the row.
// kOrder: kDestOrderWave when a page holds a multiple of 64 chunks, so that the wave's 64 consecutive chunks share
// one page and its entry is read with a scalar load; kDestOrder reads it per lane.  The choice is a template argument
// so that no tile has a branch around one of its loads.
enum TileOrder { kSourceOrder = 0, kDestOrder = 1, kDestOrderWave = 2 };
// `page` receives the entry (wave-uniform under kDestOrderWave, so its table entry can be read with a scalar load).
template <int kOrder>
__device__ __forceinline__ uint32_t ordered_chunk(const MoveRow& r, const MoveGeo& g, uint32_t vq, bool kv,
                                                  int32_t& page) {
    const uint32_t vp = fdiv(vq, g.page_chunks);
    const uint32_t ip = vq - vp * g.page_chunks.d;
    int64_t lp;
    if constexpr (kOrder == kDestOrderWave) lp = *((ci32*) r.order + __builtin_amdgcn_readfirstlane(vp));
    else lp = *(gi32*) (r.order + vp);
    page = int32_t(lp);
    if (lp < 0) return ~0u;
    const int64_t q = kv ? (lp * int64_t(g.page_size.d) - r.pos0) * int64_t(g.heads.d * g.row_chunks.d) + ip
                         : lp * int64_t(g.page_chunks.d) + ip;
    return q >= 0 && q < int64_t(r.n) ? uint32_t(q) : ~0u;
}

// kTable: the row has a page table, whose entries are loaded with the data; without one the physical page is the
// logical page and nothing but the data is loaded before the stores.  kOrder: the tiles visit the row's pages in
// destination order (the order's load comes before the data's).
template <bool kTable, int kOrder = kSourceOrder>
__device__ void tile_kv16(const MoveRow& r, const MoveGeo& g, uint64_t local) {
    const uint32_t row_bytes = g.row_chunks.d * 16u;
    const uint32_t last = uint32_t(r.n) - 1u;
    u32x4 v[kChunksPerThread];
    uint32_t q[kChunksPerThread];
    int32_t phys[kChunksPerThread], lpage[kChunksPerThread];
    // every order entry is read before the first data load, so no data load waits behind the next entry's
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        q[j] = uint32_t(local * kTileChunks) + uint32_t(j * kThreads) + threadIdx.x;
        if constexpr (kOrder != kSourceOrder) q[j] = ordered_chunk<kOrder>(r, g, q[j], true, lpage[j]);
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        // rows past the source's tokens (an image's stale-cell tail) are written as zeros
        const uint32_t row = fdiv(min(q[j], last), g.row_chunks);
        const bool live = q[j] <= last && fdiv(row, g.heads) < uint32_t(r.aux);
        v[j] = ld16(live ? r.src + uint64_t(q[j]) * 16u : zero_chunks());
        // in wave-uniform destination order the wave's chunks share the order's logical page (a lane outside the
        // row stores nothing), whose table entry is read with a scalar load
        if constexpr (kTable && kOrder == kDestOrderWave)
            phys[j] = lpage[j] >= 0 ? table_entry_uniform(r, uint32_t(lpage[j])) : -1;
        else if constexpr (kTable)
            phys[j] = table_entry<true>(r, kv_cell(r, g, row).page);
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        if (q[j] >= r.n) continue;
        const uint32_t row = fdiv(q[j], g.row_chunks);
        const uint32_t ch = q[j] - row * g.row_chunks.d;
        const KvCell c = kv_cell(r, g, row);
        const int64_t prow = pool_row(r, g, kTable ? phys[j] : int32_t(c.page), c);
        if (prow >= 0) st16(r.dst + uint64_t(prow) * row_bytes + ch * 16u, v[j]);
    }
}

// The same map from f32 rows, rounded to f16: destination chunk q holds 8 halves = 32 source bytes at q * 32.
template <bool kTable, int kOrder = kSourceOrder>
__device__ void tile_kv32(const MoveRow& r, const MoveGeo& g, uint64_t local) {
    const uint32_t row_bytes = g.row_chunks.d * 16u;
    const uint32_t last = uint32_t(r.n) - 1u;
    u32x4 a[kChunksPerThread], b[kChunksPerThread];
    uint32_t q[kChunksPerThread];
    int32_t phys[kChunksPerThread], lpage[kChunksPerThread];
    // every order entry is read before the first data load, so no data load waits behind the next entry's
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        q[j] = uint32_t(local * kTileChunks) + uint32_t(j * kThreads) + threadIdx.x;
        if constexpr (kOrder != kSourceOrder) q[j] = ordered_chunk<kOrder>(r, g, q[j], true, lpage[j]);
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        const uint32_t row = fdiv(min(q[j], last), g.row_chunks);
        const bool live = q[j] <= last && fdiv(row, g.heads) < uint32_t(r.aux);
        const uint8_t* p = live ? r.src + uint64_t(q[j]) * 32u : zero_chunks();
        a[j] = ld16(p);
        b[j] = ld16(p + 16u);
        // in wave-uniform destination order the wave's chunks share the order's logical page (a lane outside the
        // row stores nothing), whose table entry is read with a scalar load
        if constexpr (kTable && kOrder == kDestOrderWave)
            phys[j] = lpage[j] >= 0 ? table_entry_uniform(r, uint32_t(lpage[j])) : -1;
        else if constexpr (kTable)
            phys[j] = table_entry<true>(r, kv_cell(r, g, row).page);
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        if (q[j] >= r.n) continue;
        u32x4 o;
        o.x = f16_bits_rne(a[j].x) | (f16_bits_rne(a[j].y) << 16);
        o.y = f16_bits_rne(a[j].z) | (f16_bits_rne(a[j].w) << 16);
        o.z = f16_bits_rne(b[j].x) | (f16_bits_rne(b[j].y) << 16);
        o.w = f16_bits_rne(b[j].z) | (f16_bits_rne(b[j].w) << 16);
        const uint32_t row = fdiv(q[j], g.row_chunks);
        const uint32_t ch = q[j] - row * g.row_chunks.d;
        const KvCell c = kv_cell(r, g, row);
        const int64_t prow = pool_row(r, g, kTable ? phys[j] : int32_t(c.page), c);
        if (prow >= 0) st16(r.dst + uint64_t(prow) * row_bytes + ch * 16u, o);
    }
}

// Destination rows (i, h) of the (S, HV, S) recurrence, S*4 bytes each, read from head-major row h*S + i.
__device__ void tile_rec(const MoveRow& r, const MoveGeo& g, uint64_t local) {
    const uint32_t row_bytes = g.rec_chunks.d * 16u;
    u32x4 v[kChunksPerThread];
    uint32_t q[kChunksPerThread];
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        q[j] = uint32_t(local * kTileChunks) + uint32_t(j * kThreads) + threadIdx.x;
        const uint32_t row = fdiv(q[j], g.rec_chunks);
        const uint32_t ch = q[j] - row * g.rec_chunks.d;
        const uint32_t i = fdiv(row, g.v_heads);
        const uint32_t h = row - i * g.v_heads.d;
        v[j] = ld16(q[j] < r.n ? r.src + (uint64_t(h) * g.state + i) * row_bytes + ch * 16u : zero_chunks());
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j)
        if (q[j] < r.n) st16(r.dst + uint64_t(q[j]) * 16u, v[j]);
}

// Whole pages between a contiguous run and a paged pool.  Scattering, the packed source does not depend on the
// table, so its loads are issued before the table is read and the table's latency hides behind them (a
// table-first order measured about 20% slower); gathering, the table must come first.
template <bool kTable, int kOrder = kSourceOrder>
__device__ void tile_pages(const MoveRow& r, const MoveGeo& g, uint64_t local, bool scatter) {
    const uint64_t page_bytes = uint64_t(g.page_chunks.d) * 16u;
    u32x4 v[kChunksPerThread];
    int64_t dst_off[kChunksPerThread];
    if (scatter) {
        // a source-order row may start `c0` chunks into its pages (pos0: a blob split where a payload's segment
        // ends); the chunk numbers below are relative to the row's source, the page arithmetic adds c0
        const uint32_t last = uint32_t(r.n) - 1u, c0 = kOrder == kSourceOrder ? uint32_t(r.pos0) : 0u;
        uint32_t q[kChunksPerThread];
        int32_t phys[kChunksPerThread], lpage[kChunksPerThread];
#pragma unroll
        for (int j = 0; j < kChunksPerThread; ++j) {
            q[j] = uint32_t(local * kTileChunks) + uint32_t(j * kThreads) + threadIdx.x;
            if constexpr (kOrder != kSourceOrder) q[j] = ordered_chunk<kOrder>(r, g, q[j], false, lpage[j]);
        }
#pragma unroll
        for (int j = 0; j < kChunksPerThread; ++j) v[j] = ld16(q[j] <= last ? r.src + uint64_t(q[j]) * 16u : zero_chunks());
#pragma unroll
        for (int j = 0; j < kChunksPerThread; ++j) {
            if constexpr (kTable && kOrder == kDestOrderWave)
                phys[j] = lpage[j] >= 0 ? table_entry_uniform(r, uint32_t(lpage[j])) : -1;
            else
                phys[j] = table_entry<kTable>(r, fdiv(min(q[j], last) + c0, g.page_chunks));
        }
#pragma unroll
        for (int j = 0; j < kChunksPerThread; ++j) {
            if (q[j] >= r.n) continue;
            const uint32_t page = fdiv(q[j] + c0, g.page_chunks);
            const uint32_t ch = q[j] + c0 - page * g.page_chunks.d;
            if (phys[j] >= 0 && int64_t(phys[j]) < r.ld) st16(r.dst + uint64_t(phys[j]) * page_bytes + ch * 16u, v[j]);
        }
        return;
    }
    const uint32_t last = uint32_t(r.n) - 1u;
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        const uint32_t q = uint32_t(local * kTileChunks) + uint32_t(j * kThreads) + threadIdx.x;
        const uint32_t page = fdiv(min(q, last), g.page_chunks);
        const uint32_t ch = q - page * g.page_chunks.d;
        const int64_t phys = table_entry<kTable>(r, page);
        const bool placed = q <= last && phys >= 0 && phys < r.ld;
        v[j] = ld16(placed ? r.src + uint64_t(phys) * page_bytes + ch * 16u : zero_chunks());
        dst_off[j] = placed ? int64_t(q) * 16 : -1;
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j)
        if (dst_off[j] >= 0) st16(r.dst + dst_off[j], v[j]);
}

__device__ void tile_copy(const MoveRow& r, uint64_t local, bool zero) {
    u32x4 v[kChunksPerThread];
    uint64_t q[kChunksPerThread];
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) q[j] = local * kTileChunks + uint64_t(j * kThreads) + threadIdx.x;
    if (zero) {
#pragma unroll
        for (int j = 0; j < kChunksPerThread; ++j)
            if (q[j] < r.n) st16(r.dst + q[j] * 16u, u32x4{0u, 0u, 0u, 0u});
        return;
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) v[j] = ld16(q[j] < r.n ? r.src + q[j] * 16u : zero_chunks());
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j)
        if (q[j] < r.n) st16(r.dst + q[j] * 16u, v[j]);
}

// The conv history: channels [c0, c0 + kConvTileChannels) of history rows k = 0..hist-1, which are source rows
// rows - hist + k.  For a source shorter than the history the older rows come from the previous history (read
// before any of it is overwritten), or are zero for a fresh sequence, whose state starts zeroed.  Staged through
// LDS so both the row reads and the interleaved [C][hist] writes are contiguous across lanes.
__device__ void tile_conv(const MoveRow& r, uint64_t local, float (*lds)[kConvTileChannels]) {
    const int hist = r.aux & 0xFF;
    const bool fresh = ((r.aux >> 8) & 1) != 0;
    const int64_t C = int64_t(r.n);
    const int64_t c0 = int64_t(local) * kConvTileChannels;
    const int64_t nc = C - c0 < kConvTileChannels ? C - c0 : kConvTileChannels;
    const float* src = reinterpret_cast<const float*>(r.src);
    float* dst = reinterpret_cast<float*>(r.dst);
    for (int k = 0; k < hist; ++k) {
        const int64_t t = r.pos0 - hist + k;
        for (int64_t c = threadIdx.x; c < nc; c += kThreads)
            lds[k][c] = t >= 0 ? src[t * r.ld + c0 + c] : fresh ? 0.0f : dst[(c0 + c) * hist + (t + hist)];
    }
    __syncthreads();
    const int64_t n_out = nc * hist;
    for (int64_t o = threadIdx.x; o < n_out; o += kThreads) {
        const int64_t c = o / hist;
        dst[c0 * hist + o] = lds[o - c * hist][c];
    }
    __syncthreads();
}

// ---- quantizing rows (int8, q4_0) -------------------------------------------------------------------------------
// One wave quantizes one (token, head) row of 256 f32 values: lane l holds values 4l..4l+3 (one 16-byte load, the
// row's 1 KiB read coalesced).  The rules are the reference's int8 kv_append (src/prefill/kernels.cu:578-600,
// src/kernels/cuda/kv_q8.cu:29-64) and q4_0 kv_append_q4 (src/kernels/cuda/kv_q4.cu:72-129): see the oracle
// (sco_q8_row, sco_q4_row) for the exact definitions these lanes reproduce.  The divisions written with `/` are
// IEEE divisions (the library is built with correctly rounded f32 divide), the int8 quotients are formed so that
// they equal them (q8_code), and the q4 code x * id + 8.5 is one fused multiply-add, as the reference's device writer
// computes it (kv_q4.cu:84, contracted by its compilers' defaults).

// The int8 code rint(x / sf) clamped to [-127, 127], with x / sf the correctly rounded quotient, formed from y, the
// correctly rounded 1 / sf computed once per group: q0 = x * y, then one correction q = q0 + (x - q0 * sf) * y with
// the residual exact in an fma (Markstein's method: P. Markstein, "Computation of elementary functions on the IBM
// RISC System/6000 processor", IBM J. Res. Dev. 34(1), 1990).  That q equals the IEEE quotient for every f32
// significand over every f16 significand is checked exhaustively by the test suite; the operations scale exactly
// with the exponents, and where they would not (a residual below the normal range) |x / sf| < 2^-78 codes 0 both
// ways.  sf = +inf gives y = 0 and a NaN q, which codes 0 as x / inf does.  A NaN quotient (x NaN, or x infinite
// over an infinite scale) codes 0, as a NaN converts to integer 0.  Written as selects: every lane forms its
// quotient and discards it where the code is 0.
__device__ __forceinline__ uint32_t q8_code(float x, float sf, float y) {
#pragma clang fp contract(off)
    const float q0 = x * y;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, sf, x), y, q0);
    const float r = __builtin_rintf(q);
    const float c = __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
    const bool coded = sf > 0.0f && r == r;
    return coded ? uint32_t(int(c)) & 0xFFu : 0u;
}

constexpr int kQuantUnitsPerWave = kQuantUnitsPerTile / (kThreads / 64);

// Cross-lane moves inside a 16-lane DPP row (VALU operations, no LDS round trip).  A row of 16 lanes holds one
// int8 group of 64 values; half a row holds one q4_0 block of 32.
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each half row (pairs the two quads of a half)
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within the row (pairs the two halves)
constexpr int kDppRowShl4 = 0x104;     // lane i reads lane i + 4 of its row (lanes 12..15 keep their own value)
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
    return __uint_as_float(dpp<kCtrl>(__float_as_uint(v)));
}

// The maximum over a 16-lane DPP row of non-negative, non-NaN floats, as unsigned integers: for such values the bit
// patterns order as the numbers do, so the comparison needs no NaN handling and each step folds into one DPP max.
__device__ __forceinline__ float row16_max_nonneg(float a) {
    uint32_t u = __float_as_uint(a);
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppXor1, 0xF, 0xF, true)));
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppXor2, 0xF, 0xF, true)));
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppHalfMirror, 0xF, 0xF, true)));
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppMirror, 0xF, 0xF, true)));
    return __uint_as_float(u);
}

// The wave's rows of a tile, all loads (rows and their pages' table entries) issued before any row is quantized:
// four 1 KiB reads in flight per wave.
// `wave` is wave-uniform (the caller reads it with readfirstlane), so every row index, page-table entry and pool
// row below is scalar work: the vector units only carry the rows' values.
__device__ __forceinline__ int load_units(const MoveRow& r, const MoveGeo& g, uint64_t local, int lane, int wave,
                                          u32x4 (&v)[kQuantUnitsPerWave], uint32_t (&unit)[kQuantUnitsPerWave],
                                          int32_t (&phys)[kQuantUnitsPerWave]) {
    int n = 0;
#pragma unroll
    for (int i = 0; i < kQuantUnitsPerWave; ++i) {
        unit[i] = uint32_t(local) * kQuantUnitsPerTile + uint32_t(wave * kQuantUnitsPerWave + i);
        if (unit[i] < r.n) {   // uniform across the wave
            v[i] = ld16_cached(r.src + uint64_t(unit[i]) * (kQuantDim * 4) + lane * 16);
            n = i + 1;
        }
    }
#pragma unroll
    for (int i = 0; i < kQuantUnitsPerWave; ++i)
        if (i < n) phys[i] = table_entry_uniform(r, kv_cell(r, g, unit[i]).page);
    return n;
}

// kStaged (rows through a page table): the tile's rows are written together once every wave has quantized its own,
// through LDS, 16 threads a row with 16 bytes each and the scales by 16 threads with 8 bytes each, so a page's rows
// reach memory at once rather than row by row as each wave finishes one.  Through a shuffled page table the 128K carve
// took 1.428-1.478 ms against 1.492-1.500 ms written from the lanes (69.8-72.3% against 68.9-69.2% of HBM peak); the
// identity carve, whose rows land in order anyway, measured 0.6-1.4% slower staged and writes from the lanes.
template <bool kStaged>
__device__ void tile_q8(const MoveRow& r, const MoveGeo& g, uint64_t local) {
    __shared__ uint32_t s_q8_codes[kQuantUnitsPerTile][64];
    __shared__ uint64_t s_q8_scale[kQuantUnitsPerTile];
    __shared__ int64_t s_q8_prow[kQuantUnitsPerTile];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    u32x4 vs[kQuantUnitsPerWave];
    uint32_t units[kQuantUnitsPerWave];
    int32_t phys[kQuantUnitsPerWave];
    const int n_units = load_units(r, g, local, lane, wave, vs, units, phys);
#pragma unroll
    for (int i = 0; i < kQuantUnitsPerWave; ++i) {
        if (i >= n_units) break;
        const uint32_t unit = units[i];
        const u32x4 v = vs[i];
        const float x0 = __uint_as_float(v.x), x1 = __uint_as_float(v.y), x2 = __uint_as_float(v.z),
                    x3 = __uint_as_float(v.w);
        // max |x| over the 64 values of this lane's group, the 16 lanes of its DPP row (fmax is exact, so any
        // order gives the same).  It starts from 0, so NaNs never count; a group of NaNs only (which the reference's
        // fmaxf reduction leaves NaN) gets the f16 NaN 0x7E00 as its scale, and codes 0.
        const float a = row16_max_nonneg(fmaxf(fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3))), 0.0f));
        const uint32_t real = uint32_t((x0 == x0) | (x1 == x1) | (x2 == x2) | (x3 == x3));
        const bool any_real = __float_as_uint(row16_max_nonneg(__uint_as_float(real))) != 0u;
        const uint32_t sb = any_real ? f16_bits_rne_not_nan(div127(a)) : 0x7E00u;   // a is never NaN, nor a / 127
        const float sf = f32_of_f16(sb);
        const float y = recip_normal(sf);   // sf is a binary16 value: 2^-24 <= sf <= 65504 wherever it codes
        const uint32_t codes = q8_code(x0, sf, y) | (q8_code(x1, sf, y) << 8) | (q8_code(x2, sf, y) << 16) |
                               (q8_code(x3, sf, y) << 24);
        const uint32_t s1 = __builtin_amdgcn_readlane(sb, 16), s2 = __builtin_amdgcn_readlane(sb, 32),
                       s3 = __builtin_amdgcn_readlane(sb, 48);
        const int64_t prow = pool_row(r, g, phys[i], kv_cell(r, g, unit));
        const uint64_t packed = uint64_t(sb | (s1 << 16)) | (uint64_t(s2 | (s3 << 16)) << 32);
        if constexpr (kStaged) {
            const int slot = wave * kQuantUnitsPerWave + i;
            s_q8_codes[slot][lane] = codes;
            if (lane == 0) {
                s_q8_scale[slot] = packed;
                s_q8_prow[slot] = prow;
            }
        } else {
            if (prow < 0) continue;
            using g32 = __attribute__((address_space(1))) uint32_t;
            using g64 = __attribute__((address_space(1))) uint64_t;
            *(g32*) (r.dst + uint64_t(prow) * kQuantDim + lane * 4) = codes;
            if (lane == 0) *(g64*) (r.dst2 + uint64_t(prow) * 8) = packed;
        }
    }
    if constexpr (!kStaged) return;
    if (lane == 0)
        for (int i = n_units; i < kQuantUnitsPerWave; ++i) s_q8_prow[wave * kQuantUnitsPerWave + i] = -1;
    __syncthreads();
    {
        const int t = threadIdx.x, u = t >> 4, c = t & 15;
        const int64_t prow = s_q8_prow[u];
        if (prow >= 0) {
            const u32x4 v = u32x4{s_q8_codes[u][4 * c], s_q8_codes[u][4 * c + 1], s_q8_codes[u][4 * c + 2],
                                  s_q8_codes[u][4 * c + 3]};
            *(gu32x4*) (r.dst + uint64_t(prow) * kQuantDim + c * 16) = v;
        }
        if (t < kQuantUnitsPerTile / 2) {
            // units u and u + H are (cell, h) and (cell + 1, h): one 16-byte store when their scale rows are
            // consecutive (one page) and the pair starts on 16 bytes, else one 8-byte store each
            const uint32_t H = g.heads.d, th = fdiv(uint32_t(t), g.heads);
            const bool pairs = kQuantUnitsPerTile % (2 * H) == 0;
            const int u0 = pairs ? int(th * 2 * H + (uint32_t(t) - th * H)) : 2 * t;
            const int u1 = pairs ? u0 + int(H) : 2 * t + 1;
            const int64_t p0 = s_q8_prow[u0], p1 = s_q8_prow[u1];
            using g64 = __attribute__((address_space(1))) uint64_t;
            if (p0 >= 0 && p1 == p0 + 1 && (p0 & 1) == 0) {
                const uint64_t a = s_q8_scale[u0], b = s_q8_scale[u1];
                *(gu32x4*) (r.dst2 + uint64_t(p0) * 8) =
                    u32x4{uint32_t(a), uint32_t(a >> 32), uint32_t(b), uint32_t(b >> 32)};
            } else {
                if (p0 >= 0) *(g64*) (r.dst2 + uint64_t(p0) * 8) = s_q8_scale[u0];
                if (p1 >= 0) *(g64*) (r.dst2 + uint64_t(p1) * 8) = s_q8_scale[u1];
            }
        }
    }
    __syncthreads();
}

// The q4_0 block's chosen value: the candidate of largest |x|, then of larger value, then of lower index; a NaN is
// never chosen and a block of NaNs chooses +0.  One maximum decides the common case.  With f = rotl(bits(x), 1) =
// 2 * bits(|x|) + sign, the key (f ^ 1) + kQ4KeyBase orders the values by magnitude and, at equal magnitude, puts the
// positive value first; every NaN (f >= 0xFF000002) wraps below every number (f <= 0xFF000001), so none is chosen.
// The maximum key over the block's 32 values (four per lane, then a DPP max over its 8 lanes) gives the chosen value
// back.  When the largest magnitude is 0 (the block holds only zeros and NaNs) every candidate is a zero and all are
// equal as values, so the lowest index wins: that rare case (a wave vote) takes a second maximum over the zeros,
// z = ((31 - j) << 1 | sign) + 1.  Keys order as unsigned integers, so every step is one DPP max.
constexpr uint32_t kQ4KeyBase = 0x00FFFFFEu;   // -0 keys to this, +0 to one more, NaNs below it

__device__ __forceinline__ uint32_t half16_max(uint32_t u) {
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppXor1, 0xF, 0xF, true)));
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppXor2, 0xF, 0xF, true)));
    u = max(u, uint32_t(__builtin_amdgcn_update_dpp(0, int(u), kDppHalfMirror, 0xF, 0xF, true)));
    return u;
}

__device__ __forceinline__ uint32_t q4_key(float x) {
    return (__builtin_rotateleft32(__float_as_uint(x), 1) ^ 1u) + kQ4KeyBase;
}

__device__ __forceinline__ float q4_chosen(const float (&x)[4], uint32_t lb) {
    uint32_t m = max(max(q4_key(x[0]), q4_key(x[1])), max(q4_key(x[2]), q4_key(x[3])));
    m = half16_max(m);
    const uint32_t f = (m - kQ4KeyBase) ^ 1u;
    float chosen = __uint_as_float(__builtin_rotateright32(f, 1));
    if (__any(m <= kQ4KeyBase + 1u)) {
        uint32_t z = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t bits = __float_as_uint(x[k]);
            const bool zero = (bits & 0x7FFFFFFFu) == 0u;
            z = max(z, zero ? (((31u - (lb * 4u + uint32_t(k))) << 1) | (bits >> 31)) + 1u : 0u);
        }
        z = half16_max(z);
        const float first_zero = __uint_as_float(((z - 1u) & 1u) << 31);
        chosen = m < kQ4KeyBase ? 0.0f : m <= kQ4KeyBase + 1u ? first_zero : chosen;
    }
    return chosen;
}

// trunc(x * id + 8.5) clamped to [0, 15], the sum rounded once.  The clamp comes first, in float (one v_med3): a NaN sum
// (inf * 0) clamps to 0 under the maximum's NaN rule and an infinite one to 0 or 15, as a saturating conversion would
// give, so the conversion always sees a value in [0, 15].
__device__ __forceinline__ uint32_t q4_code(float x, float id) {
    const float sum = __builtin_fmaf(x, id, 8.5f);
    return uint32_t(__builtin_fminf(__builtin_fmaxf(sum, 0.0f), 15.0f));
}

__device__ void tile_q4(const MoveRow& r, const MoveGeo& g, uint64_t local) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lb = lane & 7;            // lane within its 32-value block
    const uint32_t blk = uint32_t(lane >> 3);
    u32x4 vs[kQuantUnitsPerWave];
    uint32_t units[kQuantUnitsPerWave];
    int32_t phys[kQuantUnitsPerWave];
    const int n_units = load_units(r, g, local, lane, wave, vs, units, phys);
#pragma unroll
    for (int i = 0; i < kQuantUnitsPerWave; ++i) {
        if (i >= n_units) break;
        const uint32_t unit = units[i];
        const u32x4 v = vs[i];
        const float x[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
        const float mval = q4_chosen(x, uint32_t(lb));
        const float d = mval / -8.0f;
        // 1 / d: the fast reciprocal where it is exact, the division for the rare blocks of subnormal or infinite d
        float id = recip_normal(d);
        const bool fast = recip_normal_ok(d);
        if (__any(!fast)) id = fast ? id : 1.0f / d;
        id = d != 0.0f ? id : 0.0f;
        const uint32_t q = q4_code(x[0], id) | (q4_code(x[1], id) << 8) | (q4_code(x[2], id) << 16) |
                           (q4_code(x[3], id) << 24);
        const uint32_t hi = dpp<kDppRowShl4>(q);   // lane lb + 4 holds the block's values 16 + 4 lb .. 19 + 4 lb
        const int64_t prow = pool_row(r, g, phys[i], kv_cell(r, g, unit));
        if (prow < 0) continue;
        // block `blk` of the row: {f16 d, qs[16]}, 18 bytes at 18 * blk; qs[4 lb .. 4 lb + 3] from lanes lb, lb + 4.
        // (Assembling each row into 36 aligned dwords with two more DPP moves, one store per row, measured slower:
        // 1.397 against 1.375 ms for the 128K carve.)
        uint8_t* row = r.dst + uint64_t(prow) * (kQuantDim / 32 * 18) + blk * 18;
        using g16 = __attribute__((address_space(1))) uint16_t;
        if (lb == 0) *(g16*) (row) = uint16_t(f16_bits_rne_not_nan(d));   // the chosen value is never NaN
        if (lb < 4) {
            const uint32_t bytes = q | (hi << 4);
            *(g16*) (row + 2 + 4 * lb) = uint16_t(bytes);
            *(g16*) (row + 4 + 4 * lb) = uint16_t(bytes >> 16);
        }
    }
}

// A workgroup takes tiles blockIdx.x, + gridDim.x, ...; the plan picks the grid (one workgroup per tile up to 2^20
// workgroups, then grid-stride).  `tile_row[t]` names the handoff table row of tile t (the host pads the array to an
// even count), so a workgroup finds its row with two scalar loads and no search: a vector load of the entry would
// make the wave wait, before its next tile and before it ends, for every store it issued.  The instance (kMix) compiles only its set of row kinds: the f32 rounding tile holds twice the loads
// and the quantizers need 80-90 VGPRs, and compiled into one kernel they took the plain movers from 8 to 6 waves
// per SIMD.  The quantizing instance is held to 80 VGPRs (6 waves per SIMD): at 84 it fell to 5 waves and every
// quantizing row slowed by 3-6%; the instance of every kind keeps 5 waves (at 80 VGPRs it would spill).
template <int kMix>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(kMix == kMixAll ? 5 : 6)))
sc_move_kernel(const MoveRow* __restrict__ rows, const uint16_t* __restrict__ tile_row, MoveGeo geo, uint64_t n_tiles,
               const uint32_t* __restrict__ gate, bool xcd) {
    // A gated launch moves nothing unless the word a kernel before it on the stream left at `gate` is nonzero (a
    // payload hash that matched): every workgroup reads the same word, so the launch writes all or nothing.
    if (gate && __builtin_amdgcn_readfirstlane(*gate) == 0u) return;
    __shared__ float s_conv[kMaxHist][kConvTileChannels];
    const bool wave_pages = geo.page_chunks.d % 64u == 0u;
    int cur = -1;
    MoveRow r{};
    // `xcd`: the plan numbers its tiles by XCD (plain plans without page tables; the host decides)
    const uint64_t first = xcd ? xcd_tile(blockIdx.x, gridDim.x) : uint64_t(blockIdx.x);
    for (uint64_t tile = first; tile < n_tiles; tile += gridDim.x) {
        using cu32 = __attribute__((address_space(4))) const uint32_t;
        const uint32_t pair = *((cu32*) tile_row + (tile >> 1));
        const int k = int((tile & 1) ? pair >> 16 : pair & 0xFFFFu);
        if (k != cur) { cur = k; r = rows[k]; }
        const uint64_t local = tile - r.tile0;
        switch (r.kind) {
            case kKv16:
                if (r.order && wave_pages) tile_kv16<true, kDestOrderWave>(r, geo, local);
                else if (r.order) tile_kv16<true, kDestOrder>(r, geo, local);
                else if (r.table) tile_kv16<true>(r, geo, local);
                else tile_kv16<false>(r, geo, local);
                break;
            case kKv32:
                if constexpr (kMix == kMixWide || kMix == kMixAll) {
                    if (r.order && wave_pages) tile_kv32<true, kDestOrderWave>(r, geo, local);
                    else if (r.order) tile_kv32<true, kDestOrder>(r, geo, local);
                    else if (r.table) tile_kv32<true>(r, geo, local);
                    else tile_kv32<false>(r, geo, local);
                }
                break;
            case kRec: tile_rec(r, geo, local); break;
            case kConv: tile_conv(r, local, s_conv); break;
            case kPagesScatter:
                if (r.order && wave_pages) tile_pages<true, kDestOrderWave>(r, geo, local, true);
                else if (r.order) tile_pages<true, kDestOrder>(r, geo, local, true);
                else if (r.table) tile_pages<true>(r, geo, local, true);
                else tile_pages<false>(r, geo, local, true);
                break;
            case kPagesGather:
                if (r.table) tile_pages<true>(r, geo, local, false);
                else tile_pages<false>(r, geo, local, false);
                break;
            case kCopy: tile_copy(r, local, false); break;
            case kZero: tile_copy(r, local, true); break;
            case kKvQ8:
                if constexpr (kMix == kMixQuant) {
                    tile_q8<false>(r, geo, local);
                } else if constexpr (kMix == kMixQuantPaged || kMix == kMixAll) {
                    if (r.table) tile_q8<true>(r, geo, local);
                    else tile_q8<false>(r, geo, local);
                }
                break;
            case kKvQ4:
                if constexpr (kMix == kMixQuant || kMix == kMixQuantPaged || kMix == kMixAll) tile_q4(r, geo, local);
                break;
            default: break;
        }
    }
}

// ---- batched ragged resume + append ----------------------------------------------------------------------------

__device__ __forceinline__ uint64_t shfl_up64(uint64_t v, int delta) {
    const uint32_t lo = __shfl_up(uint32_t(v), delta), hi = __shfl_up(uint32_t(v >> 32), delta);
    return (uint64_t(hi) << 32) | lo;
}
// Inclusive prefix sum across the 64 lanes of a wave (Hillis-Steele: six shuffle steps).
__device__ __forceinline__ uint64_t wave_scan(uint64_t v, int lane) {
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y = shfl_up64(v, o);
        if (lane >= o) v += y;
    }
    return v;
}

__device__ __forceinline__ uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

// Bytes of a slot's parked image (K/V blobs of ceil(L/ps) cells, 64-byte aligned, then the GDN rows).
__device__ __forceinline__ uint64_t kv_blob_stride(const BatchArgs& a, int64_t L) {
    const uint64_t ps = a.geo.page_size.d;
    const uint64_t cells = (uint64_t(L) + ps - 1) / ps * ps;
    return align_up(cells * a.geo.heads.d * a.geo.row_chunks.d * 16, 64);
}

// The batch's pre-pass, one wave: each lane one slot.  The staging offsets are an exclusive scan over the slots'
// padded image sizes.  The batch is all or nothing, like a restore that validates before its first write: if any
// slot's length is out of range or its image would run past the staging buffer, `ok` is 0, nothing is written and
// every lens_out entry is -1.
__global__ void __launch_bounds__(64) batch_prep_kernel(BatchArgs a) {
    const int lane = threadIdx.x;
    const bool live = lane < a.n_slots;
    const int64_t L = live ? a.lens[lane] : 0;
    bool ok = !live || (L >= 0 && L <= a.max_tokens);
    const uint64_t stride = live && ok ? kv_blob_stride(a, L) : 0;
    const uint64_t image = live && ok ? align_up(2 * uint64_t(a.n_qsa) * stride + a.gdn_bytes, 64) : 0;
    const uint64_t padded = align_up(image, 256);
    const uint64_t stage_end = wave_scan(padded, lane);
    if (stage_end > a.staging_bytes) ok = false;
    ok = __ballot(!ok) == 0;   // every lane agrees: the whole batch is valid
    if (live) {
        const uint64_t ps = a.geo.page_size.d;
        BatchSlot& S = a.slots[lane];
        S.len = ok ? L : -1;
        S.stage = stage_end - padded;
        S.stride = stride;
        S.need = ok ? int64_t((uint64_t(L) + uint64_t(a.chunk_tokens) + ps - 1) / ps) : 0;
        if (a.lens_out) a.lens_out[lane] = ok ? L + a.chunk_tokens : -1;
    }
    if (lane == 0) *a.ok = ok ? 1u : 0u;
}

// Every slot's logical pages into the inverse arena table (blockIdx.y = slot).
__global__ void __launch_bounds__(kThreads) batch_inverse_kernel(BatchArgs a) {
    const int slot = blockIdx.y;
    const int64_t lp = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (lp >= a.slots[slot].need) return;   // 0 for every slot of a refused batch
    const int32_t* table = reinterpret_cast<const int32_t*>(a.ptrs[2 * a.n_qsa + uint64_t(a.n_slots) * a.n_qsa * 2 + slot]);
    const int32_t p = *(gi32*) (table + lp);
    if (p >= 0 && int64_t(p) < a.arena_pages) a.inv[p] = int32_t((uint32_t(slot) << kBatchSlotShift) | uint32_t(lp));
}

// One 16 KiB tile of arena pages of K/V blob `blob` (K, V of layer blob / 2), in ascending arena order.  A page's
// chunk ip is row (h * ps + c) of the page, chunk ch: cell c of logical page lp is token lp * ps + c of its slot, from
// the staged image (whose pages have the arena's layout) below L and from the slot's chunk ([chunk][H][D], kv_append's
// mapping) in [L, L + chunk); cells past L + chunk are left alone.
// The slots' placement, staged in LDS by every workgroup of the move: a page's source address then costs the
// order's load and an LDS read, not a second global load.
struct BatchSlotsLds {
    int64_t len[kMaxBatchSlots];
    uint64_t stage[kMaxBatchSlots], stride[kMaxBatchSlots];
};

__device__ void batch_page_tile(const BatchArgs& a, const BatchSlotsLds& S, uint32_t blob, uint32_t w) {
    const MoveGeo& g = a.geo;
    const uint64_t page_bytes = uint64_t(g.page_chunks.d) * 16u, row_bytes = uint64_t(g.row_chunks.d) * 16u;
    const uint64_t* chunks = a.ptrs + 2 * a.n_qsa;
    uint8_t* arena = reinterpret_cast<uint8_t*>(a.ptrs[blob]);
    u32x4 v[kBatchChunksPerThread];
    int64_t dst[kBatchChunksPerThread];
    using gi64 = __attribute__((address_space(1))) const int64_t;
#pragma unroll
    for (int j = 0; j < kBatchChunksPerThread; ++j) {
        dst[j] = -1;
        const uint32_t vq = w * kBatchTileChunks + uint32_t(j * kThreads) + threadIdx.x;
        const uint32_t vp = fdiv(vq, g.page_chunks);
        const uint32_t ip = vq - vp * g.page_chunks.d;
        const int64_t pair = *(gi64*) (a.order + 2 * uint64_t(vp));   // (entry, arena page), little-endian
        const int32_t e = int32_t(uint32_t(pair)), phys = int32_t(uint32_t(uint64_t(pair) >> 32));
        if (e < 0) continue;
        const uint32_t slot = uint32_t(e) >> kBatchSlotShift, lp = uint32_t(e) & ((1u << kBatchSlotShift) - 1u);
        const int64_t L = S.len[slot];
        const uint32_t row = fdiv(ip, g.row_chunks), ch = ip - row * g.row_chunks.d;
        const uint32_t h = fdiv(row, g.page_size), c = row - h * g.page_size.d;
        const int64_t token = int64_t(lp) * g.page_size.d + c;
        if (token < L) {
            v[j] = ld16(a.staging + S.stage[slot] + uint64_t(blob) * S.stride[slot] + uint64_t(lp) * page_bytes +
                               ip * 16u);
        } else if (token < L + a.chunk_tokens) {
            const uint8_t* src = reinterpret_cast<const uint8_t*>(chunks[(uint64_t(slot) * a.n_qsa + blob / 2) * 2 + (blob & 1)]);
            v[j] = ld16(src + (uint64_t(token - L) * g.heads.d + h) * row_bytes + ch * 16u);
        } else {
            continue;
        }
        dst[j] = int64_t(phys) * int64_t(page_bytes) + int64_t(ip) * 16;
    }
#pragma unroll
    for (int j = 0; j < kBatchChunksPerThread; ++j)
        if (dst[j] >= 0) st16(arena + dst[j], v[j]);
}

// A refused batch writes nothing: its order holds no page (every slot's `need` is 0) and its slots' lengths are -1,
// which the GDN tiles check.
__global__ void __launch_bounds__(kThreads) sc_batch_kernel(BatchArgs a) {
    __shared__ BatchSlotsLds S;
    if (threadIdx.x < uint32_t(a.n_slots)) {
        const BatchSlot& x = a.slots[threadIdx.x];
        S.len[threadIdx.x] = x.len;
        S.stage[threadIdx.x] = x.stage;
        S.stride[threadIdx.x] = x.stride;
    }
    __syncthreads();
    const uint64_t kv_tiles = 2 * uint64_t(a.n_qsa) * a.kv_tiles;
    const uint64_t total = kv_tiles + uint64_t(a.n_slots) * a.gdn_tiles;
    const uint64_t* gdns = a.ptrs + 2 * a.n_qsa + uint64_t(a.n_slots) * a.n_qsa * 2 + a.n_slots;
    for (uint64_t tile = blockIdx.x; tile < total; tile += gridDim.x) {
        if (tile < kv_tiles) {
            const uint32_t t = uint32_t(tile);
            const uint32_t blob = __builtin_amdgcn_readfirstlane(fdiv(t, a.kv_tiles_div));
            batch_page_tile(a, S, blob, t - blob * a.kv_tiles);
        } else {
            const uint32_t t = uint32_t(tile - kv_tiles);
            const uint32_t slot = __builtin_amdgcn_readfirstlane(fdiv(t, a.gdn_tiles_div));
            if (S.len[slot] < 0) continue;
            MoveRow r{};
            r.src = a.staging + S.stage[slot] + 2 * uint64_t(a.n_qsa) * S.stride[slot];
            r.dst = reinterpret_cast<uint8_t*>(gdns[slot]);
            r.n = a.gdn_bytes / 16;
            tile_copy(r, t - slot * a.gdn_tiles, false);
        }
    }
}

// ---- synthetic inputs ----------------------------------------------------------------------------------------

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// Draw i of the stream keyed by `key` (SplitMix64 advanced i + 1 steps from the key).
__device__ __forceinline__ uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

__global__ void fill_uniform_f16_kernel(uint16_t* dst, uint64_t n, float lo, float span, uint64_t key) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x) {
        const float u = float(uint32_t(draw(key, i) >> 40)) * 0x1p-24f;
        const float x = __builtin_fmaf(span, u, lo);
        dst[i] = uint16_t(f16_bits_rne(__float_as_uint(x)));
    }
}

__global__ void fill_uniform_f32_kernel(float* dst, uint64_t n, float lo, float span, uint64_t key) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x) {
        const float u = float(uint32_t(draw(key, i) >> 40)) * 0x1p-24f;
        dst[i] = __builtin_fmaf(span, u, lo);
    }
}

__global__ void fill_normal_f32_kernel(float* dst, uint64_t n, uint64_t key) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x) {
        int64_t sum = 0;
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const uint64_t x = draw(key, i * 6 + k);
            sum += int64_t(x >> 40) + int64_t((x >> 16) & 0xFFFFFFull);
        }
        dst[i] = float(int32_t(sum - (int64_t(6) << 24))) * 0x1p-24f;
    }
}

__global__ void fill_bytes_kernel(uint8_t* dst, uint8_t value, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    const uint64_t head = (16u - (reinterpret_cast<uintptr_t>(dst) & 15u)) & 15u;
    const uint64_t pre = head < n ? head : n;
    const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid < pre) dst[gid] = value;
    const uint64_t body = (n - pre) / 16;
    const uint32_t w = uint32_t(value) * 0x01010101u;
    const u32x4 v = {w, w, w, w};
    for (uint64_t i = gid; i < body; i += stride) st16(dst + pre + i * 16, v);
    const uint64_t tail0 = pre + body * 16;
    for (uint64_t i = tail0 + gid; i < n; i += stride) dst[i] = value;
}

// Device-to-device copies, used where the source is another process's memory mapped by a memory handle (which the
// runtime's own copy may hand to a copy engine).  When source and destination share their alignment modulo 16 the
// copy is cut into 16 KiB tiles, one per workgroup, each thread issuing its four 16-byte non-temporal loads before its
// four non-temporal stores (the shape that measures fastest for a plain copy on this part: 3.3 GB in 1.10 ms against
// 1.15 ms with regular loads, three alternating pairs); one extra workgroup copies the unaligned head and the tail.
// Other pairs take a grid-stride byte loop.
constexpr uint64_t kCopyTile = 256 * 4 * 16;

__global__ void __launch_bounds__(256) copy_tiles_kernel(uint8_t* dst, const uint8_t* src, uint64_t n, uint64_t pre,
                                                        uint64_t tiles) {
    const uint32_t tid = threadIdx.x;
    if (blockIdx.x < tiles) {
        const uint64_t base = pre + uint64_t(blockIdx.x) * kCopyTile;
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = ld16(src + base + (u * 256 + tid) * 16);
#pragma unroll
        for (int u = 0; u < 4; ++u) st16(dst + base + (u * 256 + tid) * 16, v[u]);
        return;
    }
    for (uint64_t i = tid; i < pre; i += 256) dst[i] = src[i];
    const uint64_t tail0 = pre + tiles * kCopyTile;
    const uint64_t vecs = (n - tail0) / 16;
    for (uint64_t i = tid; i < vecs; i += 256) st16(dst + tail0 + i * 16, ld16(src + tail0 + i * 16));
    for (uint64_t i = tail0 + vecs * 16 + tid; i < n; i += 256) dst[i] = src[i];
}

__global__ void __launch_bounds__(256) copy_bytes_kernel(uint8_t* dst, const uint8_t* src, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * 256;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// Reads its share of the K/V bytes and folds them into one word per workgroup.
__global__ void __launch_bounds__(kThreads) decode_probe_kernel(const uint8_t* kv, uint64_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < n16; i += uint64_t(gridDim.x) * kThreads) {
        const u32x4 v = ld16(kv + i * 16);
        acc ^= v.x ^ (v.y * 3u) ^ (v.z * 5u) ^ (v.w * 7u);
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    __shared__ uint32_t s[kThreads / 64];
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = s[0] ^ s[1] ^ s[2] ^ s[3];
}

// Holds its stream for `ticks` ticks of the constant-rate wall clock, then exits: a stand-in for long work queued
// ahead of a transfer, so tests can show that an event-gated transfer does not start early.  Every exit path is
// bounded: the loop ends after `max_iters` sleeps even if the clock were not to advance.
__global__ void delay_kernel(uint64_t ticks, uint32_t max_iters) {
    const uint64_t t0 = wall_clock64();
    for (uint32_t i = 0; i < max_iters; ++i) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(100);
    }
}

// Every block of a streamed layer evicted (the reference's reset, src/kernels/cuda/kv_stream.cu:173-182).
__global__ void stream_reset_kernel(int32_t* table, int64_t n_blocks, int32_t* slot_block, int32_t* slot_stamp,
                                    int32_t* slot_ref, int64_t n_slots, int32_t* ctl) {
    const int64_t i0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x, stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = i0; i < n_blocks; i += stride) table[i] = -1;
    for (int64_t i = i0; i < n_slots; i += stride) {
        slot_block[i] = -1;
        slot_stamp[i] = -1;
        slot_ref[i] = 0;
    }
    if (i0 < 16) ctl[i0] = 0;
}

__global__ void ring_table_kernel(int32_t* table, int64_t n_blocks, int64_t n_slots) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n_blocks; i += int64_t(gridDim.x) * blockDim.x)
        table[i] = int32_t(i % n_slots);
}

// ---- destination order: the pre-pass of a plan whose rows write through page tables ------------------------------
// (OrderGroup, sc_internal.hpp.)  Three launches, one group (page table) per blockIdx.y.

// The inverse table: inv[table[lp]] = lp for the group's logical pages whose physical page is in the pool.
__global__ void __launch_bounds__(kThreads) order_scatter_kernel(const OrderGroup* __restrict__ groups) {
    const OrderGroup& G = groups[blockIdx.y];
    const int64_t lp = G.lp_lo + int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (lp >= G.lp_hi) return;
    const int32_t p = *(gi32*) (G.table + lp);
    if (p >= 0 && int64_t(p) < G.ld) G.inv[p] = int32_t(lp);
}

// Exclusive prefix of one value per thread across the workgroup; `total` gets the sum.
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t& total) {
    __shared__ uint32_t s_wave[kThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t x = v;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
    for (int w = 0; w < kThreads / 64; ++w) {
        if (w < wave) before += s_wave[w];
        total += s_wave[w];
    }
    __syncthreads();   // s_wave is reused by the next call
    return before + x - v;
}

// Entries per block of kOrderBlockPages physical pages.
__global__ void __launch_bounds__(kThreads) order_count_kernel(const OrderGroup* __restrict__ groups) {
    const OrderGroup& G = groups[blockIdx.y];
    const uint32_t b = blockIdx.x;
    if (b >= G.n_blocks) return;
    const int64_t base = int64_t(b) * kOrderBlockPages;
    uint32_t c = 0;
    for (int k = threadIdx.x; k < kOrderBlockPages; k += kThreads)
        if (base + k < G.ld && G.inv[base + k] >= 0) ++c;
    uint32_t total;
    (void) block_scan(c, total);
    if (threadIdx.x == 0) G.counts[b] = total;
}

// Each block sums the counts before it, writes its entries, ascending by physical page, at that prefix and clears them
// from inv; the last block fills the list past the last entry with -1.
__global__ void __launch_bounds__(kThreads) order_write_kernel(const OrderGroup* __restrict__ groups) {
    constexpr int kPer = kOrderBlockPages / kThreads;
    const OrderGroup& G = groups[blockIdx.y];
    const uint32_t b = blockIdx.x;
    if (b >= G.n_blocks) return;
    uint32_t before = 0;
    for (uint32_t i = threadIdx.x; i < b; i += kThreads) before += G.counts[i];
    uint32_t prefix;
    (void) block_scan(before, prefix);
    const int64_t base = int64_t(b) * kOrderBlockPages + int64_t(threadIdx.x) * kPer;
    int32_t e[kPer];
    uint32_t c = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        e[k] = base + k < G.ld ? G.inv[base + k] : -1;
        c += e[k] >= 0 ? 1u : 0u;
    }
    uint32_t total;
    uint32_t at = prefix + block_scan(c, total);
    const uint32_t width = G.pairs ? 2u : 1u;
#pragma unroll
    for (int k = 0; k < kPer; ++k)
        if (e[k] >= 0) {
            G.order[uint64_t(at) * width] = e[k];
            if (G.pairs) G.order[uint64_t(at) * width + 1] = int32_t(base + k);
            ++at;
            G.inv[base + k] = -1;
        }
    if (b + 1 == G.n_blocks)
        for (uint64_t i = (uint64_t(prefix) + total) * width + threadIdx.x; i < G.order_len * width; i += kThreads)
            G.order[i] = -1;
}

// ---- paged park / resume straight through pinned host memory ---------------------------------------------------
// (PagedImage, sc_internal.hpp.)  The blob of a tile is wave-uniform, so its pool and table pointers are read from the
// argument segment with scalar loads (indexing the argument array directly would copy it to scratch first).
__global__ void __launch_bounds__(kThreads) paged_image_kernel(PagedImage a, MoveGeo geo) {
    using karg = __attribute__((address_space(4))) const PagedImage*;
    const karg args = (karg) __builtin_amdgcn_kernarg_segment_ptr();
    const uint64_t total = uint64_t(a.n_blobs) * a.tiles_per_blob;
    for (uint64_t tile = blockIdx.x; tile < total; tile += gridDim.x) {
        const uint32_t t = uint32_t(tile);
        const uint32_t blob = __builtin_amdgcn_readfirstlane(fdiv(t, a.tiles_div));
        MoveRow r{};
        uint8_t* image = a.image + uint64_t(blob) * a.blob_stride;
        r.table = args->table[blob / 2];
        r.n = a.blob_chunks;
        r.ld = a.pool_pages;
        if (a.park) {
            r.src = args->pool[blob];
            r.dst = image;
        } else {
            r.src = image;
            r.dst = args->pool[blob];
        }
        if (r.table) tile_pages<true>(r, geo, t - blob * a.tiles_per_blob, !a.park);
        else tile_pages<false>(r, geo, t - blob * a.tiles_per_blob, !a.park);
    }
}

}  // namespace

// ---- launchers (host) ------------------------------------------------------------------------------------------

hipError_t launch_paged_image(const PagedImage& a, const MoveGeo& geo, hipStream_t stream) {
    const uint64_t tiles = uint64_t(a.n_blobs) * a.tiles_per_blob;
    if (tiles == 0) return hipSuccess;
    if (!a.image || a.n_blobs > 2u * kPagedLayers || tiles >= (uint64_t(1) << 32)) return hipErrorInvalidValue;
    const uint64_t grid = tiles < 65536 ? tiles : 65536;
    hipLaunchKernelGGL(paged_image_kernel, dim3(unsigned(grid)), dim3(kThreads), 0, stream, a, geo);
    return hipGetLastError();
}

// ---- re-pointing a plan without allocating -----------------------------------------------------------------------
// A retargeted carve plan (sc_plan_retarget) keeps its device table, tile map and order workspace and takes new rows:
// the host writes them, and the order groups, into pinned staging, and this kernel copies them into the plan's device
// table and rebuilds the tile -> row map, on the stream the launches use, so nothing is allocated and the host does
// not wait.  Workgroup b < n_rows copies row b and writes the map entries of its tiles (the last row also takes the
// pad entry of an odd tile count); workgroup n_rows copies the order groups.
namespace {
__global__ void __launch_bounds__(kThreads) retarget_kernel(const MoveRow* staged_rows, int32_t n_rows,
                                                            const OrderGroup* staged_groups, int32_t n_groups,
                                                            MoveRow* rows, uint16_t* tile_row, uint64_t n_tiles,
                                                            OrderGroup* groups) {
    const int32_t b = int32_t(blockIdx.x);
    if (b == n_rows) {
        const uint32_t* s = reinterpret_cast<const uint32_t*>(staged_groups);
        uint32_t* d = reinterpret_cast<uint32_t*>(groups);
        const uint32_t words = uint32_t(n_groups) * uint32_t(sizeof(OrderGroup) / 4);
        for (uint32_t i = threadIdx.x; i < words; i += kThreads) d[i] = s[i];
        return;
    }
    __shared__ uint64_t s_span[2];
    if (threadIdx.x == 0) {
        s_span[0] = staged_rows[b].tile0;
        s_span[1] = b + 1 < n_rows ? staged_rows[b + 1].tile0 : n_tiles + (n_tiles & 1u);
    }
    if (threadIdx.x < sizeof(MoveRow) / 4)
        reinterpret_cast<uint32_t*>(rows + b)[threadIdx.x] = reinterpret_cast<const uint32_t*>(staged_rows + b)[threadIdx.x];
    __syncthreads();
    const uint64_t t1 = s_span[1];
    for (uint64_t t = s_span[0] + threadIdx.x; t < t1; t += kThreads) tile_row[t] = uint16_t(b);
}
}  // namespace

hipError_t launch_retarget(const MoveRow* staged_rows, int32_t n_rows, const OrderGroup* staged_groups,
                           int32_t n_groups, MoveRow* rows, uint16_t* tile_row, uint64_t n_tiles, OrderGroup* groups,
                           hipStream_t stream) {
    if (n_rows < 0 || n_groups < 0 || (n_rows && (!staged_rows || !rows || !tile_row)) ||
        (n_groups && (!staged_groups || !groups)))
        return hipErrorInvalidValue;
    if (n_rows == 0 && n_groups == 0) return hipSuccess;
    hipLaunchKernelGGL(retarget_kernel, dim3(unsigned(n_rows) + 1), dim3(kThreads), 0, stream, staged_rows, n_rows,
                       staged_groups, n_groups, rows, tile_row, n_tiles, groups);
    return hipGetLastError();
}

hipError_t launch_page_order(const OrderGroup* groups, int32_t n_groups, int64_t max_pages, uint32_t max_blocks,
                             hipStream_t stream) {
    if (n_groups <= 0) return hipSuccess;
    if (!groups || n_groups > 65535 || max_pages <= 0 || max_blocks == 0) return hipErrorInvalidValue;
    const dim3 threads(kThreads);
    hipLaunchKernelGGL(order_scatter_kernel, dim3(unsigned((max_pages + kThreads - 1) / kThreads), unsigned(n_groups)),
                       threads, 0, stream, groups);
    hipLaunchKernelGGL(order_count_kernel, dim3(max_blocks, unsigned(n_groups)), threads, 0, stream, groups);
    hipLaunchKernelGGL(order_write_kernel, dim3(max_blocks, unsigned(n_groups)), threads, 0, stream, groups);
    return hipGetLastError();
}

hipError_t launch_batch(const BatchArgs& args, const OrderGroup* arena, uint32_t arena_blocks, int64_t grid,
                        hipStream_t stream) {
    if (grid <= 0 || args.n_slots < 1 || args.n_slots > kMaxBatchSlots || !args.slots || !args.ok)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(batch_prep_kernel, dim3(1), dim3(64), 0, stream, args);
    if (args.n_qsa > 0 && args.kv_tiles > 0) {
        if (!arena || !arena_blocks || args.table_pages <= 0) return hipErrorInvalidValue;
        hipLaunchKernelGGL(batch_inverse_kernel, dim3(unsigned((args.table_pages + kThreads - 1) / kThreads),
                                                      unsigned(args.n_slots)),
                           dim3(kThreads), 0, stream, args);
        hipLaunchKernelGGL(order_count_kernel, dim3(arena_blocks, 1), dim3(kThreads), 0, stream, arena);
        hipLaunchKernelGGL(order_write_kernel, dim3(arena_blocks, 1), dim3(kThreads), 0, stream, arena);
    }
    hipLaunchKernelGGL(sc_batch_kernel, dim3(unsigned(grid)), dim3(kThreads), 0, stream, args);
    return hipGetLastError();
}

hipError_t launch_stream_reset(int32_t* table, int64_t n_blocks, int32_t* slot_block, int32_t* slot_stamp,
                               int32_t* slot_ref, int64_t n_slots, int32_t* ctl, hipStream_t stream) {
    const int64_t n = n_blocks > n_slots ? n_blocks : n_slots;
    const int64_t blocks = (n + 255) / 256 < 1024 ? ((n + 255) / 256 > 0 ? (n + 255) / 256 : 1) : 1024;
    hipLaunchKernelGGL(stream_reset_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, table, n_blocks,
                       slot_block, slot_stamp, slot_ref, n_slots, ctl);
    return hipGetLastError();
}

hipError_t launch_ring_table(int32_t* table, int64_t n_blocks, int64_t n_slots, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t blocks = (n_blocks + 255) / 256 < 1024 ? (n_blocks + 255) / 256 : 1024;
    hipLaunchKernelGGL(ring_table_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, table, n_blocks, n_slots);
    return hipGetLastError();
}

hipError_t launch_move(const MoveRow* rows, const uint16_t* tile_row, const MoveGeo& geo, uint64_t n_tiles,
                       int64_t grid, int32_t mix, bool xcd, hipStream_t stream, const uint32_t* gate) {
    if (n_tiles == 0) return hipSuccess;
    if (!rows || !tile_row || grid <= 0 || mix < kMixPlain || mix > kMixQuantPaged) return hipErrorInvalidValue;
    const dim3 blocks(unsigned(uint64_t(grid) < n_tiles ? uint64_t(grid) : n_tiles)), threads(kThreads);
    switch (mix) {
        case kMixPlain:
            hipLaunchKernelGGL(sc_move_kernel<kMixPlain>, blocks, threads, 0, stream, rows, tile_row, geo, n_tiles, gate, xcd);
            break;
        case kMixWide:
            hipLaunchKernelGGL(sc_move_kernel<kMixWide>, blocks, threads, 0, stream, rows, tile_row, geo, n_tiles, gate, xcd);
            break;
        case kMixQuant:
            hipLaunchKernelGGL(sc_move_kernel<kMixQuant>, blocks, threads, 0, stream, rows, tile_row, geo, n_tiles, gate, xcd);
            break;
        case kMixQuantPaged:
            hipLaunchKernelGGL(sc_move_kernel<kMixQuantPaged>, blocks, threads, 0, stream, rows, tile_row, geo, n_tiles, gate,
                               xcd);
            break;
        default:
            hipLaunchKernelGGL(sc_move_kernel<kMixAll>, blocks, threads, 0, stream, rows, tile_row, geo, n_tiles, gate, xcd);
            break;
    }
    return hipGetLastError();
}

// ---- kv_append: one call's rows in the kernel arguments -----------------------------------------------------------
// The reference's per-layer prefill writers (kv_append, src/prefill/kernels.cu:558-625; kv_append_q4,
// src/kernels/cuda/kv_q4.cu:111-135,205-215) take their destinations as arguments and allocate nothing, so this launch
// takes its up to six rows the same way.  Row k owns tiles [k * tiles_per_row, (k + 1) * tiles_per_row); the switch
// reads the selected row with scalar loads from the argument segment (an indexed read of the argument array would
// copy it to scratch first).
namespace {
template <int kKind>
__global__ void __launch_bounds__(kThreads) sc_append_kernel(AppendRows rows, int32_t n_rows, uint64_t tiles_per_row,
                                                              MoveGeo geo) {
    const uint64_t n_tiles = uint64_t(n_rows) * tiles_per_row;
    for (uint64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int k = __builtin_amdgcn_readfirstlane(int(tile / tiles_per_row));
        MoveRow r;
        switch (k) {
            case 0: r = rows.row[0]; break;
            case 1: r = rows.row[1]; break;
            case 2: r = rows.row[2]; break;
            case 3: r = rows.row[3]; break;
            case 4: r = rows.row[4]; break;
            default: r = rows.row[5]; break;
        }
        const uint64_t local = tile - uint64_t(k) * tiles_per_row;
        if constexpr (kKind == kKv32) {
            if (r.table) tile_kv32<true>(r, geo, local);
            else tile_kv32<false>(r, geo, local);
        } else if constexpr (kKind == kKvQ8) {
            if (r.table) tile_q8<true>(r, geo, local);
            else tile_q8<false>(r, geo, local);
        } else {
            tile_q4(r, geo, local);
        }
    }
}
}  // namespace

hipError_t launch_append(const AppendRows& rows, int n_rows, uint64_t tiles_per_row, const MoveGeo& geo, int32_t kind,
                         hipStream_t stream) {
    if (n_rows <= 0 || tiles_per_row == 0) return hipSuccess;
    if (n_rows > kAppendMaxRows || (kind != kKv32 && kind != kKvQ8 && kind != kKvQ4)) return hipErrorInvalidValue;
    const uint64_t n_tiles = uint64_t(n_rows) * tiles_per_row;
    // one workgroup per tile, as the plans launch (the 12 per-layer calls at 128K measured alike with 65536 workgroups
    // for f16 and 262144 for the quantizing rows: f16 1.636 against 1.640 ms, int8 1.409 against 1.410)
    const uint64_t cap = uint64_t(1) << 20;
    const dim3 blocks(unsigned(n_tiles < cap ? n_tiles : cap)), threads(kThreads);
    switch (kind) {
        case kKv32:
            hipLaunchKernelGGL(sc_append_kernel<kKv32>, blocks, threads, 0, stream, rows, n_rows, tiles_per_row, geo);
            break;
        case kKvQ8:
            hipLaunchKernelGGL(sc_append_kernel<kKvQ8>, blocks, threads, 0, stream, rows, n_rows, tiles_per_row, geo);
            break;
        default:
            hipLaunchKernelGGL(sc_append_kernel<kKvQ4>, blocks, threads, 0, stream, rows, n_rows, tiles_per_row, geo);
            break;
    }
    return hipGetLastError();
}

static unsigned fill_grid(uint64_t n) {
    const uint64_t b = (n + 255) / 256;
    return unsigned(b < 8192 ? (b ? b : 1) : 8192);
}

uint64_t synth_key(uint64_t seed, uint64_t stream_id);

hipError_t launch_fill_uniform_f16(uint16_t* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t sid,
                                   hipStream_t stream) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(fill_uniform_f16_kernel, dim3(fill_grid(n)), dim3(256), 0, stream, dst, n, lo, hi - lo,
                       synth_key(seed, sid));
    return hipGetLastError();
}

hipError_t launch_fill_uniform_f32(float* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t sid,
                                   hipStream_t stream) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(fill_uniform_f32_kernel, dim3(fill_grid(n)), dim3(256), 0, stream, dst, n, lo, hi - lo,
                       synth_key(seed, sid));
    return hipGetLastError();
}

hipError_t launch_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t sid, hipStream_t stream) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(fill_normal_f32_kernel, dim3(fill_grid(n)), dim3(256), 0, stream, dst, n,
                       synth_key(seed, sid));
    return hipGetLastError();
}

// A plan's tile -> row table, one thread per entry: the last row whose first tile is at or before the entry (rows are in
// tile order, and a row that moves nothing shares its first tile with the next, so the row that owns the tile is the
// last of them); the padding entry past the last tile names the last row.  Built on the device from the uploaded rows
// so that a plan's creation uploads its rows only (the table is 2 bytes per 8 KiB tile: 806 KB for the 128K slot,
// whose upload from pageable memory took 0.35 ms).
__global__ void tile_rows_kernel(const MoveRow* rows, uint32_t n_rows, uint16_t* tile_row, uint64_t n_entries,
                                 uint64_t tiles) {
    const uint64_t t = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n_entries) return;
    uint32_t k = n_rows - 1;
    if (t < tiles) {
        uint32_t lo = 0, hi = n_rows - 1;   // the last row with tile0 <= t
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo + 1) / 2;
            if (rows[mid].tile0 <= t) lo = mid;
            else hi = mid - 1;
        }
        k = lo;
    }
    tile_row[t] = uint16_t(k);
}

hipError_t launch_tile_rows(const MoveRow* rows, uint32_t n_rows, uint16_t* tile_row, uint64_t n_entries, uint64_t tiles,
                            hipStream_t stream) {
    if (!n_entries) return hipSuccess;
    if (!n_rows) return hipErrorInvalidValue;
    const uint64_t blocks = (n_entries + 255) / 256;
    hipLaunchKernelGGL(tile_rows_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, rows, n_rows, tile_row, n_entries,
                       tiles);
    return hipGetLastError();
}

hipError_t launch_fill_bytes(void* dst, uint8_t value, uint64_t n, hipStream_t stream) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(fill_grid(n / 16 + 16)), dim3(256), 0, stream,
                       static_cast<uint8_t*>(dst), value, n);
    return hipGetLastError();
}

hipError_t launch_copy_bytes(void* dst, const void* src, uint64_t n, hipStream_t stream) {
    if (!n) return hipSuccess;
    auto* d = static_cast<uint8_t*>(dst);
    auto* s = static_cast<const uint8_t*>(src);
    const uintptr_t da = reinterpret_cast<uintptr_t>(d), sa = reinterpret_cast<uintptr_t>(s);
    if (((da ^ sa) & 15u) != 0) {
        const uint64_t blocks = (n + 255) / 256;
        hipLaunchKernelGGL(copy_bytes_kernel, dim3(unsigned(blocks < 16384 ? blocks : 16384)), dim3(256), 0, stream, d, s,
                           n);
        return hipGetLastError();
    }
    const uint64_t head = (16u - (da & 15u)) & 15u;
    const uint64_t pre = head < n ? head : n;
    const uint64_t tiles = (n - pre) / kCopyTile;
    if (tiles + 1 > 0x7FFFFFFFull) return hipErrorInvalidValue;   // 32 TiB: beyond any allocation here
    hipLaunchKernelGGL(copy_tiles_kernel, dim3(unsigned(tiles + 1)), dim3(256), 0, stream, d, s, n, pre, tiles);
    return hipGetLastError();
}

hipError_t launch_delay(uint64_t ticks, uint32_t max_iters, hipStream_t stream) {
    hipLaunchKernelGGL(delay_kernel, dim3(1), dim3(64), 0, stream, ticks, max_iters);
    return hipGetLastError();
}

hipError_t launch_decode_probe(const void* kv, uint64_t n_bytes, uint32_t* sink, int64_t workgroups,
                               hipStream_t stream) {
    if (workgroups <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(decode_probe_kernel, dim3(unsigned(workgroups)), dim3(kThreads), 0, stream,
                       static_cast<const uint8_t*>(kv), n_bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace sc
