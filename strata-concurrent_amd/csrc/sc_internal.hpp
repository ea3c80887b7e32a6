// sc_internal.hpp - the handoff table's row format and the launch geometry, shared by the host plan builder
// (sc_capi.cpp) and the move kernel (sc_kernels.hip).
//
// The handoff table is one row per moved blob.  Every row describes a flat space of 16-byte CHUNKS (or, for
// the conv history, of channels) and a closed-form address map from a chunk index to its source and
// destination byte offsets.  A launch walks the concatenation of all rows in TILES of kTileChunks chunks, so
// one launch moves every layer of a handoff whatever the mix of kinds.
#pragma once

#include <cstdint>
#include <string>

namespace sc {

// The C-ABI's per-thread error record (sc_last_error), for entry points defined outside sc_capi.cpp.
int record_ok();
int record_error(int code, const std::string& message);

constexpr int kThreads = 256;            // one workgroup = 4 wave64
// 16-byte chunks in flight per thread per tile: 8 KiB tiles measured faster than 16 KiB ones for the 128K carve
// (1.045-1.053 against 1.064-1.074 ms), the paged carve in source order (1.20 against 1.24 ms) and the per-layer f32
// appends (1.57 against 1.64 ms), alike for the destination-ordered paged carve; 4 KiB (1.26 ms) and 32 KiB (1.11 ms)
// tiles measured slower.
constexpr int kChunksPerThread = 2;
constexpr int kTileChunks = kThreads * kChunksPerThread;   // 512 chunks = 8 KiB per tile
// The batched resume's page tiles keep 16 KiB (4 pages of 4 KiB): config 5 measured 4.98-5.02 ms with them against
// 5.08-5.10 ms with 8 KiB tiles.
constexpr int kBatchChunksPerThread = 4;
constexpr int kBatchTileChunks = kThreads * kBatchChunksPerThread;
constexpr int kConvTileChannels = 512;   // channels per conv-history tile (LDS-staged transpose)
constexpr int kMaxHist = 4;              // d_conv - 1 rows of history the conv tile supports

// Row kinds.
enum MoveKind : int32_t {
    kKv16 = 1,          // prefill K or V rows [T][H][D] f16 -> paged pool rows (page table, pos0)
    kKv32 = 2,          // the same from f32 rows, rounded to f16 (round to nearest even)
    kRec = 3,           // recurrence [HV][S][S] -> (S, HV, S)
    kConv = 4,          // conv input rows [rows][C] -> history [C][hist] (LDS-staged transpose)
    kPagesScatter = 5,  // contiguous pages -> pool pages through the page table
    kPagesGather = 6,   // pool pages through the page table -> contiguous pages
    kCopy = 7,          // contiguous 16-byte chunks
    kZero = 8,          // zero-fill 16-byte chunks (padding and stale-cell tails of an image)
    kKvQ8 = 9,          // f32 rows [T][H][256] -> int8 codes [prow][256] + f16 scales [prow][4] (quantizing kv_append)
    kKvQ4 = 10,         // f32 rows [T][H][256] (already rotated) -> q4_0 blocks [prow][8 x 18 B]
};

// The kernel instances: each compiles the tiles of a set of row kinds, so a plan of plain moves is not held to the
// register budget of the f32 rounding or the quantizing tiles.  A plan launches the smallest instance whose set
// holds every kind it has (mix_of).
enum MoveMix : int32_t {
    kMixPlain = 0,        // kKv16, kRec, kConv, kPages*, kCopy, kZero
    kMixWide = 1,         // plain + kKv32
    kMixQuant = 2,        // plain + kKvQ8, kKvQ4
    kMixAll = 3,          // every kind
    kMixQuantPaged = 4,   // kMixQuant with the int8 rows through a page table staged in LDS (a separate instance, so
                          // that the identity carve keeps the code of the instance without the staging)
};
constexpr int32_t mix_of(bool has_kv32, bool has_quant, bool quant_tables = false) {
    return has_quant ? (has_kv32 ? kMixAll : quant_tables ? kMixQuantPaged : kMixQuant)
                     : (has_kv32 ? kMixWide : kMixPlain);
}

// Quantizing rows move one (token, head) row of 256 values per wave at a time: a tile is 16 rows (16 KiB of f32).
constexpr int kQuantUnitsPerTile = 16;
constexpr int kQuantDim = 256;

// Division by a runtime constant d >= 1 for 32-bit numerators: q = (umulhi(n, m) + n) >> s with
// s = ceil(log2 d), m = floor(2^32 * (2^s - d) / d) + 1 (the round-up method of Granlund and Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994).  The sum is formed in 64 bits.
struct FastDiv {
    uint32_t d = 1, m = 1, s = 0;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) ++s;
    f.s = s;
    f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
    return f;
}

// One row of the handoff table (device-resident, 72 bytes).
struct MoveRow {
    int32_t kind;
    int32_t aux;            // kKv*: source tokens (rows past them are zero-filled); kConv: history rows
                            // (d_conv - 1) | 0x100 when the sequence is fresh (older history reads as zero)
    uint64_t tile0;         // first global tile of this row
    const uint8_t* src;
    uint8_t* dst;
    const int32_t* table;   // page table (destination side for kKv*/kPagesScatter, source side for kPagesGather)
    uint64_t n;             // chunks (kKv*, kRec, kPages*, kCopy, kZero) or channels (kConv)
    int64_t pos0;           // kKv*: first decode cell; kConv: rows available in the source
    int64_t ld;             // kConv: source row stride in floats; kKv*, kPages*: physical pages in the pool
    uint8_t* dst2;          // kKvQ8: the f16 scale pool
    const int32_t* order;   // kKv16, kKv32, kPagesScatter through a table: the logical pages in the order of their
                            // physical pages, then -1 up to the row's last tile, rebuilt on the device before every
                            // launch; null: the tiles follow the source
};
static_assert(sizeof(MoveRow) == 80, "handoff table rows are 80 bytes");

// Destination-ordered pages.  A launch's concurrent tiles that follow the source write pages scattered over the whole
// pool when the page table is a permutation; visiting the logical pages in the order of their physical pages makes the
// writes one ascending run and scatters the reads instead, which this part takes better with non-temporal stores
// (a 3.3 GB copy of permuted 4 KiB pages measured 64% of HBM peak in source order, 67.5-68% in destination order).
// The order of one page table is rebuilt before every launch, since the table may change between launches: the
// inverse table (physical page -> logical page) is scattered into `inv`, each block of kOrderBlockPages physical
// pages counts its entries, and each block then writes its logical pages, ascending, after those of the blocks
// before it, and clears its part of `inv` for the next launch.
constexpr int kOrderBlockPages = 4096;
struct OrderGroup {
    const int32_t* table;   // logical page -> physical page
    int32_t* inv;           // [ld] physical page -> logical page; -1 between launches
    int32_t* order;         // [order_len]: the pages, then -1
    uint32_t* counts;       // [n_blocks]: entries per block of physical pages
    int64_t lp_lo, lp_hi;   // the logical pages the plan's rows of this table touch
    int64_t ld;             // physical pages in the pool
    uint64_t order_len;     // >= the pages of the rows' tiles: ceil(tiles * kTileChunks / page chunks)
    uint32_t n_blocks;
    uint32_t pairs;         // 1: order holds (entry, physical page) pairs, as the batched launch reads it
};

// Geometry every row of one plan shares.
struct MoveGeo {
    FastDiv row_chunks;     // chunks per 512-byte-class row: D*2/16 (K/V) ...
    FastDiv heads;          // n_head_kv
    FastDiv page_size;      // cells per page
    FastDiv rec_chunks;     // S*4/16
    FastDiv v_heads;        // HV
    FastDiv page_chunks;    // chunks per page: H*ps*D*2/16
    uint32_t state;         // S
    uint32_t pad;
};

// Arguments of the batched ragged resume + append launch (sc_plan_resume_append).  `ptrs` is one device block
// of pointers: [2*n_qsa arenas (K, V of layer j at 2j, 2j+1)] [n_slots*n_qsa*2 chunk sources, slot-major]
// [n_slots page tables] [n_slots GDN row bases].
//
// A launch is a pre-pass and the move.  The pre-pass (one workgroup) checks every slot's length and places its image
// in the staging buffer (a wave-level scan over the slots), then the arena's destination order is built as for a
// page table: every slot's logical pages [0, need) scattered into the inverse arena table as (slot << 25 | page),
// counted and compacted into (entry, arena page) pairs in ascending arena order.  The move then assembles each arena
// page in that order - its parked cells from the slot's staged image, its chunk cells from the slot's chunk - so the
// launch writes the arena as one ascending run, and copies every slot's GDN rows.
constexpr int kMaxBatchSlots = 64;   // one wave64 lane per slot in the offset scan
constexpr int kBatchSlotShift = 25;  // an arena entry is slot << 25 | logical page (pages < 2^25)
struct BatchSlot {
    int64_t len;       // L, or -1 when the batch is refused
    uint64_t stage;    // staging offset of the slot's image
    uint64_t stride;   // bytes between the image's K/V blobs
    int64_t need;      // logical pages the slot writes: ceil((L + chunk) / ps)
};
struct BatchArgs {
    const int64_t* lens;
    int64_t* lens_out;
    const uint8_t* staging;
    uint64_t staging_bytes;
    const uint64_t* ptrs;
    int32_t n_slots, n_qsa;
    int64_t max_tokens, chunk_tokens, arena_pages, table_pages;
    uint64_t gdn_bytes;      // all GDN rows of one slot
    MoveGeo geo;
    // the plan's workspace
    BatchSlot* slots;        // [n_slots]
    uint32_t* ok;            // 1 when every slot's length is in range and every image fits the staging buffer
    int32_t* inv;            // [arena_pages] arena page -> slot << 25 | logical page; -1 between launches
    const int32_t* order;    // [2 * order_len]: (entry, arena page) pairs in ascending arena order, then -1
    uint32_t kv_tiles;       // tiles per K/V blob: ceil(order_len pages * page chunks / kBatchTileChunks)
    FastDiv kv_tiles_div;    // kv_tiles, for the blob of a tile
    uint32_t gdn_tiles;      // tiles per slot's GDN rows
    FastDiv gdn_tiles_div;
};

// The rows of one kv_append call (sc_kv_append_async, sc_kv_append_q4_async), carried in the kernel arguments
// rather than a device table: K and V into the paged pool, into the host copy and into the staging pool.  Every row
// is of one kind (kKv32, kKvQ8 or kKvQ4) and spans the same number of tiles.
constexpr int kAppendMaxRows = 6;
struct AppendRows {
    MoveRow row[kAppendMaxRows];
};

// A paged slot parked into, or resumed from, a pinned host image by one kernel that writes or reads the mapped host
// memory itself: every K/V page goes through its layer's table between the pool and the image's packed blob, with no
// staging copy in HBM and nothing allocated.  Up to kPagedLayers QSA layers per launch, their pointers in the kernel
// arguments (read through the argument segment with scalar loads).
constexpr int kPagedLayers = 32;
struct PagedImage {
    uint8_t* pool[2 * kPagedLayers];     // K, V of each layer (device)
    const int32_t* table[kPagedLayers];  // the layer's page table (null: identity)
    uint8_t* image;                      // the image's first K/V blob of this launch (pinned host memory)
    uint64_t blob_stride;                // bytes between the image's K/V blobs
    uint64_t blob_chunks;                // 16-byte chunks per blob: cells * H * row_chunks
    int64_t pool_pages;                  // physical pages per pool
    uint32_t n_blobs, park;              // 2 * layers of this launch; 1: pool -> image, 0: image -> pool
    uint32_t tiles_per_blob;
    FastDiv tiles_div;
};

// The parallel FNV-1a (sc_hash.hip): bytes per lane segment, and where its workspace keeps what.
constexpr int kFnvLaneBytes = 256;
struct FnvWorkspace {
    uint64_t segments = 0, groups = 0;
    uint64_t off_ctl = 0, off_status = 0, stride = 0;   // stride: status words per level
    uint64_t bytes = 0;
};
FnvWorkspace fnv_workspace(uint64_t n);

// The gather fused with the hash (sc_hash_map_*): the payload [0, n) as extents sorted by offset, every byte in exactly
// one.  A self extent's bytes are already in the payload (written earlier on the stream, or left as they are); a copy
// extent's come from a contiguous source, a pages extent's from pool pages through a page table (a page whose entry is
// negative or past the pool is left as the payload holds it, as the page gather leaves it), a zero extent's are zeros.
enum HashExtentKind : uint32_t { kExtSelf = 0, kExtCopy = 1, kExtPages = 2, kExtZero = 3 };
struct HashExtent {
    uint64_t off, end;       // payload bytes [off, end), 16-byte aligned
    const uint8_t* src;      // copy: the source of byte `off`; pages: the pool
    const int32_t* table;    // pages: logical -> physical page (null: identity)
    int64_t ld;              // pages: physical pages of the pool
    uint32_t kind;
    uint32_t page_chunks;    // pages: 16-byte chunks per page
};
static_assert(sizeof(HashExtent) == 48, "hash extents are 48 bytes");
// Lanes of one hash workgroup: 256 (64 KiB) hashed 3.3 GB in 1.77 ms, against 4.84, 2.53 and 2.22 ms with 64, 128
// and 512 (more workgroups mean more look-backs per byte, larger ones fewer resident workgroups per CU).
constexpr int kFnvThreads = 256;
constexpr int kFnvGroupBytes = kFnvThreads * kFnvLaneBytes;   // the payload bytes of one hash workgroup
// The carries of a hashed input: the low byte of the running hash after each whole 64 KiB workgroup whose end lies
// strictly inside the input, one byte per boundary (fnv_carry_count).  A launch may write them (`out`); a check given
// them (`in`) starts every workgroup from the carry before it instead of looking back across workgroups, and checks
// that the low byte it ends with is the carry after it.
struct FnvCarries {
    const uint8_t* in = nullptr;
    uint8_t* out = nullptr;
};
constexpr uint64_t fnv_carry_count(uint64_t bytes) { return bytes ? (bytes - 1) / uint64_t(kFnvGroupBytes) : 0; }
// One hash workgroup's part of a map, built with the map so that the workgroup reads it in one scalar load after its
// ticket: where its payload bytes lie, the extent holding its first byte and, when all its bytes lie in at most two
// extents (a workgroup inside one blob or across one blob boundary), those two, so that its lanes gather without
// reading the extent table.
struct HashGroup {
    uint8_t* base;       // payload byte o of this workgroup is at base + o (its segment's start less the segment offset)
    uint32_t first;      // the extent holding the workgroup's first byte
    uint32_t two;        // 1: the workgroup's gathered bytes lie in x[0] and x[1]
    HashExtent x[2];     // the extent `first` and the one after it (zeros past the last)
    uint64_t pad[2];
};
static_assert(sizeof(HashGroup) == 128, "hash groups are 128 bytes");
struct HashMapArgs {
    const HashExtent* ext;   // null: the plain hash of `data`
    const HashGroup* grp;    // per workgroup (maps that gather)
    uint8_t* const* seg;     // the payload's segments: byte o is at seg[o / seg_bytes] + o % seg_bytes
    uint64_t seg_bytes;      // a multiple of kFnvGroupBytes, so no workgroup's bytes straddle two segments
    uint64_t n_total;        // payload bytes gathered (n rounded down to whole lane segments is hashed in the kernel)
    uint32_t store;          // 0: the sources are only read and hashed (a payload hashed where it lies)
};

}  // namespace sc
