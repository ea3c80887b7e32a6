// sc_capi.cpp - the extern "C" layer of libsc_handoff.so (declared in include/sc_handoff.h).
//
// Every entry point validates its whole request on the host before the first HIP call, so a refusal
// (SC_EINVAL / SC_ERANGE) has enqueued nothing and written nothing - the reference's "invalid images are
// rejected before any CUDA call/write" contract (include/strata/core/conversation_snapshot.hpp:104-105).  A HIP
// failure after that point is SC_EHIP: the destination may be partly written, as the reference's
// `transfer_failed` (conversation_snapshot.hpp:103-108).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <exception>
#include <limits>
#include <new>
#include <string>
#include <vector>

#include "sc_handoff.h"
#include "sc_internal.hpp"

namespace sc {
hipError_t launch_append(const AppendRows& rows, int n_rows, uint64_t tiles_per_row, const MoveGeo& geo, int32_t kind,
                         hipStream_t stream);
hipError_t launch_move(const MoveRow* rows, const uint16_t* tile_row, const MoveGeo& geo, uint64_t n_tiles,
                       int64_t grid, int32_t mix, bool xcd, hipStream_t stream, const uint32_t* gate = nullptr);
hipError_t launch_page_order(const OrderGroup* groups, int32_t n_groups, int64_t max_pages, uint32_t max_blocks,
                             hipStream_t stream);
hipError_t launch_retarget(const MoveRow* staged_rows, int32_t n_rows, const OrderGroup* staged_groups,
                           int32_t n_groups, MoveRow* rows, uint16_t* tile_row, uint64_t n_tiles, OrderGroup* groups,
                           hipStream_t stream);
hipError_t launch_paged_image(const PagedImage& a, const MoveGeo& geo, hipStream_t stream);
hipError_t launch_fill_uniform_f16(uint16_t* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t sid,
                                   hipStream_t stream);
hipError_t launch_fill_uniform_f32(float* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t sid,
                                   hipStream_t stream);
hipError_t launch_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t sid, hipStream_t stream);
hipError_t launch_fill_bytes(void* dst, uint8_t value, uint64_t n, hipStream_t stream);
hipError_t launch_copy_bytes(void* dst, const void* src, uint64_t n, hipStream_t stream);
hipError_t launch_tile_rows(const MoveRow* rows, uint32_t n_rows, uint16_t* tile_row, uint64_t n_entries, uint64_t tiles,
                            hipStream_t stream);
hipError_t launch_decode_probe(const void* kv, uint64_t n_bytes, uint32_t* sink, int64_t workgroups,
                               hipStream_t stream);
hipError_t launch_batch(const BatchArgs& args, const OrderGroup* arena, uint32_t arena_blocks, int64_t grid,
                        hipStream_t stream);
hipError_t launch_delay(uint64_t ticks, uint32_t max_iters, hipStream_t stream);
hipError_t launch_stream_reset(int32_t* table, int64_t n_blocks, int32_t* slot_block, int32_t* slot_stamp,
                               int32_t* slot_ref, int64_t n_slots, int32_t* ctl, hipStream_t stream);
hipError_t launch_ring_table(int32_t* table, int64_t n_blocks, int64_t n_slots, hipStream_t stream);
hipError_t launch_fnv1a64(const void* data, uint64_t n, uint64_t seed, const uint64_t* seed_dev, uint64_t* out,
                          uint32_t* fault_out, void* workspace, hipStream_t stream, uint64_t expected = 0,
                          uint32_t* verdict = nullptr, const FnvCarries& carries = {});
hipError_t launch_fnv1a64_mapped(const HashMapArgs& map, const uint8_t* tail, uint64_t seed, uint64_t* out,
                                 uint32_t* fault_out, void* workspace, hipStream_t stream, uint64_t expected = 0,
                                 uint32_t* verdict = nullptr, const FnvCarries& carries = {});
hipError_t launch_hash_groups(const HashExtent* ext, uint32_t n_ext, uint64_t bytes, uint8_t* const* segs,
                              uint32_t n_segs, uint64_t seg_bytes, HashGroup* grp, uint64_t groups, hipStream_t stream);

static uint64_t host_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// The key of synthetic stream `sid` under `seed`; element i of the stream is mix64(key + (i + 1) * golden).
uint64_t synth_key(uint64_t seed, uint64_t sid) { return host_mix64(seed ^ host_mix64(sid + 0x9E3779B97F4A7C15ull)); }
}  // namespace sc

struct CarveRetarget;   // what a carve plan keeps to be re-pointed at another prefill view (sc_plan_retarget)

struct sc_plan {
    bool batch = false;                 // a batched resume + append plan (BatchArgs) instead of a handoff table
    sc::BatchArgs batch_args{};
    uint64_t* batch_ptrs_dev = nullptr;
    sc::MoveRow* rows_dev = nullptr;
    uint16_t* tile_row_dev = nullptr;   // row index of every tile
    int n_rows = 0;
    sc::MoveGeo geo{};
    uint64_t n_tiles = 0;
    uint64_t payload = 0;
    int64_t grid = 0;
    int64_t default_grid = 0;           // what the builder chose; sc_plan_set_grid(plan, 0) returns to it
    int32_t mix = sc::kMixPlain;        // the kernel instance that holds every row kind of the plan
    bool xcd = false;                   // tiles numbered by XCD (no row of the plan goes through a page table)
    // destination order of the rows that write through page tables (OrderGroup, sc_internal.hpp)
    void* order_ws = nullptr;           // one device block: the groups, then inv / order / counts per group
    const sc::OrderGroup* order_groups = nullptr;
    int32_t n_order_groups = 0;
    int64_t order_max_pages = 0;
    uint32_t order_max_blocks = 0;
    CarveRetarget* rt = nullptr;        // carve plans only
    std::vector<sc::MoveRow> host_rows; // the table as uploaded (what sc_hash_map_create reads)
};

struct sc_hash_map {
    sc::HashExtent* ext_dev = nullptr;   // one device block: the extents, the workgroups' parts, the segments
    sc::HashGroup* grp_dev = nullptr;
    uint8_t** seg_dev = nullptr;
    uint64_t seg_bytes = 0;
    const uint8_t* tail = nullptr;       // device address of the payload's last partial lane segment
    uint64_t bytes = 0;
    bool store = true;
};

namespace {

thread_local std::string g_error;

int ok() {
    g_error.clear();
    return SC_OK;
}
int fail(int code, const std::string& message) {
    g_error = message;
    return code;
}
int snapshot_fail(const char* message) { return fail(SC_EINVAL, std::string("conversation snapshot: ") + message); }
}  // namespace

int sc::record_ok() { return ok(); }
int sc::record_error(int code, const std::string& message) { return fail(code, message); }

namespace {
int hip_fail(hipError_t e, const char* what) {
    return fail(SC_EHIP, std::string("sc_handoff ") + what + ": " + hipGetErrorString(e));
}

constexpr uint64_t kBlobAlign = 64;   // the wire codec's blob-pool alignment (conversation_wire.hpp:68-70)
uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct Geo {
    int64_t n_qsa = 0, n_gdn = 0, H = 0, D = 0, ps = 0, S = 0, HV = 0, C = 0, hist = 0;
    uint64_t row_bytes = 0, page_bytes = 0, gdn_row_bytes = 0, rec_bytes = 0;
};

bool geometry(const sc_geometry* g, Geo& o, std::string& why) {
    if (!g) { why = "missing geometry"; return false; }
    if (g->n_layers < 0 || g->qsa_interval < 1 || g->n_head_kv < 1 || g->head_dim < 1 || g->page_size < 1 ||
        g->ssm_state_size < 1 || g->ssm_v_heads < 1 || g->ssm_conv_channels < 1 || g->ssm_d_conv < 2) {
        why = "invalid model geometry";
        return false;
    }
    if (g->n_head_kv > 4096 || g->head_dim > (1 << 20) || g->page_size > (1 << 20) || g->ssm_state_size > 65536 ||
        g->ssm_v_heads > 65536 || g->ssm_conv_channels > (int64_t(1) << 30) || g->n_layers > 100000) {
        why = "model geometry beyond the supported range";
        return false;
    }
    o.n_qsa = g->n_layers / g->qsa_interval;
    o.n_gdn = g->n_layers - o.n_qsa;
    o.H = g->n_head_kv; o.D = g->head_dim; o.ps = g->page_size;
    o.S = g->ssm_state_size; o.HV = g->ssm_v_heads; o.C = g->ssm_conv_channels; o.hist = g->ssm_d_conv - 1;
    if ((o.D * 2) % 16) { why = "head_dim must make 16-byte rows (a multiple of 8)"; return false; }
    if ((o.S * 4) % 16) { why = "ssm_state_size must make 16-byte rows (a multiple of 4)"; return false; }
    if (o.hist > sc::kMaxHist) { why = "ssm_d_conv beyond the supported history"; return false; }
    o.row_bytes = uint64_t(o.D) * 2;
    o.page_bytes = uint64_t(o.H) * uint64_t(o.ps) * o.row_bytes;
    o.rec_bytes = uint64_t(o.S) * uint64_t(o.HV) * uint64_t(o.S) * 4;
    o.gdn_row_bytes = o.rec_bytes + uint64_t(o.C) * uint64_t(o.hist) * 4;
    if (o.gdn_row_bytes % 16) { why = "a GDN row must be whole 16-byte chunks (C*(d_conv-1) a multiple of 4)"; return false; }
    return true;
}

int64_t cells_of(const Geo& g, int64_t tokens) { return (tokens + g.ps - 1) / g.ps * g.ps; }

struct Blob {
    int32_t kind, layer;
    uint64_t offset, bytes;
};

// K then V of every QSA layer, then the GDN rows; each blob on a 64-byte boundary.
std::vector<Blob> image_blobs(const Geo& g, int64_t tokens, uint64_t& total) {
    std::vector<Blob> out;
    const uint64_t kv = uint64_t(cells_of(g, tokens)) * uint64_t(g.H) * g.row_bytes;
    uint64_t at = 0;
    for (int64_t j = 0; j < g.n_qsa; ++j)
        for (int32_t kind : {SC_BLOB_K, SC_BLOB_V}) {
            at = round_up(at, kBlobAlign);
            out.push_back({kind, int32_t(j), at, kv});
            at += kv;
        }
    if (g.n_gdn > 0) {
        at = round_up(at, kBlobAlign);
        out.push_back({SC_BLOB_GDN, -1, at, uint64_t(g.n_gdn) * g.gdn_row_bytes});
        at += uint64_t(g.n_gdn) * g.gdn_row_bytes;
    }
    total = round_up(at, kBlobAlign);
    return out;
}

// Zero rows for the gaps between blobs (and after the last), so an image is fully deterministic.
void gap_rows(const std::vector<Blob>& blobs, uint64_t total, uint8_t* image, std::vector<sc::MoveRow>& rows) {
    uint64_t at = 0;
    auto gap = [&](uint64_t end) {
        if (end > at) {
            sc::MoveRow r{};
            r.kind = sc::kZero; r.dst = image + at; r.n = (end - at) / 16;
            if (r.n) rows.push_back(r);
        }
    };
    for (const Blob& b : blobs) { gap(b.offset); at = b.offset + b.bytes; }
    gap(total);
}

sc::MoveGeo move_geo(const Geo& g) {
    sc::MoveGeo m{};
    m.row_chunks = sc::make_fastdiv(uint32_t(g.row_bytes / 16));
    m.heads = sc::make_fastdiv(uint32_t(g.H));
    m.page_size = sc::make_fastdiv(uint32_t(g.ps));
    m.rec_chunks = sc::make_fastdiv(uint32_t(g.S * 4 / 16));
    m.v_heads = sc::make_fastdiv(uint32_t(g.HV));
    m.page_chunks = sc::make_fastdiv(uint32_t(g.page_bytes / 16));
    m.state = uint32_t(g.S);
    return m;
}

constexpr uint64_t kMaxRowChunks = uint64_t(1) << 31;
// Workgroups per launch; larger plans stride.  Measured on the 128K handoff (48 layers, 201K tiles), four alternating
// rounds: one workgroup per tile 1.155 ms, 65536 workgroups 1.166 ms (with the rows' loads non-temporal: 1.148 and
// 1.159 ms); an earlier version of the kernel, whose loads waited on the table lookups, had measured the opposite.
constexpr uint64_t kMaxGrid = uint64_t(1) << 20;
// The batched launch takes one workgroup per tile as well: config 5's scatter (870K tiles) at a median of 7 launches,
// 65536 workgroups 5.42 ms, 262144 5.11-5.19, one per tile 5.05-5.07 (with regular loads, 65536 to 262144 had
// measured alike).
constexpr uint64_t kMaxGridBatch = kMaxGrid;
// Plans with quantizing rows take one workgroup per tile too: against 262144 workgroups, the 128K int8 carve 1.35
// against 1.38 ms, q4_0 1.24 against 1.33, K8V4 1.30 against 1.35, int8 through a shuffled table 1.49 against 1.55
// (two alternating rounds).  Before the tile's table entry was read with scalar loads, 262144 had measured fastest.

// Rows that write through a page table visit their pages in destination order when the table covers at least this
// many logical pages (fewer pages gain nothing from the pre-pass) and the pool is at most kOrderMaxSparsity times
// larger (the pre-pass reads every physical page of the pool).  sc_set_order_min_pages changes it; <= 0 turns it off.
std::atomic<int64_t> g_order_min_pages{2048};
constexpr int64_t kOrderMaxSparsity = 8;

bool quant_kind(int32_t kind) { return kind == sc::kKvQ8 || kind == sc::kKvQ4; }
// The quantizing rows keep the source order: measured on the 128K int8 carve through a shuffled table, destination
// order took it from 1.64 to 2.12 ms (1.85 ms with the order entries read by scalar loads): a quantizing row reads 4-7x
// the bytes it writes, and destination order gives up the sequential reads.
bool orderable_kind(int32_t kind) { return kind == sc::kKv16 || kind == sc::kKv32 || kind == sc::kPagesScatter; }
// A row's work items per page and per tile: 16-byte chunks, or (cell, head) rows for the quantizing kinds.
uint64_t items_per_page(int32_t kind, const Geo& g) {
    return quant_kind(kind) ? uint64_t(g.ps) * uint64_t(g.H) : g.page_bytes / 16;
}
// Whether any quantizing row writes through a page table (such plans launch the instance that stages those rows).
bool quant_tables(const std::vector<sc::MoveRow>& rows) {
    return std::any_of(rows.begin(), rows.end(), [](const sc::MoveRow& r) { return quant_kind(r.kind) && r.table; });
}
uint64_t items_per_tile(int32_t kind) {
    return kind == sc::kConv ? sc::kConvTileChannels : quant_kind(kind) ? sc::kQuantUnitsPerTile : sc::kTileChunks;
}

// The logical pages a row writes through its table: K/V rows the cells [pos0, pos0 + rows), page rows their pages.
void table_pages_of(const sc::MoveRow& r, const Geo& g, int64_t& lo, int64_t& hi) {
    if (r.kind == sc::kPagesScatter) {
        lo = 0;
        hi = int64_t((r.n + g.page_bytes / 16 - 1) / (g.page_bytes / 16));
        return;
    }
    const int64_t tokens = int64_t(r.n / (uint64_t(g.H) * (quant_kind(r.kind) ? 1 : g.row_bytes / 16)));
    lo = r.pos0 / g.ps;
    hi = (r.pos0 + tokens + g.ps - 1) / g.ps;
}

struct OrderPlan {
    std::vector<sc::OrderGroup> groups;   // device pointers filled once the workspace exists
    std::vector<int> row_group;           // per row: its group, or -1
};

OrderPlan order_plan(const std::vector<sc::MoveRow>& rows, const Geo& g) {
    OrderPlan o;
    o.row_group.assign(rows.size(), -1);
    const int64_t min_pages = g_order_min_pages.load();
    if (min_pages <= 0) return o;
    for (size_t k = 0; k < rows.size(); ++k) {
        const sc::MoveRow& r = rows[k];
        if (!r.table || !r.n || !orderable_kind(r.kind)) continue;
        if (r.kind == sc::kPagesScatter && r.pos0 != 0) continue;   // a piece of a split blob keeps the source order
        int64_t lo, hi;
        table_pages_of(r, g, lo, hi);
        int gi = -1;
        for (size_t i = 0; i < o.groups.size(); ++i)
            if (o.groups[i].table == r.table && o.groups[i].ld == r.ld) gi = int(i);
        if (gi < 0) {
            sc::OrderGroup G{};
            G.table = r.table;
            G.ld = r.ld;
            G.lp_lo = lo;
            G.lp_hi = hi;
            o.groups.push_back(G);
            gi = int(o.groups.size()) - 1;
        }
        o.groups[size_t(gi)].lp_lo = std::min(o.groups[size_t(gi)].lp_lo, lo);
        o.groups[size_t(gi)].lp_hi = std::max(o.groups[size_t(gi)].lp_hi, hi);
        o.row_group[k] = gi;
    }
    // groups too small or too sparse keep the source order
    std::vector<int> keep(o.groups.size(), -1);
    std::vector<sc::OrderGroup> kept;
    const uint64_t page_chunks = g.page_bytes / 16;
    for (size_t i = 0; i < o.groups.size(); ++i) {
        const sc::OrderGroup& G = o.groups[i];
        const int64_t m = G.lp_hi - G.lp_lo;
        if (m < min_pages || G.ld > kOrderMaxSparsity * m || G.ld <= 0 ||
            uint64_t(m) * page_chunks >= kMaxRowChunks || G.ld >= (int64_t(1) << 31))
            continue;
        keep[i] = int(kept.size());
        kept.push_back(G);
    }
    for (int& gi : o.row_group) gi = gi >= 0 ? keep[size_t(gi)] : -1;
    o.groups = std::move(kept);
    for (sc::OrderGroup& G : o.groups) G.n_blocks = uint32_t((G.ld + sc::kOrderBlockPages - 1) / sc::kOrderBlockPages);
    // the order covers every page the tiles of its rows reach (whole tiles of whole pages)
    for (size_t k = 0; k < rows.size(); ++k) {
        if (o.row_group[k] < 0) continue;
        sc::OrderGroup& G = o.groups[size_t(o.row_group[k])];
        const uint64_t per_page = items_per_page(rows[k].kind, g), per_tile = items_per_tile(rows[k].kind);
        const uint64_t tiles = (uint64_t(G.lp_hi - G.lp_lo) * per_page + per_tile - 1) / per_tile;
        G.order_len = std::max<uint64_t>(G.order_len, (tiles * per_tile + per_page - 1) / per_page);
    }
    return o;
}

// One device block for the order pre-pass: the groups, then each group's inv (set to -1), order and counts.  Fills
// the rows' order pointers.
int order_workspace(OrderPlan& o, std::vector<sc::MoveRow>& rows, sc_plan* p) {
    if (o.groups.empty()) return ok();
    auto up = [](uint64_t x) { return (x + 255) / 256 * 256; };
    uint64_t at = up(o.groups.size() * sizeof(sc::OrderGroup));
    std::vector<uint64_t> inv_at, order_at, counts_at;
    for (const sc::OrderGroup& G : o.groups) {
        inv_at.push_back(at);
        at += up(uint64_t(G.ld) * 4);
        order_at.push_back(at);
        at += up(G.order_len * 4);
        counts_at.push_back(at);
        at += up(uint64_t(G.n_blocks) * 4);
    }
    hipError_t e = hipMalloc(&p->order_ws, at);
    if (e != hipSuccess) return fail(SC_ENOMEM, std::string("sc_handoff: order workspace: ") + hipGetErrorString(e));
    uint8_t* base = static_cast<uint8_t*>(p->order_ws);
    for (size_t i = 0; i < o.groups.size(); ++i) {
        sc::OrderGroup& G = o.groups[i];
        G.inv = reinterpret_cast<int32_t*>(base + inv_at[i]);
        G.order = reinterpret_cast<int32_t*>(base + order_at[i]);
        G.counts = reinterpret_cast<uint32_t*>(base + counts_at[i]);
        p->order_max_pages = std::max(p->order_max_pages, G.lp_hi - G.lp_lo);
        p->order_max_blocks = std::max(p->order_max_blocks, G.n_blocks);
        e = hipMemset(G.inv, 0xFF, uint64_t(G.ld) * 4);   // every entry -1; each launch leaves it so
        if (e != hipSuccess) return hip_fail(e, "order workspace");
    }
    p->order_groups = reinterpret_cast<const sc::OrderGroup*>(base);
    p->n_order_groups = int32_t(o.groups.size());
    e = hipMemcpy(base, o.groups.data(), o.groups.size() * sizeof(sc::OrderGroup), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "order workspace");
    for (size_t k = 0; k < rows.size(); ++k)
        if (o.row_group[k] >= 0) rows[k].order = o.groups[size_t(o.row_group[k])].order;
    return ok();
}

// Gives every row its tile range, in row order; an ordered row spans the items of its group's pages (whole pages, in
// destination order).  Also reports which kernel instance the rows need.
int assign_tiles(std::vector<sc::MoveRow>& rows, const OrderPlan& order, const Geo& g, uint64_t& tiles, bool& quant,
                 bool& kv32) {
    tiles = 0;
    quant = kv32 = false;
    for (size_t k = 0; k < rows.size(); ++k) {
        sc::MoveRow& r = rows[k];
        if (r.n >= kMaxRowChunks) return fail(SC_ERANGE, "sc_handoff: a handoff table row beyond 2^31 chunks");
        r.tile0 = tiles;
        const uint64_t per_tile = items_per_tile(r.kind);
        const int gi = order.row_group[k];
        const uint64_t items = gi >= 0 ? uint64_t(order.groups[size_t(gi)].lp_hi - order.groups[size_t(gi)].lp_lo) *
                                             items_per_page(r.kind, g)
                                       : r.n;
        tiles += (items + per_tile - 1) / per_tile;
        quant = quant || r.kind == sc::kKvQ8 || r.kind == sc::kKvQ4;
        kv32 = kv32 || r.kind == sc::kKv32;
    }
    return SC_OK;
}

// Assigns tile ranges, uploads the table and fills the plan.  The only HIP calls a plan builder makes.  `order_out`
// (may be null) receives the order groups with their workspace pointers.
int finish_plan(std::vector<sc::MoveRow>& rows, const Geo& g, uint64_t payload, sc_plan** out,
                OrderPlan* order_out = nullptr) {
    if (rows.size() > 65535) return fail(SC_ERANGE, "sc_handoff: more than 65535 handoff table rows in one plan");
    OrderPlan order = order_plan(rows, g);
    uint64_t tiles = 0;
    bool quant = false, kv32 = false;
    if (const int rc = assign_tiles(rows, order, g, tiles, quant, kv32)) return rc;
    // rows that move nothing still own an (empty) tile range; the kernel never visits them
    sc_plan* p = new (std::nothrow) sc_plan();
    if (!p) return fail(SC_ENOMEM, "sc_handoff: plan allocation failed");
    p->n_rows = int(rows.size());
    p->geo = move_geo(g);
    p->n_tiles = tiles;
    p->payload = payload;
    p->grid = p->default_grid = int64_t(std::min<uint64_t>(tiles, kMaxGrid));
    p->mix = sc::mix_of(kv32, quant, quant_tables(rows));
    // The XCD-contiguous numbering of the tiles (xcd_tile, sc_kernels.hip) measured faster for the identity carve
    // (1.072-1.075 against 1.088-1.118 ms at 128K) and slower for a carve through shuffled tables in destination order
    // (1.164 against 1.142-1.153 ms) and for the f32 and quantizing rows, which read 2-7 times what they write
    // (per-layer f32 appends 1.90 against 1.64 ms, q4_0 1.30 against 1.20), so only plain plans without a page table
    // take it.
    p->xcd = p->mix == sc::kMixPlain &&
             std::none_of(rows.begin(), rows.end(), [](const sc::MoveRow& r) { return r.table != nullptr; });
    if (rows.empty() || tiles == 0) {   // an empty handoff (0 tokens, no running state) is a valid no-op
        *out = p;
        return ok();
    }
    // padded to an even count: the kernel reads the entries a 4-byte word (two entries) at a time; the table is built
    // on the device from the rows (tile_rows_kernel)
    const uint64_t n_entries = tiles + (tiles & 1);
    if (const int rc = order_workspace(order, rows, p)) {
        if (p->order_ws) (void) hipFree(p->order_ws);
        delete p;
        return rc;
    }
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->rows_dev), rows.size() * sizeof(sc::MoveRow));
    if (e == hipSuccess)
        e = hipMalloc(reinterpret_cast<void**>(&p->tile_row_dev), n_entries * sizeof(uint16_t));
    if (e != hipSuccess) {
        if (p->rows_dev) (void) hipFree(p->rows_dev);
        if (p->order_ws) (void) hipFree(p->order_ws);
        delete p;
        return fail(SC_ENOMEM, std::string("sc_handoff: table allocation: ") + hipGetErrorString(e));
    }
    e = hipMemcpy(p->rows_dev, rows.data(), rows.size() * sizeof(sc::MoveRow), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = sc::launch_tile_rows(p->rows_dev, uint32_t(rows.size()), p->tile_row_dev, n_entries, tiles, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        (void) hipFree(p->rows_dev);
        (void) hipFree(p->tile_row_dev);
        if (p->order_ws) (void) hipFree(p->order_ws);
        delete p;
        return hip_fail(e, "table upload");
    }
    if (order_out) *order_out = std::move(order);
    p->host_rows = rows;
    *out = p;
    return ok();
}

bool slot_identity(const sc_decode_slot* s, int64_t n_qsa) {
    if (!s->page_table) return true;
    for (int64_t j = 0; j < n_qsa; ++j)
        if (s->page_table[j]) return false;
    return true;
}

// Checks the slot can hold `cells` cells (from cell 0) and that its buffers are present and aligned.
int check_slot(const Geo& g, const sc_decode_slot* s, int64_t cells_end, bool need_gdn) {
    if (!s) return snapshot_fail("missing decode slot");
    if (s->n_pages < 0 || s->max_cells < 0 || cells_end > s->max_cells)
        return snapshot_fail("invalid K/V extent");
    if (g.n_qsa > 0) {
        if (!s->k_pool || !s->v_pool) return snapshot_fail("missing target state buffer");
        const bool identity = slot_identity(s, g.n_qsa);
        if (identity && s->max_cells > s->n_pages * g.ps) return snapshot_fail("invalid K/V extent");
        for (int64_t j = 0; j < g.n_qsa; ++j) {
            if (!s->k_pool[j] || !s->v_pool[j]) return snapshot_fail("missing target state buffer");
            if (!aligned16(s->k_pool[j]) || !aligned16(s->v_pool[j]))
                return fail(SC_EINVAL, "sc_handoff: K/V pools must be 16-byte aligned");
        }
    }
    if (need_gdn && g.n_gdn > 0) {
        if (!s->gdn_state) return snapshot_fail("missing running-state buffer");
        if (!aligned16(s->gdn_state) || g.gdn_row_bytes % 16)
            return fail(SC_EINVAL, "sc_handoff: GDN rows must be 16-byte aligned multiples of 16 bytes");
    }
    return SC_OK;
}

int check_view(const Geo& g, const sc_prefill_view* v) {
    if (!v) return snapshot_fail("missing prefill view");
    if (v->tokens < 0 || v->pos0 < 0 || v->tokens > (int64_t(1) << 30) || v->pos0 > (int64_t(1) << 30))
        return snapshot_fail("invalid K/V extent");
    if (v->kv_dtype != SC_DTYPE_F16 && v->kv_dtype != SC_DTYPE_F32)
        return fail(SC_EINVAL, "sc_handoff: unsupported prefill K/V dtype");
    if (g.n_qsa > 0 && v->tokens > 0) {
        if (!v->k || !v->v) return snapshot_fail("missing prefill K/V");
        for (int64_t j = 0; j < g.n_qsa; ++j) {
            if (!v->k[j] || !v->v[j]) return snapshot_fail("missing prefill K/V");
            if (!aligned16(v->k[j]) || !aligned16(v->v[j]))
                return fail(SC_EINVAL, "sc_handoff: prefill K/V must be 16-byte aligned");
        }
    }
    if (v->with_gdn && g.n_gdn > 0) {
        if (!v->rec || !v->conv) return snapshot_fail("missing prefill running state");
        if (v->conv_rows < 0 || v->conv_ld < g.C) return snapshot_fail("invalid conv source extent");
        for (int64_t i = 0; i < g.n_gdn; ++i) {
            if (!v->rec[i] || (!v->conv[i] && v->conv_rows > 0)) return snapshot_fail("missing prefill running state");
            if (!aligned16(v->rec[i])) return fail(SC_EINVAL, "sc_handoff: recurrent state must be 16-byte aligned");
        }
    }
    return SC_OK;
}

void kv_rows(const Geo& g, const sc_prefill_view* v, int64_t j, uint16_t* kdst, uint16_t* vdst,
             const int32_t* table, int64_t phys_pages, int64_t virtual_cells, std::vector<sc::MoveRow>& rows) {
    const uint64_t row_chunks = g.row_bytes / 16;
    const void* srcs[2] = {v->k[j], v->v[j]};
    uint16_t* dsts[2] = {kdst, vdst};
    for (int a = 0; a < 2; ++a) {
        sc::MoveRow r{};
        r.kind = v->kv_dtype == SC_DTYPE_F16 ? sc::kKv16 : sc::kKv32;
        r.src = static_cast<const uint8_t*>(srcs[a]);
        r.dst = reinterpret_cast<uint8_t*>(dsts[a]);
        r.table = table;
        r.pos0 = v->pos0;
        r.ld = phys_pages;
        // `virtual_cells` > tokens: the rows of cells [tokens, virtual_cells) are written as zeros (image tails)
        const int64_t rows_n = std::max(v->tokens, virtual_cells) * g.H;
        r.aux = int32_t(v->tokens);
        r.n = uint64_t(rows_n) * row_chunks;
        if (r.n) rows.push_back(r);
    }
}

void gdn_rows(const Geo& g, const sc_prefill_view* v, float* gdn, std::vector<sc::MoveRow>& rows) {
    const uint64_t row_floats = g.gdn_row_bytes / 4;
    for (int64_t i = 0; i < g.n_gdn; ++i) {
        float* base = gdn + uint64_t(i) * row_floats;
        sc::MoveRow rec{};
        rec.kind = sc::kRec;
        rec.src = reinterpret_cast<const uint8_t*>(v->rec[i]);
        rec.dst = reinterpret_cast<uint8_t*>(base);
        rec.n = uint64_t(g.S) * uint64_t(g.HV) * uint64_t(g.S * 4 / 16);
        rows.push_back(rec);
        sc::MoveRow conv{};
        conv.kind = sc::kConv;
        conv.aux = int32_t(g.hist) | (v->pos0 == 0 ? 0x100 : 0);   // a fresh sequence's older history is zero
        conv.src = reinterpret_cast<const uint8_t*>(v->conv[i]);
        conv.dst = reinterpret_cast<uint8_t*>(base + g.rec_bytes / 4);
        conv.n = uint64_t(g.C);
        conv.pos0 = v->conv_rows;
        conv.ld = v->conv_ld;
        rows.push_back(conv);
    }
}

// The identity-layout pools a carve writes beside the paged pool (a streamed layer's host copy, the prompt path's
// staging pool): `pools` is NULL or [n_qsa].  Returns, per layer, the K, V (and int8 scale) destinations of `format`,
// or nulls for a layer that has none; refuses half-given or misaligned pools.
// The device address of a pinned host range the device can reach, or nullptr: its first and last byte must both be
// pinned host memory mapped for the device, at device addresses `bytes - 1` apart (one mapping).  A kernel that reads
// or writes a host image itself needs this; a pageable image would fault the GPU rather than fail a copy.
uint8_t* mapped_host_range(const void* host, uint64_t bytes) {
    if (!host || bytes == 0) return nullptr;
    hipPointerAttribute_t first{}, last{};
    hipError_t e = hipPointerGetAttributes(&first, host);
    if (e == hipSuccess) e = hipPointerGetAttributes(&last, static_cast<const uint8_t*>(host) + (bytes - 1));
    if (e != hipSuccess) {
        (void) hipGetLastError();   // an unknown pointer is an answer here, not an error for the next call
        return nullptr;
    }
    if (first.type != hipMemoryTypeHost || last.type != hipMemoryTypeHost || !first.devicePointer ||
        !last.devicePointer ||
        static_cast<uint8_t*>(last.devicePointer) - static_cast<uint8_t*>(first.devicePointer) != ptrdiff_t(bytes - 1))
        return nullptr;
    return static_cast<uint8_t*>(first.devicePointer);
}

struct ExtraKv {
    uint8_t* k = nullptr;
    uint8_t* v = nullptr;
    uint16_t* ks = nullptr;
    uint16_t* vs = nullptr;
};
// Bytes per (cell, head) row of a pool of `format`: codes (or f16 values), and int8 scales.
uint64_t code_row_bytes(const Geo& g, int32_t format, bool value) {
    if (format == SC_KV_F16) return uint64_t(g.D) * 2;
    if (format == SC_KV_Q4 || (format == SC_KV_K8V4 && value)) return uint64_t(g.D) / 32 * 18;
    return uint64_t(g.D);
}
uint64_t scale_row_bytes(const Geo& g) { return uint64_t(g.D) / 64 * 2; }

// A host copy is written by the kernels themselves, so each of its pools must be pinned host memory mapped for the
// device over the rows a launch may write, rows [row0, row0 + rows) of `H` heads; checked before anything is enqueued.
int check_host_copy(const Geo& g, const ExtraKv& e, int32_t format, uint64_t row0, uint64_t rows) {
    const uint64_t cr = code_row_bytes(g, format, false), vr = code_row_bytes(g, format, true), sr = scale_row_bytes(g);
    const struct { const void* p; uint64_t row; } pools[4] = {{e.k, cr}, {e.v, vr}, {e.ks, sr}, {e.vs, sr}};
    for (const auto& q : pools)
        if (q.p && rows && !mapped_host_range(static_cast<const uint8_t*>(q.p) + row0 * q.row, rows * q.row))
            return snapshot_fail("a host copy must be pinned memory mapped for the device");
    return SC_OK;
}

// `map_cells` > 0: the pools are a host copy of that many cells (checked with check_host_copy).
int extra_kv(const Geo& g, const sc_kv_pools* pools, int32_t format, const char* what, std::vector<ExtraKv>& out,
             int64_t map_cells = 0) {
    out.assign(size_t(g.n_qsa), ExtraKv{});
    if (!pools) return SC_OK;
    for (int64_t j = 0; j < g.n_qsa; ++j) {
        const sc_kv_pools& p = pools[j];
        ExtraKv& e = out[size_t(j)];
        switch (format) {
            case SC_KV_F16:
                e.k = reinterpret_cast<uint8_t*>(p.k_pool), e.v = reinterpret_cast<uint8_t*>(p.v_pool);
                break;
            case SC_KV_INT8:
                e.k = reinterpret_cast<uint8_t*>(p.k_q), e.v = reinterpret_cast<uint8_t*>(p.v_q);
                e.ks = p.k_scale, e.vs = p.v_scale;
                break;
            case SC_KV_Q4:
                e.k = p.k_q4, e.v = p.v_q4;
                break;
            default:   // K8V4 is resident only: it has no host copy or staging pool
                if (p.k_pool || p.v_pool || p.k_q || p.v_q || p.k_scale || p.v_scale || p.k_q4 || p.v_q4)
                    return snapshot_fail("hybrid K8V4 requires an identity layout and distinct format flags");
                continue;
        }
        const bool any = e.k || e.v || e.ks || e.vs;
        const bool all = e.k && e.v && (format != SC_KV_INT8 || (e.ks && e.vs));
        if (any && !all) return fail(SC_EINVAL, std::string("sc_handoff: ") + what + " needs every pool of its format");
        const uintptr_t a = format == SC_KV_F16 ? 16 : 4;
        if (any && ((reinterpret_cast<uintptr_t>(e.k) | reinterpret_cast<uintptr_t>(e.v)) & (a - 1) ||
                    (format == SC_KV_INT8 && ((reinterpret_cast<uintptr_t>(e.ks) | reinterpret_cast<uintptr_t>(e.vs)) & 7u))))
            return fail(SC_EINVAL, std::string("sc_handoff: ") + what + " pools must be aligned as the slot's pools are");
        if (any && map_cells > 0) {
            const int rc = check_host_copy(g, e, format, 0, uint64_t(map_cells) * uint64_t(g.H));
            if (rc) return rc;
        }
    }
    return SC_OK;
}

uint64_t kv_payload(const Geo& g, int64_t tokens) { return uint64_t(tokens) * uint64_t(g.H) * g.row_bytes * 2 * uint64_t(g.n_qsa); }

// ---- slot images in every K/V format (sc_slot_layers) ----

constexpr uint64_t kAbsent = ~uint64_t(0);

// The five blob sizes of one QSA layer (conversation_snapshot.cpp:27-66): data, value data, key scales, value scales,
// pooled indexer rows.  Returns an empty string or the refusal.
std::string layer_blob_sizes(const Geo& o, const sc_geometry* g, int32_t format, bool index, int64_t tokens,
                             uint64_t (&b)[SC_N_BUF]) {
    if (format < SC_KV_F16 || format > SC_KV_K8V4) return "unknown K/V format";
    if (tokens < 0 || tokens > (int64_t(1) << 30)) return "invalid K/V extent";
    const bool q4 = format == SC_KV_Q4, int8_keys = format == SC_KV_INT8 || format == SC_KV_K8V4;
    if (g->idx_key_dim <= 0 || g->idx_key_dim > (1 << 20) || (q4 && o.D % 32) || (int8_keys && o.D % 64) ||
        (format == SC_KV_K8V4 && o.D % 32))
        return "invalid K/V geometry";
    const uint64_t cells = uint64_t(cells_of(o, tokens)), H = uint64_t(o.H), D = uint64_t(o.D);
    const uint64_t q4_head = D / 32 * 18;
    const uint64_t per_head = format == SC_KV_F16 ? 2 * D : q4 ? q4_head : D;
    b[SC_BUF_K] = cells * H * per_head;
    b[SC_BUF_V] = format == SC_KV_K8V4 ? cells * H * q4_head : b[SC_BUF_K];
    b[SC_BUF_K_SCALE] = int8_keys ? cells * H * (D / 64) * 2 : 0;
    b[SC_BUF_V_SCALE] = format == SC_KV_INT8 ? b[SC_BUF_K_SCALE] : 0;
    const uint64_t pooled_rows = index && tokens > 0 ? uint64_t(tokens) / SC_IDX_BLOCK + 1 : 0;
    b[SC_BUF_POOLED] = pooled_rows * uint64_t(g->idx_key_dim) * 4;
    return "";
}

// Offsets of every blob in the image (kAbsent for an empty one), the GDN rows last; returns the total.
uint64_t layers_layout(const Geo& o, const uint64_t (&b)[SC_N_BUF], std::vector<uint64_t>& off) {
    off.assign(size_t(o.n_qsa) * SC_N_BUF + 1, kAbsent);
    uint64_t at = 0;
    for (int64_t j = 0; j < o.n_qsa; ++j)
        for (int k = 0; k < SC_N_BUF; ++k)
            if (b[k]) {
                at = round_up(at, kBlobAlign);
                off[size_t(j) * SC_N_BUF + k] = at;
                at += b[k];
            }
    if (o.n_gdn > 0) {
        at = round_up(at, kBlobAlign);
        off.back() = at;
        at += uint64_t(o.n_gdn) * o.gdn_row_bytes;
    }
    return round_up(at, kBlobAlign);
}

// A validated sc_slot_layers request: the blob sizes, and every buffer present where its blob is nonempty.
int check_layers(const Geo& o, const sc_geometry* g, const sc_slot_layers* s, int64_t tokens, uint64_t (&b)[SC_N_BUF]) {
    if (!s) return snapshot_fail("missing decode slot");
    const std::string why = layer_blob_sizes(o, g, s->format, s->with_index != 0, tokens, b);
    if (!why.empty()) return snapshot_fail(why.c_str());
    if (s->max_cells < 0 || cells_of(o, tokens) > s->max_cells) return snapshot_fail("invalid K/V extent");
    const uint64_t pooled_rows = b[SC_BUF_POOLED] / (uint64_t(g->idx_key_dim) * 4);
    if (s->pooled_capacity < 0 || pooled_rows > uint64_t(s->pooled_capacity))
        return snapshot_fail("invalid indexer extent");
    for (int k = 0; k < SC_N_BUF; ++k) {
        if (b[k] % 16) return fail(SC_ERANGE, "sc_handoff: a K/V blob is not a whole number of 16-byte chunks");
        if (!b[k] || o.n_qsa == 0) continue;
        if (!s->buf[k]) return snapshot_fail("missing K/V buffer for the slot's format");
        for (int64_t j = 0; j < o.n_qsa; ++j)
            if (!s->buf[k][j] || !aligned16(s->buf[k][j])) return snapshot_fail("missing or misaligned K/V buffer");
    }
    if (o.n_gdn > 0 && (!s->gdn_state || !aligned16(s->gdn_state))) return snapshot_fail("missing running-state buffer");
    return SC_OK;
}

// The slot side of a carve as sc_plan_carve checked it: its pools, tables and identity-layout copies.  A carve plan
// keeps it so that a retarget re-points only the prefill side.
struct CarveTarget {
    std::vector<uint16_t*> k, v;
    std::vector<const int32_t*> table;
    int64_t n_pages = 0, max_cells = 0;
    float* gdn = nullptr;
    std::vector<ExtraKv> host, stage;
};

// The rows of a carve of `src` into `t`, and its algorithmic payload.
void carve_rows(const Geo& o, const sc_prefill_view* src, const CarveTarget& t, std::vector<sc::MoveRow>& rows,
                uint64_t& payload) {
    const int64_t logical_pages = (t.max_cells + o.ps - 1) / o.ps;
    payload = kv_payload(o, src->tokens);
    for (int64_t j = 0; j < o.n_qsa; ++j) {
        kv_rows(o, src, j, t.k[size_t(j)], t.v[size_t(j)], t.table[size_t(j)], t.n_pages, 0, rows);
        // the identity-layout copies get every carved cell, resident in the paged pool or not
        for (const ExtraKv* e : {&t.host[size_t(j)], &t.stage[size_t(j)]}) {
            if (!e->k) continue;
            kv_rows(o, src, j, reinterpret_cast<uint16_t*>(e->k), reinterpret_cast<uint16_t*>(e->v), nullptr,
                    logical_pages, 0, rows);
            payload += uint64_t(src->tokens) * uint64_t(o.H) * o.row_bytes * 2;
        }
    }
    if (src->with_gdn) {
        gdn_rows(o, src, t.gdn, rows);
        payload += uint64_t(o.n_gdn) * o.gdn_row_bytes;
    }
}

template <class F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return fail(SC_ENOMEM, "sc_handoff: host allocation failed");
    } catch (const std::exception& e) {
        return fail(SC_EINVAL, std::string("sc_handoff: ") + e.what());
    } catch (...) {
        return fail(SC_EINVAL, "sc_handoff: unknown failure");
    }
}

}  // namespace

// A carve plan's retarget state: the slot side, the capacity of the device table, tile map and order workspace as
// built, and two slots of pinned staging for new rows, each free again once the retarget that last used it has run.
struct CarveRetarget {
    Geo o;
    CarveTarget t;
    size_t rows_cap = 0;
    uint64_t tile_entries = 0;                // entries of the device tile map
    std::vector<sc::OrderGroup> built;        // the order groups as built: their workspace and its capacity
    uint8_t* staging = nullptr;               // pinned: two slots of [rows_cap rows][built.size() groups]
    uint8_t* staging_dev = nullptr;           // its device address
    uint64_t slot_bytes = 0;
    hipEvent_t done[2] = {nullptr, nullptr};  // the last retarget that read each slot
    int next = 0;
    bool grid_set = false;                    // sc_plan_set_grid chose the grid

    ~CarveRetarget() {
        for (hipEvent_t& e : done)
            if (e) (void) hipEventDestroy(e);
        if (staging) (void) hipHostFree(staging);
    }
};

namespace {
// Prepares a freshly built carve plan for retargets (sc_plan_retarget): its pinned staging and events, nothing on the
// device.  Called once per plan, when it is built.
int attach_retarget(sc_plan* p, const Geo& o, CarveTarget&& t, size_t n_rows, OrderPlan&& order) {
    auto* rt = new (std::nothrow) CarveRetarget();
    if (!rt) return fail(SC_ENOMEM, "sc_handoff: plan allocation failed");
    rt->o = o;
    rt->t = std::move(t);
    rt->rows_cap = n_rows;
    rt->tile_entries = p->n_tiles + (p->n_tiles & 1);
    rt->built = std::move(order.groups);
    rt->slot_bytes = round_up(n_rows * sizeof(sc::MoveRow) + rt->built.size() * sizeof(sc::OrderGroup) + 16, 256);
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&rt->staging), 2 * rt->slot_bytes);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void**>(&rt->staging_dev), rt->staging, 0);
    for (hipEvent_t& ev : rt->done)
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        delete rt;
        return fail(SC_ENOMEM, std::string("sc_handoff: retarget staging: ") + hipGetErrorString(e));
    }
    p->rt = rt;
    return SC_OK;
}
}  // namespace

extern "C" {

const char* sc_last_error(void) { return g_error.c_str(); }
const char* sc_version(void) { return "sc_handoff 0.1 gfx950"; }

int64_t sc_n_qsa_layers(const sc_geometry* g) { return g && g->qsa_interval > 0 ? g->n_layers / g->qsa_interval : 0; }
int64_t sc_n_gdn_layers(const sc_geometry* g) { return g ? g->n_layers - sc_n_qsa_layers(g) : 0; }
int64_t sc_gdn_row_floats(const sc_geometry* g) {
    Geo o;
    std::string why;
    return geometry(g, o, why) ? int64_t(o.gdn_row_bytes / 4) : 0;
}
int64_t sc_kv_cells(const sc_geometry* g, int64_t tokens) {
    Geo o;
    std::string why;
    return geometry(g, o, why) && tokens >= 0 ? cells_of(o, tokens) : -1;
}
uint64_t sc_payload_bytes(const sc_geometry* g, int64_t tokens) {
    Geo o;
    std::string why;
    if (!geometry(g, o, why) || tokens < 0) return 0;
    return kv_payload(o, cells_of(o, tokens)) + uint64_t(o.n_gdn) * o.gdn_row_bytes;
}

int sc_image_layout(const sc_geometry* g, int64_t tokens, sc_image_blob* blobs, int64_t* n_blobs,
                    uint64_t* total_bytes) {
    return guarded([&] {
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        if (tokens < 0 || tokens > (int64_t(1) << 30)) return snapshot_fail("invalid K/V extent");
        uint64_t total = 0;
        const auto list = image_blobs(o, tokens, total);
        if (blobs)
            for (size_t i = 0; i < list.size(); ++i)
                blobs[i] = sc_image_blob{list[i].kind, list[i].layer, list[i].offset, list[i].bytes};
        if (n_blobs) *n_blobs = int64_t(list.size());
        if (total_bytes) *total_bytes = total;
        return ok();
    });
}

int sc_plan_carve(const sc_geometry* g, const sc_prefill_view* src, const sc_decode_slot* dst, sc_plan** out) {
    return guarded([&] {
        if (!out) return fail(SC_EINVAL, "sc_handoff: missing plan output");
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        int rc = check_view(o, src);
        if (rc) return rc;
        rc = check_slot(o, dst, src->pos0 + src->tokens, src->with_gdn != 0);
        if (rc) return rc;
        CarveTarget t;
        const int64_t host_cells = (dst->max_cells + o.ps - 1) / o.ps * o.ps;
        if ((rc = extra_kv(o, dst->host, SC_KV_F16, "a host copy", t.host, host_cells)) ||
            (rc = extra_kv(o, dst->stage, SC_KV_F16, "a staging pool", t.stage)))
            return rc;
        for (int64_t j = 0; j < o.n_qsa; ++j) {
            t.k.push_back(dst->k_pool[j]);
            t.v.push_back(dst->v_pool[j]);
            t.table.push_back(dst->page_table ? dst->page_table[j] : nullptr);
        }
        t.n_pages = dst->n_pages;
        t.max_cells = dst->max_cells;
        t.gdn = src->with_gdn ? dst->gdn_state : nullptr;
        std::vector<sc::MoveRow> rows;
        uint64_t payload = 0;
        carve_rows(o, src, t, rows, payload);
        OrderPlan order;
        sc_plan* p = nullptr;
        if ((rc = finish_plan(rows, o, payload, &p, &order))) return rc;
        if ((rc = attach_retarget(p, o, std::move(t), rows.size(), std::move(order)))) {
            sc_plan_destroy(p);
            return rc;
        }
        *out = p;
        return ok();
    });
}

int sc_plan_retarget(sc_plan* plan, const sc_prefill_view* src, void* stream) {
    return guarded([&] {
        if (!plan) return fail(SC_EINVAL, "sc_handoff: missing plan");
        CarveRetarget* rt = plan->rt;
        if (!rt) return fail(SC_EINVAL, "sc_handoff: only a carve plan (sc_plan_carve) can be retargeted");
        const Geo& o = rt->o;
        int rc = check_view(o, src);
        if (rc) return rc;
        if (src->pos0 + src->tokens > rt->t.max_cells) return snapshot_fail("invalid K/V extent");
        if (src->with_gdn && o.n_gdn > 0 && !rt->t.gdn)
            return fail(SC_ERANGE, "sc_handoff: the plan was built without the GDN rows; build a plan that carves them");
        std::vector<sc::MoveRow> rows;
        uint64_t payload = 0;
        carve_rows(o, src, rt->t, rows, payload);
        OrderPlan order = order_plan(rows, o);
        // each ordered group takes the workspace its table got when the plan was built; a group the build did not
        // order (or whose pages outgrow it) keeps the source order
        std::vector<int> remap(order.groups.size(), -1);
        std::vector<sc::OrderGroup> groups;
        for (size_t i = 0; i < order.groups.size(); ++i) {
            const sc::OrderGroup& G = order.groups[i];
            for (const sc::OrderGroup& B : rt->built)
                if (B.table == G.table && B.ld == G.ld && G.order_len <= B.order_len && G.n_blocks == B.n_blocks) {
                    sc::OrderGroup X = G;
                    X.inv = B.inv;
                    X.order = B.order;
                    X.counts = B.counts;
                    remap[i] = int(groups.size());
                    groups.push_back(X);
                    break;
                }
        }
        for (int& gi : order.row_group) gi = gi >= 0 ? remap[size_t(gi)] : -1;
        order.groups = groups;
        uint64_t tiles = 0;
        bool quant = false, kv32 = false;
        if ((rc = assign_tiles(rows, order, o, tiles, quant, kv32))) return rc;
        if (rows.size() > rt->rows_cap || tiles + (tiles & 1) > rt->tile_entries)
            return fail(SC_ERANGE, "sc_handoff: the view needs a larger handoff table than the plan was built with; "
                                   "build the plan for the largest view it will carve");
        for (size_t k = 0; k < rows.size(); ++k) {
            rows[k].order = order.row_group[k] >= 0 ? groups[size_t(order.row_group[k])].order : nullptr;
        }
        // the staging slot is free once the retarget that used it two calls ago has run (normally long since)
        const int slot = rt->next;
        hipError_t e = hipEventSynchronize(rt->done[slot]);
        if (e != hipSuccess) return hip_fail(e, "retarget staging wait");
        uint8_t* host = rt->staging + uint64_t(slot) * rt->slot_bytes;
        uint8_t* dev = rt->staging_dev + uint64_t(slot) * rt->slot_bytes;
        const uint64_t groups_at = round_up(rt->rows_cap * sizeof(sc::MoveRow), 16);
        if (!rows.empty()) std::memcpy(host, rows.data(), rows.size() * sizeof(sc::MoveRow));
        if (!groups.empty()) std::memcpy(host + groups_at, groups.data(), groups.size() * sizeof(sc::OrderGroup));
        e = sc::launch_retarget(reinterpret_cast<const sc::MoveRow*>(dev), int32_t(rows.size()),
                                reinterpret_cast<const sc::OrderGroup*>(dev + groups_at), int32_t(groups.size()),
                                plan->rows_dev, plan->tile_row_dev, tiles,
                                const_cast<sc::OrderGroup*>(plan->order_groups), static_cast<hipStream_t>(stream));
        if (e == hipSuccess) e = hipEventRecord(rt->done[slot], static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "retarget");
        rt->next = slot ^ 1;
        plan->n_rows = int(rows.size());
        plan->n_tiles = tiles;
        plan->payload = payload;
        plan->mix = sc::mix_of(kv32, quant, quant_tables(rows));
        plan->default_grid = int64_t(std::min<uint64_t>(tiles, kMaxGrid));
        if (!rt->grid_set) plan->grid = plan->default_grid;
        plan->xcd = plan->mix == sc::kMixPlain &&
                    std::none_of(rows.begin(), rows.end(), [](const sc::MoveRow& r) { return r.table != nullptr; });
        plan->n_order_groups = int32_t(groups.size());
        plan->order_max_pages = 0;
        plan->order_max_blocks = 0;
        for (const sc::OrderGroup& G : groups) {
            plan->order_max_pages = std::max(plan->order_max_pages, G.lp_hi - G.lp_lo);
            plan->order_max_blocks = std::max(plan->order_max_blocks, G.n_blocks);
        }
        return ok();
    });
}

int sc_plan_carve_quant(const sc_geometry* g, const sc_prefill_view* src, const sc_quant_slot* dst, sc_plan** out) {
    return guarded([&] {
        if (!out) return fail(SC_EINVAL, "sc_handoff: missing plan output");
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        int rc = check_view(o, src);
        if (rc) return rc;
        if (src->kv_dtype != SC_DTYPE_F32) return fail(SC_EINVAL, "sc_handoff: a quantizing carve reads f32 K/V rows");
        if (o.D != sc::kQuantDim) return fail(SC_EINVAL, "sc_handoff: the quantizing carve supports head_dim 256");
        if (!dst) return snapshot_fail("missing decode slot");
        if (dst->format != SC_KV_INT8 && dst->format != SC_KV_Q4 && dst->format != SC_KV_K8V4)
            return fail(SC_EINVAL, "sc_handoff: unknown quantized K/V format");
        if (dst->n_pages < 0 || dst->max_cells < 0 || src->pos0 + src->tokens > dst->max_cells)
            return snapshot_fail("invalid K/V extent");
        const bool k_int8 = dst->format != SC_KV_Q4, v_int8 = dst->format == SC_KV_INT8;
        const bool identity = !dst->page_table || std::all_of(dst->page_table, dst->page_table + o.n_qsa,
                                                              [](const int32_t* t) { return t == nullptr; });
        if (identity && dst->max_cells > dst->n_pages * o.ps) return snapshot_fail("invalid K/V extent");
        if (o.n_qsa > 0 && (!dst->k_codes || !dst->v_codes || (k_int8 && !dst->k_scale) || (v_int8 && !dst->v_scale)))
            return snapshot_fail("missing target state buffer");
        for (int64_t j = 0; j < o.n_qsa; ++j) {
            if (!dst->k_codes[j] || !dst->v_codes[j] || (k_int8 && !dst->k_scale[j]) || (v_int8 && !dst->v_scale[j]))
                return snapshot_fail("missing target state buffer");
            if ((reinterpret_cast<uintptr_t>(dst->k_codes[j]) | reinterpret_cast<uintptr_t>(dst->v_codes[j])) & 3u ||
                (k_int8 && (reinterpret_cast<uintptr_t>(dst->k_scale[j]) & 7u)) ||
                (v_int8 && (reinterpret_cast<uintptr_t>(dst->v_scale[j]) & 7u)))
                return fail(SC_EINVAL, "sc_handoff: code pools must be 4-byte and scale pools 8-byte aligned");
        }
        if (src->with_gdn && o.n_gdn > 0) {
            if (!dst->gdn_state) return snapshot_fail("missing running-state buffer");
            if (!aligned16(dst->gdn_state) || o.gdn_row_bytes % 16)
                return fail(SC_EINVAL, "sc_handoff: GDN rows must be 16-byte aligned multiples of 16 bytes");
        }
        std::vector<ExtraKv> host, stage;
        const int64_t host_cells = (dst->max_cells + o.ps - 1) / o.ps * o.ps;
        if ((rc = extra_kv(o, dst->host, dst->format, "a host copy", host, host_cells)) ||
            (rc = extra_kv(o, dst->stage, dst->format, "a staging pool", stage)))
            return rc;
        const int64_t logical_pages = (dst->max_cells + o.ps - 1) / o.ps;
        std::vector<sc::MoveRow> rows;
        uint64_t payload = 0;
        const uint64_t units = uint64_t(src->tokens) * uint64_t(o.H);
        for (int64_t j = 0; j < o.n_qsa && units; ++j) {
            const void* srcs[2] = {src->k[j], src->v[j]};
            const bool int8[2] = {k_int8, v_int8};
            // the paged pool through the page table, then the identity-layout copies (every carved cell)
            const ExtraKv pool{static_cast<uint8_t*>(dst->k_codes[j]), static_cast<uint8_t*>(dst->v_codes[j]),
                               k_int8 ? dst->k_scale[j] : nullptr, v_int8 ? dst->v_scale[j] : nullptr};
            const ExtraKv* dests[3] = {&pool, &host[size_t(j)], &stage[size_t(j)]};
            for (int d = 0; d < 3; ++d) {
                if (!dests[d]->k) continue;
                uint8_t* codes[2] = {dests[d]->k, dests[d]->v};
                uint16_t* scales[2] = {dests[d]->ks, dests[d]->vs};
                for (int a = 0; a < 2; ++a) {
                    sc::MoveRow r{};
                    r.kind = int8[a] ? sc::kKvQ8 : sc::kKvQ4;
                    r.src = static_cast<const uint8_t*>(srcs[a]);
                    r.dst = codes[a];
                    r.dst2 = reinterpret_cast<uint8_t*>(scales[a]);
                    r.table = d == 0 && dst->page_table ? dst->page_table[j] : nullptr;
                    r.pos0 = src->pos0;
                    r.ld = d == 0 ? dst->n_pages : logical_pages;
                    r.aux = int32_t(src->tokens);
                    r.n = units;
                    rows.push_back(r);
                    payload +=
                        units * sc::kQuantDim * 4 + units * (int8[a] ? sc::kQuantDim + 8 : sc::kQuantDim / 32 * 18);
                }
            }
        }
        if (src->with_gdn) {
            gdn_rows(o, src, dst->gdn_state, rows);
            payload += 2 * uint64_t(o.n_gdn) * o.gdn_row_bytes;
        }
        // the payload of a quantizing carve counts bytes read plus bytes written (they differ)
        return finish_plan(rows, o, payload, out);
    });
}

int sc_plan_gather(const sc_geometry* g, const sc_prefill_view* src, void* image, uint64_t image_bytes,
                   sc_plan** out) {
    return guarded([&] {
        if (!out) return fail(SC_EINVAL, "sc_handoff: missing plan output");
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        int rc = check_view(o, src);
        if (rc) return rc;
        if (src->pos0 != 0) return snapshot_fail("an image starts at cell 0");
        if (!src->with_gdn && o.n_gdn > 0) return snapshot_fail("an image carries the running state");
        uint64_t total = 0;
        const auto blobs = image_blobs(o, src->tokens, total);
        if (!image || image_bytes < total) return snapshot_fail("transfer buffer smaller than the image");
        if (!aligned16(image)) return fail(SC_EINVAL, "sc_handoff: transfer buffer must be 16-byte aligned");
        if (o.gdn_row_bytes % 16) return fail(SC_EINVAL, "sc_handoff: GDN rows must be multiples of 16 bytes");
        uint8_t* base = static_cast<uint8_t*>(image);
        const int64_t cells = cells_of(o, src->tokens);
        std::vector<sc::MoveRow> rows;
        size_t b = 0;
        for (int64_t j = 0; j < o.n_qsa; ++j, b += 2)
            kv_rows(o, src, j, reinterpret_cast<uint16_t*>(base + blobs[b].offset),
                    reinterpret_cast<uint16_t*>(base + blobs[b + 1].offset), nullptr, cells / o.ps, cells, rows);
        if (o.n_gdn > 0) gdn_rows(o, src, reinterpret_cast<float*>(base + blobs[b].offset), rows);
        gap_rows(blobs, total, base, rows);
        return finish_plan(rows, o, kv_payload(o, cells) + uint64_t(o.n_gdn) * o.gdn_row_bytes, out);
    });
}

static int page_plan(const sc_geometry* g, const void* image, uint64_t image_bytes, int64_t tokens,
                     const sc_decode_slot* slot, bool scatter, sc_plan** out) {
    if (!out) return fail(SC_EINVAL, "sc_handoff: missing plan output");
    Geo o;
    std::string why;
    if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
    if (tokens < 0 || tokens > (int64_t(1) << 30)) return snapshot_fail("invalid K/V extent");
    const int64_t cells = cells_of(o, tokens);
    // the reference's extent rule (conversation_snapshot.cpp:18-25,80-84): tokens within the capacity, and the
    // page-rounded extent within the pool's pages
    int rc = check_slot(o, slot, tokens, true);
    if (rc) return rc;
    if (slot_identity(slot, o.n_qsa) && cells / o.ps > slot->n_pages) return snapshot_fail("invalid K/V extent");
    uint64_t total = 0;
    const auto blobs = image_blobs(o, tokens, total);
    if (!image || image_bytes < total) return snapshot_fail("invalid K/V payload size");
    if (!aligned16(image)) return fail(SC_EINVAL, "sc_handoff: image must be 16-byte aligned");
    uint8_t* base = const_cast<uint8_t*>(static_cast<const uint8_t*>(image));
    std::vector<sc::MoveRow> rows;
    const uint64_t pages = uint64_t(cells / o.ps);
    size_t b = 0;
    for (int64_t j = 0; j < o.n_qsa; ++j, b += 2) {
        uint16_t* pools[2] = {slot->k_pool[j], slot->v_pool[j]};
        for (int a = 0; a < 2; ++a) {
            sc::MoveRow r{};
            r.kind = scatter ? sc::kPagesScatter : sc::kPagesGather;
            uint8_t* img = base + blobs[b + a].offset;
            r.src = scatter ? img : reinterpret_cast<const uint8_t*>(pools[a]);
            r.dst = scatter ? reinterpret_cast<uint8_t*>(pools[a]) : img;
            r.table = slot->page_table ? slot->page_table[j] : nullptr;
            r.n = pages * (o.page_bytes / 16);
            r.ld = slot->n_pages;
            if (r.n) rows.push_back(r);
        }
    }
    if (o.n_gdn > 0) {
        sc::MoveRow r{};
        r.kind = sc::kCopy;
        uint8_t* img = base + blobs[b].offset;
        r.src = scatter ? img : reinterpret_cast<const uint8_t*>(slot->gdn_state);
        r.dst = scatter ? reinterpret_cast<uint8_t*>(slot->gdn_state) : img;
        r.n = uint64_t(o.n_gdn) * o.gdn_row_bytes / 16;
        rows.push_back(r);
    }
    if (!scatter) gap_rows(blobs, total, base, rows);
    return finish_plan(rows, o, kv_payload(o, cells) + uint64_t(o.n_gdn) * o.gdn_row_bytes, out);
}

// A scatter from a segmented payload: each row reading payload bytes [off, off + 16 n) of `frame` is cut where a
// segment ends, every piece reading its own segment.  A page-scatter piece keeps its place in the blob's pages (pos0:
// the chunks of the blob before it); a copy piece moves its destination with it.
struct SegSpec {
    const uint8_t* frame;
    std::vector<uint8_t*> ptr;
    uint64_t bytes;   // of every segment but the last
};
void split_rows_at_segments(std::vector<sc::MoveRow>& rows, const SegSpec& seg) {
    std::vector<sc::MoveRow> out;
    for (const sc::MoveRow& r : rows) {
        const uint64_t off = uint64_t(r.src - seg.frame), end = off + r.n * 16;
        for (uint64_t o = off; o < end;) {
            const uint64_t k = o / seg.bytes, stop = std::min(end, (k + 1) * seg.bytes);
            sc::MoveRow piece = r;
            piece.src = seg.ptr[size_t(k)] + (o - k * seg.bytes);
            piece.n = (stop - o) / 16;
            if (r.kind == sc::kPagesScatter) piece.pos0 = r.pos0 + int64_t((o - off) / 16);
            else piece.dst = r.dst + (o - off);
            out.push_back(piece);
            o = stop;
        }
    }
    rows = std::move(out);
}

// Capture / scatter with caller-placed blobs: the K and V blob of QSA layer j at k_off[j] / v_off[j] and the GDN rows
// at gdn_off inside one buffer, plus zero-filled ranges (capture only).  Everything is checked before the plan exists.
static int map_plan(const sc_geometry* g, void* buf, uint64_t buf_bytes, const sc_blob_map* map, int64_t tokens,
                    const sc_decode_slot* slot, bool scatter, sc_plan** out, const SegSpec* seg = nullptr) {
    if (!out) return fail(SC_EINVAL, "sc_handoff: missing plan output");
    Geo o;
    std::string why;
    if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
    if (tokens < 0 || tokens > (int64_t(1) << 30)) return snapshot_fail("invalid K/V extent");
    int rc = check_slot(o, slot, tokens, true);
    if (rc) return rc;
    const int64_t cells = cells_of(o, tokens);
    if (slot_identity(slot, o.n_qsa) && cells / o.ps > slot->n_pages) return snapshot_fail("invalid K/V extent");
    if (!map || (o.n_qsa > 0 && (!map->k_off || !map->v_off)) || map->n_zero < 0 || (map->n_zero && !map->zero))
        return fail(SC_EINVAL, "sc_handoff: missing blob map");
    if (!buf || !aligned16(buf)) return fail(SC_EINVAL, "sc_handoff: the blob buffer must be 16-byte aligned");
    const uint64_t kv_bytes = uint64_t(cells) * uint64_t(o.H) * o.row_bytes;
    const uint64_t gdn_bytes = uint64_t(o.n_gdn) * o.gdn_row_bytes;
    struct Range { uint64_t at, n; };
    std::vector<Range> used;
    auto place = [&](uint64_t at, uint64_t n) {
        if (at % 16 || at > buf_bytes || n > buf_bytes - at) return false;
        if (n) used.push_back({at, n});
        return true;
    };
    for (int64_t j = 0; j < o.n_qsa; ++j)
        if (!place(map->k_off[j], kv_bytes) || !place(map->v_off[j], kv_bytes))
            return snapshot_fail("a K/V blob lies outside the buffer or off a 16-byte boundary");
    if (o.n_gdn > 0 && !place(map->gdn_off, gdn_bytes))
        return snapshot_fail("the running-state blob lies outside the buffer or off a 16-byte boundary");
    for (int64_t z = 0; z < map->n_zero && !scatter; ++z)
        if (map->zero[2 * z + 1] % 16 || !place(map->zero[2 * z], map->zero[2 * z + 1]))
            return fail(SC_EINVAL, "sc_handoff: a zero range must be 16-byte aligned, whole chunks, inside the buffer");
    std::sort(used.begin(), used.end(), [](const Range& a, const Range& b) { return a.at < b.at; });
    for (size_t i = 1; i < used.size(); ++i)
        if (used[i].at < used[i - 1].at + used[i - 1].n) return fail(SC_EINVAL, "sc_handoff: blobs overlap in the buffer");
    uint8_t* base = static_cast<uint8_t*>(buf);
    std::vector<sc::MoveRow> rows;
    const uint64_t pages = uint64_t(cells / o.ps);
    for (int64_t j = 0; j < o.n_qsa; ++j) {
        uint16_t* pools[2] = {slot->k_pool[j], slot->v_pool[j]};
        const uint64_t offs[2] = {map->k_off[j], map->v_off[j]};
        for (int a = 0; a < 2; ++a) {
            sc::MoveRow r{};
            r.kind = scatter ? sc::kPagesScatter : sc::kPagesGather;
            r.src = scatter ? base + offs[a] : reinterpret_cast<const uint8_t*>(pools[a]);
            r.dst = scatter ? reinterpret_cast<uint8_t*>(pools[a]) : base + offs[a];
            r.table = slot->page_table ? slot->page_table[j] : nullptr;
            r.n = pages * (o.page_bytes / 16);
            r.ld = slot->n_pages;
            if (r.n) rows.push_back(r);
        }
    }
    if (o.n_gdn > 0) {
        sc::MoveRow r{};
        r.kind = sc::kCopy;
        r.src = scatter ? base + map->gdn_off : reinterpret_cast<const uint8_t*>(slot->gdn_state);
        r.dst = scatter ? reinterpret_cast<uint8_t*>(slot->gdn_state) : base + map->gdn_off;
        r.n = gdn_bytes / 16;
        rows.push_back(r);
    }
    for (int64_t z = 0; z < map->n_zero && !scatter; ++z) {
        sc::MoveRow r{};
        r.kind = sc::kZero;
        r.dst = base + map->zero[2 * z];
        r.n = map->zero[2 * z + 1] / 16;
        if (r.n) rows.push_back(r);
    }
    if (seg) split_rows_at_segments(rows, *seg);
    return finish_plan(rows, o, 2 * kv_bytes * uint64_t(o.n_qsa) + gdn_bytes, out);
}

int sc_plan_capture_map(const sc_geometry* g, const sc_decode_slot* src, int64_t tokens, void* dst, uint64_t dst_bytes,
                        const sc_blob_map* map, sc_plan** out) {
    return guarded([&] { return map_plan(g, dst, dst_bytes, map, tokens, src, false, out); });
}

int sc_plan_scatter_map(const sc_geometry* g, const void* src, uint64_t src_bytes, const sc_blob_map* map,
                        int64_t tokens, const sc_decode_slot* dst, sc_plan** out) {
    return guarded([&] {
        return map_plan(g, const_cast<void*>(src), src_bytes, map, tokens, dst, true, out);
    });
}

int sc_plan_scatter(const sc_geometry* g, const void* image, uint64_t image_bytes, int64_t tokens,
                    const sc_decode_slot* dst, sc_plan** out) {
    return guarded([&] { return page_plan(g, image, image_bytes, tokens, dst, true, out); });
}

int sc_plan_capture(const sc_geometry* g, const sc_decode_slot* src, int64_t tokens, void* image,
                    uint64_t image_bytes, sc_plan** out) {
    return guarded([&] { return page_plan(g, image, image_bytes, tokens, src, false, out); });
}

int sc_plan_copies(const sc_copy* copies, int32_t n, sc_plan** out) {
    return guarded([&] {
        if (!out || n < 0 || (n && !copies)) return fail(SC_EINVAL, "sc_handoff: missing copy plan argument");
        std::vector<sc::MoveRow> rows;
        std::vector<std::pair<uintptr_t, uintptr_t>> spans;
        uint64_t payload = 0;
        for (int32_t i = 0; i < n; ++i) {
            const sc_copy& c = copies[i];
            if (!c.bytes) continue;
            if (!c.dst || !c.src || !aligned16(c.dst) || !aligned16(c.src) || c.bytes % 16)
                return fail(SC_EINVAL, "sc_handoff: copies are whole 16-byte chunks between 16-byte aligned addresses");
            sc::MoveRow r{};
            r.kind = sc::kCopy;
            r.src = static_cast<const uint8_t*>(c.src);
            r.dst = static_cast<uint8_t*>(c.dst);
            r.n = c.bytes / 16;
            rows.push_back(r);
            spans.push_back({reinterpret_cast<uintptr_t>(c.dst), reinterpret_cast<uintptr_t>(c.dst) + c.bytes});
            payload += c.bytes;
        }
        std::sort(spans.begin(), spans.end());
        for (size_t i = 1; i < spans.size(); ++i)
            if (spans[i].first < spans[i - 1].second)
                return fail(SC_EINVAL, "sc_handoff: two copies of a copy plan write the same bytes");
        // the rows need no geometry; a unit one keeps the plan's divisors defined
        Geo unit;
        unit.H = unit.ps = unit.HV = 1;
        unit.D = 8;
        unit.S = 4;
        unit.row_bytes = unit.page_bytes = 16;
        return finish_plan(rows, unit, payload, out);
    });
}

int sc_layer_blob_bytes(const sc_geometry* g, int32_t format, int32_t with_index, int64_t tokens, uint64_t* bytes) {
    return guarded([&] {
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        uint64_t b[SC_N_BUF];
        why = layer_blob_sizes(o, g, format, with_index != 0, tokens, b);
        if (!why.empty()) return snapshot_fail(why.c_str());
        if (bytes) std::copy(b, b + SC_N_BUF, bytes);
        return ok();
    });
}

int sc_image_layout_layers(const sc_geometry* g, int32_t format, int32_t with_index, int64_t tokens, uint64_t* offsets,
                           uint64_t* total_bytes) {
    return guarded([&] {
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        uint64_t b[SC_N_BUF];
        why = layer_blob_sizes(o, g, format, with_index != 0, tokens, b);
        if (!why.empty()) return snapshot_fail(why.c_str());
        std::vector<uint64_t> off;
        const uint64_t total = layers_layout(o, b, off);
        if (offsets) std::copy(off.begin(), off.end(), offsets);
        if (total_bytes) *total_bytes = total;
        return ok();
    });
}

// One launch moving every blob of an sc_slot_layers slot between the slot (identity pools: a blob is a prefix of
// its buffer) and a buffer laid out by `map` (or the standard image when map is NULL).
static int layers_plan(const sc_geometry* g, void* buf, uint64_t buf_bytes, const sc_layers_map* map, int64_t tokens,
                       const sc_slot_layers* slot, bool scatter, sc_plan** out, const SegSpec* seg = nullptr) {
    if (!out) return fail(SC_EINVAL, "sc_handoff: missing plan output");
    Geo o;
    std::string why;
    if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
    uint64_t b[SC_N_BUF];
    int rc = check_layers(o, g, slot, tokens, b);
    if (rc) return rc;
    if (!buf || !aligned16(buf)) return fail(SC_EINVAL, "sc_handoff: the blob buffer must be 16-byte aligned");
    std::vector<uint64_t> std_off, zero;
    const uint64_t* off = nullptr;
    if (map) {
        if (!map->off || map->n_zero < 0 || (map->n_zero && !map->zero))
            return fail(SC_EINVAL, "sc_handoff: missing blob map");
        off = map->off;
        if (!scatter) zero.assign(map->zero, map->zero + 2 * map->n_zero);
    } else {
        const uint64_t total = layers_layout(o, b, std_off);
        if (total > buf_bytes) return snapshot_fail("invalid K/V payload size");
        off = std_off.data();
        if (!scatter) {   // a capture clears the gaps of the standard image
            uint64_t at = 0;
            auto gap = [&](uint64_t end) {
                if (end > at) { zero.push_back(at); zero.push_back(end - at); }
            };
            for (int64_t j = 0; j < o.n_qsa; ++j)
                for (int k = 0; k < SC_N_BUF; ++k)
                    if (b[k]) {
                        gap(off[size_t(j) * SC_N_BUF + k]);
                        at = off[size_t(j) * SC_N_BUF + k] + b[k];
                    }
            if (o.n_gdn > 0) {
                gap(off[size_t(o.n_qsa) * SC_N_BUF]);
                at = off[size_t(o.n_qsa) * SC_N_BUF] + uint64_t(o.n_gdn) * o.gdn_row_bytes;
            }
            gap(total);
        }
    }
    struct Range { uint64_t at, n; };
    std::vector<Range> used;
    auto place = [&](uint64_t at, uint64_t n) {
        if (at % 16 || at > buf_bytes || n > buf_bytes - at) return false;
        if (n) used.push_back({at, n});
        return true;
    };
    const uint64_t gdn_bytes = uint64_t(o.n_gdn) * o.gdn_row_bytes;
    for (int64_t j = 0; j < o.n_qsa; ++j)
        for (int k = 0; k < SC_N_BUF; ++k) {
            const uint64_t at = off[size_t(j) * SC_N_BUF + k];
            if (!b[k]) {
                if (at != kAbsent) return snapshot_fail("a blob map places a blob the slot's format does not have");
                continue;
            }
            if (!place(at, b[k])) return snapshot_fail("a K/V blob lies outside the buffer or off a 16-byte boundary");
        }
    const uint64_t gdn_at = off[size_t(o.n_qsa) * SC_N_BUF];
    if (o.n_gdn > 0 && !place(gdn_at, gdn_bytes))
        return snapshot_fail("the running-state blob lies outside the buffer or off a 16-byte boundary");
    for (size_t z = 0; z < zero.size(); z += 2)
        if (zero[z + 1] % 16 || !place(zero[z], zero[z + 1]))
            return fail(SC_EINVAL, "sc_handoff: a zero range must be 16-byte aligned, whole chunks, inside the buffer");
    std::sort(used.begin(), used.end(), [](const Range& x, const Range& y) { return x.at < y.at; });
    for (size_t i = 1; i < used.size(); ++i)
        if (used[i].at < used[i - 1].at + used[i - 1].n) return fail(SC_EINVAL, "sc_handoff: blobs overlap in the buffer");
    uint8_t* base = static_cast<uint8_t*>(buf);
    std::vector<sc::MoveRow> rows;
    uint64_t moved = 0;
    auto copy = [&](uint8_t* slot_side, uint64_t at, uint64_t n) {
        sc::MoveRow r{};
        r.kind = sc::kCopy;
        r.src = scatter ? base + at : slot_side;
        r.dst = scatter ? slot_side : base + at;
        r.n = n / 16;
        if (r.n) rows.push_back(r);
        moved += n;
    };
    for (int64_t j = 0; j < o.n_qsa; ++j)
        for (int k = 0; k < SC_N_BUF; ++k)
            if (b[k]) copy(static_cast<uint8_t*>(slot->buf[k][j]), off[size_t(j) * SC_N_BUF + k], b[k]);
    if (o.n_gdn > 0) copy(reinterpret_cast<uint8_t*>(slot->gdn_state), gdn_at, gdn_bytes);
    for (size_t z = 0; z < zero.size(); z += 2) {
        sc::MoveRow r{};
        r.kind = sc::kZero;
        r.dst = base + zero[z];
        r.n = zero[z + 1] / 16;
        if (r.n) rows.push_back(r);
    }
    if (seg) split_rows_at_segments(rows, *seg);
    return finish_plan(rows, o, moved, out);
}

int sc_plan_capture_layers(const sc_geometry* g, const sc_slot_layers* src, int64_t tokens, void* dst,
                           uint64_t dst_bytes, const sc_layers_map* map, sc_plan** out) {
    return guarded([&] { return layers_plan(g, dst, dst_bytes, map, tokens, src, false, out); });
}

int sc_plan_scatter_layers(const sc_geometry* g, const void* src, uint64_t src_bytes, const sc_layers_map* map,
                           int64_t tokens, const sc_slot_layers* dst, sc_plan** out) {
    return guarded([&] { return layers_plan(g, const_cast<void*>(src), src_bytes, map, tokens, dst, true, out); });
}

// The segments of a segmented payload of `bytes`, as a SegSpec whose frame is the first segment.
static int seg_spec(const sc_segments* s, uint64_t bytes, SegSpec& spec) {
    if (!s || s->n < 1 || s->n > SC_IPC_MAX_SEGMENTS || !s->ptr || s->segment_bytes == 0 || s->segment_bytes % 16)
        return fail(SC_EINVAL, "sc_handoff: a segmented payload needs 1 to SC_IPC_MAX_SEGMENTS segments of whole chunks");
    if (uint64_t(s->n) < (bytes + s->segment_bytes - 1) / s->segment_bytes)
        return fail(SC_ERANGE, "sc_handoff: the segments are smaller than the payload");
    spec.ptr.clear();
    for (int32_t k = 0; k < s->n; ++k) spec.ptr.push_back(static_cast<uint8_t*>(s->ptr[k]));
    for (uint8_t* q : spec.ptr)
        if (!q || !aligned16(q)) return fail(SC_EINVAL, "sc_handoff: every segment is 16-byte aligned device memory");
    spec.frame = spec.ptr[0];
    spec.bytes = s->segment_bytes;
    return SC_OK;
}

int sc_plan_scatter_map_segments(const sc_geometry* g, const sc_segments* src, uint64_t src_bytes,
                                 const sc_blob_map* map, int64_t tokens, const sc_decode_slot* dst, sc_plan** out) {
    return guarded([&] {
        SegSpec spec;
        if (const int rc = seg_spec(src, src_bytes, spec)) return rc;
        return map_plan(g, const_cast<uint8_t*>(spec.frame), src_bytes, map, tokens, dst, true, out, &spec);
    });
}

int sc_plan_scatter_layers_segments(const sc_geometry* g, const sc_segments* src, uint64_t src_bytes,
                                    const sc_layers_map* map, int64_t tokens, const sc_slot_layers* dst,
                                    sc_plan** out) {
    return guarded([&] {
        SegSpec spec;
        if (const int rc = seg_spec(src, src_bytes, spec)) return rc;
        return layers_plan(g, const_cast<uint8_t*>(spec.frame), src_bytes, map, tokens, dst, true, out, &spec);
    });
}

namespace {
// The order pre-pass of a plan with destination-ordered rows; it writes only the plan's own workspace, so launches
// of one plan on different streams must not overlap.
hipError_t launch_order(const sc_plan* plan, hipStream_t stream) {
    if (!plan->n_order_groups || !plan->n_tiles) return hipSuccess;
    return sc::launch_page_order(plan->order_groups, plan->n_order_groups, plan->order_max_pages, plan->order_max_blocks,
                                 stream);
}
}  // namespace

int64_t sc_set_order_min_pages(int64_t pages) { return g_order_min_pages.exchange(pages); }

int sc_plan_order_groups(const sc_plan* plan) { return plan ? plan->n_order_groups : 0; }

int sc_plan_launch(const sc_plan* plan, void* stream) {
    if (!plan) return fail(SC_EINVAL, "sc_handoff: missing plan");
    if (plan->batch) {
        const hipError_t e = sc::launch_batch(plan->batch_args, plan->order_groups, plan->order_max_blocks, plan->grid,
                                              static_cast<hipStream_t>(stream));
        return e == hipSuccess ? ok() : hip_fail(e, "batch launch");
    }
    hipError_t e = launch_order(plan, static_cast<hipStream_t>(stream));
    if (e == hipSuccess)
        e = sc::launch_move(plan->rows_dev, plan->tile_row_dev, plan->geo, plan->n_tiles, plan->grid, plan->mix,
                            plan->xcd, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "move launch");
}

int sc_plan_launch_gated(const sc_plan* plan, const uint32_t* gate, void* stream) {
    if (!plan || !gate || (reinterpret_cast<uintptr_t>(gate) & 3u))
        return fail(SC_EINVAL, "sc_handoff: a gated launch needs a plan and a 4-byte aligned gate word");
    if (plan->batch) return fail(SC_EINVAL, "sc_handoff: a batched plan is all or nothing on its own lengths");
    hipError_t e = launch_order(plan, static_cast<hipStream_t>(stream));
    if (e == hipSuccess)
        e = sc::launch_move(plan->rows_dev, plan->tile_row_dev, plan->geo, plan->n_tiles, plan->grid, plan->mix,
                            plan->xcd, static_cast<hipStream_t>(stream), gate);
    return e == hipSuccess ? ok() : hip_fail(e, "move launch");
}

uint64_t sc_plan_payload_bytes(const sc_plan* plan) { return plan ? plan->payload : 0; }

int sc_plan_set_grid(sc_plan* plan, int64_t workgroups) {
    if (!plan || workgroups < 0 || workgroups > (int64_t(1) << 30)) return fail(SC_EINVAL, "sc_handoff: invalid grid");
    plan->grid = workgroups == 0 ? plan->default_grid : workgroups;
    if (plan->rt) plan->rt->grid_set = workgroups != 0;
    return ok();
}

int sc_plan_destroy(sc_plan* plan) {
    if (!plan) return ok();
    hipError_t e = plan->rows_dev ? hipFree(plan->rows_dev) : hipSuccess;
    const hipError_t e2 = plan->tile_row_dev ? hipFree(plan->tile_row_dev) : hipSuccess;
    const hipError_t e3 = plan->batch_ptrs_dev ? hipFree(plan->batch_ptrs_dev) : hipSuccess;
    const hipError_t e4 = plan->order_ws ? hipFree(plan->order_ws) : hipSuccess;
    if (e == hipSuccess) e = e2;
    if (e == hipSuccess) e = e3;
    if (e == hipSuccess) e = e4;
    delete plan->rt;
    delete plan;
    return e == hipSuccess ? ok() : hip_fail(e, "table free");
}

// ---- capture plans fused with the payload hash -------------------------------------------------------------------

}  // extern "C"

namespace {
// The extents of the payload [0, bytes) that `n_plans` capture plans write, their rows' destinations taken relative to
// `frame` (the payload they were built for); the bytes no row writes become self extents.
int capture_extents(const sc_plan* const* plans, int32_t n_plans, const uint8_t* frame, uint64_t bytes,
                    std::vector<sc::HashExtent>& ext) {
    std::vector<sc::HashExtent> rows;
    for (int32_t i = 0; i < n_plans; ++i) {
        const sc_plan* p = plans[i];
        if (!p || p->batch) return fail(SC_EINVAL, "sc_handoff: a hash map reads the rows of capture plans");
        for (const sc::MoveRow& r : p->host_rows) {
            sc::HashExtent x{};
            switch (r.kind) {
                case sc::kCopy: x.kind = sc::kExtCopy; x.src = r.src; break;
                case sc::kZero: x.kind = sc::kExtZero; break;
                case sc::kPagesGather:
                    x.kind = sc::kExtPages;
                    x.src = r.src;
                    x.table = r.table;
                    x.ld = r.ld;
                    x.page_chunks = p->geo.page_chunks.d;
                    break;
                default:
                    return fail(SC_EINVAL, "sc_handoff: only capture plans (page gathers, copies and zero fills into "
                                           "the payload) can be fused with its hash");
            }
            if (r.dst < frame || uint64_t(r.dst - frame) > bytes || r.n * 16 > bytes - uint64_t(r.dst - frame))
                return fail(SC_EINVAL, "sc_handoff: a row of the plan writes outside the hashed payload");
            x.off = uint64_t(r.dst - frame);
            x.end = x.off + r.n * 16;
            // pages through the identity table, every one inside the pool, are one contiguous source: page k of
            // the row is pool page k, so payload byte o comes from src + (o - off)
            if (x.kind == sc::kExtPages && !x.table && x.page_chunks &&
                (r.n + x.page_chunks - 1) / x.page_chunks <= uint64_t(std::max<int64_t>(x.ld, 0)))
                x = sc::HashExtent{x.off, x.end, x.src, nullptr, 0, sc::kExtCopy, 0};
            if (x.end > x.off) rows.push_back(x);
        }
    }
    std::sort(rows.begin(), rows.end(), [](const sc::HashExtent& a, const sc::HashExtent& b) { return a.off < b.off; });
    ext.clear();
    uint64_t at = 0;
    for (const sc::HashExtent& x : rows) {
        if (x.off < at) return fail(SC_EINVAL, "sc_handoff: two rows of the plans write the same payload bytes");
        if (x.off > at) ext.push_back(sc::HashExtent{at, x.off, nullptr, nullptr, 0, sc::kExtSelf, 0});
        ext.push_back(x);
        at = x.end;
    }
    if (at < bytes || ext.empty()) ext.push_back(sc::HashExtent{at, bytes, nullptr, nullptr, 0, sc::kExtSelf, 0});
    return SC_OK;
}

// Checks a segmented payload of `bytes` and lists its segments.
int segment_list(const sc_segments* s, uint64_t bytes, std::vector<uint8_t*>& segs) {
    if (!s || s->n < 1 || s->n > SC_IPC_MAX_SEGMENTS || !s->ptr)
        return fail(SC_EINVAL, "sc_handoff: a segmented payload needs 1 to SC_IPC_MAX_SEGMENTS segments");
    if (s->segment_bytes == 0 || s->segment_bytes % uint64_t(sc::kFnvGroupBytes))
        return fail(SC_EINVAL, "sc_handoff: segments of a hashed payload are whole multiples of 64 KiB");
    if (uint64_t(s->n) < (bytes + s->segment_bytes - 1) / s->segment_bytes)
        return fail(SC_ERANGE, "sc_handoff: the segments are smaller than the payload");
    segs.clear();
    for (int32_t k = 0; k < s->n; ++k) segs.push_back(static_cast<uint8_t*>(s->ptr[k]));
    for (uint8_t* q : segs)
        if (!q || !aligned16(q)) return fail(SC_EINVAL, "sc_handoff: every segment is 16-byte aligned device memory");
    return SC_OK;
}

// Makes a map in one device block: the extents and the segment table uploaded, each workgroup's part (sc::HashGroup)
// built from them on the device (hash_groups_kernel), waited for before the map is handed out.  A map that only reads
// (no extents) is hashed by the plain kernel from the segment table alone, so it needs nothing else.
int make_hash_map(const std::vector<sc::HashExtent>& ext, uint64_t bytes, const std::vector<uint8_t*>& segs,
                  uint64_t seg_bytes, bool store, sc_hash_map** out) {
    const sc::FnvWorkspace w = sc::fnv_workspace(bytes);
    const uint64_t n_grp = store ? std::max<uint64_t>(w.groups, 1) : 1;
    if (ext.size() >= (uint64_t(1) << 32) || segs.empty())
        return fail(SC_ERANGE, "sc_handoff: a hash map holds fewer than 2^32 extents and at least one segment");
    auto* m = new (std::nothrow) sc_hash_map();
    if (!m) return fail(SC_ENOMEM, "sc_handoff: hash map allocation failed");
    const uint64_t ext_bytes = round_up(ext.size() * sizeof(sc::HashExtent), 256);
    const uint64_t grp_bytes = round_up(n_grp * sizeof(sc::HashGroup), 256);
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&m->ext_dev), ext_bytes + grp_bytes + segs.size() * 8);
    if (err != hipSuccess) {
        delete m;
        return fail(SC_ENOMEM, std::string("sc_handoff: hash map: ") + hipGetErrorString(err));
    }
    uint8_t* block = reinterpret_cast<uint8_t*>(m->ext_dev);
    m->grp_dev = reinterpret_cast<sc::HashGroup*>(block + ext_bytes);
    m->seg_dev = reinterpret_cast<uint8_t**>(block + ext_bytes + grp_bytes);
    if (!ext.empty()) err = hipMemcpy(m->ext_dev, ext.data(), ext.size() * sizeof(sc::HashExtent), hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(m->seg_dev, segs.data(), segs.size() * 8, hipMemcpyHostToDevice);
    if (err == hipSuccess && store && !ext.empty())
        err = sc::launch_hash_groups(m->ext_dev, uint32_t(ext.size()), bytes, m->seg_dev, uint32_t(segs.size()),
                                     seg_bytes, m->grp_dev, w.groups, nullptr);
    if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
    if (err != hipSuccess) {
        (void) hipFree(m->ext_dev);
        delete m;
        return hip_fail(err, "hash map upload");
    }
    const uint64_t n_full = bytes & ~uint64_t(sc::kFnvLaneBytes - 1);
    m->seg_bytes = seg_bytes;
    m->tail = segs[size_t(std::min<uint64_t>(n_full / seg_bytes, segs.size() - 1))] + n_full % seg_bytes;
    m->bytes = bytes;
    m->store = store;
    *out = m;
    return ok();
}

int hash_map_args(const sc_hash_map* map, const uint32_t* fault, const void* workspace, uint64_t workspace_bytes) {
    if (!map) return fail(SC_EINVAL, "sc_handoff: missing hash map");
    if (reinterpret_cast<uintptr_t>(fault) & 3u) return fail(SC_EINVAL, "sc_handoff: the hash fault word must be 4-byte aligned");
    if (!workspace || workspace_bytes < sc::fnv_workspace(map->bytes).bytes)
        return fail(SC_EINVAL, "sc_handoff: hash workspace smaller than sc_fnv1a64_workspace_bytes()");
    if (reinterpret_cast<uintptr_t>(workspace) & 15u) return fail(SC_EINVAL, "sc_handoff: hash workspace must be 16-byte aligned");
    return SC_OK;
}
}  // namespace

extern "C" {

int sc_hash_map_create(const sc_plan* const* plans, int32_t n_plans, void* payload, uint64_t bytes, sc_hash_map** out) {
    return guarded([&] {
        if (!out || (n_plans && !plans) || n_plans < 0) return fail(SC_EINVAL, "sc_handoff: missing hash map argument");
        if ((bytes && !payload) || !aligned16(payload) || bytes % 16)
            return fail(SC_EINVAL, "sc_handoff: a hashed payload is 16-byte aligned and whole 16-byte chunks");
        if (bytes > (uint64_t(1) << 46)) return fail(SC_ERANGE, "sc_handoff: hash input beyond 2^46 bytes");
        std::vector<sc::HashExtent> ext;
        if (const int rc = capture_extents(plans, n_plans, static_cast<uint8_t*>(payload), bytes, ext)) return rc;
        return make_hash_map(ext, bytes, {static_cast<uint8_t*>(payload)}, uint64_t(1) << 62, true, out);
    });
}

int sc_hash_map_create_segments(const sc_plan* const* plans, int32_t n_plans, const void* frame, uint64_t bytes,
                                const sc_segments* into, sc_hash_map** out) {
    return guarded([&] {
        if (!out || (n_plans && !plans) || n_plans < 0 || !frame)
            return fail(SC_EINVAL, "sc_handoff: missing hash map argument");
        if (!aligned16(frame) || bytes % 16)
            return fail(SC_EINVAL, "sc_handoff: a hashed payload is 16-byte aligned and whole 16-byte chunks");
        if (bytes > (uint64_t(1) << 46)) return fail(SC_ERANGE, "sc_handoff: hash input beyond 2^46 bytes");
        std::vector<uint8_t*> segs;
        if (const int rc = segment_list(into, bytes, segs)) return rc;
        std::vector<sc::HashExtent> ext;
        if (const int rc = capture_extents(plans, n_plans, static_cast<const uint8_t*>(frame), bytes, ext)) return rc;
        return make_hash_map(ext, bytes, segs, into->segment_bytes, true, out);
    });
}

int sc_hash_map_create_read(const sc_segments* from, uint64_t bytes, sc_hash_map** out) {
    return guarded([&] {
        if (!out) return fail(SC_EINVAL, "sc_handoff: missing hash map argument");
        if (bytes % 16) return fail(SC_EINVAL, "sc_handoff: a hashed payload is whole 16-byte chunks");
        std::vector<uint8_t*> segs;
        if (const int rc = segment_list(from, bytes, segs)) return rc;
        return make_hash_map({}, bytes, segs, from->segment_bytes, false, out);
    });
}

int sc_hash_map_launch(const sc_hash_map* map, uint64_t seed, uint64_t* out, uint32_t* fault, void* workspace,
                       uint64_t workspace_bytes, void* stream) {
    if (const int rc = hash_map_args(map, fault, workspace, workspace_bytes)) return rc;
    if (!out || !fault) return fail(SC_EINVAL, "sc_handoff: missing hash output or fault word");
    const sc::HashMapArgs a{map->ext_dev, map->grp_dev, map->seg_dev, map->seg_bytes, map->bytes, map->store ? 1u : 0u};
    const hipError_t e =
        sc::launch_fnv1a64_mapped(a, map->tail, seed, out, fault, workspace, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "mapped hash launch");
}

int sc_hash_map_check_async(const sc_hash_map* map, uint64_t seed, uint64_t expected, uint64_t* out, uint32_t* verdict,
                            uint32_t* fault, void* workspace, uint64_t workspace_bytes, void* stream) {
    if (const int rc = hash_map_args(map, fault, workspace, workspace_bytes)) return rc;
    if (!out || !verdict || (reinterpret_cast<uintptr_t>(verdict) & 3u))
        return fail(SC_EINVAL, "sc_handoff: missing hash output, or a verdict word that is not 4-byte aligned");
    const sc::HashMapArgs a{map->ext_dev, map->grp_dev, map->seg_dev, map->seg_bytes, map->bytes, map->store ? 1u : 0u};
    const hipError_t e = sc::launch_fnv1a64_mapped(a, map->tail, seed, out, fault, workspace,
                                                   static_cast<hipStream_t>(stream), expected, verdict);
    return e == hipSuccess ? ok() : hip_fail(e, "mapped hash launch");
}

int sc_hash_map_launch_carry(const sc_hash_map* map, uint64_t seed, uint64_t* out, uint32_t* fault, uint8_t* carry_out,
                             void* workspace, uint64_t workspace_bytes, void* stream) {
    if (const int rc = hash_map_args(map, fault, workspace, workspace_bytes)) return rc;
    if (!out || !fault) return fail(SC_EINVAL, "sc_handoff: missing hash output or fault word");
    if (!carry_out && sc::fnv_carry_count(map->bytes)) return fail(SC_EINVAL, "sc_handoff: missing carry output");
    const sc::HashMapArgs a{map->ext_dev, map->grp_dev, map->seg_dev, map->seg_bytes, map->bytes, map->store ? 1u : 0u};
    sc::FnvCarries c;
    c.out = carry_out;
    const hipError_t e = sc::launch_fnv1a64_mapped(a, map->tail, seed, out, fault, workspace,
                                                   static_cast<hipStream_t>(stream), 0, nullptr, c);
    return e == hipSuccess ? ok() : hip_fail(e, "mapped hash launch");
}

int sc_hash_map_check_carried_async(const sc_hash_map* map, uint64_t seed, uint64_t expected, const uint8_t* carry,
                                    uint64_t* out, uint32_t* verdict, uint32_t* fault, void* workspace,
                                    uint64_t workspace_bytes, void* stream) {
    if (const int rc = hash_map_args(map, fault, workspace, workspace_bytes)) return rc;
    if (!out || !verdict || (reinterpret_cast<uintptr_t>(verdict) & 3u))
        return fail(SC_EINVAL, "sc_handoff: missing hash output, or a verdict word that is not 4-byte aligned");
    if (!carry && sc::fnv_carry_count(map->bytes)) return fail(SC_EINVAL, "sc_handoff: missing carries");
    if (map->store)
        return fail(SC_EINVAL, "sc_handoff: a check with carries reads the payload where it lies (sc_hash_map_create_read)");
    const sc::HashMapArgs a{map->ext_dev, map->grp_dev, map->seg_dev, map->seg_bytes, map->bytes, 0u};
    sc::FnvCarries c;
    c.in = carry;
    const hipError_t e = sc::launch_fnv1a64_mapped(a, map->tail, seed, out, fault, workspace,
                                                   static_cast<hipStream_t>(stream), expected, verdict, c);
    return e == hipSuccess ? ok() : hip_fail(e, "mapped hash launch");
}

int sc_hash_map_destroy(sc_hash_map* map) {
    if (!map) return ok();
    const hipError_t e = map->ext_dev ? hipFree(map->ext_dev) : hipSuccess;
    delete map;
    return e == hipSuccess ? ok() : hip_fail(e, "hash map free");
}

#define SC_HIP(call, what)                                    \
    do {                                                      \
        const hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return hip_fail(e_, what);      \
    } while (0)

// ---- kv_append: the per-layer prefill writers ---------------------------------------------------------------------

namespace {

bool misaligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; }

// One destination set of a kv_append call: K and V codes (f16 rows, int8 codes or q4_0 blocks), the int8 scales,
// and the page table (NULL: identity, the layout of the host copy and of the staging pool).
struct AppendDest {
    void* k;
    void* v;
    uint16_t* ks;
    uint16_t* vs;
    const int32_t* table;
    bool host_copy = false;   // written by the kernel straight into host memory
};

// Checks and lays out the rows of one call.  `kind` is sc::kKv32, kKvQ8 or kKvQ4; `dests` holds the pool first.
int append_launch(int32_t kind, const float* K, const float* V, int64_t T, int64_t pos0, int64_t H, int64_t D,
                  int64_t page_size, const AppendDest* dests, int n_dests, void* stream) {
    if (pos0 < 0 || T > (int64_t(1) << 30) || pos0 > (int64_t(1) << 30) || page_size < 1 || page_size > (1 << 20))
        return fail(SC_EINVAL, "sc_handoff: kv_append: invalid extent (pos0, T or page_size)");
    if (!K || !V) return fail(SC_EINVAL, "sc_handoff: kv_append: missing K or V");
    if (misaligned(K, 16) || misaligned(V, 16))
        return fail(SC_EINVAL, "sc_handoff: kv_append: K and V must be 16-byte aligned");
    // the tiles index a row's chunks (f16 rows) or (token, head) rows (quantized) with 32-bit integers
    const uint64_t units = uint64_t(T) * uint64_t(H) * (kind == sc::kKv32 ? uint64_t(D * 2 / 16) : 1u);
    if (units >= kMaxRowChunks)
        return fail(SC_ERANGE, "sc_handoff: kv_append: one call's K or V beyond 2^31 chunks (split the chunk)");
    const uintptr_t code_align = kind == sc::kKv32 ? 16 : kind == sc::kKvQ8 ? 4 : 2;
    sc::AppendRows rows{};
    int n = 0;
    for (int d = 0; d < n_dests; ++d) {
        const AppendDest& a = dests[d];
        if (!a.k || !a.v || (kind == sc::kKvQ8 && (!a.ks || !a.vs)))
            return fail(SC_EINVAL, kind == sc::kKvQ8 ? "sc_handoff: kv_append: int8 destinations need K and V codes "
                                                       "and both scale arrays"
                                                     : "sc_handoff: kv_append: a destination needs both K and V");
        if (misaligned(a.k, code_align) || misaligned(a.v, code_align) ||
            (kind == sc::kKvQ8 && (misaligned(a.ks, 8) || misaligned(a.vs, 8))))
            return fail(SC_EINVAL, "sc_handoff: kv_append: f16 pools must be 16-byte, int8 codes 4-byte, int8 scales "
                                   "8-byte and q4_0 pools 2-byte aligned");
        if (a.host_copy) {
            // the pages of cells [pos0, pos0 + T) of the identity layout, which the kernel writes in host memory
            const uint64_t first = uint64_t(pos0 / page_size), end = uint64_t((pos0 + T + page_size - 1) / page_size);
            const uint64_t row0 = first * uint64_t(page_size) * uint64_t(H), rows_n = (end - first) * uint64_t(page_size) * uint64_t(H);
            const uint64_t code_row = kind == sc::kKv32 ? uint64_t(D) * 2 : kind == sc::kKvQ8 ? uint64_t(D) : uint64_t(D) / 32 * 18;
            const struct { const void* p; uint64_t row; } pools[4] = {
                {a.k, code_row}, {a.v, code_row}, {a.ks, uint64_t(D) / 64 * 2}, {a.vs, uint64_t(D) / 64 * 2}};
            for (const auto& q : pools)
                if (q.p && !mapped_host_range(static_cast<const uint8_t*>(q.p) + row0 * q.row, rows_n * q.row))
                    return fail(SC_EINVAL, "sc_handoff: kv_append: a host copy must be pinned memory mapped for the "
                                           "device");
        }
        const float* srcs[2] = {K, V};
        void* codes[2] = {a.k, a.v};
        uint16_t* scales[2] = {a.ks, a.vs};
        for (int kv = 0; kv < 2; ++kv) {
            sc::MoveRow& r = rows.row[n++];
            r.kind = kind;
            r.src = reinterpret_cast<const uint8_t*>(srcs[kv]);
            r.dst = static_cast<uint8_t*>(codes[kv]);
            r.dst2 = reinterpret_cast<uint8_t*>(scales[kv]);
            r.table = a.table;
            r.pos0 = pos0;
            r.ld = std::numeric_limits<int64_t>::max();   // the reference bounds no page: the caller sized the pools
            r.aux = int32_t(T);
            r.n = units;
        }
    }
    const uint64_t per_tile = kind == sc::kKv32 ? sc::kTileChunks : sc::kQuantUnitsPerTile;
    const uint64_t tiles = (rows.row[0].n + per_tile - 1) / per_tile;
    sc::MoveGeo geo{};
    geo.row_chunks = sc::make_fastdiv(uint32_t(D * 2 / 16));
    geo.heads = sc::make_fastdiv(uint32_t(H));
    geo.page_size = sc::make_fastdiv(uint32_t(page_size));
    SC_HIP(sc::launch_append(rows, n, tiles, geo, kind, static_cast<hipStream_t>(stream)), "kv_append launch");
    return ok();
}

}  // namespace

int sc_kv_append_async(const float* K, const float* V, int64_t T, int64_t pos0, const int32_t* page_table,
                       int64_t page_size, uint16_t* k_pool, uint16_t* v_pool, int8_t* k_q, int8_t* v_q,
                       uint16_t* k_scale, uint16_t* v_scale, void* stream, const sc_kv_pools* host,
                       const sc_kv_pools* stage) {
    return guarded([&] {
        if (T <= 0) return ok();   // the reference launches nothing (src/prefill/kernels.cu:617)
        // f16 when the f16 pools are given, else int8 codes + scales (kernels.cu:576-582)
        const bool f16 = k_pool != nullptr;
        AppendDest dests[3];
        int n = 0;
        dests[n++] = f16 ? AppendDest{k_pool, v_pool, nullptr, nullptr, page_table}
                         : AppendDest{k_q, v_q, k_scale, v_scale, page_table};
        for (const sc_kv_pools* p : {host, stage}) {
            if (!p || !(f16 ? static_cast<const void*>(p->k_pool) : static_cast<const void*>(p->k_q))) continue;
            dests[n++] = f16 ? AppendDest{p->k_pool, p->v_pool, nullptr, nullptr, nullptr, p == host}
                             : AppendDest{p->k_q, p->v_q, p->k_scale, p->v_scale, nullptr, p == host};
        }
        return append_launch(f16 ? sc::kKv32 : sc::kKvQ8, K, V, T, pos0, 2, 256, page_size, dests, n, stream);
    });
}

int sc_kv_append_q4_async(uint8_t* k_q4, uint8_t* v_q4, const int32_t* page_table, int64_t pos0, int64_t T,
                          const float* K, const float* V, int64_t n_head_kv, int64_t head_dim, int64_t page_size,
                          void* stream, const sc_kv_pools* host, const sc_kv_pools* stage) {
    return guarded([&] {
        if (T <= 0) return ok();   // src/kernels/cuda/kv_q4.cu:207
        if (head_dim != sc::kQuantDim)
            return fail(SC_EINVAL, "sc_handoff: kv_append_q4: head_dim must be 256 (the Hadamard transform's size)");
        if (n_head_kv < 1 || n_head_kv > 4096) return fail(SC_EINVAL, "sc_handoff: kv_append_q4: invalid n_head_kv");
        AppendDest dests[3];
        int n = 0;
        dests[n++] = AppendDest{k_q4, v_q4, nullptr, nullptr, page_table};
        for (const sc_kv_pools* p : {host, stage})
            if (p && p->k_q4) dests[n++] = AppendDest{p->k_q4, p->v_q4, nullptr, nullptr, nullptr, p == host};
        return append_launch(sc::kKvQ4, K, V, T, pos0, n_head_kv, head_dim, page_size, dests, n, stream);
    });
}

// ---- batched ragged resume + append ----------------------------------------------------------------------------

static uint64_t image_bytes_of(const Geo& o, int64_t tokens) {
    uint64_t total = 0;
    image_blobs(o, tokens, total);
    return total;
}

int sc_batch_staging_layout(const sc_geometry* g, const int64_t* lens, int32_t n_slots, uint64_t* offsets,
                            uint64_t* total_bytes) {
    return guarded([&] {
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        if (n_slots < 1 || n_slots > sc::kMaxBatchSlots || !lens) return fail(SC_EINVAL, "sc_handoff: invalid slot count");
        uint64_t at = 0;
        for (int32_t i = 0; i < n_slots; ++i) {
            if (lens[i] < 0 || lens[i] > (int64_t(1) << 30)) return snapshot_fail("invalid K/V extent");
            if (offsets) offsets[i] = at;
            at += round_up(image_bytes_of(o, lens[i]), 256);
        }
        if (total_bytes) *total_bytes = at;
        return ok();
    });
}

int sc_plan_resume_append(const sc_geometry* g, const sc_batch_desc* d, sc_plan** out) {
    return guarded([&] {
        if (!out || !d) return fail(SC_EINVAL, "sc_handoff: missing plan output or descriptor");
        Geo o;
        std::string why;
        if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
        if (d->n_slots < 1 || d->n_slots > sc::kMaxBatchSlots) return fail(SC_ERANGE, "sc_handoff: 1 to 64 slots per batch");
        if (!d->lens || !d->staging || d->max_tokens < 0 || d->max_tokens > (int64_t(1) << 30) || d->chunk_tokens < 0 ||
            d->chunk_tokens > (int64_t(1) << 30))
            return snapshot_fail("invalid K/V extent");
        if (d->arena_pages < 0 || d->table_pages < (d->max_tokens + d->chunk_tokens + o.ps - 1) / o.ps)
            return snapshot_fail("invalid K/V extent");
        // arena entries carry the logical page in 25 bits and the arena page in 31
        if (d->table_pages >= (int64_t(1) << sc::kBatchSlotShift) || d->arena_pages >= (int64_t(1) << 31))
            return fail(SC_ERANGE, "sc_handoff: page tables beyond 2^25 pages or an arena beyond 2^31 pages");
        // the launch indexes a slot's chunks with 32-bit integers
        if (uint64_t(d->max_tokens / o.ps) * (o.page_bytes / 16) >= kMaxRowChunks ||
            uint64_t(d->chunk_tokens) * uint64_t(o.H) * (o.row_bytes / 16) >= kMaxRowChunks ||
            uint64_t(o.n_gdn) * o.gdn_row_bytes / 16 >= kMaxRowChunks)
            return fail(SC_ERANGE, "sc_handoff: a slot beyond 2^31 chunks");
        if (o.n_gdn > 0 && (!d->gdn || o.gdn_row_bytes % 16)) return snapshot_fail("missing running-state buffer");
        if (o.n_qsa > 0 && (!d->arena_k || !d->arena_v || !d->tables || (d->chunk_tokens && (!d->chunk_k || !d->chunk_v))))
            return snapshot_fail("missing target state buffer");
        if (!aligned16(d->staging)) return fail(SC_EINVAL, "sc_handoff: staging must be 16-byte aligned");
        // the pointer block: arenas, chunk sources, tables, GDN rows
        const size_t n_chunk = size_t(d->n_slots) * size_t(o.n_qsa) * 2;
        std::vector<uint64_t> ptrs;
        ptrs.reserve(size_t(o.n_qsa) * 2 + n_chunk + size_t(d->n_slots) * 2);
        for (int64_t j = 0; j < o.n_qsa; ++j) {
            if (!d->arena_k[j] || !d->arena_v[j] || !aligned16(d->arena_k[j]) || !aligned16(d->arena_v[j]))
                return snapshot_fail("missing target state buffer");
            ptrs.push_back(reinterpret_cast<uint64_t>(d->arena_k[j]));
            ptrs.push_back(reinterpret_cast<uint64_t>(d->arena_v[j]));
        }
        for (int32_t i = 0; i < d->n_slots; ++i)
            for (int64_t j = 0; j < o.n_qsa; ++j) {
                const void* k = d->chunk_tokens ? d->chunk_k[size_t(i) * size_t(o.n_qsa) + size_t(j)] : nullptr;
                const void* v = d->chunk_tokens ? d->chunk_v[size_t(i) * size_t(o.n_qsa) + size_t(j)] : nullptr;
                if (d->chunk_tokens && (!k || !v || !aligned16(k) || !aligned16(v)))
                    return snapshot_fail("missing prefill K/V");
                ptrs.push_back(reinterpret_cast<uint64_t>(k));
                ptrs.push_back(reinterpret_cast<uint64_t>(v));
            }
        for (int32_t i = 0; i < d->n_slots; ++i) {
            if (o.n_qsa > 0 && !d->tables[i]) return snapshot_fail("missing page table");
            ptrs.push_back(reinterpret_cast<uint64_t>(o.n_qsa > 0 ? d->tables[i] : nullptr));
        }
        for (int32_t i = 0; i < d->n_slots; ++i) {
            float* rows = o.n_gdn > 0 ? d->gdn[i] : nullptr;
            if (o.n_gdn > 0 && (!rows || !aligned16(rows))) return snapshot_fail("missing running-state buffer");
            ptrs.push_back(reinterpret_cast<uint64_t>(rows));
        }
        sc::BatchArgs a{};
        a.lens = d->lens;
        a.lens_out = d->lens_out;
        a.staging = static_cast<const uint8_t*>(d->staging);
        a.staging_bytes = d->staging_bytes;
        a.n_slots = d->n_slots;
        a.n_qsa = int32_t(o.n_qsa);
        a.max_tokens = d->max_tokens;
        a.chunk_tokens = d->chunk_tokens;
        a.arena_pages = d->arena_pages;
        a.table_pages = d->table_pages;
        a.gdn_bytes = uint64_t(o.n_gdn) * o.gdn_row_bytes;
        a.geo = move_geo(o);
        // The arena pages a launch can write: at most every arena page, at most every slot at max_tokens.  The K/V
        // tiles of a blob cover that many pages in ascending arena order; pages past the ones the lengths reach are
        // -1 entries and move nothing.
        const uint64_t page_chunks = o.page_bytes / 16;
        const uint64_t slot_pages = uint64_t((d->max_tokens + d->chunk_tokens + o.ps - 1) / o.ps);
        const uint64_t pages = o.n_qsa > 0 ? std::min<uint64_t>(uint64_t(d->arena_pages), slot_pages * uint64_t(d->n_slots))
                                           : 0;
        const uint64_t kv_tiles = (pages * page_chunks + sc::kBatchTileChunks - 1) / sc::kBatchTileChunks;
        if (kv_tiles * sc::kBatchTileChunks >= kMaxRowChunks)
            return fail(SC_ERANGE, "sc_handoff: an arena beyond 2^31 chunks");
        const uint64_t order_len = (kv_tiles * sc::kBatchTileChunks + page_chunks - 1) / page_chunks;
        a.kv_tiles = uint32_t(kv_tiles);
        a.kv_tiles_div = sc::make_fastdiv(uint32_t(std::max<uint64_t>(kv_tiles, 1)));
        a.gdn_tiles = uint32_t((a.gdn_bytes / 16 + sc::kTileChunks - 1) / sc::kTileChunks);
        a.gdn_tiles_div = sc::make_fastdiv(std::max<uint32_t>(a.gdn_tiles, 1));
        const uint64_t tiles = 2 * uint64_t(o.n_qsa) * kv_tiles + uint64_t(d->n_slots) * a.gdn_tiles;
        sc_plan* p = new (std::nothrow) sc_plan();
        if (!p) return fail(SC_ENOMEM, "sc_handoff: plan allocation failed");
        p->batch = true;
        p->grid = p->default_grid = int64_t(std::min<uint64_t>(std::max<uint64_t>(tiles, 1), kMaxGridBatch));
        p->payload = 0;   // depends on the device-resident lengths
        // workspace: [slots][ok][arena order group][inv][order pairs][counts]
        auto up = [](uint64_t x) { return (x + 255) / 256 * 256; };
        const uint32_t n_blocks = uint32_t((uint64_t(d->arena_pages) + sc::kOrderBlockPages - 1) / sc::kOrderBlockPages);
        const uint64_t at_ok = up(sizeof(sc::BatchSlot) * sc::kMaxBatchSlots), at_group = at_ok + 256,
                       at_inv = at_group + up(sizeof(sc::OrderGroup)), at_order = at_inv + up(uint64_t(d->arena_pages) * 4),
                       at_counts = at_order + up(2 * order_len * 4), ws_bytes = at_counts + up(uint64_t(n_blocks) * 4);
        auto release = [&] {
            if (p->batch_ptrs_dev) (void) hipFree(p->batch_ptrs_dev);
            if (p->order_ws) (void) hipFree(p->order_ws);
            delete p;
        };
        hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->batch_ptrs_dev), ptrs.size() * sizeof(uint64_t));
        if (e == hipSuccess) e = hipMalloc(&p->order_ws, ws_bytes);
        if (e != hipSuccess) {
            release();
            return fail(SC_ENOMEM, std::string("sc_handoff: batch allocation: ") + hipGetErrorString(e));
        }
        uint8_t* ws = static_cast<uint8_t*>(p->order_ws);
        a.slots = reinterpret_cast<sc::BatchSlot*>(ws);
        a.ok = reinterpret_cast<uint32_t*>(ws + at_ok);
        a.inv = reinterpret_cast<int32_t*>(ws + at_inv);
        a.order = reinterpret_cast<const int32_t*>(ws + at_order);
        sc::OrderGroup arena{};
        arena.inv = a.inv;
        arena.order = reinterpret_cast<int32_t*>(ws + at_order);
        arena.counts = reinterpret_cast<uint32_t*>(ws + at_counts);
        arena.lp_hi = int64_t(pages);
        arena.ld = d->arena_pages;
        arena.order_len = order_len;
        arena.n_blocks = n_blocks;
        arena.pairs = 1;
        p->order_groups = reinterpret_cast<const sc::OrderGroup*>(ws + at_group);
        p->order_max_blocks = n_blocks;
        e = hipMemcpy(p->batch_ptrs_dev, ptrs.data(), ptrs.size() * sizeof(uint64_t), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(ws + at_group, &arena, sizeof arena, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemset(ws, 0, at_group);   // slots and ok: nothing valid before the first launch
        if (e == hipSuccess && d->arena_pages) e = hipMemset(a.inv, 0xFF, uint64_t(d->arena_pages) * 4);
        if (e != hipSuccess) {
            release();
            return hip_fail(e, "batch workspace");
        }
        a.ptrs = p->batch_ptrs_dev;
        p->batch_args = a;
        *out = p;
        return ok();
    });
}

// ---- park / resume --------------------------------------------------------------------------------------------

static int dma_image(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens, uint8_t* host,
                     uint64_t image_bytes, bool park, void* stream, void* done) {
    Geo o;
    std::string why;
    if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
    if (tokens < 0 || tokens > (int64_t(1) << 30)) return snapshot_fail("invalid K/V extent");
    const int64_t cells = cells_of(o, tokens);
    int rc = check_slot(o, slot, tokens, true);
    if (rc) return rc;
    const bool identity = slot_identity(slot, o.n_qsa);
    if (identity && cells / o.ps > slot->n_pages) return snapshot_fail("invalid K/V extent");
    uint64_t total = 0;
    const auto blobs = image_blobs(o, tokens, total);
    if (!host || image_bytes < total) return snapshot_fail("invalid K/V payload size");
    // a paged slot's pages are moved by a kernel that reads or writes the image itself
    uint8_t* host_dev = nullptr;
    if (!identity && o.n_qsa > 0 && total > 0) {
        host_dev = mapped_host_range(host, total);
        if (!host_dev) return snapshot_fail("a paged slot's host image must be pinned memory mapped for the device");
    }
    if (park) {
        // the gaps between blobs are never copied; clear them so the image is deterministic
        uint64_t at = 0;
        for (const Blob& b : blobs) {
            if (b.offset > at) std::memset(host + at, 0, b.offset - at);
            at = b.offset + b.bytes;
        }
        if (total > at) std::memset(host + at, 0, total - at);
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    size_t b = 0;
    // A paged slot: its pages go through the tables between the pools and the pinned image, moved by a kernel that
    // reads or writes the host memory itself (measured at 95-99% of a plain DMA of the same bytes), kPagedLayers
    // layers per launch.  The K/V blobs of an image are equal and 64-byte aligned, so blob b sits at b * stride.
    if (!identity && o.n_qsa > 0) {
        const uint64_t stride = blobs.size() > 1 ? blobs[1].offset : round_up(blobs[0].bytes, kBlobAlign);
        const uint64_t chunks = blobs[0].bytes / 16;
        const uint64_t tiles = (chunks + sc::kTileChunks - 1) / sc::kTileChunks;
        if (chunks >= kMaxRowChunks || tiles * 2 * sc::kPagedLayers >= (uint64_t(1) << 32))
            return fail(SC_ERANGE, "sc_handoff: a K/V blob beyond 2^31 chunks");
        for (int64_t j0 = 0; j0 < o.n_qsa; j0 += sc::kPagedLayers) {
            const int64_t n = std::min<int64_t>(sc::kPagedLayers, o.n_qsa - j0);
            sc::PagedImage a{};
            for (int64_t j = 0; j < n; ++j) {
                a.pool[2 * j] = reinterpret_cast<uint8_t*>(slot->k_pool[j0 + j]);
                a.pool[2 * j + 1] = reinterpret_cast<uint8_t*>(slot->v_pool[j0 + j]);
                a.table[j] = slot->page_table ? slot->page_table[j0 + j] : nullptr;
            }
            a.image = host_dev + uint64_t(2 * j0) * stride;
            a.blob_stride = stride;
            a.blob_chunks = chunks;
            a.pool_pages = slot->n_pages;
            a.n_blobs = uint32_t(2 * n);
            a.park = park ? 1u : 0u;
            a.tiles_per_blob = uint32_t(tiles);
            a.tiles_div = sc::make_fastdiv(uint32_t(std::max<uint64_t>(tiles, 1)));
            const hipError_t e = sc::launch_paged_image(a, move_geo(o), s);
            if (e != hipSuccess) return hip_fail(e, park ? "paged park" : "paged resume");
        }
        b = 2 * size_t(o.n_qsa);
    }
    for (int64_t j = identity ? 0 : o.n_qsa; j < o.n_qsa; ++j, b += 2) {
        uint16_t* pools[2] = {slot->k_pool[j], slot->v_pool[j]};
        for (int a = 0; a < 2; ++a) {
            const Blob& blob = blobs[b + a];
            if (!blob.bytes) continue;
            const hipError_t e = park ? hipMemcpyAsync(host + blob.offset, pools[a], blob.bytes, hipMemcpyDeviceToHost, s)
                                      : hipMemcpyAsync(pools[a], host + blob.offset, blob.bytes, hipMemcpyHostToDevice, s);
            if (e != hipSuccess) return hip_fail(e, park ? "park copy" : "resume copy");
        }
    }
    if (o.n_gdn > 0) {
        const Blob& blob = blobs[b];
        const hipError_t e = park ? hipMemcpyAsync(host + blob.offset, slot->gdn_state, blob.bytes, hipMemcpyDeviceToHost, s)
                                  : hipMemcpyAsync(slot->gdn_state, host + blob.offset, blob.bytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_fail(e, park ? "park copy" : "resume copy");
    }
    if (done) {
        const hipError_t e = hipEventRecord(static_cast<hipEvent_t>(done), s);
        if (e != hipSuccess) return hip_fail(e, "event record");
    }
    return ok();
}

// Park / resume of an sc_slot_layers slot: one copy per blob between its buffers' prefixes and the pinned image.
static int dma_layers(const sc_geometry* g, const sc_slot_layers* slot, int64_t tokens, uint8_t* host,
                      uint64_t image_bytes, bool park, void* stream, void* done) {
    Geo o;
    std::string why;
    if (!geometry(g, o, why)) return snapshot_fail(why.c_str());
    uint64_t b[SC_N_BUF];
    int rc = check_layers(o, g, slot, tokens, b);
    if (rc) return rc;
    std::vector<uint64_t> off;
    const uint64_t total = layers_layout(o, b, off);
    if (!host || image_bytes < total) return snapshot_fail("invalid K/V payload size");
    struct Item { uint8_t* dev; uint64_t at, n; };
    std::vector<Item> items;
    for (int64_t j = 0; j < o.n_qsa; ++j)
        for (int k = 0; k < SC_N_BUF; ++k)
            if (b[k]) items.push_back({static_cast<uint8_t*>(slot->buf[k][j]), off[size_t(j) * SC_N_BUF + k], b[k]});
    if (o.n_gdn > 0)
        items.push_back({reinterpret_cast<uint8_t*>(slot->gdn_state), off.back(), uint64_t(o.n_gdn) * o.gdn_row_bytes});
    if (park) {   // the gaps are never copied; clear them so the image is deterministic
        uint64_t at = 0;
        for (const Item& it : items) {
            if (it.at > at) std::memset(host + at, 0, it.at - at);
            at = it.at + it.n;
        }
        if (total > at) std::memset(host + at, 0, total - at);
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (const Item& it : items) {
        const hipError_t e = park ? hipMemcpyAsync(host + it.at, it.dev, it.n, hipMemcpyDeviceToHost, s)
                                  : hipMemcpyAsync(it.dev, host + it.at, it.n, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_fail(e, park ? "park copy" : "resume copy");
    }
    if (done) {
        const hipError_t e = hipEventRecord(static_cast<hipEvent_t>(done), s);
        if (e != hipSuccess) return hip_fail(e, "event record");
    }
    return ok();
}

int sc_park_layers_async(const sc_geometry* g, const sc_slot_layers* slot, int64_t tokens, void* host_image,
                         uint64_t image_bytes, void* stream, void* done) {
    return guarded([&] { return dma_layers(g, slot, tokens, static_cast<uint8_t*>(host_image), image_bytes, true, stream, done); });
}

int sc_resume_layers_async(const sc_geometry* g, const void* host_image, uint64_t image_bytes, int64_t tokens,
                           const sc_slot_layers* slot, void* stream, void* done) {
    return guarded([&] {
        return dma_layers(g, slot, tokens, const_cast<uint8_t*>(static_cast<const uint8_t*>(host_image)), image_bytes,
                          false, stream, done);
    });
}

int sc_park_async(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens, void* host_image,
                  uint64_t image_bytes, void* stream, void* done) {
    return guarded([&] { return dma_image(g, slot, tokens, static_cast<uint8_t*>(host_image), image_bytes, true, stream, done); });
}

int sc_resume_async(const sc_geometry* g, const void* host_image, uint64_t image_bytes, int64_t tokens,
                    const sc_decode_slot* slot, void* stream, void* done) {
    return guarded([&] {
        return dma_image(g, slot, tokens, const_cast<uint8_t*>(static_cast<const uint8_t*>(host_image)), image_bytes,
                         false, stream, done);
    });
}

// ---- block movers ----------------------------------------------------------------------------------------------

static int check_runs(const sc_kv_runs* r) {
    if (!r || r->n < 1 || r->n > 4) return fail(SC_EINVAL, "sc_handoff: invalid block runs");
    for (int a = 0; a < r->n; ++a)
        if (!r->src[a] || !r->dst[a] || !r->len[a]) return fail(SC_EINVAL, "sc_handoff: invalid block runs");
    return SC_OK;
}

int sc_kv_ring_restore(const sc_kv_runs* runs, int64_t b0, int64_t b1, int64_t n_slots, void* stream) {
    if (int rc = check_runs(runs)) return rc;
    if (b0 < 0 || b1 < b0 || n_slots < 1) return fail(SC_EINVAL, "sc_handoff: invalid ring range");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int64_t b = b0; b < b1;) {
        const int64_t slot = b % n_slots, run = std::min<int64_t>(b1 - b, n_slots - slot);   // up to the ring's end
        for (int a = 0; a < runs->n; ++a) {
            const uint64_t len = runs->len[a];
            const hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(runs->dst[a]) + uint64_t(slot) * len,
                                                static_cast<const uint8_t*>(runs->src[a]) + uint64_t(b) * len,
                                                uint64_t(run) * len, hipMemcpyDefault, s);
            if (e != hipSuccess) return hip_fail(e, "ring restore");
        }
        b += run;
    }
    return ok();
}

int sc_kv_stage_from_host(const sc_kv_runs* runs, int64_t n_blocks, void* stream) {
    if (n_blocks <= 0) return ok();
    if (int rc = check_runs(runs)) return rc;
    for (int a = 0; a < runs->n; ++a) {
        const hipError_t e = hipMemcpyAsync(runs->dst[a], runs->src[a], uint64_t(n_blocks) * runs->len[a],
                                            hipMemcpyDefault, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "stage");
    }
    return ok();
}

int sc_kv_ring_table(int32_t* page_table, int64_t n_blocks, int64_t n_slots, void* stream) {
    if (n_blocks < 0 || n_slots < 1 || (n_blocks && !page_table)) return fail(SC_EINVAL, "sc_handoff: invalid ring table");
    SC_HIP(sc::launch_ring_table(page_table, n_blocks, n_slots, static_cast<hipStream_t>(stream)), "ring table");
    return ok();
}

int sc_kv_stream_reset(int32_t* page_table, int64_t n_blocks, int32_t* slot_block, int32_t* slot_stamp,
                       int32_t* slot_ref, int64_t n_slots, int32_t* ctl, void* stream) {
    if (n_blocks < 0 || n_slots < 0 || !page_table || !slot_block || !slot_stamp || !slot_ref || !ctl)
        return fail(SC_EINVAL, "sc_handoff: invalid streaming map");
    SC_HIP(sc::launch_stream_reset(page_table, n_blocks, slot_block, slot_stamp, slot_ref, n_slots, ctl,
                                   static_cast<hipStream_t>(stream)), "stream reset");
    return ok();
}

uint64_t sc_kv_block_bytes(int64_t n_head_kv, int64_t head_dim, int64_t page_size, int32_t format) {
    const uint64_t rows = uint64_t(n_head_kv) * uint64_t(page_size);
    if (format == 2) return rows * uint64_t(head_dim / 32) * 18 * 2;                       // q4_0: 18 B per 32
    if (format == 1) return rows * uint64_t(head_dim) * 2 + rows * uint64_t(head_dim / 64) * 2 * 2;   // int8 + scales
    return rows * uint64_t(head_dim) * 2 * 2;                                                 // f16 K and V
}

// ---- FNV-1a 64 of device bytes -----------------------------------------------------------------------------------

uint64_t sc_fnv1a64_workspace_bytes(uint64_t bytes) { return sc::fnv_workspace(bytes).bytes; }

// The checks every asynchronous form makes before it enqueues anything.
static int check_fnv_args(const void* data, uint64_t bytes, const void* out, const uint32_t* fault, bool fault_required,
                          const void* workspace, uint64_t workspace_bytes) {
    if (!out || (bytes && !data)) return fail(SC_EINVAL, "sc_handoff: missing hash input or output");
    if (fault_required && !fault) return fail(SC_EINVAL, "sc_handoff: missing hash fault word");
    if (reinterpret_cast<uintptr_t>(fault) & 3u) return fail(SC_EINVAL, "sc_handoff: the hash fault word must be 4-byte aligned");
    if (!workspace || workspace_bytes < sc::fnv_workspace(bytes).bytes)
        return fail(SC_EINVAL, "sc_handoff: hash workspace smaller than sc_fnv1a64_workspace_bytes()");
    if (reinterpret_cast<uintptr_t>(workspace) & 15u) return fail(SC_EINVAL, "sc_handoff: hash workspace must be 16-byte aligned");
    if (bytes > (uint64_t(1) << 46)) return fail(SC_ERANGE, "sc_handoff: hash input beyond 2^46 bytes");
    return SC_OK;
}

int sc_fnv1a64_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, uint32_t* fault, void* workspace,
                     uint64_t workspace_bytes, void* stream) {
    if (const int rc = check_fnv_args(data, bytes, out, fault, true, workspace, workspace_bytes)) return rc;
    SC_HIP(sc::launch_fnv1a64(data, bytes, seed, nullptr, out, fault, workspace, static_cast<hipStream_t>(stream)),
           "hash launch");
    return ok();
}

int sc_fnv1a64_check_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t expected, uint64_t* out,
                           uint32_t* verdict, uint32_t* fault, void* workspace, uint64_t workspace_bytes, void* stream) {
    if (!verdict) return fail(SC_EINVAL, "sc_handoff: missing hash verdict");
    if (reinterpret_cast<uintptr_t>(verdict) & 3u) return fail(SC_EINVAL, "sc_handoff: the verdict must be 4-byte aligned");
    if (const int rc = check_fnv_args(data, bytes, out, fault, false, workspace, workspace_bytes)) return rc;
    SC_HIP(sc::launch_fnv1a64(data, bytes, seed, nullptr, out, fault, workspace, static_cast<hipStream_t>(stream),
                              expected, verdict),
           "hash launch");
    return ok();
}

uint64_t sc_fnv1a64_carry_bytes(uint64_t bytes) { return sc::fnv_carry_count(bytes); }

int sc_fnv1a64_carry_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, uint32_t* fault,
                           uint8_t* carry_out, void* workspace, uint64_t workspace_bytes, void* stream) {
    if (const int rc = check_fnv_args(data, bytes, out, fault, true, workspace, workspace_bytes)) return rc;
    if (!carry_out && sc::fnv_carry_count(bytes)) return fail(SC_EINVAL, "sc_handoff: missing carry output");
    sc::FnvCarries c;
    c.out = carry_out;
    SC_HIP(sc::launch_fnv1a64(data, bytes, seed, nullptr, out, fault, workspace, static_cast<hipStream_t>(stream), 0,
                              nullptr, c),
           "hash launch");
    return ok();
}

int sc_fnv1a64_check_carried_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t expected,
                                   const uint8_t* carry, uint64_t* out, uint32_t* verdict, uint32_t* fault,
                                   void* workspace, uint64_t workspace_bytes, void* stream) {
    if (!verdict) return fail(SC_EINVAL, "sc_handoff: missing hash verdict");
    if (reinterpret_cast<uintptr_t>(verdict) & 3u) return fail(SC_EINVAL, "sc_handoff: the verdict must be 4-byte aligned");
    if (const int rc = check_fnv_args(data, bytes, out, fault, false, workspace, workspace_bytes)) return rc;
    if (!carry && sc::fnv_carry_count(bytes)) return fail(SC_EINVAL, "sc_handoff: missing carries");
    sc::FnvCarries c;
    c.in = carry;
    SC_HIP(sc::launch_fnv1a64(data, bytes, seed, nullptr, out, fault, workspace, static_cast<hipStream_t>(stream),
                              expected, verdict, c),
           "hash launch");
    return ok();
}

int sc_fnv1a64_chain_async(const void* data, uint64_t bytes, uint64_t* state, uint32_t* fault, void* workspace,
                           uint64_t workspace_bytes, void* stream) {
    if (reinterpret_cast<uintptr_t>(state) & 7u) return fail(SC_EINVAL, "sc_handoff: hash state must be 8-byte aligned");
    if (const int rc = check_fnv_args(data, bytes, state, fault, true, workspace, workspace_bytes)) return rc;
    SC_HIP(sc::launch_fnv1a64(data, bytes, 0, state, state, fault, workspace, static_cast<hipStream_t>(stream)),
           "hash launch");
    return ok();
}

int sc_fnv1a64_device(const void* data, uint64_t bytes, uint64_t seed, uint64_t* hash) {
    if (!hash || (bytes && !data)) return fail(SC_EINVAL, "sc_handoff: missing hash input or output");
    if (bytes > (uint64_t(1) << 46)) return fail(SC_ERANGE, "sc_handoff: hash input beyond 2^46 bytes");
    const uint64_t ws_bytes = (sc::fnv_workspace(bytes).bytes + 255) / 256 * 256;
    void* ws = nullptr;
    hipError_t e = hipMalloc(&ws, ws_bytes + 256);
    if (e != hipSuccess) return fail(SC_ENOMEM, std::string("sc_handoff: hash workspace: ") + hipGetErrorString(e));
    // the result and the fault word after the workspace, read back together
    uint64_t* out = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(ws) + ws_bytes);
    uint32_t* fault = reinterpret_cast<uint32_t*>(out + 1);
    uint64_t back[2] = {0, 0};
    e = sc::launch_fnv1a64(data, bytes, seed, nullptr, out, fault, ws, nullptr);
    if (e == hipSuccess) e = hipMemcpy(back, out, sizeof back, hipMemcpyDeviceToHost);
    const hipError_t f = hipFree(ws);
    if (e != hipSuccess) return hip_fail(e, "hash");
    if (f != hipSuccess) return hip_fail(f, "hash workspace free");
    if (uint32_t(back[1]))
        return fail(SC_ETIMEOUT, "sc_handoff: a look-back wait of the hash kernel ran out; the hash is not valid");
    *hash = back[0];
    return ok();
}

// ---- plumbing --------------------------------------------------------------------------------------------------

int sc_device_count(int* count) {
    if (!count) return fail(SC_EINVAL, "sc_handoff: missing output");
    *count = 0;
    SC_HIP(hipGetDeviceCount(count), "device count");
    return ok();
}
int sc_get_device(int* device) {
    if (!device) return fail(SC_EINVAL, "sc_handoff: missing output");
    SC_HIP(hipGetDevice(device), "get device");
    return ok();
}
int sc_set_device(int device) {
    SC_HIP(hipSetDevice(device), "set device");
    return ok();
}
int sc_device_alloc(void** ptr, uint64_t bytes) {
    if (!ptr) return fail(SC_EINVAL, "sc_handoff: missing pointer");
    const hipError_t e = hipMalloc(ptr, bytes ? bytes : 16);
    return e == hipSuccess ? ok() : fail(SC_ENOMEM, std::string("sc_handoff: device allocation: ") + hipGetErrorString(e));
}
int sc_device_free(void* ptr) {
    SC_HIP(hipFree(ptr), "device free");
    return ok();
}
int sc_host_alloc(void** ptr, uint64_t bytes) {
    if (!ptr) return fail(SC_EINVAL, "sc_handoff: missing pointer");
    const hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 16, hipHostMallocDefault);
    return e == hipSuccess ? ok() : fail(SC_ENOMEM, std::string("sc_handoff: pinned allocation: ") + hipGetErrorString(e));
}
int sc_host_range_mapped(const void* host, uint64_t bytes, int32_t* mapped) {
    if (!mapped) return fail(SC_EINVAL, "sc_handoff: missing output");
    *mapped = mapped_host_range(host, bytes) ? 1 : 0;
    return ok();
}

int sc_host_free(void* ptr) {
    SC_HIP(hipHostFree(ptr), "pinned free");
    return ok();
}
int sc_copy_async(void* dst, const void* src, uint64_t bytes, void* stream) {
    if (!bytes) return ok();
    if (!dst || !src) return fail(SC_EINVAL, "sc_handoff: missing copy buffer");
    SC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, static_cast<hipStream_t>(stream)), "copy");
    return ok();
}
int sc_fill_bytes_async(void* dst, uint8_t value, uint64_t bytes, void* stream) {
    if (!bytes) return ok();
    if (!dst) return fail(SC_EINVAL, "sc_handoff: missing fill buffer");
    SC_HIP(sc::launch_fill_bytes(dst, value, bytes, static_cast<hipStream_t>(stream)), "fill");
    return ok();
}
int sc_stream_create(void** stream) {
    if (!stream) return fail(SC_EINVAL, "sc_handoff: missing stream");
    hipStream_t s = nullptr;
    SC_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream create");
    *stream = s;
    return ok();
}
int sc_stream_destroy(void* stream) {
    SC_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)), "stream destroy");
    return ok();
}
int sc_stream_sync(void* stream) {
    SC_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "stream sync");
    return ok();
}
int sc_device_sync(void) {
    SC_HIP(hipDeviceSynchronize(), "device sync");
    return ok();
}
int sc_event_create(void** event) {
    if (!event) return fail(SC_EINVAL, "sc_handoff: missing event");
    hipEvent_t ev = nullptr;
    SC_HIP(hipEventCreate(&ev), "event create");
    *event = ev;
    return ok();
}
int sc_event_destroy(void* event) {
    SC_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)), "event destroy");
    return ok();
}
int sc_event_record(void* event, void* stream) {
    SC_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)), "event record");
    return ok();
}
int sc_event_sync(void* event) {
    SC_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)), "event sync");
    return ok();
}
int sc_event_elapsed_ms(void* start, void* end, float* ms) {
    if (!ms) return fail(SC_EINVAL, "sc_handoff: missing output");
    SC_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)), "event elapsed");
    return ok();
}
int sc_stream_wait_event(void* stream, void* event) {
    SC_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0), "stream wait");
    return ok();
}

int sc_copy_device_async(void* dst, const void* src, uint64_t bytes, void* stream) {
    if (!bytes) return ok();
    if (!dst || !src) return fail(SC_EINVAL, "sc_handoff: missing copy buffer");
    SC_HIP(sc::launch_copy_bytes(dst, src, bytes, static_cast<hipStream_t>(stream)), "device copy");
    return ok();
}

// ---- same-GPU hand-off between processes ------------------------------------------------------------------------

struct sc_ipc_export {
    std::vector<void*> ptr;
    std::vector<uint64_t> bytes;
    std::vector<hipIpcMemHandle_t> handle;
};
struct sc_ipc_import {
    std::vector<void*> ptr;
    std::vector<uint64_t> bytes;
};

static void ipc_export_free(sc_ipc_export* ex) {
    for (void* p : ex->ptr) (void) hipFree(p);
    delete ex;
}

int sc_ipc_export_create(uint64_t capacity, uint64_t segment_bytes, sc_ipc_export** out) {
    if (!out) return fail(SC_EINVAL, "sc_handoff: missing output");
    *out = nullptr;
    if (!capacity || segment_bytes < 4096 || segment_bytes % 4096 || segment_bytes > SC_IPC_MAX_SEGMENT)
        return fail(SC_ERANGE, "sc_handoff: IPC segments are 4 KiB multiples of at most 1 GiB, over a nonzero capacity");
    const uint64_t n = (capacity + segment_bytes - 1) / segment_bytes;
    if (n > SC_IPC_MAX_SEGMENTS) return fail(SC_ERANGE, "sc_handoff: more than SC_IPC_MAX_SEGMENTS IPC segments");
    auto* ex = new (std::nothrow) sc_ipc_export;
    if (!ex) return fail(SC_ENOMEM, "sc_handoff: out of host memory");
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t left = capacity - i * segment_bytes;
        const uint64_t b = left < segment_bytes ? (left + 4095) & ~uint64_t(4095) : segment_bytes;
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, b);
        if (e != hipSuccess) {
            ipc_export_free(ex);
            return fail(SC_ENOMEM, std::string("sc_handoff: IPC segment allocation: ") + hipGetErrorString(e));
        }
        ex->ptr.push_back(p);
        ex->bytes.push_back(b);
        hipIpcMemHandle_t h;
        e = hipIpcGetMemHandle(&h, p);
        if (e != hipSuccess) {
            ipc_export_free(ex);
            return hip_fail(e, "IPC handle");
        }
        ex->handle.push_back(h);
    }
    *out = ex;
    return ok();
}

int32_t sc_ipc_export_count(const sc_ipc_export* ex) { return ex ? int32_t(ex->ptr.size()) : 0; }

int sc_ipc_export_segments(const sc_ipc_export* ex, sc_ipc_segment* segments, int32_t max_segments) {
    if (!ex || !segments) return fail(SC_EINVAL, "sc_handoff: missing export or output");
    if (max_segments < int32_t(ex->ptr.size())) return fail(SC_ERANGE, "sc_handoff: room for fewer segments than exported");
    static_assert(sizeof(hipIpcMemHandle_t) == SC_IPC_HANDLE_BYTES, "hipIpcMemHandle_t is 64 bytes");
    for (size_t i = 0; i < ex->ptr.size(); ++i) {
        std::memcpy(segments[i].handle, &ex->handle[i], SC_IPC_HANDLE_BYTES);
        segments[i].bytes = ex->bytes[i];
    }
    return ok();
}

/// Copy `bytes` between a contiguous buffer and a list of segments (to_segments: buffer -> segments).
static int segmented_copy(const std::vector<void*>& ptr, const std::vector<uint64_t>& seg_bytes, void* buffer,
                          uint64_t bytes, bool to_segments, hipStream_t stream) {
    uint64_t total = 0;
    for (uint64_t b : seg_bytes) total += b;
    if (bytes > total) return fail(SC_ERANGE, "sc_handoff: the payload is larger than the IPC segments");
    if (bytes && !buffer) return fail(SC_EINVAL, "sc_handoff: missing payload buffer");
    uint64_t off = 0;
    for (size_t i = 0; i < ptr.size() && off < bytes; ++i) {
        const uint64_t n = std::min(seg_bytes[i], bytes - off);
        uint8_t* b = static_cast<uint8_t*>(buffer) + off;
        const hipError_t e = to_segments ? sc::launch_copy_bytes(ptr[i], b, n, stream)
                                         : sc::launch_copy_bytes(b, ptr[i], n, stream);
        if (e != hipSuccess) return hip_fail(e, "IPC segment copy");
        off += n;
    }
    return ok();
}

int sc_ipc_export_stage(sc_ipc_export* ex, const void* device_payload, uint64_t bytes, void* stream) {
    if (!ex) return fail(SC_EINVAL, "sc_handoff: missing export");
    return segmented_copy(ex->ptr, ex->bytes, const_cast<void*>(device_payload), bytes, true,
                          static_cast<hipStream_t>(stream));
}

int sc_ipc_export_destroy(sc_ipc_export* ex) {
    if (ex) ipc_export_free(ex);
    return ok();
}

int sc_ipc_import_open(const sc_ipc_segment* segments, int32_t n_segments, sc_ipc_import** out) {
    if (!out || (n_segments && !segments)) return fail(SC_EINVAL, "sc_handoff: missing segments or output");
    *out = nullptr;
    if (n_segments < 1 || n_segments > SC_IPC_MAX_SEGMENTS)
        return fail(SC_ERANGE, "sc_handoff: 1 to SC_IPC_MAX_SEGMENTS IPC segments");
    for (int32_t i = 0; i < n_segments; ++i)
        if (segments[i].bytes == 0 || segments[i].bytes > SC_IPC_MAX_SEGMENT)
            return fail(SC_ERANGE, "sc_handoff: an IPC segment is empty or larger than SC_IPC_MAX_SEGMENT");
    auto* im = new (std::nothrow) sc_ipc_import;
    if (!im) return fail(SC_ENOMEM, "sc_handoff: out of host memory");
    for (int32_t i = 0; i < n_segments; ++i) {
        hipIpcMemHandle_t h;
        std::memcpy(&h, segments[i].handle, SC_IPC_HANDLE_BYTES);
        void* p = nullptr;
        const hipError_t e = hipIpcOpenMemHandle(&p, h, hipIpcMemLazyEnablePeerAccess);
        if (e != hipSuccess) {
            for (void* q : im->ptr) (void) hipIpcCloseMemHandle(q);
            delete im;
            return hip_fail(e, "IPC open");
        }
        im->ptr.push_back(p);
        im->bytes.push_back(segments[i].bytes);
    }
    *out = im;
    return ok();
}

// The segments' device addresses in payload order and the size every one but the last has (refused when the sizes
// are not uniform, so the list is an sc_segments).
static int segments_layout(const std::vector<void*>& ptr, const std::vector<uint64_t>& bytes, void** out, int32_t max,
                           int32_t* n, uint64_t* segment_bytes) {
    if (!n || !segment_bytes || (max && !out)) return fail(SC_EINVAL, "sc_handoff: missing layout output");
    if (max < int32_t(ptr.size())) return fail(SC_ERANGE, "sc_handoff: room for fewer segments than there are");
    for (size_t i = 0; i + 1 < bytes.size(); ++i)
        if (bytes[i] != bytes[0]) return fail(SC_EINVAL, "sc_handoff: the segments are not of one size");
    for (size_t i = 0; i < ptr.size(); ++i) out[i] = ptr[i];
    *n = int32_t(ptr.size());
    *segment_bytes = bytes.empty() ? 0 : bytes[0];
    return ok();
}

int sc_ipc_export_layout(const sc_ipc_export* ex, void** ptr, int32_t max_segments, int32_t* n, uint64_t* segment_bytes) {
    if (!ex) return fail(SC_EINVAL, "sc_handoff: missing export");
    return segments_layout(ex->ptr, ex->bytes, ptr, max_segments, n, segment_bytes);
}

int sc_ipc_import_layout(const sc_ipc_import* im, void** ptr, int32_t max_segments, int32_t* n, uint64_t* segment_bytes) {
    if (!im) return fail(SC_EINVAL, "sc_handoff: missing import");
    return segments_layout(im->ptr, im->bytes, ptr, max_segments, n, segment_bytes);
}

int sc_ipc_import_fetch(sc_ipc_import* im, void* device_dst, uint64_t bytes, void* stream) {
    if (!im) return fail(SC_EINVAL, "sc_handoff: missing import");
    return segmented_copy(im->ptr, im->bytes, device_dst, bytes, false, static_cast<hipStream_t>(stream));
}

int sc_ipc_import_close(sc_ipc_import* im) {
    if (!im) return ok();
    hipError_t first = hipSuccess;
    for (void* p : im->ptr) {
        const hipError_t e = hipIpcCloseMemHandle(p);
        if (first == hipSuccess) first = e;
    }
    delete im;
    return first == hipSuccess ? ok() : hip_fail(first, "IPC close");
}

int sc_probe_link(uint64_t bytes, int iters, double* h2d_gbps, double* d2h_gbps) {
    if (!bytes || iters < 1 || !h2d_gbps || !d2h_gbps) return fail(SC_EINVAL, "sc_handoff: invalid probe request");
    void* h = nullptr;
    void* d = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipStream_t s = nullptr;
    int rc = SC_OK;
    auto cleanup = [&] {
        if (e0) (void) hipEventDestroy(e0);
        if (e1) (void) hipEventDestroy(e1);
        if (s) (void) hipStreamDestroy(s);
        if (d) (void) hipFree(d);
        if (h) (void) hipHostFree(h);
    };
    hipError_t e = hipHostMalloc(&h, bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&d, bytes);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) { cleanup(); return hip_fail(e, "probe setup"); }
    std::memset(h, 0, bytes);   // fault the pages in before timing
    for (int dir = 0; dir < 2 && rc == SC_OK; ++dir) {
        const hipMemcpyKind kind = dir == 0 ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
        void* to = dir == 0 ? d : h;
        const void* from = dir == 0 ? h : d;
        float ms = 0.f;
        e = hipMemcpyAsync(to, from, bytes, kind, s);   // warm-up: context up, copy engine primed
        if (e == hipSuccess) e = hipEventRecord(e0, s);
        for (int i = 0; i < iters && e == hipSuccess; ++i) e = hipMemcpyAsync(to, from, bytes, kind, s);
        if (e == hipSuccess) e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e != hipSuccess) { rc = hip_fail(e, "probe copy"); break; }
        const double gbps = ms > 0.f ? double(bytes) * iters / (double(ms) * 1e-3) / 1e9 : -1.0;
        (dir == 0 ? *h2d_gbps : *d2h_gbps) = gbps;
    }
    cleanup();
    return rc == SC_OK ? ok() : rc;
}

int sc_fill_uniform_f16(uint16_t* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t stream_id,
                        void* stream) {
    if (n && !dst) return fail(SC_EINVAL, "sc_handoff: missing fill buffer");
    SC_HIP(sc::launch_fill_uniform_f16(dst, n, lo, hi, seed, stream_id, static_cast<hipStream_t>(stream)), "fill");
    return ok();
}
int sc_fill_uniform_f32(float* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t stream_id,
                        void* stream) {
    if (n && !dst) return fail(SC_EINVAL, "sc_handoff: missing fill buffer");
    SC_HIP(sc::launch_fill_uniform_f32(dst, n, lo, hi, seed, stream_id, static_cast<hipStream_t>(stream)), "fill");
    return ok();
}
int sc_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t stream_id, void* stream) {
    if (n && !dst) return fail(SC_EINVAL, "sc_handoff: missing fill buffer");
    SC_HIP(sc::launch_fill_normal_f32(dst, n, seed, stream_id, static_cast<hipStream_t>(stream)), "fill");
    return ok();
}
int sc_decode_probe(const void* kv, uint64_t n_bytes, uint32_t* sink, int64_t workgroups, void* stream) {
    if (!kv || !sink || workgroups <= 0 || workgroups > (int64_t(1) << 20) || (n_bytes % 16))
        return fail(SC_EINVAL, "sc_handoff: invalid decode probe request");
    SC_HIP(sc::launch_decode_probe(kv, n_bytes, sink, workgroups, static_cast<hipStream_t>(stream)), "decode probe");
    return ok();
}

int sc_delay_async(uint32_t microseconds, void* stream) {
    if (microseconds > 2000000u) return fail(SC_EINVAL, "sc_handoff: a delay is at most 2 s");
    int dev = 0, khz = 0;
    SC_HIP(hipGetDevice(&dev), "hipGetDevice");
    SC_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), "wall clock rate");
    if (khz <= 0) return fail(SC_EHIP, "sc_handoff: the device reports no wall clock rate");
    const uint64_t ticks = uint64_t(microseconds) * uint64_t(khz) / 1000u;
    // one sleep of 100 * 64 clocks lasts well over a microsecond, so `microseconds` sleeps outlast the request
    SC_HIP(sc::launch_delay(ticks, microseconds + 16u, static_cast<hipStream_t>(stream)), "delay");
    return ok();
}

}  // extern "C"
