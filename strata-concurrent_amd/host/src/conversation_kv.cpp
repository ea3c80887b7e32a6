// conversation_kv.cpp - one QSA layer's K/V between its pools and a ConversationKv.
//
// Semantics of the reference's per-layer functions (src/core/conversation_snapshot.cpp:12-262), restated:
//   * the extent is page-granular: cells = ceil(upto / page_size) * page_size, and each of the five buffers
//     (k, v, k_scale, v_scale, pooled) is the identity-layout prefix of its pool (:27-67);
//   * a streamed (mode 1) or ring (mode 2) layer is read from and written to its authoritative host copy (:69-78);
//   * every check runs before the first copy, with the reference's messages (:18-25, :80-103, :175-194);
//   * a save may keep the whole pages of an earlier image strictly before the first rewritten token (:145-171);
//   * a restore of a streamed layer evicts its VRAM slots and a ring layer refills its window (:205-214).
// The copies go through libsc_handoff.so on this thread's transfer stream; each public call waits once.
#include "strata/core/conversation_snapshot.hpp"
#include "strata/kernels/kv_stream.hpp"

#include "transfer.hpp"

#include <array>
#include <cstring>
#include <limits>

namespace strata::core {
namespace detail {

bool checked_add(size_t& total, size_t n) {
    if (n > std::numeric_limits<size_t>::max() - total) return false;
    total += n;
    return true;
}

bool checked_product(size_t& out, std::initializer_list<uint64_t> factors) {
    size_t value = 1;
    for (uint64_t f : factors) {
        if (f > std::numeric_limits<size_t>::max() || (f && value > std::numeric_limits<size_t>::max() / f))
            return false;
        value *= size_t(f);
    }
    out = value;
    return true;
}

}  // namespace detail

namespace {

using detail::checked_product;

constexpr int kHybridFormat = 3;   // the image format of K8V4; never a block-mover format

// The five buffers of one layer image, in the order ConversationKv declares them.
struct KvExtent {
    int format = 0;
    int64_t cells = 0, pooled_rows = 0, page_size = 0;
    std::array<size_t, 5> sizes{};   // k, v, k_scale, v_scale, pooled
};

bool fail(std::string& error, const char* what) {
    error = std::string("conversation snapshot: ") + what;
    return false;
}

bool kv_extent(const QsaState& st, const ModelGeometry& g, int64_t upto, bool index, KvExtent& e,
               std::string& error) {
    const auto gran = strata::kernels::qsa_granules();
    if (upto < 0 || upto > st.max_cells || upto > std::numeric_limits<int64_t>::max() - (gran.page_size - 1))
        return fail(error, "invalid K/V extent");
    if (st.kv_hybrid && (st.kv_mode != 0 || st.kv_q4 || st.kv_int8))
        return fail(error, "hybrid K8V4 requires an identity layout and distinct format flags");
    const bool int8_keys = st.kv_int8 || st.kv_hybrid;
    if (g.n_head_kv <= 0 || g.head_dim <= 0 || g.head_dim > INT32_MAX || g.idx_key_dim <= 0 ||
        (st.kv_q4 && g.head_dim % 32) || (int8_keys && !st.kv_q4 && g.head_dim % 64))
        return fail(error, "invalid K/V geometry");
    e.page_size = gran.page_size;
    e.cells = (upto + gran.page_size - 1) / gran.page_size * gran.page_size;
    e.pooled_rows = index && upto > 0 ? upto / gran.idx_block + 1 : 0;   // completed rows plus the moving spare
    e.format = st.kv_hybrid ? kHybridFormat : qsa_kv_format(st);
    const uint64_t per_head = st.kv_q4 ? strata::kernels::kv_q4_bytes_per_head(int(g.head_dim))
                                       : uint64_t(g.head_dim) * (int8_keys ? 1 : 2);
    const uint64_t scale_groups = int8_keys && !st.kv_q4 ? uint64_t(g.head_dim / strata::kernels::KV_Q8_GROUP) * 2 : 0;
    size_t data = 0, scales = 0, pooled = 0;
    if (!checked_product(data, {uint64_t(e.cells), uint64_t(g.n_head_kv), per_head}) ||
        !checked_product(scales, {uint64_t(e.cells), uint64_t(g.n_head_kv), scale_groups}) ||
        !checked_product(pooled, {uint64_t(e.pooled_rows), uint64_t(g.idx_key_dim), sizeof(float)}))
        return fail(error, "K/V byte count overflow");
    size_t value_data = data, value_scales = scales;
    if (st.kv_hybrid) {   // V is rotated q4_0 and carries no separate scales
        if (!checked_product(value_data, {uint64_t(e.cells), uint64_t(g.n_head_kv),
                                          strata::kernels::kv_q4_bytes_per_head(int(g.head_dim))}))
            return fail(error, "hybrid V byte count overflow");
        value_scales = 0;
    }
    e.sizes = {data, value_data, scales, value_scales, pooled};
    return true;
}

// Where the authoritative bytes of each buffer live: the VRAM pools, or the host copy of a streamed/ring layer.
std::array<void*, 5> kv_sources(const QsaState& st, bool resident = false) {
    const bool host = st.kv_mode != 0 && !resident;
    if (st.kv_hybrid) return {st.k_q, st.v_q4, st.k_scale, nullptr, st.idx_pooled};
    if (st.kv_q4) return {host ? st.host.k_q4 : st.k_q4, host ? st.host.v_q4 : st.v_q4, nullptr, nullptr, st.idx_pooled};
    if (st.kv_int8)
        return {host ? (void*) st.host.k_q : (void*) st.k_q, host ? (void*) st.host.v_q : (void*) st.v_q,
                host ? st.host.k_scale : st.k_scale, host ? st.host.v_scale : st.v_scale, st.idx_pooled};
    return {host ? st.host.k_pool : st.k_pool, host ? st.host.v_pool : st.v_pool, nullptr, nullptr, st.idx_pooled};
}

bool kv_state_valid(const QsaState& st, const KvExtent& e, int64_t upto, std::string& error) {
    if (upto < 0 || upto > st.max_cells || st.n_pages < 0 || e.cells / e.page_size > st.n_pages || st.kv_mode < 0 ||
        st.kv_mode > 2 || st.n_slots <= 0 || (st.kv_mode == 0 && st.n_slots < st.n_pages) ||
        e.pooled_rows > st.idx_pooled_rows || (st.kv_mode != 0 && !st.host.present()))
        return fail(error, "invalid K/V extent or missing authoritative host pool");
    if (st.kv_mode == 1) {
        const auto& m = st.map;
        if (m.n_blocks != st.n_pages || m.n_slots != st.n_slots || !m.page_table || !m.slot_block || !m.slot_stamp ||
            !m.slot_ref || !m.ctl || !m.miss_block || !m.miss_slot)
            return fail(error, "invalid streaming map");
    }
    if (st.kv_mode == 2) {
        const bool pools_ok = st.kv_q4 ? st.k_q4 && st.v_q4
                            : st.kv_int8 ? st.k_q && st.v_q && st.k_scale && st.v_scale
                                         : st.k_pool && st.v_pool;
        if (!st.page_table || !pools_ok) return fail(error, "invalid draft ring");
    }
    return true;
}

std::array<ConversationBuffer*, 5> buffers(ConversationKv& kv) { return {&kv.k, &kv.v, &kv.k_scale, &kv.v_scale, &kv.pooled}; }
std::array<const ConversationBuffer*, 5> buffers(const ConversationKv& kv) {
    return {&kv.k, &kv.v, &kv.k_scale, &kv.v_scale, &kv.pooled};
}

// Enqueues one copy; a missing endpoint with bytes to move is the reference's "missing state buffer".
bool copy_piece(void* dst, const void* src, size_t n, std::string& error) {
    if (!n) return true;
    if (!dst || !src) return fail(error, "missing state buffer");
    return detail::enqueue_copy(dst, src, n, error, "conversation snapshot copy");
}

}  // namespace

namespace detail {

// The save of one layer with its copies enqueued but not yet waited for (the whole-session save waits once).
bool kv_save_enqueue(ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto, bool index,
                     std::string& error, int64_t unchanged_tokens, size_t* reused_bytes) {
    KvExtent e;
    if (!kv_extent(st, g, upto, index, e, error) || !kv_state_valid(st, e, upto, error)) return false;
    if (unchanged_tokens < 0 || unchanged_tokens > upto || unchanged_tokens > image.cells)
        return fail(error, "invalid unchanged prefix");
    const auto gran = strata::kernels::qsa_granules();
    const int64_t whole_cells = unchanged_tokens / e.page_size * e.page_size;
    image.format = e.format;
    image.cells = e.cells;
    image.heads = g.n_head_kv;
    image.head_dim = g.head_dim;
    image.page_size = e.page_size;
    image.pooled_rows = e.pooled_rows;
    image.idx_dim = g.idx_key_dim;
    const auto src = kv_sources(st);
    const auto dst = buffers(image);
    for (size_t i = 0; i < dst.size(); ++i) {
        // Whole pages (or completed indexer rows) strictly before the first rewritten token are unchanged; the
        // partial page and the moving spare row are always copied again.
        const size_t keep = i == 4 ? (index ? size_t(unchanged_tokens / gran.idx_block) * size_t(g.idx_key_dim) * 4 : 0)
                                   : e.cells ? e.sizes[i] / size_t(e.cells) * size_t(whole_cells) : 0;
        if (keep > dst[i]->size()) return fail(error, "missing reusable prefix");
        dst[i]->resize(e.sizes[i]);
        const uint8_t* from = static_cast<const uint8_t*>(src[i]);
        if (!dst[i]->visit(keep, e.sizes[i] - keep, [&](uint8_t* p, size_t n, size_t at) {
                return copy_piece(p, from ? from + at : nullptr, n, error);
            }))
            return false;
        if (reused_bytes) *reused_bytes += keep;
    }
    return true;
}

// The restore of one layer with its copies (and the residency fix-up) enqueued on the transfer stream.
bool kv_restore_enqueue(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                        bool index, std::string& error) {
    const auto src = buffers(image);
    const auto dst = kv_sources(st);
    for (size_t i = 0; i < src.size(); ++i) {
        uint8_t* to = static_cast<uint8_t*>(dst[i]);
        if (!src[i]->visit(0, src[i]->size(), [&](const uint8_t* p, size_t n, size_t at) {
                return copy_piece(to ? to + at : nullptr, p, n, error);
            }))
            return false;
    }
    (void) index;
    void* stream = transfer_stream();
    // The VRAM slots of a streamed layer still hold the outgoing conversation: evict them all, so the resolve
    // refills from the restored host copy before any attention reads.  A ring refills its window from the host.
    if (st.kv_mode == 1) strata::kernels::kv_stream_reset(st.map, stream);
    if (st.kv_mode == 2 && upto > 0) {
        strata::kernels::QsaShapes s = strata::kernels::qsa_real_shapes();
        s.n_head_kv = g.n_head_kv;
        s.head_dim = g.head_dim;
        s.page_size = image.page_size;
        const int64_t end = (upto + s.page_size - 1) / s.page_size;
        strata::kernels::kv_ring_restore(qsa_attn_pools(st), st.host, qsa_kv_format(st),
                                         std::max<int64_t>(0, end - st.n_slots), end, st.n_slots, s, stream);
    }
    return true;
}

}  // namespace detail

bool conversation_kv_capture_bytes(const ConversationKv& image, const QsaState& st, const ModelGeometry& g,
                                   int64_t upto, bool index, size_t& bytes, std::string& error) {
    KvExtent e;
    if (!kv_extent(st, g, upto, index, e, error) || !kv_state_valid(st, e, upto, error)) return false;
    const auto held = buffers(image);
    bytes = 0;
    for (size_t i = 0; i < held.size(); ++i) {
        const size_t n = held[i]->allocation_peak(e.sizes[i]);
        if (n == SIZE_MAX || !detail::checked_add(bytes, n)) return fail(error, "segmented K/V allocation overflow");
    }
    return true;
}

size_t conversation_kv_bytes(const QsaState& st, const ModelGeometry& g, int64_t upto, bool index) {
    size_t bytes = 0;
    std::string error;
    return conversation_kv_capture_bytes(ConversationKv{}, st, g, upto, index, bytes, error) ? bytes : 0;
}

bool conversation_kv_save(ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                          bool index, std::string& error, int64_t unchanged_tokens, size_t* reused_bytes) {
    if (!detail::kv_save_enqueue(image, st, g, upto, index, error, unchanged_tokens, reused_bytes)) {
        std::string ignored;
        detail::finish_transfers(ignored, "");   // never leave copies in flight into a buffer the caller may free
        return false;
    }
    return detail::finish_transfers(error, "conversation snapshot copy");
}

bool conversation_kv_validate(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                              bool index, std::string& error) {
    KvExtent e;
    if (!kv_extent(st, g, upto, index, e, error) || !kv_state_valid(st, e, upto, error)) return false;
    if (image.format != e.format || image.cells != e.cells || image.heads != g.n_head_kv ||
        image.head_dim != g.head_dim || image.page_size != e.page_size || image.pooled_rows != e.pooled_rows ||
        image.idx_dim != g.idx_key_dim)
        return fail(error, "incompatible K/V geometry");
    const auto held = buffers(image);
    for (size_t i = 0; i < held.size(); ++i)
        if (held[i]->size() != e.sizes[i]) return fail(error, "invalid K/V payload size");
    const auto targets = kv_sources(st);
    for (size_t i = 0; i < held.size(); ++i)
        if (e.sizes[i] && !targets[i]) return fail(error, "missing target state buffer");
    return true;
}

bool conversation_kv_restore(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                             bool index, std::string& error) {
    if (!conversation_kv_validate(image, st, g, upto, index, error)) return false;
    if (!detail::kv_restore_enqueue(image, st, g, upto, index, error)) {
        std::string ignored;
        detail::finish_transfers(ignored, "");
        return false;
    }
    return detail::finish_transfers(error, "conversation snapshot residency restore");
}

bool conversation_kv_verify(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                            bool index, uint64_t& fingerprint, std::string& error) {
    if (!conversation_kv_validate(image, st, g, upto, index, error)) return false;
    static constexpr size_t kChunk = 65536;
    std::vector<uint8_t> staging(kChunk);
    uint64_t hash = 1469598103934665603ull;   // the engine's FNV-1a seed (src/core/conversation_snapshot.cpp:225)
    // Reads `bytes` of device/host state in 64 KiB pieces and compares them with the image's bytes.
    auto compare = [&](const uint8_t* state, const uint8_t* expected, size_t bytes, bool fold) {
        for (size_t at = 0; at < bytes;) {
            const size_t n = std::min(kChunk, bytes - at);
            if (!copy_piece(staging.data(), state + at, n, error) ||
                !detail::finish_transfers(error, "conversation snapshot copy"))
                return false;
            if (std::memcmp(staging.data(), expected + at, n) != 0) return fail(error, "restored K/V bytes differ");
            if (fold)
                for (size_t i = 0; i < n; ++i) { hash ^= staging[i]; hash *= 1099511628211ull; }
            at += n;
        }
        return true;
    };
    const auto saved = buffers(image);
    const auto authoritative = kv_sources(st);
    for (size_t i = 0; i < saved.size(); ++i) {
        const uint8_t* base = static_cast<const uint8_t*>(authoritative[i]);
        if (!saved[i]->visit(0, saved[i]->size(), [&](const uint8_t* p, size_t n, size_t at) {
                return compare(base + at, p, n, true);
            }))
            return false;
    }
    if (st.kv_mode == 2 && image.cells > 0) {   // the ring's resident window must hold the image's last pages
        const auto resident = kv_sources(st, true);
        const int64_t end = image.cells / image.page_size, begin = std::max<int64_t>(0, end - st.n_slots);
        for (size_t i = 0; i < 4; ++i) {
            if (saved[i]->empty()) continue;
            const size_t page_bytes = saved[i]->size() / size_t(end);
            const uint8_t* ring = static_cast<const uint8_t*>(resident[i]);
            for (int64_t page = begin; page < end; ++page)
                if (!saved[i]->visit(size_t(page) * page_bytes, page_bytes, [&](const uint8_t* p, size_t n, size_t at) {
                        const size_t slot_at = size_t(page % st.n_slots) * page_bytes + (at - size_t(page) * page_bytes);
                        return compare(ring + slot_at, p, n, false);
                    }))
                    return false;
        }
    }
    fingerprint = hash;
    return true;
}

}  // namespace strata::core
