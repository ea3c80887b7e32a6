// snapshot_spec.cpp - the descriptors of a conversation image (snapshot_spec.hpp).
#include "snapshot_spec.hpp"

#include "strata/kernels/kv_stream.hpp"

#include <algorithm>
#include <limits>

namespace strata::core::spec {

bool refuse(std::string& error, const char* what) {
    error = std::string("conversation snapshot: ") + what;
    return false;
}

bool add(size_t& total, size_t n) {
    if (n > std::numeric_limits<size_t>::max() - total) return false;
    total += n;
    return true;
}

bool mul(size_t& out, std::initializer_list<uint64_t> factors) {
    unsigned __int128 acc = 1;
    for (uint64_t f : factors) {
        acc *= f;
        if (acc > std::numeric_limits<size_t>::max()) return false;
    }
    out = size_t(acc);
    return true;
}

// ---- the per-format layout of a layer image ---------------------------------------------------------------------------

namespace {

// The eight pool members QsaState and KvHostPools share (include/strata/core/layer.hpp:204-215,
// include/strata/kernels/kv_stream.hpp:30-39).
enum class Pool : uint8_t { none, f16_k, f16_v, q8_k, q8_v, scale_k, scale_v, q4_k, q4_v };
// What one cell of one KV head takes in a buffer: a 16-bit row is 2D bytes, an int8 row D, a q4_0 row D/32 blocks of 18
// bytes (kv_q4.hpp:21-28), the int8 scales one f16 per 64 values (kv_q8.hpp:22).
enum class Unit : uint8_t { none, row_f16, row_q8, row_q4, q8_scales };

struct Format {
    std::array<Unit, 4> unit;   // k, v, k_scale, v_scale
    std::array<Pool, 4> pool;
    bool host_authoritative;    // a streamed or ring layer of this format keeps its authoritative copy on the host
};

// Indexed by image format: f16, int8, q4_0 (the block movers' KvFormat values) and K8V4 (int8 K + q4_0 V, resident
// only; src/core/conversation_snapshot.cpp's format 3).
constexpr std::array<Format, 4> kFormats{{
    {{Unit::row_f16, Unit::row_f16, Unit::none, Unit::none}, {Pool::f16_k, Pool::f16_v, Pool::none, Pool::none}, true},
    {{Unit::row_q8, Unit::row_q8, Unit::q8_scales, Unit::q8_scales},
     {Pool::q8_k, Pool::q8_v, Pool::scale_k, Pool::scale_v}, true},
    {{Unit::row_q4, Unit::row_q4, Unit::none, Unit::none}, {Pool::q4_k, Pool::q4_v, Pool::none, Pool::none}, true},
    {{Unit::row_q8, Unit::row_q4, Unit::q8_scales, Unit::none}, {Pool::q8_k, Pool::q4_v, Pool::scale_k, Pool::none},
     false},
}};

template <class Pools>
uint8_t* member(const Pools& p, Pool which) {
    switch (which) {
        case Pool::f16_k: return reinterpret_cast<uint8_t*>(p.k_pool);
        case Pool::f16_v: return reinterpret_cast<uint8_t*>(p.v_pool);
        case Pool::q8_k: return reinterpret_cast<uint8_t*>(p.k_q);
        case Pool::q8_v: return reinterpret_cast<uint8_t*>(p.v_q);
        case Pool::scale_k: return reinterpret_cast<uint8_t*>(p.k_scale);
        case Pool::scale_v: return reinterpret_cast<uint8_t*>(p.v_scale);
        case Pool::q4_k: return reinterpret_cast<uint8_t*>(p.k_q4);
        case Pool::q4_v: return reinterpret_cast<uint8_t*>(p.v_q4);
        default: return nullptr;
    }
}

uint64_t unit_bytes(Unit u, int64_t head_dim) {
    switch (u) {
        case Unit::row_f16: return uint64_t(head_dim) * 2;
        case Unit::row_q8: return uint64_t(head_dim);
        case Unit::row_q4: return strata::kernels::kv_q4_bytes_per_head(int(head_dim));
        case Unit::q8_scales: return uint64_t(head_dim / strata::kernels::KV_Q8_GROUP) * 2;
        default: return 0;
    }
}

// A head_dim the format can hold: int8 scales group 64 values, q4_0 blocks 32.
bool holds(const Format& f, int64_t head_dim) {
    for (Unit u : f.unit) {
        if (u == Unit::q8_scales && head_dim % strata::kernels::KV_Q8_GROUP) return false;
        if (u == Unit::row_q4 && head_dim % strata::kernels::QK4_0) return false;
    }
    return true;
}

int image_format(const QsaState& st) { return st.kv_hybrid ? kK8V4 : st.kv_q4 ? 2 : st.kv_int8 ? 1 : 0; }

bool streaming_map_complete(const QsaState& st) {
    const auto& m = st.map;
    return m.n_blocks == st.n_pages && m.n_slots == st.n_slots && m.page_table && m.slot_block && m.slot_stamp &&
           m.slot_ref && m.ctl && m.miss_block && m.miss_slot;
}

}  // namespace

size_t LayerSpec::unchanged_bytes(int b, int64_t unchanged_tokens) const {
    if (b == kPooled) return bytes[kPooled] ? size_t(unchanged_tokens / idx_block) * idx_row_bytes : 0;
    if (!cells) return 0;
    const int64_t whole_cells = unchanged_tokens / page_size * page_size;
    return bytes[size_t(b)] / size_t(cells) * size_t(whole_cells);
}

bool describe_layer(const QsaState& st, const ModelGeometry& g, int64_t upto, bool include_index, LayerSpec& out,
                    std::string& error) {
    const auto gran = strata::kernels::qsa_granules();
    // the request, then the format flags, then the geometry the format needs
    if (upto < 0 || upto > st.max_cells || upto > std::numeric_limits<int64_t>::max() - (gran.page_size - 1))
        return refuse(error, "invalid K/V extent");
    if (st.kv_hybrid && (st.kv_mode != 0 || st.kv_q4 || st.kv_int8))
        return refuse(error, "hybrid K8V4 requires an identity layout and distinct format flags");
    const int fmt = image_format(st);
    const Format& f = kFormats[size_t(fmt)];
    if (g.n_head_kv <= 0 || g.head_dim <= 0 || g.head_dim > INT32_MAX || g.idx_key_dim <= 0 || !holds(f, g.head_dim))
        return refuse(error, "invalid K/V geometry");

    LayerSpec s;
    s.format = fmt;
    s.page_size = gran.page_size;
    s.idx_block = gran.idx_block;
    s.cells = (upto + gran.page_size - 1) / gran.page_size * gran.page_size;
    s.pooled_rows = include_index && upto > 0 ? upto / gran.idx_block + 1 : 0;
    for (size_t b = 0; b < 4; ++b)
        if (!mul(s.bytes[b], {uint64_t(s.cells), uint64_t(g.n_head_kv), unit_bytes(f.unit[b], g.head_dim)}))
            return refuse(error, fmt == kK8V4 && b == kV ? "hybrid V byte count overflow" : "K/V byte count overflow");
    if (!mul(s.idx_row_bytes, {uint64_t(g.idx_key_dim), sizeof(float)}) ||
        !mul(s.bytes[kPooled], {uint64_t(s.pooled_rows), s.idx_row_bytes}))
        return refuse(error, "K/V byte count overflow");

    // the layer's pools can take the extent, and a streamed or ring layer has its host copy
    const bool host_copy = st.kv_mode != 0;
    if (upto > st.max_cells || st.n_pages < 0 || s.cells / s.page_size > st.n_pages || st.kv_mode < 0 ||
        st.kv_mode > 2 || st.n_slots <= 0 || (st.kv_mode == 0 && st.n_slots < st.n_pages) ||
        s.pooled_rows > st.idx_pooled_rows || (host_copy && !st.host.present()))
        return refuse(error, "invalid K/V extent or missing authoritative host pool");
    if (st.kv_mode == 1 && !streaming_map_complete(st)) return refuse(error, "invalid streaming map");
    for (size_t b = 0; b < 4; ++b) {
        s.resident[b] = member(st, f.pool[b]);
        s.state[b] = host_copy && f.host_authoritative ? member(st.host, f.pool[b]) : s.resident[b];
    }
    s.resident[kPooled] = s.state[kPooled] = reinterpret_cast<uint8_t*>(st.idx_pooled);
    if (st.kv_mode == 2) {   // a ring's window lives in its VRAM pools: every pool of the format must exist
        bool window = st.page_table != nullptr;
        for (size_t b = 0; b < 4; ++b) window = window && (f.pool[b] == Pool::none || s.resident[b] != nullptr);
        if (!window) return refuse(error, "invalid draft ring");
    }
    out = s;
    return true;
}

std::array<ConversationBuffer*, kBufs> buffers_of(ConversationKv& image) {
    return {&image.k, &image.v, &image.k_scale, &image.v_scale, &image.pooled};
}
std::array<const ConversationBuffer*, kBufs> buffers_of(const ConversationKv& image) {
    return {&image.k, &image.v, &image.k_scale, &image.v_scale, &image.pooled};
}

bool image_matches(const ConversationKv& image, const LayerSpec& s, const ModelGeometry& g, std::string& error) {
    if (image.format != s.format || image.cells != s.cells || image.heads != g.n_head_kv ||
        image.head_dim != g.head_dim || image.page_size != s.page_size || image.pooled_rows != s.pooled_rows ||
        image.idx_dim != g.idx_key_dim)
        return refuse(error, "incompatible K/V geometry");
    const auto held = buffers_of(image);
    for (size_t b = 0; b < kBufs; ++b)
        if (held[b]->size() != s.bytes[b]) return refuse(error, "invalid K/V payload size");
    for (size_t b = 0; b < kBufs; ++b)
        if (s.bytes[b] && !s.state[b]) return refuse(error, "missing target state buffer");
    return true;
}

void stamp(ConversationKv& image, const LayerSpec& s, const ModelGeometry& g) {
    image.format = s.format;
    image.cells = s.cells;
    image.heads = g.n_head_kv;
    image.head_dim = g.head_dim;
    image.page_size = s.page_size;
    image.pooled_rows = s.pooled_rows;
    image.idx_dim = g.idx_key_dim;
}

// ---- running state ---------------------------------------------------------------------------------------------------

std::array<int64_t, 18> geometry_key(const ModelGeometry& g) {
    return {g.n_embd, g.n_layers, g.qsa_interval, g.ssm_state_size, g.ssm_k_heads, g.ssm_v_heads, g.ssm_d_conv,
            g.ssm_conv_channels, g.ssm_value_dim, g.n_head, g.n_head_kv, g.head_dim, g.idx_q_heads, g.idx_key_dim,
            g.hc, g.hc_lr, g.n_expert, g.n_ff};
}

size_t owned_layers(const SessionState& ss) { return size_t(std::max<int64_t>(ss.qsa_alloc, 0)); }
const QsaState& owned_layer(const SessionState& ss, size_t j) { return ss.qsa_states[size_t(ss.qsa_ord0) + j]; }

bool running_state_targets(const SessionState& ss, const ModelGeometry& g, size_t tokens, ConversationStateSizes& z,
                           std::string& error) {
    if (!conversation_session_sizes(g, ss, z, error)) return false;
    const size_t layers = owned_layers(ss);
    if (ss.max_cells < 0 || tokens > uint64_t(ss.max_cells) || (z.gdn && !ss.gdn_state) || (layers && !ss.qsa_states))
        return refuse(error, "invalid session running-state targets");
    const uint64_t block = uint64_t(strata::kernels::qsa_granules().idx_block);
    for (size_t j = 0; j < layers; ++j) {
        const QsaState& st = owned_layer(ss, j);
        // the spare row a restore rebuilds sits at row tokens / block, which must be inside the pooled rows
        const bool buffers = st.idx_tail && st.idx_dead && st.idx_block_pos && st.idx_pooled;
        const bool room = st.max_cells >= 0 && tokens <= uint64_t(st.max_cells) &&
                          (!tokens || tokens / block < uint64_t(std::max<int64_t>(0, st.idx_pooled_rows)));
        size_t spare_end = 0;
        if (!buffers || !room || !mul(spare_end, {tokens / block + 1, uint64_t(g.idx_key_dim), sizeof(float)}))
            return refuse(error, "invalid indexer running-state target");
    }
    return true;
}

bool image_keys_ordered(const std::vector<ConversationImageKey>& images, size_t tokens) {
    for (size_t i = 0; i < images.size(); ++i) {
        const int64_t start = images[i].start;
        if (start < 0 || uint64_t(start) >= tokens || (i && start <= images[i - 1].start)) return false;
    }
    return true;
}

// ---- a snapshot's shape ------------------------------------------------------------------------------------------------

int64_t stage_count(const ConversationStageSet& stages) { return stages.empty() ? 0 : stages.count; }

bool stages_tile_model(const ConversationStageSet& stages, const SessionState& main, const ModelGeometry& g,
                       std::string& error) {
    if (stages.empty()) return true;
    if (stages.count > int64_t(std::numeric_limits<size_t>::max() / sizeof(ConversationStageSnapshot)))
        return refuse(error, "too many layer-split stages");
    const int64_t n_qsa = g.n_qsa_layers();
    int64_t expected_lo = main.layer_hi;
    for (const ConversationStage* s = stages.stages; s != stages.stages + stages.count; ++s) {
        if (!s->session) return refuse(error, "layer-split stage has no session");
        const SessionState& ss = *s->session;
        ConversationStateSizes z;
        if (!conversation_session_sizes(g, ss, z, error)) return false;
        if (ss.layer_lo != expected_lo || ss.layer_lo >= ss.layer_hi || ss.layer_hi > g.n_layers)
            return refuse(error, "layer-split stages do not tile the model");
        if (ss.qsa_ord0 < ss.layer_lo / std::max<int64_t>(g.qsa_interval, 1))
            return refuse(error, "layer-split stage carve starts before its layer range");
        if (ss.qsa_alloc > n_qsa - ss.qsa_ord0) return refuse(error, "layer-split stage carve past the last QSA layer");
        expected_lo = ss.layer_hi;
    }
    if (expected_lo != g.n_layers) return refuse(error, "layer-split stages do not cover the whole model");
    return true;
}

namespace {

bool is_prefix(const std::vector<int32_t>& shorter, const std::vector<int32_t>& longer) {
    return shorter.size() <= longer.size() && std::equal(shorter.begin(), shorter.end(), longer.begin());
}

// A retained checkpoint of the view: a prefix of the live tokens whose image keys are the live keys it covers, with
// one part per later stage when the model is split.
bool checkpoint_consistent(const ConversationCheckpoint& c, const ConversationView& view, const SessionState& ss,
                           const ConversationStageSet& stages, const ModelGeometry& g, std::string& error) {
    if (c.ids.empty() || !is_prefix(c.ids, view.ids)) return refuse(error, "checkpoint is not a live token prefix");
    if (int64_t(c.stage_parts.size()) != stage_count(stages))
        return refuse(error, stages.empty() ? "layer-split parking is not supported"
                                            : "checkpoint is missing a layer-split stage part");
    if (!conversation_checkpoint_validate(c, ss, g, error)) return false;
    for (size_t i = 0; i < c.stage_parts.size(); ++i) {
        const ConversationCheckpoint& part = c.stage_parts[i];
        if (part.ids.size() != c.ids.size() || !part.imgs.empty() || !part.stage_parts.empty())
            return refuse(error, "layer-split checkpoint part is not a live token prefix");
        if (!conversation_checkpoint_validate(part, *stages.stages[i].session, g, error)) return false;
    }
    // the live keys that start inside the checkpoint, in order, are exactly the checkpoint's keys
    auto held = c.imgs.begin();
    for (const ConversationImageKey& key : view.images) {
        if (uint64_t(key.start) >= c.ids.size()) break;
        if (held == c.imgs.end() || !(*held == key)) return refuse(error, "checkpoint image identity differs");
        ++held;
    }
    if (held != c.imgs.end()) return refuse(error, "checkpoint image prefix differs");
    return true;
}

}  // namespace

bool view_consistent(const ConversationView& view, const SessionState& ss, const ConversationStageSet& stages,
                     const ModelGeometry& g, std::string& error) {
    ConversationStateSizes z;
    if (!running_state_targets(ss, g, view.ids.size(), z, error)) return false;
    const bool ids_ok = !view.ids.empty() && std::none_of(view.ids.begin(), view.ids.end(), [](int32_t id) { return id < 0; });
    if (!ids_ok || !image_keys_ordered(view.images, view.ids.size()))
        return refuse(error, "invalid live token/image metadata");
    for (const ConversationCheckpoint& c : view.checkpoints)
        if (!checkpoint_consistent(c, view, ss, stages, g, error)) return false;
    return true;
}

namespace {

// Host bytes of a retained checkpoint's payloads and directories, its stage parts included.
bool checkpoint_bytes(const ConversationCheckpoint& c, size_t& total) {
    size_t ids = 0, keys = 0, parts = 0;
    if (!mul(ids, {c.ids.size(), sizeof(int32_t)}) || !mul(keys, {c.imgs.size(), sizeof(ConversationImageKey)}) ||
        !mul(parts, {c.stage_parts.capacity(), sizeof(ConversationCheckpoint)}))
        return false;
    for (size_t n : {ids, keys, c.gdn.size(), c.ple.size(), c.tails.size(), c.dead.size(), c.block_pos.size(), parts})
        if (!add(total, n)) return false;
    return std::all_of(c.stage_parts.begin(), c.stage_parts.end(),
                       [&](const ConversationCheckpoint& part) { return checkpoint_bytes(part, total); });
}

// The running state and directory entries a session contributes: `directory_entries` ConversationKv entries, the
// owned layers' indexer state, the GDN rows and the PLE history.
bool session_state_bytes(const SessionState& ss, const ConversationStateSizes& z, uint64_t directory_entries,
                         size_t& total) {
    const uint64_t layers = owned_layers(ss);
    size_t directory = 0, tails = 0, dead = 0, positions = 0;
    return mul(directory, {directory_entries, sizeof(ConversationKv)}) && mul(tails, {layers, z.tail}) &&
           mul(dead, {layers, z.dead}) && mul(positions, {layers, z.block_pos}) && add(total, directory) &&
           add(total, tails) && add(total, dead) && add(total, positions) && add(total, z.gdn) &&
           add(total, ss.ple_hist ? z.ple : 0);
}

}  // namespace

bool snapshot_estimate(const ConversationView& view, const SessionState& ss, const ConversationStageSet& stages,
                       const ModelGeometry& g, const QsaState& draft, size_t& bytes, std::string& error) {
    ConversationStateSizes z;
    if (!conversation_session_sizes(g, ss, z, error)) return false;
    const int64_t tokens = int64_t(view.ids.size());
    const size_t layers = owned_layers(ss);
    // the main session: token ids and image keys, the checkpoint directory, its layers plus the draft
    size_t ids = 0, keys = 0, checkpoints = 0;
    if (!mul(ids, {view.ids.size(), sizeof(int32_t)}) || !mul(keys, {view.images.size(), sizeof(ConversationImageKey)}) ||
        !mul(checkpoints, {view.checkpoints.size(), sizeof(ConversationCheckpoint)}))
        return refuse(error, "snapshot metadata byte count overflow");
    if (!add(bytes, ids) || !add(bytes, keys) || !add(bytes, checkpoints) ||
        !session_state_bytes(ss, z, uint64_t(layers) + 1, bytes))
        return refuse(error, "snapshot byte count overflow");
    for (const ConversationCheckpoint& c : view.checkpoints)
        if (!checkpoint_bytes(c, bytes)) return refuse(error, "checkpoint byte count overflow");
    for (size_t j = 0; j <= layers; ++j) {
        const bool is_draft = j == layers;
        const size_t n = conversation_kv_bytes(is_draft ? draft : owned_layer(ss, j), g, tokens, !is_draft);
        if (!n || !add(bytes, n)) return refuse(error, "invalid or overflowing K/V byte estimate");
    }
    // every later stage: a directory entry, its own copy of the ids, its running state and its layers
    if (stages.empty()) return true;
    size_t directory = 0;
    if (!mul(directory, {uint64_t(stages.count), sizeof(ConversationStageSnapshot)}) || !add(bytes, directory))
        return refuse(error, "layer-split stage directory overflow");
    for (int64_t i = 0; i < stages.count; ++i) {
        const SessionState& part = *stages.stages[i].session;
        ConversationStateSizes pz;
        if (!running_state_targets(part, g, size_t(tokens), pz, error)) return false;
        if (!add(bytes, ids) || !session_state_bytes(part, pz, owned_layers(part), bytes))
            return refuse(error, "stage byte count overflow");
        for (size_t j = 0; j < owned_layers(part); ++j) {
            const size_t n = conversation_kv_bytes(owned_layer(part, j), g, tokens, true);
            if (!n || !add(bytes, n)) return refuse(error, "invalid or overflowing stage K/V byte estimate");
        }
    }
    return true;
}

}  // namespace strata::core::spec

namespace strata::core {

bool conversation_state_sizes(const ModelGeometry& g, ConversationStateSizes& z, std::string& error) {
    z = {};
    const auto key = spec::geometry_key(g);
    for (size_t i = 0; i < key.size(); ++i)   // every dimension positive; only the layer count may be zero
        if (key[i] < (i == 1 ? 0 : 1)) return spec::refuse(error, "invalid model geometry");
    const uint64_t block = uint64_t(strata::kernels::qsa_granules().idx_block);
    size_t row = 0, history = 0;
    const bool sized =
        spec::mul(row, {uint64_t(g.ssm_state_size), uint64_t(g.ssm_v_heads), uint64_t(g.ssm_state_size)}) &&
        spec::mul(history, {uint64_t(g.ssm_conv_channels), uint64_t(g.ssm_d_conv - 1)}) && spec::add(row, history) &&
        spec::mul(z.gdn, {uint64_t(g.n_gdn_layers()), row, sizeof(float)}) &&
        spec::mul(z.ple, {uint64_t(strata::kernels::NG_HIST), uint64_t(strata::kernels::NG_HC_DIM), sizeof(float)}) &&
        spec::mul(z.tail, {block - 1, uint64_t(g.idx_key_dim), sizeof(float)}) &&
        spec::mul(z.dead, {uint64_t(g.idx_key_dim), sizeof(float)});
    if (!sized) return spec::refuse(error, "running-state byte count overflow");
    z.block_pos = sizeof(int32_t);
    size_t all = 0;
    const uint64_t n_qsa = uint64_t(g.n_qsa_layers());
    if (!spec::mul(all, {n_qsa, z.tail}) || !spec::mul(all, {n_qsa, z.dead}) || !spec::mul(all, {n_qsa, z.block_pos}))
        return spec::refuse(error, "indexer byte count overflow");
    return true;
}

bool conversation_session_sizes(const ModelGeometry& g, const SessionState& ss, ConversationStateSizes& z,
                                std::string& error) {
    if (!conversation_state_sizes(g, z, error)) return false;
    const int64_t n_gdn = g.n_gdn_layers(), n_qsa = g.n_qsa_layers();
    const bool carve = ss.gdn_alloc >= 0 && ss.gdn_alloc <= n_gdn && ss.qsa_ord0 >= 0 && ss.qsa_alloc >= 0 &&
                       ss.qsa_ord0 <= n_qsa && ss.qsa_alloc <= n_qsa - ss.qsa_ord0;
    if (!carve) return spec::refuse(error, "invalid session layer carve");
    z.gdn = n_gdn > 0 ? z.gdn / size_t(n_gdn) * size_t(ss.gdn_alloc) : 0;   // only the rows this session owns
    return true;
}

}  // namespace strata::core
