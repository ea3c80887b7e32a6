// conversation_state.cpp - a whole session's running state and K/V between the device and a SavedConversation.
//
// Semantics of the reference's session-level functions (src/core/conversation_state.cpp:14-512), restated over
// libsc_handoff.so: the geometry key and sizes (:14-19, :180-214), checkpoint save/validate/restore including the
// indexer's spare-row rebuild and the PLE token window (:216-267), the byte estimates (:269-358), and the
// snapshot save / validate / restore with the layer-split stage parts (:360-512).  The differences are in how
// bytes move, not in what moves: the copies of one call are enqueued together on the transfer stream and waited
// for once, and pinned image segments make them DMAs.
#include "strata/core/conversation_snapshot.hpp"

#include "transfer.hpp"

#include <algorithm>
#include <array>
#include <limits>

namespace strata::core {
namespace detail {
bool checked_add(size_t& total, size_t n);
bool checked_product(size_t& out, std::initializer_list<uint64_t> factors);
bool kv_save_enqueue(ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto, bool index,
                     std::string& error, int64_t unchanged_tokens, size_t* reused_bytes);
bool kv_restore_enqueue(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                        bool index, std::string& error);
}  // namespace detail

namespace {

using detail::checked_add;
using detail::checked_product;

std::array<int64_t, 18> geometry_key(const ModelGeometry& g) {
    return {g.n_embd, g.n_layers, g.qsa_interval, g.ssm_state_size, g.ssm_k_heads, g.ssm_v_heads, g.ssm_d_conv,
            g.ssm_conv_channels, g.ssm_value_dim, g.n_head, g.n_head_kv, g.head_dim, g.idx_q_heads, g.idx_key_dim,
            g.hc, g.hc_lr, g.n_expert, g.n_ff};
}

bool fail(std::string& error, const char* what) {
    error = std::string("conversation snapshot: ") + what;
    return false;
}

bool sync(std::string& error) { return detail::device_synchronize(error, "conversation snapshot synchronize"); }
bool wait(std::string& error) { return detail::finish_transfers(error, "conversation snapshot running-state copy"); }

bool copy(void* dst, const void* src, size_t n, std::string& error) {
    if (!n) return true;
    if (!dst || !src) return fail(error, "missing running-state buffer");
    return detail::enqueue_copy(dst, src, n, error, "conversation snapshot running-state copy");
}

// Drains whatever a failed call left enqueued, so no copy lands in a buffer after the caller has moved on.
void drain() {
    std::string ignored;
    detail::finish_transfers(ignored, "");
}

size_t owned_qsa(const SessionState& ss) { return size_t(std::max<int64_t>(ss.qsa_alloc, 0)); }
const QsaState& owned(const SessionState& ss, size_t j) { return ss.qsa_states[size_t(ss.qsa_ord0) + j]; }

bool image_keys_ok(const std::vector<ConversationImageKey>& images, size_t tokens) {
    int64_t prev = -1;
    for (const ConversationImageKey& k : images) {
        if (k.start <= prev || k.start < 0 || uint64_t(k.start) >= tokens) return false;
        prev = k.start;
    }
    return true;
}

int64_t stage_count(const ConversationStageSet& s) { return s.empty() ? 0 : s.count; }

bool checkpoint_targets(const SessionState& ss, const ModelGeometry& g, size_t tokens, ConversationStateSizes& z,
                        std::string& error) {
    if (!conversation_session_sizes(g, ss, z, error)) return false;
    if (ss.max_cells < 0 || tokens > uint64_t(ss.max_cells) || (z.gdn && !ss.gdn_state) ||
        (owned_qsa(ss) && !ss.qsa_states))
        return fail(error, "invalid session running-state targets");
    const uint64_t block = uint64_t(strata::kernels::qsa_granules().idx_block);
    for (size_t j = 0; j < owned_qsa(ss); ++j) {
        const QsaState& st = owned(ss, j);
        size_t pooled = 0;
        if (!st.idx_tail || !st.idx_dead || !st.idx_block_pos || !st.idx_pooled || st.max_cells < 0 ||
            tokens > uint64_t(st.max_cells) ||
            (tokens && tokens / block >= uint64_t(std::max<int64_t>(0, st.idx_pooled_rows))) ||
            !checked_product(pooled, {tokens / block + 1, uint64_t(g.idx_key_dim), sizeof(float)}))
            return fail(error, "invalid indexer running-state target");
    }
    return true;
}

// The stages, with the main session, must tile [0, n_layers): increasing, disjoint, complete.
bool stage_set_validate(const ConversationStageSet& stages, const SessionState& main_ss, const ModelGeometry& g,
                        std::string& error) {
    if (stages.empty()) return true;
    if (stages.count > int64_t(std::numeric_limits<size_t>::max() / sizeof(ConversationStageSnapshot)))
        return fail(error, "too many layer-split stages");
    const int64_t n_qsa = g.n_qsa_layers();
    int64_t next = main_ss.layer_hi;
    for (int64_t i = 0; i < stages.count; ++i) {
        const SessionState* ss = stages.stages[i].session;
        if (!ss) return fail(error, "layer-split stage has no session");
        ConversationStateSizes z;
        if (!conversation_session_sizes(g, *ss, z, error)) return false;
        if (ss->layer_lo != next || ss->layer_lo >= ss->layer_hi || ss->layer_hi > g.n_layers)
            return fail(error, "layer-split stages do not tile the model");
        if (ss->qsa_ord0 < ss->layer_lo / std::max<int64_t>(g.qsa_interval, 1))
            return fail(error, "layer-split stage carve starts before its layer range");
        if (ss->qsa_alloc > n_qsa - ss->qsa_ord0) return fail(error, "layer-split stage carve past the last QSA layer");
        next = ss->layer_hi;
    }
    if (next != g.n_layers) return fail(error, "layer-split stages do not cover the whole model");
    return true;
}

bool stage_kv_bytes(const SessionState& ss, const ModelGeometry& g, int64_t upto, size_t& total, std::string& error) {
    ConversationStateSizes z;
    if (!conversation_session_sizes(g, ss, z, error) || !checkpoint_targets(ss, g, size_t(upto), z, error)) return false;
    const size_t layers = owned_qsa(ss);
    size_t directory = 0, tails = 0, dead = 0, positions = 0, ids = 0;
    if (!checked_product(directory, {layers, sizeof(ConversationKv)}) || !checked_product(tails, {layers, z.tail}) ||
        !checked_product(dead, {layers, z.dead}) || !checked_product(positions, {layers, z.block_pos}) ||
        !checked_product(ids, {uint64_t(upto), sizeof(int32_t)}))
        return fail(error, "stage byte count overflow");
    for (size_t n : {directory, ids, tails, dead, positions, z.gdn, ss.ple_hist ? z.ple : size_t(0)})
        if (!checked_add(total, n)) return fail(error, "stage byte count overflow");
    for (size_t j = 0; j < layers; ++j) {
        const size_t n = conversation_kv_bytes(owned(ss, j), g, upto, true);
        if (!n || !checked_add(total, n)) return fail(error, "invalid or overflowing stage K/V byte estimate");
    }
    return true;
}

bool view_validate(const ConversationView& view, const SessionState& ss, const ConversationStageSet& stages,
                   const ModelGeometry& g, std::string& error) {
    ConversationStateSizes z;
    if (!checkpoint_targets(ss, g, view.ids.size(), z, error)) return false;
    if (view.ids.empty() || !image_keys_ok(view.images, view.ids.size()) ||
        std::any_of(view.ids.begin(), view.ids.end(), [](int32_t id) { return id < 0; }))
        return fail(error, "invalid live token/image metadata");
    for (const ConversationCheckpoint& c : view.checkpoints) {
        if (c.ids.empty() || c.ids.size() > view.ids.size() || !std::equal(c.ids.begin(), c.ids.end(), view.ids.begin()))
            return fail(error, "checkpoint is not a live token prefix");
        if (int64_t(c.stage_parts.size()) != stage_count(stages))
            return fail(error, stages.empty() ? "layer-split parking is not supported"
                                              : "checkpoint is missing a layer-split stage part");
        if (!conversation_checkpoint_validate(c, ss, g, error)) return false;
        for (size_t i = 0; i < c.stage_parts.size(); ++i) {
            const ConversationCheckpoint& part = c.stage_parts[i];
            if (part.ids.size() != c.ids.size() || !part.imgs.empty() || !part.stage_parts.empty())
                return fail(error, "layer-split checkpoint part is not a live token prefix");
            if (!conversation_checkpoint_validate(part, *stages.stages[i].session, g, error)) return false;
        }
        size_t k = 0;
        for (const ConversationImageKey& key : view.images) {
            if (uint64_t(key.start) >= c.ids.size()) break;
            if (k >= c.imgs.size() || !(c.imgs[k++] == key)) return fail(error, "checkpoint image identity differs");
        }
        if (k != c.imgs.size()) return fail(error, "checkpoint image prefix differs");
    }
    return true;
}

bool metadata_bytes(const ConversationCheckpoint& c, size_t& total) {
    size_t ids = 0, images = 0;
    if (!checked_product(ids, {c.ids.size(), sizeof(int32_t)}) ||
        !checked_product(images, {c.imgs.size(), sizeof(ConversationImageKey)}))
        return false;
    for (size_t n : {ids, images, c.gdn.size(), c.ple.size(), c.tails.size(), c.dead.size(), c.block_pos.size()})
        if (!checked_add(total, n)) return false;
    if (!checked_product(images, {c.stage_parts.capacity(), sizeof(ConversationCheckpoint)}) ||
        !checked_add(total, images))
        return false;
    for (const ConversationCheckpoint& part : c.stage_parts)
        if (!metadata_bytes(part, total)) return false;
    return true;
}

// The main session's own estimate: running state, indexer payloads, its QSA layers' K/V and the draft's.
bool main_snapshot_bytes(const ConversationView& view, const SessionState& ss, const ModelGeometry& g,
                         const QsaState& draft, size_t& bytes, std::string& error) {
    ConversationStateSizes z;
    if (!conversation_session_sizes(g, ss, z, error)) return false;
    const uint64_t qsa = owned_qsa(ss);
    size_t ids = 0, images = 0, checkpoints = 0, layers = 0, tails = 0, dead = 0, positions = 0;
    if (!checked_product(ids, {view.ids.size(), sizeof(int32_t)}) ||
        !checked_product(images, {view.images.size(), sizeof(ConversationImageKey)}) ||
        !checked_product(checkpoints, {view.checkpoints.size(), sizeof(ConversationCheckpoint)}) ||
        !checked_product(layers, {qsa + 1, sizeof(ConversationKv)}) || !checked_product(tails, {qsa, z.tail}) ||
        !checked_product(dead, {qsa, z.dead}) || !checked_product(positions, {qsa, z.block_pos}))
        return fail(error, "snapshot metadata byte count overflow");
    for (size_t n : {ids, images, checkpoints, layers, tails, dead, positions, z.gdn, ss.ple_hist ? z.ple : size_t(0)})
        if (!checked_add(bytes, n)) return fail(error, "snapshot byte count overflow");
    for (const ConversationCheckpoint& c : view.checkpoints)
        if (!metadata_bytes(c, bytes)) return fail(error, "checkpoint byte count overflow");
    const int64_t upto = int64_t(view.ids.size());
    for (uint64_t i = 0; i <= qsa; ++i) {
        const QsaState& st = i == qsa ? draft : owned(ss, size_t(i));
        const size_t n = conversation_kv_bytes(st, g, upto, i != qsa);
        if (!n || !checked_add(bytes, n)) return fail(error, "invalid or overflowing K/V byte estimate");
    }
    return true;
}

bool stage_directory_bytes(const ConversationStageSet& stages, size_t& bytes, std::string& error) {
    if (stages.empty()) return true;
    size_t directory = 0;
    if (!checked_product(directory, {uint64_t(stages.count), sizeof(ConversationStageSnapshot)}) ||
        !checked_add(bytes, directory))
        return fail(error, "layer-split stage directory overflow");
    return true;
}

// Enqueues a checkpoint save's copies (running state and per-layer indexer state) without waiting.
bool checkpoint_save_enqueue(ConversationCheckpoint& c, const SessionState& ss, const ModelGeometry& g,
                             std::string& error) {
    ConversationStateSizes z;
    if (!checkpoint_targets(ss, g, c.ids.size(), z, error)) return false;
    const size_t layers = owned_qsa(ss);
    c.gdn.resize(z.gdn);
    c.ple.resize(ss.ple_hist ? z.ple : 0);
    c.tails.resize(layers * z.tail);
    c.dead.resize(layers * z.dead);
    c.block_pos.resize(layers * z.block_pos);
    if (!copy(c.gdn.data(), ss.gdn_state, c.gdn.size(), error) || !copy(c.ple.data(), ss.ple_hist, c.ple.size(), error))
        return false;
    for (size_t j = 0; j < layers; ++j) {
        const QsaState& st = owned(ss, j);
        if (!copy(c.tails.data() + j * z.tail, st.idx_tail, z.tail, error) ||
            !copy(c.dead.data() + j * z.dead, st.idx_dead, z.dead, error) ||
            !copy(c.block_pos.data() + j * z.block_pos, st.idx_block_pos, z.block_pos, error))
            return false;
    }
    return true;
}

}  // namespace

bool conversation_state_sizes(const ModelGeometry& g, ConversationStateSizes& z, std::string& error) {
    z = {};
    const auto key = geometry_key(g);
    for (size_t i = 0; i < key.size(); ++i)
        if (key[i] < 0 || (i != 1 && key[i] == 0)) return fail(error, "invalid model geometry");
    size_t recurrence = 0, convolution = 0;
    const uint64_t block = uint64_t(strata::kernels::qsa_granules().idx_block);
    if (!checked_product(recurrence, {uint64_t(g.ssm_state_size), uint64_t(g.ssm_v_heads), uint64_t(g.ssm_state_size)}) ||
        !checked_product(convolution, {uint64_t(g.ssm_conv_channels), uint64_t(g.ssm_d_conv - 1)}) ||
        !checked_add(recurrence, convolution) ||
        !checked_product(z.gdn, {uint64_t(g.n_gdn_layers()), recurrence, sizeof(float)}) ||
        !checked_product(z.ple, {uint64_t(strata::kernels::NG_HIST), uint64_t(strata::kernels::NG_HC_DIM), sizeof(float)}) ||
        !checked_product(z.tail, {block - 1, uint64_t(g.idx_key_dim), sizeof(float)}) ||
        !checked_product(z.dead, {uint64_t(g.idx_key_dim), sizeof(float)}))
        return fail(error, "running-state byte count overflow");
    z.block_pos = sizeof(int32_t);
    size_t total = 0;
    const uint64_t n_qsa = uint64_t(g.n_qsa_layers());
    if (!checked_product(total, {n_qsa, z.tail}) || !checked_product(total, {n_qsa, z.dead}) ||
        !checked_product(total, {n_qsa, z.block_pos}))
        return fail(error, "indexer byte count overflow");
    return true;
}

bool conversation_session_sizes(const ModelGeometry& g, const SessionState& ss, ConversationStateSizes& z,
                                std::string& error) {
    if (!conversation_state_sizes(g, z, error)) return false;
    const int64_t n_gdn = g.n_gdn_layers(), n_qsa = g.n_qsa_layers();
    if (ss.gdn_alloc < 0 || ss.gdn_alloc > n_gdn || ss.qsa_ord0 < 0 || ss.qsa_alloc < 0 || ss.qsa_ord0 > n_qsa ||
        ss.qsa_alloc > n_qsa - ss.qsa_ord0)
        return fail(error, "invalid session layer carve");
    z.gdn = n_gdn > 0 ? z.gdn / size_t(n_gdn) * size_t(ss.gdn_alloc) : 0;   // the rows this session owns
    return true;
}

bool conversation_checkpoint_validate(const ConversationCheckpoint& c, const SessionState& ss, const ModelGeometry& g,
                                      std::string& error) {
    ConversationStateSizes z;
    if (!checkpoint_targets(ss, g, c.ids.size(), z, error)) return false;
    const size_t layers = owned_qsa(ss);
    if (c.gdn.size() != z.gdn || c.ple.size() != (ss.ple_hist ? z.ple : 0) || c.tails.size() != layers * z.tail ||
        c.dead.size() != layers * z.dead || c.block_pos.size() != layers * z.block_pos ||
        !image_keys_ok(c.imgs, c.ids.size()))
        return fail(error, "invalid checkpoint running-state payload");
    return true;
}

bool conversation_checkpoint_save(ConversationCheckpoint& c, const SessionState& ss, const ModelGeometry& g,
                                  std::string& error) {
    if (!checkpoint_save_enqueue(c, ss, g, error)) {
        drain();
        return false;
    }
    return wait(error);
}

bool conversation_checkpoint_restore(const ConversationCheckpoint& c, SessionState& ss, const ModelGeometry& g,
                                     std::string& error) {
    if (!conversation_checkpoint_validate(c, ss, g, error)) return false;
    ConversationStateSizes z;
    if (!conversation_session_sizes(g, ss, z, error)) return false;
    bool ok = copy(ss.gdn_state, c.gdn.data(), c.gdn.size(), error) && copy(ss.ple_hist, c.ple.data(), c.ple.size(), error);
    const size_t block = size_t(strata::kernels::qsa_granules().idx_block);
    for (size_t j = 0; ok && j < owned_qsa(ss); ++j) {
        const QsaState& st = owned(ss, j);
        ok = copy(st.idx_tail, c.tails.data() + j * z.tail, z.tail, error) &&
             copy(st.idx_dead, c.dead.data() + j * z.dead, z.dead, error) &&
             copy(st.idx_block_pos, c.block_pos.data() + j * z.block_pos, z.block_pos, error);
        // The indexer's moving spare row is a copy of the spare key: rebuild it at the checkpoint's block, which
        // may be earlier than where the outgoing conversation had it.
        if (ok && !c.ids.empty())
            ok = copy(st.idx_pooled + (c.ids.size() / block) * size_t(g.idx_key_dim), c.dead.data() + j * z.dead,
                      z.dead, error);
    }
    if (!ok) {
        drain();
        return false;
    }
    const size_t tokens = c.ids.size();
    ss.ple_prev[0] = tokens >= 2 ? c.ids[tokens - 2] : -1;
    ss.ple_prev[1] = tokens >= 1 ? c.ids[tokens - 1] : -1;
    return wait(error) && sync(error);
}

bool conversation_snapshot_bytes(const ConversationView& view, const SessionState& ss,
                                 const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                 size_t& bytes, std::string& error) {
    bytes = 0;
    if (!stage_set_validate(stages, ss, g, error) || !view_validate(view, ss, stages, g, error) ||
        !main_snapshot_bytes(view, ss, g, draft, bytes, error) || !stage_directory_bytes(stages, bytes, error))
        return false;
    const int64_t upto = int64_t(view.ids.size());
    for (int64_t i = 0; i < stage_count(stages); ++i)
        if (!stage_kv_bytes(*stages.stages[i].session, g, upto, bytes, error)) return false;
    return true;
}

bool conversation_snapshot_bytes(const ConversationView& view, const SessionState& ss, const ModelGeometry& g,
                                 const QsaState& draft, size_t& bytes, std::string& error) {
    return conversation_snapshot_bytes(view, ss, ConversationStageSet{}, g, draft, bytes, error);
}

bool conversation_snapshot_capture_bytes(const ConversationKvReuse& reuse, const ConversationView& view,
                                         const SessionState& ss, const ConversationStageSet& stages,
                                         const ModelGeometry& g, const QsaState& draft, size_t& bytes,
                                         std::string& error) {
    if (!conversation_snapshot_bytes(view, ss, stages, g, draft, bytes, error)) return false;
    if (reuse.kv.empty()) return true;
    // Retained pages are the single-GPU optimization: exactly the main session's layers plus the draft.
    const size_t layers = owned_qsa(ss) + 1;
    if (reuse.kv.size() != layers || reuse.unchanged_tokens < 0 || reuse.unchanged_tokens > reuse.captured_tokens ||
        reuse.unchanged_tokens > int64_t(view.ids.size()))
        return fail(error, "invalid retained K/V prefix");
    for (size_t i = 0; i < layers; ++i) {
        const bool index = i + 1 != layers;
        const QsaState& st = index ? owned(ss, i) : draft;
        if (!conversation_kv_validate(reuse.kv[i], st, g, reuse.captured_tokens, index, error)) return false;
        const size_t fresh = conversation_kv_bytes(st, g, int64_t(view.ids.size()), index);
        size_t retained = 0;
        if (!conversation_kv_capture_bytes(reuse.kv[i], st, g, int64_t(view.ids.size()), index, retained, error))
            return false;
        bytes -= fresh;
        if (!checked_add(bytes, retained)) return fail(error, "retained K/V allocation overflow");
    }
    size_t directory = 0;
    if (!checked_product(directory, {reuse.kv.capacity() - layers, sizeof(ConversationKv)}) ||
        !checked_add(bytes, directory))
        return fail(error, "retained K/V directory overflow");
    return true;
}

bool conversation_snapshot_capture_bytes(const ConversationKvReuse& reuse, const ConversationView& view,
                                         const SessionState& ss, const ModelGeometry& g, const QsaState& draft,
                                         size_t& bytes, std::string& error) {
    return conversation_snapshot_capture_bytes(reuse, view, ss, ConversationStageSet{}, g, draft, bytes, error);
}

bool conversation_snapshot_save(SavedConversation& image, const ConversationView& view, const SessionState& ss,
                                const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                std::string& error, ConversationKvReuse reuse, size_t* reused_bytes) {
    size_t estimate = 0;
    if (!conversation_snapshot_capture_bytes(reuse, view, ss, stages, g, draft, estimate, error)) return false;
    SavedConversation captured;   // built aside, so a failure publishes nothing
    captured.geometry = geometry_key(g);
    captured.layer_lo = ss.layer_lo;
    captured.layer_hi = ss.layer_hi;
    captured.live.ids = view.ids;
    captured.live.imgs = view.images;
    captured.cvec = view.cvec;
    captured.checkpoints = view.checkpoints;
    const int64_t unchanged = reuse.kv.empty() ? 0 : reuse.unchanged_tokens;
    captured.kv = std::move(reuse.kv);
    const size_t layers = owned_qsa(ss);
    captured.kv.resize(layers + 1);
    const int64_t upto = int64_t(view.ids.size());
    auto failed = [&] { drain(); return false; };
    {
        const detail::OnDevice on(stages.main_device);
        if (!sync(error) || !checkpoint_save_enqueue(captured.live, ss, g, error)) return failed();
        for (size_t j = 0; j < layers; ++j)
            if (!detail::kv_save_enqueue(captured.kv[j], owned(ss, j), g, upto, true, error, unchanged, reused_bytes))
                return failed();
        if (!wait(error)) return false;
    }
    {
        // The draft's last cell may not have been computed when the output cap was reached: its partial page is
        // always captured again (one token earlier than the main layers' unchanged prefix).
        const detail::OnDevice on(stages.empty() ? -1 : stages.draft_device);
        if (!stages.empty() && !sync(error)) return false;
        if (!detail::kv_save_enqueue(captured.kv.back(), draft, g, upto, false, error,
                                     std::max<int64_t>(0, unchanged - 1), reused_bytes) ||
            !wait(error))
            return failed();
    }
    captured.stage_parts.resize(size_t(stage_count(stages)));
    for (int64_t i = 0; i < stage_count(stages); ++i) {
        const ConversationStage& stage = stages.stages[i];
        const SessionState& stage_ss = *stage.session;
        ConversationStageSnapshot& part = captured.stage_parts[size_t(i)];
        part.layer_lo = stage_ss.layer_lo;
        part.layer_hi = stage_ss.layer_hi;
        part.state.ids = view.ids;
        part.kv.resize(owned_qsa(stage_ss));
        const detail::OnDevice on(stage.device);
        if (!sync(error) || !checkpoint_save_enqueue(part.state, stage_ss, g, error)) return failed();
        for (size_t j = 0; j < part.kv.size(); ++j)
            if (!detail::kv_save_enqueue(part.kv[j], owned(stage_ss, j), g, upto, true, error, 0, nullptr))
                return failed();
        if (!wait(error)) return false;
    }
    image = std::move(captured);
    return true;
}

bool conversation_snapshot_save(SavedConversation& image, const ConversationView& view, const SessionState& ss,
                                const ModelGeometry& g, const QsaState& draft, std::string& error,
                                ConversationKvReuse reuse, size_t* reused_bytes) {
    return conversation_snapshot_save(image, view, ss, ConversationStageSet{}, g, draft, error, std::move(reuse),
                                      reused_bytes);
}

bool conversation_snapshot_validate(const SavedConversation& image, const SessionState& ss,
                                    const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                    std::string& error) {
    if (!stage_set_validate(stages, ss, g, error)) return false;
    if (!image.live.stage_parts.empty()) return fail(error, "layer-split parking is not supported");
    if (int64_t(image.stage_parts.size()) != stage_count(stages))
        return fail(error, stages.empty() ? "layer-split parking is not supported"
                                          : "snapshot is missing a layer-split stage part");
    if (image.geometry != geometry_key(g)) return fail(error, "incompatible runtime geometry");
    if (image.layer_lo != ss.layer_lo || image.layer_hi != ss.layer_hi)
        return fail(error, "snapshot from another session layer range");
    const ConversationView view{image.live.ids, image.live.imgs, image.checkpoints, image.cvec};
    if (!view_validate(view, ss, stages, g, error) || !conversation_checkpoint_validate(image.live, ss, g, error))
        return false;
    const size_t layers = owned_qsa(ss);
    if (image.kv.size() != layers + 1) return fail(error, "invalid K/V layer count");
    const int64_t upto = int64_t(image.live.ids.size());
    for (size_t j = 0; j < layers; ++j)
        if (!conversation_kv_validate(image.kv[j], owned(ss, j), g, upto, true, error)) return false;
    if (!conversation_kv_validate(image.kv.back(), draft, g, upto, false, error)) return false;
    for (size_t i = 0; i < image.stage_parts.size(); ++i) {
        const ConversationStageSnapshot& part = image.stage_parts[i];
        const SessionState& stage_ss = *stages.stages[i].session;
        if (part.layer_lo != stage_ss.layer_lo || part.layer_hi != stage_ss.layer_hi)
            return fail(error, "layer-split stage part from another session layer range");
        if (!part.state.imgs.empty() || !part.state.stage_parts.empty() || part.state.ids.size() != image.live.ids.size() ||
            !std::equal(part.state.ids.begin(), part.state.ids.end(), image.live.ids.begin()))
            return fail(error, "layer-split stage part is not a live token prefix");
        if (!conversation_checkpoint_validate(part.state, stage_ss, g, error)) return false;
        if (part.kv.size() != owned_qsa(stage_ss)) return fail(error, "invalid layer-split stage K/V layer count");
        for (size_t j = 0; j < part.kv.size(); ++j)
            if (!conversation_kv_validate(part.kv[j], owned(stage_ss, j), g, upto, true, error)) return false;
    }
    return true;
}

bool conversation_snapshot_validate(const SavedConversation& image, const SessionState& ss, const ModelGeometry& g,
                                    const QsaState& draft, std::string& error) {
    return conversation_snapshot_validate(image, ss, ConversationStageSet{}, g, draft, error);
}

ConversationRestore conversation_snapshot_restore(const SavedConversation& image, SessionState& ss,
                                                  const ConversationStageSet& stages, const ModelGeometry& g,
                                                  const QsaState& draft, std::string& error) {
    // Nothing is written until the whole image - main session, draft, every stage - has validated.
    if (!conversation_snapshot_validate(image, ss, stages, g, draft, error)) return ConversationRestore::invalid;
    const int64_t upto = int64_t(image.live.ids.size());
    auto failed = [&] { drain(); return ConversationRestore::transfer_failed; };
    {
        const detail::OnDevice on(stages.main_device);
        if (!sync(error)) return ConversationRestore::transfer_failed;
        for (size_t j = 0; j < owned_qsa(ss); ++j)
            if (!detail::kv_restore_enqueue(image.kv[j], owned(ss, j), g, upto, true, error)) return failed();
        if (!wait(error)) return ConversationRestore::transfer_failed;
    }
    {
        const detail::OnDevice on(stages.empty() ? -1 : stages.draft_device);
        if (!detail::kv_restore_enqueue(image.kv.back(), draft, g, upto, false, error) || !wait(error)) return failed();
    }
    {
        const detail::OnDevice on(stages.main_device);
        if (!conversation_checkpoint_restore(image.live, ss, g, error)) return ConversationRestore::transfer_failed;
    }
    for (size_t i = 0; i < image.stage_parts.size(); ++i) {
        const ConversationStage& stage = stages.stages[i];
        const ConversationStageSnapshot& part = image.stage_parts[i];
        const detail::OnDevice on(stage.device);
        for (size_t j = 0; j < part.kv.size(); ++j)
            if (!detail::kv_restore_enqueue(part.kv[j], owned(*stage.session, j), g, upto, true, error)) return failed();
        if (!wait(error) || !conversation_checkpoint_restore(part.state, *stage.session, g, error))
            return ConversationRestore::transfer_failed;
    }
    return ConversationRestore::restored;
}

ConversationRestore conversation_snapshot_restore(const SavedConversation& image, SessionState& ss,
                                                  const ModelGeometry& g, const QsaState& draft, std::string& error) {
    return conversation_snapshot_restore(image, ss, ConversationStageSet{}, g, draft, error);
}

}  // namespace strata::core
