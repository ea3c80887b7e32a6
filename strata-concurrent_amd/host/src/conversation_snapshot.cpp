// conversation_snapshot.cpp - park and mount of a conversation: the engine interface of
// include/strata/core/conversation_snapshot.hpp (the reference's include/strata/core/conversation_snapshot.hpp:9-141),
// built from snapshot_spec's descriptors and run as snapshot_transfer batches.
//
// Every call first describes everything it will move - which refuses an invalid request before anything is written -
// and then runs the transfer, one batch per device scope.  Whole-conversation calls synchronize the device before a
// capture and after a restore, the engine's contract (conversation_snapshot.hpp:11); per-layer and per-checkpoint
// calls wait for their own copies only.  A failure after the first write of a restore is `transfer_failed`.
#include "strata/core/conversation_snapshot.hpp"

#include "snapshot_spec.hpp"
#include "snapshot_transfer.hpp"

#include <algorithm>

namespace strata::core {
namespace {

using spec::refuse;

// ---- one layer's K/V ----------------------------------------------------------------------------------------------------

// Stamps and sizes `image` for layer spec `s` and adds the copies of everything not retained: whole pages before the
// first of `unchanged_tokens` rewritten tokens stay as an earlier capture of this conversation left them.
bool plan_layer_capture(ConversationKv& image, const spec::LayerSpec& s, const ModelGeometry& g, int64_t tokens,
                        int64_t unchanged_tokens, size_t* reused_bytes, xfer::CaptureBatch& batch, std::string& error) {
    if (unchanged_tokens < 0 || unchanged_tokens > tokens || unchanged_tokens > image.cells)
        return refuse(error, "invalid unchanged prefix");
    const auto held = spec::buffers_of(image);
    std::array<size_t, spec::kBufs> kept{};
    for (size_t b = 0; b < spec::kBufs; ++b) {
        kept[b] = s.unchanged_bytes(int(b), unchanged_tokens);
        if (kept[b] > held[b]->size()) return refuse(error, "missing reusable prefix");
    }
    spec::stamp(image, s, g);
    for (size_t b = 0; b < spec::kBufs; ++b) {
        held[b]->resize(s.bytes[b]);
        batch.legs.push_back({s.state[b], held[b], nullptr, s.bytes[b], kept[b], xfer::Kind::kv});
        if (reused_bytes) *reused_bytes += kept[b];
    }
    return true;
}

void plan_layer_restore(const ConversationKv& image, const spec::LayerSpec& s, const QsaState& st,
                        const ModelGeometry& g, int64_t tokens, xfer::RestoreBatch& batch) {
    const auto held = spec::buffers_of(image);
    for (size_t b = 0; b < spec::kBufs; ++b)
        batch.legs.push_back({s.state[b], held[b], nullptr, s.bytes[b], 0, xfer::Kind::kv});
    if (st.kv_mode != 0) batch.residency.push_back({&st, tokens, image.page_size, g.n_head_kv, g.head_dim});
}

bool layer_capture(ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t tokens, bool index,
                   int64_t unchanged_tokens, size_t* reused_bytes, xfer::CaptureBatch& batch, std::string& error) {
    spec::LayerSpec s;
    return spec::describe_layer(st, g, tokens, index, s, error) &&
           plan_layer_capture(image, s, g, tokens, unchanged_tokens, reused_bytes, batch, error);
}

// ---- running state --------------------------------------------------------------------------------------------------------

// The running state of a session against a checkpoint: the GDN rows, the PLE history and, per owned QSA layer, the
// indexer's tail rows, spare key and block position (src/core/conversation_state.cpp:228-251).
void plan_running_capture(ConversationCheckpoint& c, const SessionState& ss, const ConversationStateSizes& z,
                          xfer::CaptureBatch& batch) {
    const size_t layers = spec::owned_layers(ss);
    c.gdn.resize(z.gdn);
    c.ple.resize(ss.ple_hist ? z.ple : 0);
    c.tails.resize(layers * z.tail);
    c.dead.resize(layers * z.dead);
    c.block_pos.resize(layers * z.block_pos);
    auto leg = [&](void* state, std::vector<uint8_t>& held, size_t at, size_t n) {
        batch.legs.push_back({static_cast<uint8_t*>(state), nullptr, held.data() + at, n, 0, xfer::Kind::running});
    };
    leg(ss.gdn_state, c.gdn, 0, c.gdn.size());
    leg(ss.ple_hist, c.ple, 0, c.ple.size());
    for (size_t j = 0; j < layers; ++j) {
        const QsaState& st = spec::owned_layer(ss, j);
        leg(st.idx_tail, c.tails, j * z.tail, z.tail);
        leg(st.idx_dead, c.dead, j * z.dead, z.dead);
        leg(st.idx_block_pos, c.block_pos, j * z.block_pos, z.block_pos);
    }
}

void plan_running_restore(const ConversationCheckpoint& c, const SessionState& ss, const ConversationStateSizes& z,
                          const ModelGeometry& g, xfer::RestoreBatch& batch) {
    const size_t layers = spec::owned_layers(ss);
    auto leg = [&](void* state, const std::vector<uint8_t>& held, size_t at, size_t n) {
        batch.legs.push_back({static_cast<uint8_t*>(state), nullptr, held.data() + at, n, 0, xfer::Kind::running});
    };
    leg(ss.gdn_state, c.gdn, 0, c.gdn.size());
    leg(ss.ple_hist, c.ple, 0, c.ple.size());
    for (size_t j = 0; j < layers; ++j) {
        const QsaState& st = spec::owned_layer(ss, j);
        leg(st.idx_tail, c.tails, j * z.tail, z.tail);
        leg(st.idx_dead, c.dead, j * z.dead, z.dead);
        leg(st.idx_block_pos, c.block_pos, j * z.block_pos, z.block_pos);
    }
    if (c.ids.empty()) return;
    // The indexer's moving spare row is a copy of its spare key; the restored conversation's spare row sits at the
    // checkpoint's block, which may be earlier than where the outgoing conversation had it.
    const size_t spare_row = c.ids.size() / size_t(strata::kernels::qsa_granules().idx_block);
    for (size_t j = 0; j < layers; ++j) {
        const QsaState& st = spec::owned_layer(ss, j);
        leg(st.idx_pooled + spare_row * size_t(g.idx_key_dim), c.dead, j * z.dead, z.dead);
    }
}

// The token window the PLE history continues from (src/core/conversation_state.cpp:259-262).
void set_ple_window(SessionState& ss, const std::vector<int32_t>& ids) {
    const size_t n = ids.size();
    ss.ple_prev[0] = n >= 2 ? ids[n - 2] : -1;
    ss.ple_prev[1] = n >= 1 ? ids[n - 1] : -1;
}

// ---- a whole snapshot ---------------------------------------------------------------------------------------------------

bool stage_part_consistent(const ConversationStageSnapshot& part, const SessionState& stage, const SavedConversation& image,
                           const ModelGeometry& g, std::string& error) {
    if (part.layer_lo != stage.layer_lo || part.layer_hi != stage.layer_hi)
        return refuse(error, "layer-split stage part from another session layer range");
    const auto& ids = part.state.ids;
    if (!part.state.imgs.empty() || !part.state.stage_parts.empty() || ids != image.live.ids)
        return refuse(error, "layer-split stage part is not a live token prefix");
    if (!conversation_checkpoint_validate(part.state, stage, g, error)) return false;
    if (part.kv.size() != spec::owned_layers(stage)) return refuse(error, "invalid layer-split stage K/V layer count");
    const int64_t tokens = int64_t(image.live.ids.size());
    for (size_t j = 0; j < part.kv.size(); ++j)
        if (!conversation_kv_validate(part.kv[j], spec::owned_layer(stage, j), g, tokens, true, error)) return false;
    return true;
}

}  // namespace

// ---- one layer --------------------------------------------------------------------------------------------------------------

bool conversation_kv_capture_bytes(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                                   bool include_index, size_t& bytes, std::string& error) {
    spec::LayerSpec s;
    if (!spec::describe_layer(st, g, upto, include_index, s, error)) return false;
    const auto held = spec::buffers_of(image);
    bytes = 0;
    for (size_t b = 0; b < spec::kBufs; ++b) {
        const size_t peak = held[b]->allocation_peak(s.bytes[b]);
        if (peak == SIZE_MAX || !spec::add(bytes, peak)) return refuse(error, "segmented K/V allocation overflow");
    }
    return true;
}

size_t conversation_kv_bytes(const QsaState& st, const ModelGeometry& g, int64_t upto, bool include_index) {
    size_t bytes = 0;
    std::string ignored;
    return conversation_kv_capture_bytes(ConversationKv{}, st, g, upto, include_index, bytes, ignored) ? bytes : 0;
}

bool conversation_kv_save(ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                          bool include_index, std::string& error, int64_t unchanged_tokens, size_t* reused_bytes) {
    std::vector<xfer::CaptureBatch> plan(1);
    return layer_capture(image, st, g, upto, include_index, unchanged_tokens, reused_bytes, plan[0], error) &&
           xfer::run(plan, error);
}

bool conversation_kv_validate(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                              bool include_index, std::string& error) {
    spec::LayerSpec s;
    return spec::describe_layer(st, g, upto, include_index, s, error) && spec::image_matches(image, s, g, error);
}

bool conversation_kv_restore(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                             bool include_index, std::string& error) {
    spec::LayerSpec s;
    if (!spec::describe_layer(st, g, upto, include_index, s, error) || !spec::image_matches(image, s, g, error))
        return false;
    std::vector<xfer::RestoreBatch> plan(1);
    plan_layer_restore(image, s, st, g, upto, plan[0]);
    return xfer::run(plan, error);
}

bool conversation_kv_verify(const ConversationKv& image, const QsaState& st, const ModelGeometry& g, int64_t upto,
                            bool include_index, uint64_t& fingerprint, std::string& error) {
    spec::LayerSpec s;
    if (!spec::describe_layer(st, g, upto, include_index, s, error) || !spec::image_matches(image, s, g, error))
        return false;
    uint64_t fnv = 1469598103934665603ull;   // the engine's FNV-1a seed (src/core/conversation_snapshot.cpp:225)
    const auto held = spec::buffers_of(image);
    for (size_t b = 0; b < spec::kBufs; ++b)
        if (!xfer::read_back_equal(s.state[b], *held[b], 0, held[b]->size(), &fnv, error)) return false;
    if (st.kv_mode == 2 && image.cells > 0) {
        // a ring's resident window must hold the image's last n_slots pages, page p in slot p % n_slots
        const int64_t end = image.cells / image.page_size, begin = std::max<int64_t>(0, end - st.n_slots);
        for (size_t b = 0; b < 4; ++b) {
            if (held[b]->empty()) continue;
            const size_t page_bytes = held[b]->size() / size_t(end);
            for (int64_t page = begin; page < end; ++page)
                if (!xfer::read_back_equal(s.resident[b] + size_t(page % st.n_slots) * page_bytes, *held[b],
                                           size_t(page) * page_bytes, page_bytes, nullptr, error))
                    return false;
        }
    }
    fingerprint = fnv;
    return true;
}

// ---- running state ------------------------------------------------------------------------------------------------------

bool conversation_checkpoint_validate(const ConversationCheckpoint& c, const SessionState& ss, const ModelGeometry& g,
                                      std::string& error) {
    ConversationStateSizes z;
    if (!spec::running_state_targets(ss, g, c.ids.size(), z, error)) return false;
    const size_t layers = spec::owned_layers(ss);
    const bool sized = c.gdn.size() == z.gdn && c.ple.size() == (ss.ple_hist ? z.ple : 0) &&
                       c.tails.size() == layers * z.tail && c.dead.size() == layers * z.dead &&
                       c.block_pos.size() == layers * z.block_pos;
    if (!sized || !spec::image_keys_ordered(c.imgs, c.ids.size()))
        return refuse(error, "invalid checkpoint running-state payload");
    return true;
}

bool conversation_checkpoint_save(ConversationCheckpoint& c, const SessionState& ss, const ModelGeometry& g,
                                  std::string& error) {
    ConversationStateSizes z;
    if (!spec::running_state_targets(ss, g, c.ids.size(), z, error)) return false;
    std::vector<xfer::CaptureBatch> plan(1);
    plan_running_capture(c, ss, z, plan[0]);
    return xfer::run(plan, error);
}

bool conversation_checkpoint_restore(const ConversationCheckpoint& c, SessionState& ss, const ModelGeometry& g,
                                     std::string& error) {
    ConversationStateSizes z;
    if (!conversation_checkpoint_validate(c, ss, g, error) || !conversation_session_sizes(g, ss, z, error)) return false;
    std::vector<xfer::RestoreBatch> plan(1);
    plan[0].sync_after = true;
    plan_running_restore(c, ss, z, g, plan[0]);
    if (!xfer::run(plan, error)) return false;
    set_ple_window(ss, c.ids);
    return true;
}

// ---- a whole snapshot ---------------------------------------------------------------------------------------------------

bool conversation_snapshot_bytes(const ConversationView& view, const SessionState& ss,
                                 const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                 size_t& bytes, std::string& error) {
    bytes = 0;
    return spec::stages_tile_model(stages, ss, g, error) && spec::view_consistent(view, ss, stages, g, error) &&
           spec::snapshot_estimate(view, ss, stages, g, draft, bytes, error);
}

bool conversation_snapshot_capture_bytes(const ConversationKvReuse& reuse, const ConversationView& view,
                                         const SessionState& ss, const ConversationStageSet& stages,
                                         const ModelGeometry& g, const QsaState& draft, size_t& bytes,
                                         std::string& error) {
    if (!conversation_snapshot_bytes(view, ss, stages, g, draft, bytes, error)) return false;
    if (reuse.kv.empty()) return true;
    // Retained pages serve the single-GPU capture: exactly the main session's layers, then the draft.
    const size_t layers = spec::owned_layers(ss) + 1;
    const int64_t tokens = int64_t(view.ids.size());
    if (reuse.kv.size() != layers || reuse.unchanged_tokens < 0 || reuse.unchanged_tokens > reuse.captured_tokens ||
        reuse.unchanged_tokens > tokens)
        return refuse(error, "invalid retained K/V prefix");
    for (size_t j = 0; j < layers; ++j) {
        const bool is_draft = j + 1 == layers;
        const QsaState& st = is_draft ? draft : spec::owned_layer(ss, j);
        if (!conversation_kv_validate(reuse.kv[j], st, g, reuse.captured_tokens, !is_draft, error)) return false;
        // the retained buffers grow in place: admit their peak instead of a fresh capture's
        size_t retained = 0;
        if (!conversation_kv_capture_bytes(reuse.kv[j], st, g, tokens, !is_draft, retained, error)) return false;
        bytes -= conversation_kv_bytes(st, g, tokens, !is_draft);
        if (!spec::add(bytes, retained)) return refuse(error, "retained K/V allocation overflow");
    }
    size_t spare = 0;
    if (!spec::mul(spare, {reuse.kv.capacity() - layers, sizeof(ConversationKv)}) || !spec::add(bytes, spare))
        return refuse(error, "retained K/V directory overflow");
    return true;
}

bool conversation_snapshot_save(SavedConversation& image, const ConversationView& view, const SessionState& ss,
                                const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                std::string& error, ConversationKvReuse reuse, size_t* reused_bytes) {
    size_t admitted = 0;
    if (!conversation_snapshot_capture_bytes(reuse, view, ss, stages, g, draft, admitted, error)) return false;
    const int64_t tokens = int64_t(view.ids.size());
    const int64_t unchanged = reuse.kv.empty() ? 0 : reuse.unchanged_tokens;
    const size_t layers = spec::owned_layers(ss);
    const int64_t n_stages = spec::stage_count(stages);

    SavedConversation out;   // built aside: a failure publishes nothing
    out.geometry = spec::geometry_key(g);
    out.layer_lo = ss.layer_lo;
    out.layer_hi = ss.layer_hi;
    out.live.ids = view.ids;
    out.live.imgs = view.images;
    out.cvec = view.cvec;
    out.checkpoints = view.checkpoints;
    out.kv = std::move(reuse.kv);
    out.kv.resize(layers + 1);
    out.stage_parts.resize(size_t(n_stages));

    std::vector<xfer::CaptureBatch> plan(2 + size_t(n_stages));
    ConversationStateSizes z;
    // the main session: its running state, then its layers
    xfer::CaptureBatch& main = plan[0];
    main.device = stages.main_device;
    main.sync_before = true;
    if (!spec::running_state_targets(ss, g, size_t(tokens), z, error)) return false;
    plan_running_capture(out.live, ss, z, main);
    for (size_t j = 0; j < layers; ++j)
        if (!layer_capture(out.kv[j], spec::owned_layer(ss, j), g, tokens, true, unchanged, reused_bytes, main, error))
            return false;
    // the draft: its last cell may not have been computed when the output cap was reached, so its partial page is
    // always taken again (its unchanged prefix is one token shorter than the main layers')
    xfer::CaptureBatch& dr = plan[1];
    dr.device = stages.empty() ? -1 : stages.draft_device;
    dr.sync_before = !stages.empty();
    if (!layer_capture(out.kv.back(), draft, g, tokens, false, std::max<int64_t>(0, unchanged - 1), reused_bytes, dr,
                       error))
        return false;
    // each later stage of a layer split: its running state and its layers, on its own device
    for (int64_t i = 0; i < n_stages; ++i) {
        const ConversationStage& stage = stages.stages[i];
        const SessionState& part_ss = *stage.session;
        ConversationStageSnapshot& part = out.stage_parts[size_t(i)];
        part.layer_lo = part_ss.layer_lo;
        part.layer_hi = part_ss.layer_hi;
        part.state.ids = view.ids;
        part.kv.resize(spec::owned_layers(part_ss));
        xfer::CaptureBatch& b = plan[2 + size_t(i)];
        b.device = stage.device;
        b.sync_before = true;
        ConversationStateSizes pz;
        if (!spec::running_state_targets(part_ss, g, size_t(tokens), pz, error)) return false;
        plan_running_capture(part.state, part_ss, pz, b);
        for (size_t j = 0; j < part.kv.size(); ++j)
            if (!layer_capture(part.kv[j], spec::owned_layer(part_ss, j), g, tokens, true, 0, nullptr, b, error))
                return false;
    }
    if (!xfer::run(plan, error)) return false;
    image = std::move(out);
    return true;
}

bool conversation_snapshot_validate(const SavedConversation& image, const SessionState& ss,
                                    const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                    std::string& error) {
    if (!spec::stages_tile_model(stages, ss, g, error)) return false;
    if (!image.live.stage_parts.empty()) return refuse(error, "layer-split parking is not supported");
    if (int64_t(image.stage_parts.size()) != spec::stage_count(stages))
        return refuse(error, stages.empty() ? "layer-split parking is not supported"
                                            : "snapshot is missing a layer-split stage part");
    if (image.geometry != spec::geometry_key(g)) return refuse(error, "incompatible runtime geometry");
    if (image.layer_lo != ss.layer_lo || image.layer_hi != ss.layer_hi)
        return refuse(error, "snapshot from another session layer range");
    const ConversationView view{image.live.ids, image.live.imgs, image.checkpoints, image.cvec};
    if (!spec::view_consistent(view, ss, stages, g, error) ||
        !conversation_checkpoint_validate(image.live, ss, g, error))
        return false;
    const size_t layers = spec::owned_layers(ss);
    if (image.kv.size() != layers + 1) return refuse(error, "invalid K/V layer count");
    const int64_t tokens = int64_t(image.live.ids.size());
    for (size_t j = 0; j <= layers; ++j) {
        const bool is_draft = j == layers;
        if (!conversation_kv_validate(image.kv[j], is_draft ? draft : spec::owned_layer(ss, j), g, tokens, !is_draft,
                                      error))
            return false;
    }
    for (size_t i = 0; i < image.stage_parts.size(); ++i)
        if (!stage_part_consistent(image.stage_parts[i], *stages.stages[i].session, image, g, error)) return false;
    return true;
}

ConversationRestore conversation_snapshot_restore(const SavedConversation& image, SessionState& ss,
                                                  const ConversationStageSet& stages, const ModelGeometry& g,
                                                  const QsaState& draft, std::string& error) {
    // Nothing is written until the whole image - main session, draft, every stage - has validated.
    if (!conversation_snapshot_validate(image, ss, stages, g, draft, error)) return ConversationRestore::invalid;
    const int64_t tokens = int64_t(image.live.ids.size());
    const size_t layers = spec::owned_layers(ss);
    std::vector<xfer::RestoreBatch> plan(2 + image.stage_parts.size());
    ConversationStateSizes z;
    // the main session's layers and running state, after a device synchronization
    xfer::RestoreBatch& main = plan[0];
    main.device = stages.main_device;
    main.sync_before = true;
    for (size_t j = 0; j < layers; ++j) {
        const QsaState& st = spec::owned_layer(ss, j);
        spec::LayerSpec s;
        if (!spec::describe_layer(st, g, tokens, true, s, error)) return ConversationRestore::invalid;
        plan_layer_restore(image.kv[j], s, st, g, tokens, main);
    }
    if (!conversation_session_sizes(g, ss, z, error)) return ConversationRestore::invalid;
    plan_running_restore(image.live, ss, z, g, main);
    // the draft's layer; the device is synchronized once the main session's and the draft's bytes have landed
    xfer::RestoreBatch& dr = plan[1];
    dr.device = stages.empty() ? -1 : stages.draft_device;
    dr.sync_after = true;
    spec::LayerSpec ds;
    if (!spec::describe_layer(draft, g, tokens, false, ds, error)) return ConversationRestore::invalid;
    plan_layer_restore(image.kv.back(), ds, draft, g, tokens, dr);
    for (size_t i = 0; i < image.stage_parts.size(); ++i) {
        const ConversationStage& stage = stages.stages[i];
        const ConversationStageSnapshot& part = image.stage_parts[i];
        xfer::RestoreBatch& b = plan[2 + i];
        b.device = stage.device;
        b.sync_after = true;
        for (size_t j = 0; j < part.kv.size(); ++j) {
            const QsaState& st = spec::owned_layer(*stage.session, j);
            spec::LayerSpec s;
            if (!spec::describe_layer(st, g, tokens, true, s, error)) return ConversationRestore::invalid;
            plan_layer_restore(part.kv[j], s, st, g, tokens, b);
        }
        ConversationStateSizes pz;
        if (!conversation_session_sizes(g, *stage.session, pz, error)) return ConversationRestore::invalid;
        plan_running_restore(part.state, *stage.session, pz, g, b);
    }
    if (!xfer::run(plan, error)) return ConversationRestore::transfer_failed;
    set_ple_window(ss, image.live.ids);
    for (size_t i = 0; i < image.stage_parts.size(); ++i) set_ple_window(*stages.stages[i].session, image.live.ids);
    return ConversationRestore::restored;
}

// ---- the single-GPU forms: an empty stage set --------------------------------------------------------------------------

bool conversation_snapshot_bytes(const ConversationView& view, const SessionState& ss, const ModelGeometry& g,
                                 const QsaState& draft, size_t& bytes, std::string& error) {
    return conversation_snapshot_bytes(view, ss, ConversationStageSet{}, g, draft, bytes, error);
}

bool conversation_snapshot_capture_bytes(const ConversationKvReuse& reuse, const ConversationView& view,
                                         const SessionState& ss, const ModelGeometry& g, const QsaState& draft,
                                         size_t& bytes, std::string& error) {
    return conversation_snapshot_capture_bytes(reuse, view, ss, ConversationStageSet{}, g, draft, bytes, error);
}

bool conversation_snapshot_save(SavedConversation& image, const ConversationView& view, const SessionState& ss,
                                const ModelGeometry& g, const QsaState& draft, std::string& error,
                                ConversationKvReuse reuse, size_t* reused_bytes) {
    return conversation_snapshot_save(image, view, ss, ConversationStageSet{}, g, draft, error, std::move(reuse),
                                      reused_bytes);
}

bool conversation_snapshot_validate(const SavedConversation& image, const SessionState& ss, const ModelGeometry& g,
                                    const QsaState& draft, std::string& error) {
    return conversation_snapshot_validate(image, ss, ConversationStageSet{}, g, draft, error);
}

ConversationRestore conversation_snapshot_restore(const SavedConversation& image, SessionState& ss,
                                                  const ModelGeometry& g, const QsaState& draft, std::string& error) {
    return conversation_snapshot_restore(image, ss, ConversationStageSet{}, g, draft, error);
}

}  // namespace strata::core
