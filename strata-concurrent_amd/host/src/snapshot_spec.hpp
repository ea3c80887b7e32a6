// snapshot_spec.hpp - what a conversation image holds, written down as data.
//
// A parked conversation is a set of byte ranges of session state.  This header describes them: the five buffers of
// one QSA layer's K/V image (LayerSpec, with a per-format table saying which pool holds each buffer and how many
// bytes a cell of it takes), the running state of a session (the parts of a ConversationCheckpoint), and the checks
// that refuse a request before anything is written.  The public functions (conversation_snapshot.cpp) assemble these
// descriptors into transfer batches (snapshot_transfer.hpp) and run them; they hold no layout arithmetic of their own.
//
// The refusals and their messages are the engine's contract (include/strata/core/conversation_snapshot.hpp:9-141,
// src/core/conversation_snapshot.cpp:18-103, src/core/conversation_state.cpp:21-214): callers match on them, and the
// reference's own snapshot and validation tests run against this library.
#pragma once

#include "strata/core/conversation_snapshot.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <string>

namespace strata::core::spec {

/// Records `what` as the refusal, with the engine's prefix, and returns false.
bool refuse(std::string& error, const char* what);
/// `total += n` / `out = product`, false on size_t overflow (nothing is assigned then).
bool add(size_t& total, size_t n);
bool mul(size_t& out, std::initializer_list<uint64_t> factors);

// ---- one QSA layer's K/V image --------------------------------------------------------------------------------------

/// The buffers of a layer image, in ConversationKv's member order.
enum Buf : int { kK = 0, kV, kKScale, kVScale, kPooled, kBufs };
/// Image format of K8V4 (int8 K + q4_0 V); the block movers never see it.
inline constexpr int kK8V4 = 3;

struct LayerSpec {
    int format = 0;                            // 0 f16, 1 int8, 2 q4_0, 3 K8V4
    int64_t cells = 0;                         // page-granular extent: ceil(upto / page_size) * page_size
    int64_t pooled_rows = 0;                   // indexer rows: completed blocks plus the moving spare (0 without index)
    int64_t page_size = 0;
    int64_t idx_block = 0;
    size_t idx_row_bytes = 0;                  // one pooled row
    std::array<size_t, kBufs> bytes{};         // image bytes per buffer
    std::array<uint8_t*, kBufs> state{};       // authoritative bytes: the pools, or a streamed/ring layer's host copy
    std::array<uint8_t*, kBufs> resident{};    // the VRAM pools (what a ring's window holds)

    /// Leading bytes of buffer `b` that are unchanged when the first `unchanged_tokens` tokens are: whole pages (and
    /// whole indexer blocks) strictly before the first rewritten token.  The partial page and the moving spare row
    /// always change.
    size_t unchanged_bytes(int b, int64_t unchanged_tokens) const;
};

/// Describes one layer at `upto` tokens; refuses what conversation_kv_save / _validate / _restore refuse before
/// touching an image.
bool describe_layer(const QsaState& st, const ModelGeometry& g, int64_t upto, bool include_index, LayerSpec& out,
                    std::string& error);
/// The image was taken at this spec: same format, extents, geometry and buffer sizes, and every target exists.
bool image_matches(const ConversationKv& image, const LayerSpec& spec, const ModelGeometry& g, std::string& error);
/// Writes the spec's metadata into an image being captured.
void stamp(ConversationKv& image, const LayerSpec& spec, const ModelGeometry& g);
std::array<ConversationBuffer*, kBufs> buffers_of(ConversationKv& image);
std::array<const ConversationBuffer*, kBufs> buffers_of(const ConversationKv& image);

// ---- a session's running state ---------------------------------------------------------------------------------------

/// The image's geometry key: every ModelGeometry field, in declaration order.
std::array<int64_t, 18> geometry_key(const ModelGeometry& g);
/// The QSA layers a session owns (its carve of the global QSA ordinals).
size_t owned_layers(const SessionState& ss);
const QsaState& owned_layer(const SessionState& ss, size_t j);
/// Checks that `ss` can hold (and yield) the running state of `tokens` tokens; `z` gets its per-part sizes.
bool running_state_targets(const SessionState& ss, const ModelGeometry& g, size_t tokens, ConversationStateSizes& z,
                           std::string& error);
/// Strictly increasing image starts, each inside [0, tokens).
bool image_keys_ordered(const std::vector<ConversationImageKey>& images, size_t tokens);

// ---- a snapshot's shape -----------------------------------------------------------------------------------------------

int64_t stage_count(const ConversationStageSet& stages);
/// The main session and the stages tile [0, n_layers) in order.
bool stages_tile_model(const ConversationStageSet& stages, const SessionState& main, const ModelGeometry& g,
                       std::string& error);
/// The live tokens, image keys and retained checkpoints of a view are consistent with the sessions.
bool view_consistent(const ConversationView& view, const SessionState& ss, const ConversationStageSet& stages,
                     const ModelGeometry& g, std::string& error);
/// Host bytes a snapshot of `view` takes (directory entries, running state and every layer's K/V).
bool snapshot_estimate(const ConversationView& view, const SessionState& ss, const ConversationStageSet& stages,
                       const ModelGeometry& g, const QsaState& draft, size_t& bytes, std::string& error);

}  // namespace strata::core::spec
