// conversation_snapshot.hpp - park and mount of a conversation: the engine interface of the handoff.
//
// The reference's API (include/strata/core/conversation_snapshot.hpp:9-141) with the same names, arguments,
// results and error strings, implemented over libsc_handoff.so's C-ABI instead of synchronous per-segment
// cudaMemcpy: every copy of one call is enqueued with hipMemcpyAsync on the library's transfer stream (pinned
// segments make them DMAs) and the call synchronizes once before it returns, so callers see the same synchronous
// contract.  Invalid requests are refused before the first copy or write; a failure after it is
// `transfer_failed` (the session must not be used).
#pragma once

#include "strata/core/conversation_cache.hpp"
#include "strata/core/engine_types.hpp"
#include "strata/kernels/kv_stream.hpp"   // the block movers (the reference reaches them through layer.hpp)

#include <cstdint>
#include <string>
#include <vector>

namespace strata::core {

// The caller synchronizes the device before saving, and after restoring all layers.
// include_index is false for the draft layer (its attention has no indexer).
size_t conversation_kv_bytes(const QsaState& state, const ModelGeometry& g, int64_t upto, bool include_index);
bool conversation_kv_save(ConversationKv& image, const QsaState& state, const ModelGeometry& g, int64_t upto,
                          bool include_index, std::string& error, int64_t unchanged_tokens = 0,
                          size_t* reused_bytes = nullptr);
bool conversation_kv_capture_bytes(const ConversationKv& image, const QsaState& state, const ModelGeometry& g,
                                   int64_t upto, bool include_index, size_t& bytes, std::string& error);
bool conversation_kv_validate(const ConversationKv& image, const QsaState& state, const ModelGeometry& g,
                              int64_t upto, bool include_index, std::string& error);
bool conversation_kv_restore(const ConversationKv& image, const QsaState& state, const ModelGeometry& g,
                             int64_t upto, bool include_index, std::string& error);
bool conversation_kv_verify(const ConversationKv& image, const QsaState& state, const ModelGeometry& g,
                            int64_t upto, bool include_index, uint64_t& fingerprint, std::string& error);

struct ConversationStateSizes {
    size_t gdn = 0, ple = 0, tail = 0, dead = 0, block_pos = 0;
};
bool conversation_state_sizes(const ModelGeometry& g, ConversationStateSizes& sizes, std::string& error);
bool conversation_session_sizes(const ModelGeometry& g, const SessionState& session, ConversationStateSizes& sizes,
                                std::string& error);
bool conversation_checkpoint_validate(const ConversationCheckpoint& checkpoint, const SessionState& session,
                                      const ModelGeometry& g, std::string& error);
bool conversation_checkpoint_save(ConversationCheckpoint& checkpoint, const SessionState& session,
                                  const ModelGeometry& g, std::string& error);
bool conversation_checkpoint_restore(const ConversationCheckpoint& checkpoint, SessionState& session,
                                     const ModelGeometry& g, std::string& error);

struct ConversationView {
    const std::vector<int32_t>& ids;
    const std::vector<ConversationImageKey>& images;
    const std::vector<ConversationCheckpoint>& checkpoints;
    bool cvec;
};

struct ConversationStage {
    SessionState* session = nullptr;
    int device = -1;
};
struct ConversationStageSet {
    const ConversationStage* stages = nullptr;
    int64_t count = 0;
    int main_device = -1;
    int draft_device = -1;
    bool empty() const { return stages == nullptr || count <= 0; }
};

bool conversation_snapshot_bytes(const ConversationView& view, const SessionState& session, const ModelGeometry& g,
                                 const QsaState& draft, size_t& bytes, std::string& error);
bool conversation_snapshot_capture_bytes(const ConversationKvReuse& reuse, const ConversationView& view,
                                         const SessionState& session, const ModelGeometry& g, const QsaState& draft,
                                         size_t& bytes, std::string& error);
bool conversation_snapshot_save(SavedConversation& image, const ConversationView& view, const SessionState& session,
                                const ModelGeometry& g, const QsaState& draft, std::string& error,
                                ConversationKvReuse reuse = {}, size_t* reused_bytes = nullptr);
bool conversation_snapshot_validate(const SavedConversation& image, const SessionState& session,
                                    const ModelGeometry& g, const QsaState& draft, std::string& error);
enum class ConversationRestore { restored, invalid, transfer_failed };
ConversationRestore conversation_snapshot_restore(const SavedConversation& image, SessionState& session,
                                                  const ModelGeometry& g, const QsaState& draft, std::string& error);

// The same five with a layer split (stages tile [layer_hi of the main session, n_layers)); an empty set is
// exactly the single-GPU path.
bool conversation_snapshot_bytes(const ConversationView& view, const SessionState& session,
                                 const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                 size_t& bytes, std::string& error);
bool conversation_snapshot_capture_bytes(const ConversationKvReuse& reuse, const ConversationView& view,
                                         const SessionState& session, const ConversationStageSet& stages,
                                         const ModelGeometry& g, const QsaState& draft, size_t& bytes,
                                         std::string& error);
bool conversation_snapshot_save(SavedConversation& image, const ConversationView& view, const SessionState& session,
                                const ConversationStageSet& stages, const ModelGeometry& g, const QsaState& draft,
                                std::string& error, ConversationKvReuse reuse = {}, size_t* reused_bytes = nullptr);
bool conversation_snapshot_validate(const SavedConversation& image, const SessionState& session,
                                    const ConversationStageSet& stages, const ModelGeometry& g,
                                    const QsaState& draft, std::string& error);
ConversationRestore conversation_snapshot_restore(const SavedConversation& image, SessionState& session,
                                                  const ConversationStageSet& stages, const ModelGeometry& g,
                                                  const QsaState& draft, std::string& error);

}  // namespace strata::core
