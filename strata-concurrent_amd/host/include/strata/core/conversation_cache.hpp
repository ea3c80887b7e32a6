// conversation_cache.hpp - the park image types.
//
// The reference's image types (include/strata/core/conversation_cache.hpp:51-162), same members and the same
// byte accounting (`bytes()` is what a RAM budget admits): a checkpoint of running state, one layer's K/V, the
// reusable K/V of an earlier image, one later stage of a layer split, and the whole parked conversation.  The
// LRU park store that holds images (ConversationCache) is scheduling policy and is not part of this library.
#pragma once

#include "strata/core/conversation_buffer.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <vector>

namespace strata::core {

constexpr int64_t kNoOwner = -1;

struct ConversationImageKey {
    int64_t start = 0;
    uint64_t hash = 0;
    bool operator==(const ConversationImageKey& o) const { return start == o.start && hash == o.hash; }
};

/// Running state without K/V: GDN rows, PLE history and the indexer's per-layer tail / spare key / block position.
struct ConversationCheckpoint {
    std::vector<int32_t> ids;
    std::vector<ConversationImageKey> imgs;
    std::vector<uint8_t> gdn, ple, tails, dead, block_pos;
    uint64_t used = 0;
    std::vector<ConversationCheckpoint> stage_parts;   // one per later stage of a layer split

    size_t bytes() const {
        size_t n = ids.capacity() * sizeof(int32_t) + imgs.capacity() * sizeof(ConversationImageKey) +
                   gdn.capacity() + ple.capacity() + tails.capacity() + dead.capacity() + block_pos.capacity() +
                   stage_parts.capacity() * sizeof(ConversationCheckpoint);
        for (const ConversationCheckpoint& part : stage_parts) n += part.bytes();
        return n;
    }
};

/// One QSA layer's K/V: the identity-layout prefix of its pools (k, v, and the int8 scales) plus the indexer's
/// completed pooled rows and its moving spare row.
struct ConversationKv {
    int format = 0;
    int64_t cells = 0, heads = 0, head_dim = 0, page_size = 0, pooled_rows = 0, idx_dim = 0;
    ConversationBuffer k, v, k_scale, v_scale, pooled;
    size_t bytes() const { return k.bytes() + v.bytes() + k_scale.bytes() + v_scale.bytes() + pooled.bytes(); }
};

struct ConversationKvReuse {
    std::vector<ConversationKv> kv;
    int64_t captured_tokens = 0, unchanged_tokens = 0;
    size_t bytes() const {
        size_t n = kv.capacity() * sizeof(ConversationKv);
        for (const ConversationKv& layer : kv) n += layer.bytes();
        return n;
    }
};

struct ConversationStageSnapshot {
    int64_t layer_lo = 0, layer_hi = 0;
    ConversationCheckpoint state;
    std::vector<ConversationKv> kv;
    size_t bytes() const {
        size_t n = state.bytes() + kv.capacity() * sizeof(ConversationKv);
        for (const ConversationKv& k : kv) n += k.bytes();
        return n;
    }
};

struct SavedConversation {
    std::array<int64_t, 18> geometry{};
    int64_t layer_lo = 0, layer_hi = 0;
    ConversationCheckpoint live;
    std::vector<ConversationCheckpoint> checkpoints;
    std::vector<ConversationKv> kv;                      // main layers, then the draft layer
    std::vector<ConversationStageSnapshot> stage_parts;  // empty on one GPU
    bool cvec = true;
    int64_t owner = kNoOwner;

    size_t bytes() const {
        size_t n = live.bytes() + checkpoints.capacity() * sizeof(ConversationCheckpoint) +
                   kv.capacity() * sizeof(ConversationKv) + stage_parts.capacity() * sizeof(ConversationStageSnapshot);
        for (const ConversationCheckpoint& c : checkpoints) n += c.bytes();
        for (const ConversationKv& k : kv) n += k.bytes();
        for (const ConversationStageSnapshot& part : stage_parts) n += part.bytes();
        return n;
    }
};

}  // namespace strata::core
