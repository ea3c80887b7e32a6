// wire_internal.hpp - the codec's pieces the device payload path (conversation_wire_device.cpp) builds on.
#pragma once

#include "strata/core/conversation_wire.hpp"

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace strata::core::detail {

/// One pool entry of a payload: which buffer of the image (the address of its ConversationBuffer or vector), its
/// absolute offset in the payload and its size.
struct WireBlobAt {
    const void* who = nullptr;
    uint64_t offset = 0;
    uint64_t bytes = 0;
};

/// Buffers of an image laid out at a stated size whatever they hold: their bytes live elsewhere (on the device).
using WireSizes = std::vector<std::pair<const void*, uint64_t>>;

/// The bytes of a payload before its blob pool (header, records, zero pad) and where every pool entry goes.
bool wire_head(const SavedConversation& image, const WireIdentity& identity, const WireSizes& sizes,
               std::vector<uint8_t>& head, std::vector<WireBlobAt>& pool, WirePlan& plan, std::string& error);

/// Parses a payload's head (bytes [0, blob_pool_off) suffice) with every check of conversation_wire_decode except the
/// payload hash; the image's buffers stay empty and `blobs` says where each one lies in the payload (by the address of
/// the buffer inside `image`, which is built in place: on a refusal it holds a partial parse and must be discarded).
bool wire_locate(const uint8_t* head, uint64_t head_bytes, SavedConversation& image, WireDecoded& info,
                 const WireExpect& expect, std::vector<WireBlobAt>& blobs, std::string& error);

}  // namespace strata::core::detail
