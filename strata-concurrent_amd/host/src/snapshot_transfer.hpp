// snapshot_transfer.hpp - moving the byte ranges snapshot_spec describes, between a session and an image.
//
// A transfer is a list of batches, one per device scope (the main session, the draft, each later stage of a layer
// split).  A batch is a list of legs - one contiguous range of session state and where it sits in the image: a
// segmented ConversationBuffer (K/V) or flat running-state bytes - plus the residency work a restored layer needs.
// Each batch is checked whole before its first copy, enqueued on this thread's transfer stream (one hipMemcpyAsync per
// leg and image segment; pinned segments make them DMAs) and waited for once.
#pragma once

#include "snapshot_spec.hpp"

#include <vector>

namespace strata::core::xfer {

/// Which refusal and copy-failure messages a leg carries: the engine names K/V and running-state copies apart.
enum class Kind : uint8_t { kv, running };

template <class Buffer, class Bytes>
struct BasicLeg {
    uint8_t* state = nullptr;     // session side: device memory, or a streamed layer's authoritative host copy
    Buffer* segmented = nullptr;  // image side: a K/V buffer ...
    Bytes* flat = nullptr;        // ... or running-state bytes
    size_t bytes = 0;
    size_t from = 0;              // a capture leaves [0, from) of the image as it is (retained from an earlier image)
    Kind kind = Kind::kv;
};
using CaptureLeg = BasicLeg<ConversationBuffer, uint8_t>;        // state -> image
using RestoreLeg = BasicLeg<const ConversationBuffer, const uint8_t>;   // image -> state

/// After a layer's restore copies, on the same stream: a streamed layer's VRAM slots still hold the outgoing
/// conversation and are all evicted; a ring refills its window from the restored host copy.
struct Residency {
    const QsaState* layer = nullptr;
    int64_t tokens = 0, page_size = 0, n_head_kv = 0, head_dim = 0;
};

template <class Leg>
struct Batch {
    int device = -1;            // made current for the batch (-1 leaves the current device)
    bool sync_before = false;   // synchronize the device before the first copy (the engine's sync before a save)
    bool sync_after = false;    // synchronize the device after the last copy (the engine's sync after a restore)
    std::vector<Leg> legs;
    std::vector<Residency> residency;
};
using CaptureBatch = Batch<CaptureLeg>;
using RestoreBatch = Batch<RestoreLeg>;

/// Runs the batches in order.  Refusals (an absent endpoint) come before any copy of their batch; a copy or
/// synchronization failure returns false with the runtime's reason and leaves nothing in flight.
bool run(const std::vector<CaptureBatch>& batches, std::string& error);
bool run(const std::vector<RestoreBatch>& batches, std::string& error);

/// Reads `bytes` of session state at `state` back in 64 KiB pieces and compares them with `held` from `offset`;
/// each piece read is folded into `*fnv` when it is given.  False with "restored K/V bytes differ" on a difference.
bool read_back_equal(const uint8_t* state, const ConversationBuffer& held, size_t offset, size_t bytes, uint64_t* fnv,
                     std::string& error);

}  // namespace strata::core::xfer
