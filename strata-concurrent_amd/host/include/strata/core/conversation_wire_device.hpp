// conversation_wire_device.hpp - hand-off payloads written straight from a decode slot, and mounted straight into
// one, in device memory.
//
// The reference builds a payload on the host: the slot is first saved to host buffers (conversation_snapshot_save,
// synchronous per-16-MiB cudaMemcpy), then the codec walks those buffers and hashes every byte on one CPU core
// (src/core/conversation_wire.cpp:400-480), and the receiver hashes the payload again before decoding it
// (src/core/handoff.cpp:1133-1136).  This library keeps the payload format and moves the heavy parts to the GPU:
//
//   encode   the host lays out the head (header, records) with the codec, then on one stream: the head and the few
//            small host blobs are copied in, ONE launch of the move kernel gathers every K/V page and GDN row of the
//            slot into its pool offset (and zeroes the pool's gaps), and the parallel device FNV-1a hashes the whole
//            payload.  The payload is then already what the wire carries: park it with one D2H copy, or hand the
//            device buffer to another process on the same GPU.
//   decode   the head is read back and parsed with every check of conversation_wire_decode; the payload hash is
//            verified on the device; only then does ONE launch scatter the pool into the slot (nothing is written
//            on a refusal), and the small host blobs are copied out into the returned image.
//
// Scope: the slot's QSA layers carry f16 K/V without indexer rows (format 0), the first image K/V records are those
// layers in order, and the live checkpoint's gdn blob is the slot's GDN rows.  Everything else of the image - the
// records that follow (a draft layer), the live checkpoint's ids, keys and small buffers, retained checkpoints - is
// host data carried as is.  A layer-split image carries one stage part per later stage (the reference's
// conversation_snapshot_save, src/core/conversation_state.cpp:397-413): given the stages' own slots, their K/V records
// and GDN rows are gathered from and scattered into those slots by launches of their own, the rest of each part's
// running state travels as host data (f16 slots).  Without stages, a layer-split payload is refused.
#pragma once

#include "strata/core/conversation_wire.hpp"

#include "sc_handoff.h"

#include <array>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace strata::core {

namespace detail {
struct WireBlobAt;   // one pool entry of a payload (the codec's internals)
}

/// The host side of a conversation whose K/V and GDN rows live in a decode slot.
struct WireDeviceConversation {
    std::array<int64_t, 18> geometry{};   // SavedConversation::geometry (the engine's geometry key)
    int64_t layer_lo = 0, layer_hi = 0;
    bool cvec = true;
    int64_t idx_dim = 0;                  // the K/V records' idx_dim (ModelGeometry::idx_key_dim)
    ConversationCheckpoint live;          // ids, keys, used and the small buffers; its gdn must be empty (it is the slot's)
    std::vector<ConversationCheckpoint> checkpoints;
    std::vector<ConversationKv> trailing_kv;   // host K/V records after the slot's layers (the draft layer)
};

/// One later stage of a layer split (ConversationStageSnapshot, include/strata/core/conversation_cache.hpp): its own
/// decode slot, laid out by its own geometry (the QSA layers and GDN rows the stage owns), its layer range, and the host
/// half of its running state: `state.ids` are the live ids, ple / tails / dead / block_pos host bytes, gdn empty (the
/// slot's rows).  A decoder fills `state` of the stages it mounts into.
struct WireDeviceStage {
    sc_geometry geometry{};
    sc_decode_slot slot{};
    int64_t layer_lo = 0, layer_hi = 0;
    ConversationCheckpoint state;
};

class WireDeviceEncoder {
public:
    WireDeviceEncoder() = default;
    ~WireDeviceEncoder();
    WireDeviceEncoder(const WireDeviceEncoder&) = delete;
    WireDeviceEncoder& operator=(const WireDeviceEncoder&) = delete;

    /// Lays out the payload of `conv` carrying the slot's state for `tokens` tokens (== conv.live.ids.size()).
    bool plan(const sc_geometry& g, const sc_decode_slot& slot, int64_t tokens, const WireDeviceConversation& conv,
              const WireIdentity& identity, std::string& error);
    /// The same with a layer split: `slot` holds the main session's layers and each of `stages` a later stage's; the
    /// payload carries one stage part per stage, in order.
    bool plan(const sc_geometry& g, const sc_decode_slot& slot, int64_t tokens, const WireDeviceConversation& conv,
              const std::vector<WireDeviceStage>& stages, const WireIdentity& identity, std::string& error);
    /// The same for a slot in any K/V format (sc_slot_layers: int8, q4_0, K8V4 or f16, with the indexer's pooled rows
    /// when slot.with_index): its layers become K/V records of slot.format whose data, scale and pooled-row blobs are
    /// gathered from the slot's identity pools.
    bool plan(const sc_geometry& g, const sc_slot_layers& slot, int64_t tokens, const WireDeviceConversation& conv,
              const WireIdentity& identity, std::string& error);
    const WirePlan& layout() const { return plan_; }
    uint64_t bytes() const { return plan_.total_bytes; }
    /// Enqueues the whole encode on `stream` into `payload` (16-byte aligned device memory of at least bytes()): the
    /// gather fused with the payload hash (one read of the slot), which also writes the head and the small host blobs
    /// from their device copy (or they are copied in first, for a head that is not whole 16-byte chunks).  When `gathered` (a
    /// hipEvent_t) is given the gather runs on its own first and the event is recorded once every payload byte is in
    /// place and before the hash runs, so a copy of the payload on another stream (a park) can start while the hash
    /// is computed.
    bool encode(void* payload, uint64_t capacity, void* stream, std::string& error, void* gathered = nullptr);
    /// Enqueues the encode into a segmented payload (`into`: the same-GPU hand-off's exported segments, byte o at
    /// into.ptr[o / segment_bytes] + o % segment_bytes, segment_bytes a multiple of 64 KiB): the gather fused with the
    /// hash writing the head, the small blobs and every slot blob into its segments, cut wherever a segment ends.  The payload bytes are exactly encode()'s; nothing is staged in between.
    bool encode_segments(const sc_segments& into, void* stream, std::string& error);
    /// The payload hash of the last encode; waits for it.
    bool payload_hash(uint64_t& hash, std::string& error);
    /// Later encodes also write the payload's carries (sc_fnv1a64_carry_bytes(bytes()) bytes of device memory at
    /// `carry`, e.g. beside an exported payload): the low byte of the running hash after every 64 KiB, which lets a
    /// decoder given them check the hash without the kernel's look-back (WireDeviceDecoder::set_carry).  Null stops it.
    void set_carry(uint8_t* carry) { carry_ = carry; }

private:
    void settle();
    bool mark_launched(void* stream, std::string& error);
    void release();
    bool stage(const SavedConversation& img, const std::vector<std::pair<const void*, uint64_t>>& sizes,
               const std::vector<const void*>& device, const WireIdentity& identity,
               std::vector<detail::WireBlobAt>& pool, std::string& error);
    /// The capture plans of the slot (and of each stage part) writing the pool of a payload at `base`.
    bool capture_plans(void* base, uint64_t capacity, std::vector<sc_plan*>& plans, std::string& error);

    sc_geometry g_{};
    sc_decode_slot slot_{};
    // a later stage's slot (own copies of its pointer arrays) and where its blobs sit in the payload
    struct StagePlan {
        sc_geometry g{};
        sc_decode_slot slot{};
        std::vector<uint16_t*> k, v;
        std::vector<uint64_t> k_off, v_off;
        uint64_t gdn_off = 0;
        sc_plan* plan = nullptr;
    };
    std::vector<StagePlan> stage_plans_;
    bool layered_ = false;                             // an sc_slot_layers slot (lay_off_) rather than f16 pools
    sc_slot_layers layers_{};
    std::array<std::vector<void*>, SC_N_BUF> layer_bufs_;
    std::vector<uint64_t> lay_off_;                    // sc_layers_map offsets of the slot's blobs in the payload
    int64_t tokens_ = 0;
    WirePlan plan_{};
    std::vector<uint64_t> k_off_, v_off_, zero_;
    uint64_t gdn_off_ = 0;
    struct Upload { uint64_t offset, bytes, staged_at; };
    std::vector<Upload> uploads_;      // the head and the small host blobs, staged in pinned memory
    uint8_t* staged_ = nullptr;        // pinned
    uint64_t staged_bytes_ = 0;
    // The same bytes in device memory, copied once at plan time, when every upload is whole 16-byte chunks at a 16-byte
    // offset (staged_rows_): the encode then writes them by copy rows of its gather (copies_, an sc_plan_copies plan
    // built with the capture plans) instead of copying them in from pinned memory before it.
    uint8_t* staged_dev_ = nullptr;
    bool staged_rows_ = false;
    sc_plan* copies_ = nullptr;
    void* hash_ws_ = nullptr;          // device
    uint64_t hash_ws_bytes_ = 0;
    uint64_t* hash_host_ = nullptr;    // pinned (64 B); the hash's last kernel stores the payload hash here
    // and the launch's fault word right after it (1: a wait ran out and the hash is not valid)
    uint32_t* hash_fault_host() { return reinterpret_cast<uint32_t*>(hash_host_ + 1); }
    void* last_stream_ = nullptr;
    void* done_ = nullptr;     // hipEvent_t recorded after each encode's launches; settle() waits on it before the
    bool launched_ = false;    // plans, maps or buffers those launches read are destroyed
    sc_plan* capture_ = nullptr;
    sc_hash_map* hash_map_ = nullptr;  // the capture plans' rows fused with the payload hash (one read of the slot)
    void* capture_target_ = nullptr;   // the payload the capture plan was built for
    sc_hash_map* seg_map_ = nullptr;   // the same into the segments of seg_target_
    std::vector<void*> seg_target_;
    uint64_t seg_bytes_ = 0;
    uint8_t* carry_ = nullptr;         // device: where encodes write the payload's carries (null: not written)
};

class WireDeviceDecoder {
public:
    WireDeviceDecoder() = default;
    ~WireDeviceDecoder();
    WireDeviceDecoder(const WireDeviceDecoder&) = delete;
    WireDeviceDecoder& operator=(const WireDeviceDecoder&) = delete;

    /// Waits for the device (so a payload still arriving on any stream is complete), reads the head of the payload at
    /// `payload` (device memory, `bytes` long), checks it against `expect` and against the slot's shape, and plans the
    /// scatter.  Nothing is written anywhere.  A decoder may be opened again for the next payload: it keeps its staging,
    /// streams, events and hash words, and keeps its scatter plan when the payload's place, the slot and the blob
    /// offsets are the ones it was built for (the same-shaped payload of the next hand-off), so an engine that holds
    /// one decoder per slot pays the allocations once.
    bool open(const void* payload, uint64_t bytes, const sc_geometry& g, const sc_decode_slot& slot,
              const WireExpect& expect, std::string& error);
    /// The same for a layer-split payload: `slot` takes the main session's layers and each stage's slot its stage
    /// part (layer ranges and shapes must match, in order).  After restore, the parts' host halves are in the returned
    /// image's stage_parts.
    bool open(const void* payload, uint64_t bytes, const sc_geometry& g, const sc_decode_slot& slot,
              const std::vector<WireDeviceStage>& stages, const WireExpect& expect, std::string& error);
    /// The same for a slot in any K/V format: the first K/V records must be the slot's layers in its format, with the
    /// indexer's rows exactly when slot.with_index.
    bool open(const void* payload, uint64_t bytes, const sc_geometry& g, const sc_slot_layers& slot,
              const WireExpect& expect, std::string& error);
    /// The same three for a payload held in segments (another process's exported segments, imported: byte o at
    /// from.ptr[o / segment_bytes] + o % segment_bytes): the head is read from them, the hash checked over them where
    /// they lie, and every blob scattered straight from them, cut where a segment ends.  Nothing is copied first.
    bool open(const sc_segments& from, uint64_t bytes, const sc_geometry& g, const sc_decode_slot& slot,
              const std::vector<WireDeviceStage>& stages, const WireExpect& expect, std::string& error);
    bool open(const sc_segments& from, uint64_t bytes, const sc_geometry& g, const sc_slot_layers& slot,
              const WireExpect& expect, std::string& error);
    int64_t tokens() const { return tokens_; }
    const WireDecoded& info() const { return info_; }
    /// Verifies the payload hash on the device (when `expect` asked for it), then scatters the K/V and GDN rows into the
    /// slot and copies every other blob into `image` (whose slot-resident K/V buffers and live gdn stay empty).
    /// Synchronous.  A refusal writes nothing to the slot.
    bool restore(void* stream, SavedConversation& image, std::string& error);
    /// The payload's carries, as the encoder wrote them (device memory, sc_fnv1a64_carry_bytes(bytes) bytes): restore
    /// then checks the hash starting every 64 KiB from its carry instead of looking back across the payload, with the
    /// same verdict - a payload or carries that are not what was hashed is refused and nothing is mounted.  Null (the
    /// default) checks without them.  Kept until the next open().
    void set_carry(const uint8_t* carry) { carry_ = carry; }

private:
    void release();
    void drop_open();   // what one open holds; the buffers and the cached plans stay
    bool open_f16(const void* payload, const sc_segments* segs, uint64_t bytes, const sc_geometry& g,
                  const sc_decode_slot& slot, const std::vector<WireDeviceStage>& stages, const WireExpect& expect,
                  std::string& error);
    bool open_layers(const void* payload, const sc_segments* segs, uint64_t bytes, const sc_geometry& g,
                     const sc_slot_layers& slot, const WireExpect& expect, std::string& error);
    bool read_head(const void* payload, const sc_segments* segs, uint64_t bytes, const WireExpect& expect,
                   std::vector<detail::WireBlobAt>& blobs, std::string& error);
    /// Copies payload bytes [off, off + n) to `dst` on `stream`, a piece per segment they lie in.
    bool copy_payload(void* dst, uint64_t off, uint64_t n, void* stream, std::string& error);
    sc_segments segments() const { return sc_segments{int32_t(seg_.size()), seg_bytes_, seg_.data()}; }
    bool finish_open(const void* payload, uint64_t bytes, const WireExpect& expect,
                     const std::vector<detail::WireBlobAt>& blobs, const std::vector<const void*>& device,
                     std::string& error);

    const uint8_t* payload_ = nullptr;
    uint64_t bytes_ = 0;
    WireExpect expect_{};
    WireDecoded info_{};
    int64_t tokens_ = 0;
    SavedConversation head_image_;
    struct Download { void* who; bool buffer; uint64_t offset, bytes, staged_at; };
    std::vector<Download> downloads_;   // blobs that go back to the host image (by address inside head_image_)
    uint8_t* staged_ = nullptr;         // pinned host staging of the downloads (64-byte aligned pieces)
    void* side_ = nullptr;              // the downloads' stream, beside the hash
    void* ev_start_ = nullptr;
    void* ev_done_ = nullptr;
    sc_plan* scatter_ = nullptr;
    bool opened_ = false;   // the last open succeeded (the kept scatter plan alone does not say so: a refused open
                            // keeps it for the next one)
    std::vector<sc_plan*> stage_scatters_;   // one per stage part, gated by the same hash verdict
    void* hash_ws_ = nullptr;
    uint64_t hash_ws_bytes_ = 0;
    std::vector<void*> seg_;          // a segmented payload's segments (empty: the payload is at payload_)
    uint64_t seg_bytes_ = 0;
    sc_hash_map* read_map_ = nullptr; // the hash of a segmented payload where it lies
    const uint8_t* carry_ = nullptr;  // device: the payload's carries (null: the check looks back)
    std::vector<uint8_t> plan_key_;   // what scatter_ was built for (empty: nothing, or a plan not kept across opens)
    std::vector<uint8_t> map_key_;    // what read_map_ was built for
    uint64_t staged_cap_ = 0;         // bytes at staged_
    uint8_t* head_pinned_ = nullptr;  // pinned: the payload's head is read into it (kept across opens; a read into
    uint64_t head_cap_ = 0;           // pageable memory took 0.28 ms for the 128K head, against ~0.02 ms here)
    uint64_t* hash_dev_ = nullptr;    // device: the hash check's verdict word
    uint64_t* hash_host_ = nullptr;   // pinned (64 B); the hash's last kernel stores the payload hash here
    // and the launch's fault word right after it, so the host sees both words the device verdict is made of
    uint32_t* hash_fault_host() { return reinterpret_cast<uint32_t*>(hash_host_ + 1); }
};

}  // namespace strata::core
