// conversation_wire.hpp - the hand-off payload codec: a parked conversation as one self-describing byte stream.
//
// The engine interface of the reference's codec (include/strata/core/conversation_wire.hpp:170-460): the same format
// constants, record layouts, entry points, sinks and sources, with the same meaning, so a prefill instance built on
// this library and a decode instance built on the reference read each other's payloads.  The implementation
// (host/src/conversation_wire.cpp) is this library's own.
//
// The payload:   header(256)  records  zero pad to 64  blob pool
//   header    magic 'SR4H', version 1, flags (cvec, has stage parts, partial), the 18 geometry values, the layer
//             range, the record counts, the live token count, the pool's offset and size, the caller's geometry and
//             pack hashes, the total payload size, and two words that must be zero (the payload hash travels out of
//             band: a hash stored inside the bytes it covers would be self-referential).
//   records   the K/V records (main layers, then the draft layer), the live CHECKPOINT, the retained checkpoints,
//             the STAGE records of a layer split, and an END record whose kind spells 'END!'.  Every record is
//             {u32 kind, u32 flags = 0, u64 body bytes} + body; every buffer is a BLOBREF {u64 bytes, u64 offset}
//             into the pool ({0, 0} for an empty one).
//   pool      every non-empty buffer, in the order its BLOBREF was written, each starting 64-byte aligned (relative to
//             the payload start), with zero bytes between: the payload is a pure function of the image.
//
// The device path of this library (conversation_wire_device.hpp) writes the same payload straight from a decode
// slot: the pool of a K/V + running-state image IS the transfer-buffer image the GPU gathers.
#pragma once

#include "strata/core/conversation_cache.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace strata::core {

// ---- format constants (an ABI: the values are the reference's, conversation_wire.hpp:178-207) ------------------------
inline constexpr uint32_t kWireMagic = 0x48345253u;   // 'S','R','4','H' little-endian
inline constexpr uint16_t kWireFormatVersion = 1;
inline constexpr uint64_t kWireHeaderSpecBytes = 232;
inline constexpr uint64_t kWireHeaderRecordBytes = 256;
inline constexpr uint64_t kWireRecordHeaderBytes = 16;
inline constexpr uint64_t kWireBlobAlign = 64;
inline constexpr uint64_t kWireHashSeed = 1469598103934665603ull;   // the FNV-1a seed of every reference call site
inline constexpr uint64_t kWireChunkBytes = 1ull << 20;             // the largest single read or write
inline constexpr int kWireMaxCheckpointDepth = 8;
inline constexpr int64_t kWireMaxKvRecords = 4096;
inline constexpr int64_t kWireMaxCheckpoints = 1 << 20;
inline constexpr int64_t kWireMaxStageParts = 64;
inline constexpr int64_t kWireMaxImages = 1 << 16;

enum WireRecordKind : uint32_t {
    kWireRecordKv = 1,
    kWireRecordCheckpoint = 2,
    kWireRecordStage = 3,
    kWireRecordEnd = 0x21444E45u,   // 'E','N','D','!'
};

enum WireHeaderFlags : uint16_t {
    kWireFlagCvec = 1u,
    kWireFlagHasStageParts = 2u,
    kWireFlagPartial = 4u,   // never valid on a finished payload: writers never set it, readers refuse it
    kWireFlagKnown = kWireFlagCvec | kWireFlagHasStageParts | kWireFlagPartial,
};

/// The header record as it lies in the payload (little-endian, no padding holes).
struct WireHeaderRecord {
    uint32_t magic;
    uint16_t fmt_version;
    uint16_t flags;
    uint64_t geometry[18];
    uint64_t layer_lo;
    uint64_t layer_hi;
    int64_t n_kv;
    int64_t n_checkpoints;
    int64_t n_stage_parts;
    int64_t live_tokens;
    uint64_t blob_pool_off;
    uint64_t blob_pool_bytes;
    uint64_t geom_hash;
    uint64_t pack_hash;
    uint64_t payload_bytes;
    uint64_t payload_hash;   // always zero on the wire
    uint64_t reserved;       // always zero
};
static_assert(sizeof(WireHeaderRecord) == kWireHeaderRecordBytes);
static_assert(offsetof(WireHeaderRecord, geometry) == 8 && offsetof(WireHeaderRecord, layer_lo) == 152);
static_assert(offsetof(WireHeaderRecord, n_kv) == 168 && offsetof(WireHeaderRecord, live_tokens) == 192);
static_assert(offsetof(WireHeaderRecord, blob_pool_off) == 200 && offsetof(WireHeaderRecord, pack_hash) == 224);
static_assert(offsetof(WireHeaderRecord, payload_bytes) == kWireHeaderSpecBytes);
static_assert(offsetof(WireHeaderRecord, reserved) == 248);

// ---- sinks: where an encode writes, strictly in payload order, in chunks of any size -----------------------------------
class WireSink {
public:
    virtual ~WireSink() = default;
    virtual bool write(const uint8_t* data, size_t bytes) = 0;
    /// Why the last write was refused (appended to the codec's own message).
    virtual std::string refusal() const { return {}; }
};

class VectorWireSink final : public WireSink {
public:
    explicit VectorWireSink(size_t reserve_bytes = 0) { bytes_.reserve(reserve_bytes); }
    bool write(const uint8_t* data, size_t bytes) override;
    const std::vector<uint8_t>& data() const { return bytes_; }
    std::vector<uint8_t>& data() { return bytes_; }

private:
    std::vector<uint8_t> bytes_;
};

/// Into a hand-off slot: through a file descriptor at `offset` (pwrite), or into a mapping.  Refuses past `capacity`.
class SlotWireSink final : public WireSink {
public:
    SlotWireSink(int fd, uint64_t offset, uint64_t capacity);
    SlotWireSink(uint8_t* mapping, uint64_t capacity);
    bool write(const uint8_t* data, size_t bytes) override;
    std::string refusal() const override { return error_; }
    uint64_t written() const { return pos_; }
    const std::string& error() const { return error_; }

private:
    int fd_ = -1;
    uint64_t base_ = 0;
    uint8_t* map_ = nullptr;
    uint64_t pos_ = 0, capacity_ = 0;
    std::string error_;
};

// ---- sources: random access by payload offset -------------------------------------------------------------------------
class WireSource {
public:
    virtual ~WireSource() = default;
    virtual uint64_t size() const = 0;
    /// Fill [offset, offset + bytes) or fail; never a short read.
    virtual bool read(uint8_t* dst, uint64_t offset, size_t bytes) const = 0;
    /// A pointer to [offset, offset + bytes) when the source is memory, else null (the codec then reads in chunks).
    virtual const uint8_t* span(uint64_t /*offset*/, size_t /*bytes*/) const { return nullptr; }
};

class SpanWireSource final : public WireSource {
public:
    SpanWireSource(const uint8_t* data, uint64_t bytes) : p_(data), n_(bytes) {}
    uint64_t size() const override { return n_; }
    bool read(uint8_t* dst, uint64_t offset, size_t bytes) const override;
    const uint8_t* span(uint64_t offset, size_t bytes) const override;

private:
    const uint8_t* p_ = nullptr;
    uint64_t n_ = 0;
};

class FileWireSource final : public WireSource {
public:
    FileWireSource(int fd, uint64_t offset, uint64_t bytes) : fd_(fd), base_(offset), n_(bytes) {}
    uint64_t size() const override { return n_; }
    bool read(uint8_t* dst, uint64_t offset, size_t bytes) const override;

private:
    int fd_ = -1;
    uint64_t base_ = 0, n_ = 0;
};

// ---- encode ---------------------------------------------------------------------------------------------------------
/// The caller's identity values, carried in the header and compared by the receiver.
struct WireIdentity {
    uint64_t geom_hash = 0;
    uint64_t pack_hash = 0;
};

/// Everything about a payload that is known without writing it.
struct WirePlan {
    uint64_t body_bytes = 0;        ///< the record stream, header excluded
    uint64_t blob_pool_off = 0;
    uint64_t blob_pool_bytes = 0;
    uint64_t total_bytes = 0;
    int64_t n_kv = 0, n_checkpoints = 0, n_stage_parts = 0, live_tokens = 0;
    uint16_t flags = 0;
    size_t blobs = 0;               ///< pool entries (empty buffers have none)
};

struct WireEncoded {
    uint64_t bytes = 0;
    uint64_t payload_hash = 0;      ///< FNV-1a over the bytes written, from kWireHashSeed
    uint64_t blob_pool_bytes = 0;
    size_t blobs = 0;
};

bool conversation_wire_plan(const SavedConversation& image, WirePlan& plan, std::string& error);
bool conversation_wire_plan(const SavedConversation& image, int max_checkpoint_depth, WirePlan& plan,
                            std::string& error);
bool conversation_wire_encode(const SavedConversation& image, WireSink& sink, const WireIdentity& identity,
                              WireEncoded& out, std::string& error);
bool conversation_wire_encode(const SavedConversation& image, WireSink& sink, const WireIdentity& identity,
                              int max_checkpoint_depth, WirePlan& plan, WireEncoded& out, std::string& error);

// ---- decode ---------------------------------------------------------------------------------------------------------
/// What the receiver requires before it writes anything.
struct WireExpect {
    std::array<int64_t, 18> geometry{};
    bool check_geometry = false;
    uint64_t geom_hash = 0, pack_hash = 0;
    bool check_hashes = false;
    uint64_t payload_hash = 0;
    bool check_payload_hash = false;
    int64_t stage_parts = -1;          ///< -1: no check
    uint64_t max_payload_bytes = 0;    ///< 0: no bound
    int max_checkpoint_depth = kWireMaxCheckpointDepth;
};

struct WireDecoded {
    uint64_t bytes = 0;
    uint64_t payload_hash = 0;
    uint64_t geom_hash = 0, pack_hash = 0;
    std::array<int64_t, 18> geometry{};
    int64_t layer_lo = 0, layer_hi = 0;
    int64_t n_kv = 0, n_checkpoints = 0, n_stage_parts = 0, live_tokens = 0;
    uint16_t flags = 0;
    bool cvec = true;
    uint64_t blob_pool_off = 0, blob_pool_bytes = 0;
    size_t blobs = 0;
};

/// All or nothing: on false `image` is untouched and `error` names the refusal.  `image.owner` comes back kNoOwner.
bool conversation_wire_decode(const WireSource& source, SavedConversation& image, WireDecoded& info,
                              const WireExpect& expect, std::string& error);
bool conversation_wire_decode(const uint8_t* data, uint64_t bytes, SavedConversation& image, WireDecoded& info,
                              const WireExpect& expect, std::string& error);

/// The header alone, with its self-consistency checks (not the geometry, the hashes or the body).
bool conversation_wire_peek(const uint8_t* data, uint64_t bytes, WireHeaderRecord& header, std::string& error);

/// FNV-1a 64 of a payload as written, from kWireHashSeed.
uint64_t conversation_wire_payload_hash(const uint8_t* data, uint64_t bytes);

/// One line describing a header, for refusal messages and logs.
std::string conversation_wire_describe(const WireHeaderRecord& header);

/// The engine's FNV-1a 64 byte loop (the reference's fnv1a64, include/strata/core/pinned.hpp:173).
uint64_t fnv1a64(const uint8_t* data, uint64_t bytes, uint64_t seed);

}  // namespace strata::core
