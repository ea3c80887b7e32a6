// handoff.hpp - the hand-off arena: the shared tmpfs file through which a prefill instance passes a conversation
// payload to a decode instance (the reference's include/strata/core/handoff.hpp, same API and same file format).
//
// The file, the two 4 KiB headers and the slot state machine are an ABI between processes: a prefill instance built
// from this library and a decode instance built from the reference (or the other way round) hand payloads to each
// other through one arena file.  Every offset, magic, state value, flag bit, sizing rule and the publish order below
// are therefore the reference's, and the tests check them against an independent table and against the reference's
// own implementation on the same file.  The code is this library's.
//
//   arena file  = arena header (4096 B)
//                 + per tier t, in ascending token order: tier_slot_count[t] x (slot header (4096 B) + tier_slot_bytes[t])
//   slot life   = FREE -> CLAIMED (claim, under the file lock) -> READY (payload written without the lock, then the
//                 48-byte metadata block [96,144), a release fence, and one 8-byte store of state+flags at [24,32))
//                 -> FREE (release on the reader's ACK, or reclaim: dead claimer, expired lease, dead reader)
//
// A reader only copies from a READY slot whose nonce and client id are the ones it was told, whose pack and geometry
// hashes are the arena's, and whose payload fits the slot.  Decisions (claim, publish's ownership check, release,
// abort, cancel, reclaim) are taken under an exclusive flock of the file plus a process-local mutex; header reads take
// a shared flock; payload bytes are never written or read under the lock.
//
// The payload movers between HBM and a slot (pinned staging, parallel host copies, the device hash) are in
// handoff_device.hpp; this file is host-only and makes no device call.  Its three additions to the reference's API
// (claim_window, read_window, reserve) serve those movers.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace strata::core {

/// FNV-1a 64 over bytes from `seed` (the engine's hash, declared with the payload codec).  The default seed is the one
/// every reference call site uses (include/strata/core/pinned.hpp:173).
uint64_t fnv1a64(const uint8_t* data, uint64_t bytes, uint64_t seed);
inline uint64_t fnv1a64(const uint8_t* data, uint64_t bytes) { return fnv1a64(data, bytes, 1469598103934665603ull); }

// ---- constants of the file format (include/strata/core/handoff.hpp:152-214) ----
inline constexpr uint64_t kHandoffHeaderBytes = 4096;            ///< the arena header and every slot header
inline constexpr uint32_t kHandoffVersion = 1;
inline constexpr int kHandoffMaxTiers = 8;
inline constexpr uint64_t kHandoffSlackBytes = 64ull << 20;      ///< per slot, over the priced payload
inline constexpr uint64_t kHandoffDefaultLeaseMs = 300000ull;    ///< STRATA_HANDOFF_LEASE_MS overrides it

enum HandoffSlotState : uint32_t { kHandoffFree = 0, kHandoffClaimed = 1, kHandoffReady = 2 };
enum HandoffSlotFlags : uint32_t { kHandoffFlagCancelled = 1u, kHandoffFlagAbandoned = 2u, kHandoffFlagPartial = 4u };

inline constexpr uint64_t kArenaMagicOffset = 0;
inline constexpr uint64_t kArenaVersionOffset = 16;
inline constexpr uint64_t kArenaHeaderBytesOffset = 20;
inline constexpr uint64_t kArenaTierCountOffset = 24;
inline constexpr uint64_t kArenaSlotTotalOffset = 32;
inline constexpr uint64_t kArenaBytesOffset = 40;
inline constexpr uint64_t kArenaPackHashOffset = 48;
inline constexpr uint64_t kArenaGeomHashOffset = 56;
inline constexpr uint64_t kArenaCreatedPidOffset = 64;
inline constexpr uint64_t kArenaCreatedStartOffset = 72;
inline constexpr uint64_t kArenaTierMaxTokensOffset = 80;
inline constexpr uint64_t kArenaTierSlotCountOffset = 144;
inline constexpr uint64_t kArenaTierSlotBytesOffset = 208;
inline constexpr uint64_t kArenaTierSlotOffOffset = 272;
inline constexpr uint64_t kArenaReservedOffset = 336;

inline constexpr uint64_t kSlotMagicOffset = 0;
inline constexpr uint64_t kSlotVersionOffset = 16;
inline constexpr uint64_t kSlotHeaderBytesOffset = 20;
inline constexpr uint64_t kSlotStateOffset = 24;
inline constexpr uint64_t kSlotFlagsOffset = 28;
inline constexpr uint64_t kSlotTierOffset = 32;
inline constexpr uint64_t kSlotOwnerOffset = 40;
inline constexpr uint64_t kSlotOwnerStartOffset = 48;
inline constexpr uint64_t kSlotNonceOffset = 56;
inline constexpr uint64_t kSlotClientOffset = 64;
inline constexpr uint64_t kSlotRequestOffset = 72;
inline constexpr uint64_t kSlotPackHashOffset = 80;
inline constexpr uint64_t kSlotGeomHashOffset = 88;
inline constexpr uint64_t kSlotTokensOffset = 96;
inline constexpr uint64_t kSlotPayloadBytesOffset = 104;
inline constexpr uint64_t kSlotPayloadHashOffset = 112;
inline constexpr uint64_t kSlotClaimedMsOffset = 120;
inline constexpr uint64_t kSlotPublishedMsOffset = 128;
inline constexpr uint64_t kSlotSeqOffset = 136;
inline constexpr uint64_t kSlotReservedOffset = 144;
/// Publish writes [96,144) first (tokens .. seq) and then, after a release fence, the 8 bytes of state+flags.
inline constexpr uint64_t kSlotPublishBlockOffset = 96;
inline constexpr uint64_t kSlotPublishBlockBytes = 48;
inline constexpr uint64_t kSlotPublishStateBytes = 8;

/// The arena header as it lies in the file (include/strata/core/handoff.hpp:218-253).  The magic is 16 raw bytes
/// with no terminator.
struct HandoffArenaHeader {
    char magic[16];
    uint32_t version;
    uint32_t header_bytes;
    uint32_t tier_count;
    uint32_t pad;
    uint64_t slot_total;
    uint64_t arena_bytes;
    uint64_t pack_hash;
    uint64_t geom_hash;
    uint64_t created_pid;
    uint64_t created_start;
    uint64_t tier_max_tokens[kHandoffMaxTiers];
    uint64_t tier_slot_count[kHandoffMaxTiers];
    uint64_t tier_slot_bytes[kHandoffMaxTiers];
    uint64_t tier_slot_off[kHandoffMaxTiers];
    uint64_t reserved[kHandoffMaxTiers];
};

/// A slot header as it lies in the file (include/strata/core/handoff.hpp:255-301).
struct HandoffSlotHeader {
    char magic[16];
    uint32_t version;
    uint32_t header_bytes;
    uint32_t state;
    uint32_t flags;
    uint32_t tier;
    uint32_t pad;
    uint64_t owner_pid;
    uint64_t owner_start;
    uint64_t nonce;
    uint64_t client_id;
    uint64_t request_id;
    uint64_t pack_hash;
    uint64_t geom_hash;
    uint64_t tokens;
    uint64_t payload_bytes;
    uint64_t payload_hash;
    uint64_t claimed_ms;
    uint64_t published_ms;
    uint64_t seq;
    uint64_t reserved[7];
};

static_assert(sizeof(HandoffArenaHeader) == 400 && sizeof(HandoffArenaHeader) <= kHandoffHeaderBytes);
static_assert(sizeof(HandoffSlotHeader) == 200 && sizeof(HandoffSlotHeader) <= kHandoffHeaderBytes);
static_assert(offsetof(HandoffArenaHeader, version) == kArenaVersionOffset &&
              offsetof(HandoffArenaHeader, header_bytes) == kArenaHeaderBytesOffset &&
              offsetof(HandoffArenaHeader, tier_count) == kArenaTierCountOffset &&
              offsetof(HandoffArenaHeader, slot_total) == kArenaSlotTotalOffset &&
              offsetof(HandoffArenaHeader, arena_bytes) == kArenaBytesOffset &&
              offsetof(HandoffArenaHeader, pack_hash) == kArenaPackHashOffset &&
              offsetof(HandoffArenaHeader, geom_hash) == kArenaGeomHashOffset &&
              offsetof(HandoffArenaHeader, created_pid) == kArenaCreatedPidOffset &&
              offsetof(HandoffArenaHeader, created_start) == kArenaCreatedStartOffset &&
              offsetof(HandoffArenaHeader, tier_max_tokens) == kArenaTierMaxTokensOffset &&
              offsetof(HandoffArenaHeader, tier_slot_count) == kArenaTierSlotCountOffset &&
              offsetof(HandoffArenaHeader, tier_slot_bytes) == kArenaTierSlotBytesOffset &&
              offsetof(HandoffArenaHeader, tier_slot_off) == kArenaTierSlotOffOffset &&
              offsetof(HandoffArenaHeader, reserved) == kArenaReservedOffset);
static_assert(offsetof(HandoffSlotHeader, version) == kSlotVersionOffset &&
              offsetof(HandoffSlotHeader, header_bytes) == kSlotHeaderBytesOffset &&
              offsetof(HandoffSlotHeader, state) == kSlotStateOffset &&
              offsetof(HandoffSlotHeader, flags) == kSlotFlagsOffset &&
              offsetof(HandoffSlotHeader, tier) == kSlotTierOffset &&
              offsetof(HandoffSlotHeader, owner_pid) == kSlotOwnerOffset &&
              offsetof(HandoffSlotHeader, owner_start) == kSlotOwnerStartOffset &&
              offsetof(HandoffSlotHeader, nonce) == kSlotNonceOffset &&
              offsetof(HandoffSlotHeader, client_id) == kSlotClientOffset &&
              offsetof(HandoffSlotHeader, request_id) == kSlotRequestOffset &&
              offsetof(HandoffSlotHeader, pack_hash) == kSlotPackHashOffset &&
              offsetof(HandoffSlotHeader, geom_hash) == kSlotGeomHashOffset &&
              offsetof(HandoffSlotHeader, tokens) == kSlotTokensOffset &&
              offsetof(HandoffSlotHeader, payload_bytes) == kSlotPayloadBytesOffset &&
              offsetof(HandoffSlotHeader, payload_hash) == kSlotPayloadHashOffset &&
              offsetof(HandoffSlotHeader, claimed_ms) == kSlotClaimedMsOffset &&
              offsetof(HandoffSlotHeader, published_ms) == kSlotPublishedMsOffset &&
              offsetof(HandoffSlotHeader, seq) == kSlotSeqOffset &&
              offsetof(HandoffSlotHeader, reserved) == kSlotReservedOffset);
static_assert(kSlotPublishBlockOffset == kSlotTokensOffset &&
              kSlotPublishBlockOffset + kSlotPublishBlockBytes == kSlotReservedOffset);

// ---- identity (include/strata/core/handoff.hpp:306-329) ----

/// One later stage of a layer split: the layers [layer_lo, layer_hi) it holds.
struct HandoffSplitStage {
    int64_t layer_lo = 0;
    int64_t layer_hi = 0;
};
/// The whole split: the main carve, the later stages in engine order, and whether the draft model binds to the last
/// stage.  Two instances whose splits differ write different payloads for one conversation.
struct HandoffSplit {
    int64_t main_lo = 0;
    int64_t main_hi = 0;
    std::vector<HandoffSplitStage> stages;
    bool draft_on_last = true;
};
/// "main=<lo>..<hi>|<lo>..<hi>,...|n=<stages>|draft=<last|main>": no space and no slash, so it names a directory.
std::string handoff_split_spec(const HandoffSplit& split);
/// FNV-1a from the engine seed over "strata-handoff-geom-v1", the 18 geometry words (little-endian u64 each) and the
/// split spec; a zero result is reported as 1 (zero means "unset" in the header).
uint64_t handoff_geom_hash(const std::array<int64_t, 18>& geometry, const std::string& split_spec);
/// "<dir>/<pack16>-<split_spec>[/<instance>]/arena", pack16 = 16 lowercase hex digits.
std::string handoff_arena_path(const std::string& handoff_dir, uint64_t pack_hash, const std::string& split_spec,
                               const std::string& instance);

inline uint64_t handoff_round_up_64(uint64_t n) { return (n + 63ull) & ~63ull; }

// ---- sizing (include/strata/core/handoff.hpp:333-366) ----

struct HandoffTierSpec {
    uint64_t max_tokens = 0;   ///< the context length of the tier
    uint64_t slot_count = 0;   ///< slots in the tier's group
};

/// The arena's layout, computed once from priced payload sizes (never from the machine's memory).
struct HandoffSizing {
    std::vector<HandoffTierSpec> tiers;
    std::vector<uint64_t> payload_bytes;   ///< as priced
    std::vector<uint64_t> slot_bytes;      ///< round_up_64(payload) + kHandoffSlackBytes
    std::vector<uint64_t> slot_off;        ///< file offset of each tier's first slot
    uint64_t slot_total = 0;
    uint64_t arena_bytes = 0;
    uint64_t max_tokens = 0;
    /// "slots 2,2,2 (tiers 1024,16384,131072), max 131072 tokens, arena 8.20 GiB (<bytes> B)"
    std::string describe;
};

/// `pricer(tier_tokens, payload_bytes, err)`: the payload size of a conversation of `tier_tokens` tokens.
using HandoffPricer = std::function<bool(uint64_t tier_tokens, uint64_t& payload_bytes, std::string& err)>;

/// Tiers must be 1..8, ascending by token count, each with at least one slot and a nonzero token count.
bool handoff_size_arena(const std::vector<HandoffTierSpec>& tiers, const HandoffPricer& pricer, HandoffSizing& out,
                        std::string& err);
bool handoff_size_arena(const std::vector<HandoffTierSpec>& tiers, const std::vector<uint64_t>& payload_bytes,
                        HandoffSizing& out, std::string& err);

// ---- what the arena hands out (include/strata/core/handoff.hpp:369-430) ----

/// One slot header as read, plus where the slot lies.
struct HandoffSlotInfo {
    int index = -1;
    uint64_t base = 0;       ///< file offset of the slot header
    uint64_t capacity = 0;   ///< payload bytes the slot holds
    uint32_t state = kHandoffFree;
    uint32_t flags = 0;
    uint32_t tier = 0;
    uint64_t owner_pid = 0, owner_start = 0, nonce = 0;
    uint64_t client_id = 0, request_id = 0;
    uint64_t pack_hash = 0, geom_hash = 0;
    uint64_t tokens = 0, payload_bytes = 0, payload_hash = 0;
    uint64_t claimed_ms = 0, published_ms = 0, seq = 0;
};

/// A slot this process claimed.
struct HandoffClaim {
    int index = -1;
    uint64_t base = 0;          ///< file offset of the slot header
    uint64_t payload_off = 0;   ///< base + 4096
    uint64_t capacity = 0;
    uint32_t tier = 0;          ///< the tier whose group the slot is in (may be above the one asked for)
    uint64_t nonce = 0;
};

/// One slot reclaim() took back, and why.
struct HandoffReclaim {
    int index = -1;
    uint32_t was_state = 0;
    uint32_t flags = 0;
    uint64_t owner_pid = 0, client_id = 0, nonce = 0, payload_bytes = 0;
    uint64_t age_ms = 0;
    std::string why;
};

/// A published payload mapped read-only; unmapped when this object goes.
struct HandoffPayload {
    const uint8_t* data = nullptr;
    uint64_t bytes = 0;
    int index = -1;
    uint32_t tier = 0;
    uint64_t nonce = 0, client_id = 0, request_id = 0;
    uint64_t tokens = 0, payload_bytes = 0, payload_hash = 0, seq = 0;

    HandoffPayload() = default;
    ~HandoffPayload();
    HandoffPayload(const HandoffPayload&) = delete;
    HandoffPayload& operator=(const HandoffPayload&) = delete;
    HandoffPayload(HandoffPayload&& o) noexcept;
    HandoffPayload& operator=(HandoffPayload&& o) noexcept;
    bool valid() const { return data != nullptr; }
    /// Adopt a mapping (`map`, `map_bytes` are what is unmapped); `data` points at the first payload byte.
    void bind_mapping(void* map, uint64_t map_bytes, const uint8_t* data, uint64_t payload_bytes);
    void unbind();

  private:
    void* map_ = nullptr;
    uint64_t map_bytes_ = 0;
};

// ---- the arena (include/strata/core/handoff.hpp:432-551) ----

class HandoffArena {
  public:
    HandoffArena();   ///< the lease starts at STRATA_HANDOFF_LEASE_MS when set, else kHandoffDefaultLeaseMs
    ~HandoffArena();
    HandoffArena(const HandoffArena&) = delete;
    HandoffArena& operator=(const HandoffArena&) = delete;
    HandoffArena(HandoffArena&& o) noexcept;
    HandoffArena& operator=(HandoffArena&& o) noexcept;

    // -- the writer (the prefill instance) --

    /// Create (or re-open) the arena file at `path`: parent directories, a free-space check before the file is sized,
    /// the header and every slot FREE.  An existing file must have the sizing's size and both hashes; if another live
    /// process created it the open is refused (one writer per arena) unless `allow_existing_writer`, which only the
    /// tests set (two processes contending for one slot); if its creator is dead the slot table is rebuilt.
    bool open_writer(const std::string& path, const HandoffSizing& sizing, uint64_t pack_hash, uint64_t geom_hash,
                     std::string& err, bool allow_existing_writer = false);
    void set_lease_ms(uint64_t ms) { lease_ms_ = ms; }
    uint64_t lease_ms() const { return lease_ms_; }
    /// The pid behind a client id, so a READY slot whose reader died is reclaimed at once.
    void note_client_pid(uint64_t client_id, uint64_t pid);
    /// Free every slot whose claimer died, whose lease expired, or whose registered reader died.
    std::vector<HandoffReclaim> reclaim(std::string* err = nullptr);
    /// Claim a FREE (or reclaimable) slot in the smallest tier group >= `tier`.  "no free handoff slot" is a
    /// temporary condition.
    bool claim(uint32_t tier, uint64_t client_id, uint64_t request_id, HandoffClaim& out, std::string& err);
    /// Write payload bytes at `offset` into the claimed slot (no lock held).
    bool write_payload(const HandoffClaim& c, uint64_t offset, const void* data, uint64_t bytes, std::string& err);
    /// Publish: refused unless the slot is still this claim's and not cancelled.
    bool publish(const HandoffClaim& c, uint64_t tokens, uint64_t payload_bytes, uint64_t payload_hash,
                 std::string& err);
    /// Free the slot of `nonce` (the reader's ACK).  The body is left as it is.
    bool release(int index, uint64_t nonce, std::string& err);
    /// Give up a claim without publishing (sets the partial flag).
    bool abort_claim(int index, uint64_t nonce, std::string& err);
    /// Mark a job cancelled; its publish is then refused.
    bool cancel(int index, uint64_t nonce, std::string& err);

    // -- this library's additions for the device mover (handoff_device.hpp) --

    /// The claim's first payload byte inside one writable mapping of the whole arena that the writer keeps until it
    /// closes the arena, so payload copies into slots run on the host's parallel memory bandwidth (a file write to one
    /// tmpfs file is serialized) and page tables are set up once, not per hand-off.  Null + err when the claim does
    /// not match this arena's slot table.
    uint8_t* claim_window(const HandoffClaim& c, std::string& err);
    /// Writer: commit every page of the arena file now (posix_fallocate: a full filesystem is an error here instead
    /// of a SIGBUS in the middle of a payload copy) and populate its mapping, so the first hand-off through each slot
    /// does not pay page allocation and faults.  Reader: map the file read-only with its page tables populated.
    bool reserve(std::string& err);
    /// Reader: every check of read_slot, then the slot's first payload byte inside one read-only mapping of the whole
    /// arena that the reader keeps until it closes the arena (no mapping is made or torn down per read; tearing down
    /// a 3 GB mapping costs ~17 ms).  `info` is the slot header as checked.  Null + err on refusal.
    const uint8_t* read_window(int index, uint64_t expect_nonce, uint64_t client_id, HandoffSlotInfo& info,
                               std::string& err);

    // -- the reader (a decode instance) --

    /// Open an existing arena read-only: magic, version and header size first, then the file size, then both hashes.
    bool open_reader(const std::string& path, uint64_t pack_hash, uint64_t geom_hash, std::string& err);
    /// Map a READY slot's payload read-only, after checking nonce, client, the slot's hashes, its size and seq.
    bool read_slot(int index, uint64_t expect_nonce, uint64_t client_id, HandoffPayload& out, std::string& err);
    /// FNV-1a of a mapped payload from the engine seed.
    static uint64_t payload_hash_of(const HandoffPayload& p);

    // -- either side --
    bool valid() const { return fd_ >= 0; }
    bool is_writer() const { return writer_; }
    const std::string& path() const { return path_; }
    const HandoffArenaHeader& header() const { return hdr_; }
    uint64_t arena_bytes() const { return hdr_.arena_bytes; }
    uint64_t slot_total() const { return hdr_.slot_total; }
    uint32_t tier_count() const { return hdr_.tier_count; }
    uint64_t tier_max_tokens(uint32_t tier) const;
    uint64_t tier_slot_bytes(uint32_t tier) const;
    uint64_t tier_slot_count(uint32_t tier) const;
    uint64_t tier_slot_off(uint32_t tier) const;
    /// The largest tier's token count (tiers ascend, so the last one).
    uint64_t max_tokens() const { return hdr_.tier_count ? hdr_.tier_max_tokens[hdr_.tier_count - 1] : 0; }
    /// "slots .. (tiers ..), max .. tokens, arena .. GiB, pack hash <16 hex>, geometry hash <16 hex>"
    std::string describe() const;
    /// One slot header, read under a shared lock.
    bool slot_info(int index, HandoffSlotInfo& out) const;
    /// "<free>/<total>"
    std::string free_slots(std::string* err = nullptr) const;

  private:
    struct Place {
        uint64_t base = 0;
        uint64_t capacity = 0;
        uint32_t tier = 0;
    };

    void close_();
    bool adopt_header_(const HandoffArenaHeader& h, uint64_t file_bytes, std::string& err);
    bool place_(int index, Place& p) const;
    bool load_slot_(int index, HandoffSlotHeader& s, Place& p) const;
    bool store_(uint64_t off, const void* data, uint64_t n) const;
    bool format_(const HandoffSizing& sizing, uint64_t pack_hash, uint64_t geom_hash, std::string& err);
    bool lease_over_(uint64_t stamp_ms) const;
    bool reader_gone_(uint64_t client_id) const;
    std::vector<HandoffReclaim> sweep_(std::string* err);   // needs the lock
    uint64_t count_free_() const;                           // needs the lock

    bool map_all_(bool populate, std::string& err);
    bool ready_slot_(int index, uint64_t expect_nonce, uint64_t client_id, HandoffSlotHeader& s, Place& p,
                     std::string& err) const;

    int fd_ = -1;
    bool writer_ = false;
    uint8_t* map_ = nullptr;      ///< the whole file, mapped once for the device movers (writable for the writer)
    uint64_t map_bytes_ = 0;
    std::string path_;
    HandoffArenaHeader hdr_{};
    std::vector<Place> places_;   ///< every slot's offset, tier and capacity, from the header
    uint64_t lease_ms_ = kHandoffDefaultLeaseMs;
    std::vector<std::pair<uint64_t, uint64_t>> client_pids_;
    /// The flock belongs to the open file description, which every thread of this process shares; the mutex keeps
    /// two threads from taking one decision at once.
    mutable std::mutex mu_;
};

// ---- liveness and clock (include/strata/core/handoff.hpp:554-558) ----

/// /proc/<pid> exists (when /proc itself is missing the answer is "alive").
bool handoff_pid_alive(uint64_t pid);
/// Field 22 (starttime) of /proc/<pid>/stat, 0 when unknown.
uint64_t handoff_proc_start_time(uint64_t pid);
/// Alive and, when both start times are known, the same process (not a recycled pid).
bool handoff_claim_alive(uint64_t pid, uint64_t start_time);
/// CLOCK_MONOTONIC in milliseconds.
uint64_t handoff_now_ms();

}  // namespace strata::core
