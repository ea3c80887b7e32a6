// handoff_device.hpp - moving hand-off payloads between HBM and slots of the hand-off arena (handoff.hpp).
//
// The reference's prefill instance hands a payload to the arena from host memory (HandoffArena::write_payload, one
// pwrite) after its codec copied it off the device, and its decode instance maps the slot and hashes it byte by byte
// on the CPU (HandoffArena::payload_hash_of) before the codec copies it back (src/core/handoff.cpp:821-841,
// 1053-1136).  Here the payload lives in HBM on both sides and the mover streams it through pinned staging:
//
//   writer: HBM --DMA--> pinned chunk k --host threads--> slot (the arena's mapped window)     chunks k+1.. in flight
//   reader: slot --host threads--> pinned chunk k --DMA--> HBM                                 chunk k-1 in flight
//
// Tmpfs pages are filled by several threads through a mapping (one file's write path is serialized), DMA and host
// copies of neighbouring chunks overlap, and the payload's FNV-1a (the arena's payload_hash) is computed on the
// device beside the copies: over the whole payload while the writer's chunks drain, and on the reader chunk by chunk
// as each lands in HBM, the running hash chained on the device.  The slot protocol is untouched: the writer
// still publishes through HandoffArena::publish, the reader still checks the slot with HandoffArena::read_slot, and a
// slot written here reads back through the reference's own reader.
#pragma once

#include "strata/core/handoff.hpp"

#include <condition_variable>
#include <cstdint>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace strata::core {

struct HandoffMoverConfig {
    uint64_t chunk_bytes = 64ull << 20;   ///< one pinned staging buffer (a multiple of 4 KiB)
    int depth = 4;                        ///< staging buffers in flight (2..16)
    int threads = 8;                      ///< host threads copying between staging and the slot (1..64)
};

/// What one transfer measured (host wall clock around the whole call, and the bytes moved).
struct HandoffMoveStats {
    uint64_t bytes = 0;
    double ms = 0.0;
    double hash_ms = 0.0;   ///< the part of `ms` spent waiting for the device hash after the copies (reader)
    double copy_ms = 0.0;   ///< host threads copying between staging and the slot
    double wait_ms = 0.0;   ///< waiting for DMA (a staging buffer's event, the stream at the end)
    bool wrote_device = false;   ///< a failed read that had already written device memory
    bool device_error = false;   ///< the failure was a device call's
    bool hash_fault = false;     ///< the device hash did not complete (a bounded wait of its kernel ran out)
};

/// A fixed set of host threads that split one copy between them (the calling thread takes part).
class HandoffCopyCrew {
  public:
    explicit HandoffCopyCrew(int threads);
    ~HandoffCopyCrew();
    HandoffCopyCrew(const HandoffCopyCrew&) = delete;
    HandoffCopyCrew& operator=(const HandoffCopyCrew&) = delete;
    /// memcpy(dst, src, n) in pieces of at least 1 MiB spread over the crew; returns when every piece is done.
    void copy(void* dst, const void* src, uint64_t n);
    int size() const { return (int) workers_.size() + 1; }

  private:
    void work();
    void take_pieces();
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable wake_, idle_;
    uint64_t round_ = 0;
    int busy_ = 0;
    bool stop_ = false;
    uint8_t* dst_ = nullptr;
    const uint8_t* src_ = nullptr;
    uint64_t n_ = 0, piece_ = 0;
    uint64_t next_ = 0;   // guarded by mu_ (pieces are >= 1 MiB, so the lock is taken rarely)
};

class HandoffMover {
  public:
    HandoffMover() = default;
    ~HandoffMover();
    HandoffMover(const HandoffMover&) = delete;
    HandoffMover& operator=(const HandoffMover&) = delete;

    /// Pinned staging, events, a hash stream and the copy crew, on the current device.
    bool init(const HandoffMoverConfig& cfg, std::string& err);
    bool ready() const { return !stage_.empty(); }
    const HandoffMoverConfig& config() const { return cfg_; }

    /// Writer: `bytes` of device memory at `device_src` (ordered after the work already on `stream`) into the claimed
    /// slot from payload offset 0.  With `hash`, also the FNV-1a of those bytes (engine seed), computed on the device
    /// beside the copies.  Returns when the bytes are in the slot; the slot stays CLAIMED.
    bool write_from_device(HandoffArena& arena, const HandoffClaim& claim, const void* device_src, uint64_t bytes,
                           void* stream, uint64_t* hash, std::string& err);
    /// write_from_device, then HandoffArena::publish with the device hash.
    bool publish_from_device(HandoffArena& arena, const HandoffClaim& claim, const void* device_src, uint64_t bytes,
                             uint64_t tokens, void* stream, std::string& err);
    /// Reader: the READY slot's payload (every check of HandoffArena::read_slot) into `device_dst` (room for
    /// `dst_capacity` bytes), on `stream`.  Refuses before any device write when the slot does not qualify or does not
    /// fit; after the copy, refuses if the slot no longer holds the same publication (released or reclaimed while it
    /// was read) and, with `verify`, if the device FNV-1a of the copied bytes differs from the slot's payload_hash.
    /// `info` is the slot as it was read.  Returns when the bytes are in device memory.
    bool read_to_device(HandoffArena& arena, int index, uint64_t nonce, uint64_t client_id, void* device_dst,
                        uint64_t dst_capacity, void* stream, bool verify, HandoffSlotInfo& info, std::string& err);

    const HandoffMoveStats& last() const { return last_; }

  private:
    uint64_t* hash_space_(uint64_t bytes, std::string& err);
    bool hash_on_device_(const void* data, uint64_t bytes, void* stream, std::string& err);
    bool fetch_hash_(uint64_t* out, std::string& err);
    void release_();

    HandoffMoverConfig cfg_{};
    std::vector<void*> stage_;    ///< pinned staging buffers
    std::vector<void*> done_;     ///< one event per staging buffer: its last DMA finished
    void* entry_ = nullptr;       ///< event: the caller's stream at entry (the hash stream waits on it)
    void* hash_stream_ = nullptr;
    void* hash_ws_ = nullptr;     ///< device hash workspace (grown on demand) + the u64 result / running hash at its end,
                                  ///< then the u32 fault word of the hash launches (sc_fnv1a64_async)
    uint64_t hash_ws_bytes_ = 0;
    uint64_t* hash_host_ = nullptr;   ///< pinned landing place of the device hash and its fault word
    /// The two words moved between the device and hash_host_: the hash, then the fault word (in the low half).
    static constexpr int kHashWords = 2;
    static uint32_t* fault_word(uint64_t* hash) { return reinterpret_cast<uint32_t*>(hash + 1); }
    HandoffCopyCrew* crew_ = nullptr;
    HandoffMoveStats last_{};
};

}  // namespace strata::core
