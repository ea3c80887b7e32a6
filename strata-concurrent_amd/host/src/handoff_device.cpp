// handoff_device.cpp - the device movers of the hand-off arena (see handoff_device.hpp).  Every device call goes
// through libsc_handoff.so's C-ABI (pinned and device memory, async copies, events, the device FNV-1a).
#include "strata/core/handoff_device.hpp"

#include "sc_handoff.h"

#include <algorithm>
#include <chrono>
#include <cstring>

namespace strata::core {

namespace {

constexpr uint64_t kEngineSeed = 1469598103934665603ull;

std::string abi_error(const char* what) { return std::string(what) + ": " + sc_last_error(); }

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace

// ================================ the copy crew ================================

HandoffCopyCrew::HandoffCopyCrew(int threads) {
    for (int i = 1; i < threads; ++i) workers_.emplace_back([this] { work(); });
}

HandoffCopyCrew::~HandoffCopyCrew() {
    {
        std::lock_guard<std::mutex> lk(mu_);
        stop_ = true;
    }
    wake_.notify_all();
    for (std::thread& t : workers_) t.join();
}

void HandoffCopyCrew::take_pieces() {
    for (;;) {
        uint64_t at, n;
        uint8_t* dst;
        const uint8_t* src;
        {
            std::lock_guard<std::mutex> lk(mu_);
            if (next_ >= n_) return;
            at = next_;
            n = std::min(piece_, n_ - at);
            next_ += n;
            dst = dst_;
            src = src_;
        }
        std::memcpy(dst + at, src + at, (size_t) n);
    }
}

void HandoffCopyCrew::work() {
    uint64_t seen = 0;
    for (;;) {
        {
            std::unique_lock<std::mutex> lk(mu_);
            wake_.wait(lk, [&] { return stop_ || round_ != seen; });
            if (stop_) return;
            seen = round_;
            ++busy_;   // counted before taking any piece, so copy() cannot return while one is being copied
        }
        take_pieces();
        {
            std::lock_guard<std::mutex> lk(mu_);
            if (--busy_ == 0) idle_.notify_all();
        }
    }
}

void HandoffCopyCrew::copy(void* dst, const void* src, uint64_t n) {
    if (n == 0) return;
    if (workers_.empty() || n < (2ull << 20)) {
        std::memcpy(dst, src, (size_t) n);
        return;
    }
    {
        std::lock_guard<std::mutex> lk(mu_);
        dst_ = static_cast<uint8_t*>(dst);
        src_ = static_cast<const uint8_t*>(src);
        n_ = n;
        // about four pieces per thread, 64 KiB multiples, at least 1 MiB
        const uint64_t share = n / (uint64_t) (4 * size());
        piece_ = std::max<uint64_t>(1ull << 20, (share + 65535) & ~65535ull);
        next_ = 0;
        ++round_;
    }
    wake_.notify_all();
    take_pieces();
    std::unique_lock<std::mutex> lk(mu_);
    idle_.wait(lk, [&] { return busy_ == 0 && next_ >= n_; });
}

// ================================ the mover ================================

HandoffMover::~HandoffMover() { release_(); }

void HandoffMover::release_() {
    delete crew_;
    crew_ = nullptr;
    for (void* e : done_) sc_event_destroy(e);
    for (void* p : stage_) sc_host_free(p);
    done_.clear();
    stage_.clear();
    if (entry_) sc_event_destroy(entry_);
    if (hash_stream_) sc_stream_destroy(hash_stream_);
    if (hash_ws_) sc_device_free(hash_ws_);
    if (hash_host_) sc_host_free(hash_host_);
    entry_ = hash_stream_ = hash_ws_ = nullptr;
    hash_host_ = nullptr;
    hash_ws_bytes_ = 0;
}

bool HandoffMover::init(const HandoffMoverConfig& cfg, std::string& err) {
    release_();
    if (cfg.chunk_bytes < 4096 || cfg.chunk_bytes % 4096 || cfg.chunk_bytes > (1ull << 30) || cfg.depth < 2 ||
        cfg.depth > 16 || cfg.threads < 1 || cfg.threads > 64) {
        err = "handoff mover: chunk_bytes must be a multiple of 4 KiB up to 1 GiB, depth 2..16, threads 1..64";
        return false;
    }
    cfg_ = cfg;
    for (int i = 0; i < cfg.depth; ++i) {
        void* p = nullptr;
        void* e = nullptr;
        if (sc_host_alloc(&p, cfg.chunk_bytes) != SC_OK) { err = abi_error("handoff mover staging"); release_(); return false; }
        stage_.push_back(p);
        if (sc_event_create(&e) != SC_OK) { err = abi_error("handoff mover event"); release_(); return false; }
        done_.push_back(e);
    }
    void* h = nullptr;
    if (sc_event_create(&entry_) != SC_OK || sc_stream_create(&hash_stream_) != SC_OK ||
        sc_host_alloc(&h, kHashWords * sizeof(uint64_t)) != SC_OK) {
        err = abi_error("handoff mover set-up");
        release_();
        return false;
    }
    hash_host_ = static_cast<uint64_t*>(h);
    crew_ = new HandoffCopyCrew(cfg.threads);
    return true;
}

/// The hash workspace, grown to serve inputs of `bytes` bytes, and the device words after it: the result (or the
/// running hash of a chained hash), then the launch's fault word.  Only called while nothing is queued on the hash
/// stream.
uint64_t* HandoffMover::hash_space_(uint64_t bytes, std::string& err) {
    const uint64_t need = (sc_fnv1a64_workspace_bytes(bytes) + 255) & ~255ull;
    if (need + 256 > hash_ws_bytes_) {
        if (hash_ws_) sc_device_free(hash_ws_);
        hash_ws_ = nullptr;
        hash_ws_bytes_ = 0;
        const uint64_t grow = std::max<uint64_t>(need + 256, 1ull << 20);
        if (sc_device_alloc(&hash_ws_, grow) != SC_OK) {
            err = abi_error("handoff mover hash workspace");
            last_.device_error = true;
            return nullptr;
        }
        hash_ws_bytes_ = grow;
    }
    return reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(hash_ws_) + hash_ws_bytes_ - 256);
}

/// Enqueue the device FNV-1a of `bytes` at `data` on the hash stream, after the work on `stream` so far; the result
/// lands in pinned memory (fetch_hash_ waits for it).
bool HandoffMover::hash_on_device_(const void* data, uint64_t bytes, void* stream, std::string& err) {
    uint64_t* dev_out = hash_space_(bytes, err);
    if (!dev_out) return false;
    if (sc_event_record(entry_, stream) != SC_OK || sc_stream_wait_event(hash_stream_, entry_) != SC_OK ||
        sc_fnv1a64_async(data, bytes, kEngineSeed, dev_out, fault_word(dev_out), hash_ws_, hash_ws_bytes_ - 256,
                         hash_stream_) != SC_OK ||
        sc_copy_async(hash_host_, dev_out, kHashWords * sizeof(uint64_t), hash_stream_) != SC_OK) {
        err = abi_error("handoff mover hash");
        last_.device_error = true;
        return false;
    }
    return true;
}

bool HandoffMover::fetch_hash_(uint64_t* out, std::string& err) {
    if (sc_stream_sync(hash_stream_) != SC_OK) {
        err = abi_error("handoff mover hash wait");
        last_.device_error = true;
        return false;
    }
    if (*fault_word(hash_host_)) {   // a wait of the hash kernel ran out: the word beside it is not the hash
        err = "handoff mover: the payload hash did not complete on the device (a look-back wait ran out)";
        last_.hash_fault = true;
        return false;
    }
    *out = *hash_host_;
    return true;
}

bool HandoffMover::write_from_device(HandoffArena& arena, const HandoffClaim& claim, const void* device_src,
                                     uint64_t bytes, void* stream, uint64_t* hash, std::string& err) {
    const auto t0 = std::chrono::steady_clock::now();
    last_ = HandoffMoveStats{};
    if (!ready()) { err = "handoff mover: not initialised"; return false; }
    if (bytes && !device_src) { err = "handoff mover: no device payload"; return false; }
    if (bytes > claim.capacity) {
        err = "handoff slot " + std::to_string(claim.index) + " holds " + std::to_string(claim.capacity) +
              " B and the payload is " + std::to_string(bytes) + " B";
        return false;
    }
    uint8_t* window = arena.claim_window(claim, err);
    if (!window) return false;
    if (hash) {
        if (bytes == 0) *hash = kEngineSeed;
        else if (!hash_on_device_(device_src, bytes, stream, err)) return false;
    }
    const uint64_t C = cfg_.chunk_bytes;
    const uint64_t n_chunks = (bytes + C - 1) / C;
    const uint64_t R = (uint64_t) cfg_.depth;
    const auto* src = static_cast<const uint8_t*>(device_src);
    auto enqueue = [&](uint64_t k) {
        const uint64_t len = std::min(C, bytes - k * C);
        return sc_copy_async(stage_[k % R], src + k * C, len, stream) == SC_OK &&
               sc_event_record(done_[k % R], stream) == SC_OK;
    };
    bool ok = true;
    uint64_t issued = 0;
    for (; issued < std::min(R, n_chunks) && ok; ++issued) ok = enqueue(issued);
    for (uint64_t k = 0; k < n_chunks && ok; ++k) {
        const auto tw = std::chrono::steady_clock::now();
        ok = sc_event_sync(done_[k % R]) == SC_OK;
        if (!ok) break;
        const auto tc = std::chrono::steady_clock::now();
        crew_->copy(window + k * C, stage_[k % R], std::min(C, bytes - k * C));
        last_.wait_ms += std::chrono::duration<double, std::milli>(tc - tw).count();
        last_.copy_ms += ms_since(tc);
        if (issued < n_chunks) ok = enqueue(issued++);
    }
    if (!ok) {
        err = abi_error("handoff mover device-to-slot copy");
        last_.device_error = true;
        sc_stream_sync(stream);
        if (hash) sc_stream_sync(hash_stream_);
        return false;
    }
    if (hash && bytes && !fetch_hash_(hash, err)) return false;
    last_.bytes = bytes;
    last_.ms = ms_since(t0);
    return true;
}

bool HandoffMover::publish_from_device(HandoffArena& arena, const HandoffClaim& claim, const void* device_src,
                                       uint64_t bytes, uint64_t tokens, void* stream, std::string& err) {
    uint64_t h = 0;
    const auto t0 = std::chrono::steady_clock::now();
    if (!write_from_device(arena, claim, device_src, bytes, stream, &h, err)) return false;
    if (!arena.publish(claim, tokens, bytes, h, err)) return false;
    last_.ms = ms_since(t0);
    return true;
}

bool HandoffMover::read_to_device(HandoffArena& arena, int index, uint64_t nonce, uint64_t client_id, void* device_dst,
                                  uint64_t dst_capacity, void* stream, bool verify, HandoffSlotInfo& info,
                                  std::string& err) {
    const auto t0 = std::chrono::steady_clock::now();
    last_ = HandoffMoveStats{};
    info = HandoffSlotInfo{};
    if (!ready()) { err = "handoff mover: not initialised"; return false; }
    const uint8_t* data = arena.read_window(index, nonce, client_id, info, err);
    if (!data) return false;
    const uint64_t bytes = info.payload_bytes;
    if (bytes > dst_capacity) {
        err = "handoff slot " + std::to_string(index) + " holds a " + std::to_string(bytes) +
              " B payload and the device buffer has room for " + std::to_string(dst_capacity) + " B";
        return false;
    }
    if (bytes && !device_dst) { err = "handoff mover: no device buffer"; return false; }
    const uint64_t C = cfg_.chunk_bytes;
    const uint64_t n_chunks = (bytes + C - 1) / C;
    const uint64_t R = (uint64_t) cfg_.depth;
    auto* dst = static_cast<uint8_t*>(device_dst);
    // with `verify`, each chunk is hashed on the hash stream as soon as its DMA is done, continuing the running hash
    // in device memory (seeded from pinned memory first), so the check ends a chunk's hash after the last copy
    uint64_t* state = nullptr;
    const bool chain = verify && bytes != 0;
    if (chain) {
        state = hash_space_(std::min(C, bytes), err);
        if (!state) return false;
        hash_host_[0] = kEngineSeed;   // the running hash, and a clear fault word for the chain to or into
        hash_host_[1] = 0;
        if (sc_copy_async(state, hash_host_, kHashWords * sizeof(uint64_t), hash_stream_) != SC_OK) {
            err = abi_error("handoff mover hash seed");
            last_.device_error = true;
            return false;
        }
    }
    last_.wrote_device = bytes != 0;
    bool ok = true;
    for (uint64_t k = 0; k < n_chunks && ok; ++k) {
        const auto tw = std::chrono::steady_clock::now();
        if (k >= R) ok = sc_event_sync(done_[k % R]) == SC_OK;   // the DMA that last read this staging buffer is done
        if (!ok) break;
        const auto tc = std::chrono::steady_clock::now();
        const uint64_t len = std::min(C, bytes - k * C);
        crew_->copy(stage_[k % R], data + k * C, len);
        last_.wait_ms += std::chrono::duration<double, std::milli>(tc - tw).count();
        last_.copy_ms += ms_since(tc);
        ok = sc_copy_async(dst + k * C, stage_[k % R], len, stream) == SC_OK &&
             sc_event_record(done_[k % R], stream) == SC_OK;
        if (ok && chain)
            ok = sc_stream_wait_event(hash_stream_, done_[k % R]) == SC_OK &&
                 sc_fnv1a64_chain_async(dst + k * C, len, state, fault_word(state), hash_ws_, hash_ws_bytes_ - 256,
                                        hash_stream_) == SC_OK;
    }
    const auto tf = std::chrono::steady_clock::now();
    if (ok) ok = sc_stream_sync(stream) == SC_OK;
    last_.wait_ms += ms_since(tf);
    if (!ok) {
        err = abi_error("handoff mover slot-to-device copy");
        last_.device_error = true;
        sc_stream_sync(stream);
        if (chain) sc_stream_sync(hash_stream_);   // nothing may still read the caller's buffer after we return
        return false;
    }
    // the writer may only reuse the slot after our ACK, or after its lease: a publication that moved while we copied
    // is refused rather than mounted
    HandoffSlotInfo after;
    if (!arena.slot_info(index, after) || after.state != kHandoffReady || after.nonce != nonce ||
        after.payload_bytes != bytes || after.payload_hash != info.payload_hash || after.published_ms != info.published_ms) {
        err = "handoff slot " + std::to_string(index) + " was released or reclaimed while it was read";
        if (chain) sc_stream_sync(hash_stream_);
        return false;
    }
    if (verify) {
        const auto th = std::chrono::steady_clock::now();
        uint64_t h = kEngineSeed;
        if (chain) {
            if (sc_copy_async(hash_host_, state, kHashWords * sizeof(uint64_t), hash_stream_) != SC_OK) {
                err = abi_error("handoff mover hash");
                last_.device_error = true;
                sc_stream_sync(hash_stream_);
                return false;
            }
            if (!fetch_hash_(&h, err)) return false;
        }
        last_.hash_ms = ms_since(th);
        if (h != info.payload_hash) {
            char buf[160];
            std::snprintf(buf, sizeof buf, "handoff slot %d: the payload hash is %016llx but the slot records %016llx",
                          index, (unsigned long long) h, (unsigned long long) info.payload_hash);
            err = buf;
            return false;
        }
    }
    last_.bytes = bytes;
    last_.ms = ms_since(t0);
    return true;
}

}  // namespace strata::core
